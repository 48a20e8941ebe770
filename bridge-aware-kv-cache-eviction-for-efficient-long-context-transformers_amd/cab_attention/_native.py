"""ctypes binding of libcab_hip.so (the C ABI declared in include/cab_hip.h).

There is exactly one implementation of every stage: the HIP kernels in this
library. Nothing here falls back to another code path: a missing library, a
CPU tensor or an ABI error raises.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
import threading

import torch

# The in-tree build; CAB_HIP_LIB names another build of the same library (the
# host-sanitized one that tests/test_host_sanitizers.py runs the ABI checks on).
LIB_PATH = pathlib.Path(os.environ.get("CAB_HIP_LIB") or
                        pathlib.Path(__file__).resolve().with_name("libcab_hip.so"))
ABI_VERSION = 10

CAB_OK, CAB_EINVAL, CAB_EDTYPE, CAB_ESHAPE, CAB_EWORKSPACE, CAB_EHIP = range(6)
CAB_F32, CAB_F16, CAB_BF16 = 0, 1, 2
NORMALIZATIONS = {"none": 0, "minmax": 1}
FORMULAS = {"additive": 0, "multiplicative": 1, "augmented": 2}

# Every symbol the header declares, with its ctypes signature.
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_ptr = ctypes.c_void_p
_f32 = ctypes.c_float
_i64x4 = ctypes.POINTER(ctypes.c_int64)
SIGNATURES = {
    "cab_abi_version": (ctypes.c_int, []),
    "cab_last_error": (ctypes.c_char_p, []),
    "cab_coarsen_maxl2": (ctypes.c_int, [_ptr, _ptr, ctypes.c_int, _i64, _i64, _i64, _i64,
                                         _i64x4, _i64x4, _i32, _ptr, _ptr, _ptr, _ptr, _ptr]),
    "cab_block_frc_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, ctypes.c_int,
                                                        ctypes.c_int]),
    "cab_block_frc": (ctypes.c_int, [_ptr, _ptr, ctypes.c_int, _i64, _i64, _i64, _i64, _f32, _f32,
                                     _f32, ctypes.c_int, ctypes.c_int, _ptr, _ptr, _ptr, _ptr,
                                     ctypes.c_size_t, _ptr]),
    "cab_block_topk": (ctypes.c_int, [_ptr, _i64, _i64, _i64, _i32, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, _ptr, _ptr, _ptr, _ptr]),
    "cab_block_topk_hybrid": (ctypes.c_int, [_ptr, _ptr, _i64, _i64, _i64, _i32, _i32, ctypes.c_int,
                                             ctypes.c_int, ctypes.c_int, _ptr, _ptr, _ptr, _ptr]),
    "cab_block_sparse_attn_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, _i64, _i64, _i64, _i64,
                                                                _i32]),
    "cab_block_sparse_attn_workspace_bytes_k": (ctypes.c_size_t, [ctypes.c_int, _i64, _i64, _i64,
                                                                  _i64, _i32, _i32]),
    "cab_block_sparse_attn_fwd": (ctypes.c_int, [_ptr, _ptr, _ptr, ctypes.c_int, _i64, _i64, _i64,
                                                 _i64, _i64x4, _i64x4, _i64x4, _i64x4, _i32, _ptr,
                                                 _ptr, _i32, _f32, ctypes.c_int, _ptr, _ptr, _ptr,
                                                 ctypes.c_size_t, _ptr]),
    "cab_block_sparse_attn_pack_v": (ctypes.c_int, [_ptr, ctypes.c_int, _i64, _i64, _i64, _i64,
                                                    _i64x4, _i32, _ptr, ctypes.c_size_t, _ptr]),
    "cab_block_sparse_attn_fwd_packed": (ctypes.c_int, [_ptr, _ptr, _ptr, ctypes.c_int, _i64, _i64,
                                                        _i64, _i64, _i64x4, _i64x4, _i64x4, _i32,
                                                        _ptr, _ptr, _i32, _f32, ctypes.c_int, _ptr,
                                                        _ptr, ctypes.c_size_t, _ptr]),
    "cab_flash_attn_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, _i64, _i64, _i64, _i64]),
    "cab_flash_attn_fwd": (ctypes.c_int, [_ptr, _ptr, _ptr, ctypes.c_int, _i64, _i64, _i64, _i64,
                                          _i64, _i64, _i64x4, _i64x4, _i64x4, _i64x4, _f32,
                                          ctypes.c_int, _ptr, _ptr, _ptr, ctypes.c_size_t, _ptr]),
    "cab_attn_key_scores": (ctypes.c_int, [_ptr, _ptr, _ptr, ctypes.c_int, _i64, _i64, _i64, _i64,
                                           _i64, _i64, _i64x4, _i64x4, _f32, ctypes.c_int, _ptr,
                                           _i64x4, ctypes.c_int, _ptr]),
    "cab_evict_select_workspace_bytes": (ctypes.c_size_t, [_i64]),
    "cab_evict_select": (ctypes.c_int, [_ptr, _i64, _ptr, _i64, _i32, _i32, _i32, ctypes.c_int,
                                        ctypes.c_int, _ptr, _ptr, _ptr, _ptr, ctypes.c_size_t,
                                        _ptr]),
    "cab_evict_select_noalloc": (ctypes.c_int, [_ptr, _i64, _ptr, _i64, _i32, _i32, _i32,
                                                ctypes.c_int, ctypes.c_int, _ptr, _ptr, _ptr,
                                                _ptr]),
    "cab_evict_connectivity": (ctypes.c_int, [_ptr, _i64, _i64, _ptr, _ptr, _ptr]),
    "cab_kv_gather": (ctypes.c_int, [ctypes.POINTER(_ptr), ctypes.POINTER(_ptr), _i32, _i64, _i64,
                                     _i64, _i64, _i64x4, _i64x4, _ptr, _i64, _ptr]),
    "cab_token_frc": (ctypes.c_int, [_ptr, ctypes.c_int, _i64, _i64, _ptr, _ptr, _ptr, _ptr]),
    "cab_attention_symmetrize": (ctypes.c_int, [_ptr, ctypes.c_int, _i64, _i64, _i64, _i64, _i64x4,
                                                _ptr, _i64, _ptr]),
    "cab_token_frc_keys_workspace_bytes": (ctypes.c_size_t, [_i64, _i64]),
    "cab_token_frc_from_keys": (ctypes.c_int, [_ptr, ctypes.c_int, _i64, _i64, _i64, _i64, _i64x4,
                                               _ptr, _ptr, _ptr, _ptr, _ptr, ctypes.c_size_t,
                                               _ptr]),
}

_lock = threading.Lock()
_lib = None


class CabError(RuntimeError):
    """A libcab_hip call failed (status code + message from cab_last_error)."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.status = status


def load() -> ctypes.CDLL:
    """Open libcab_hip.so once (torch must be imported first: the library binds
    to the HIP runtime torch already loaded)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                    "(hipcc, gfx950). There is no fallback implementation.")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            ver = lib.cab_abi_version()
            if ver != ABI_VERSION:
                raise RuntimeError(f"libcab_hip ABI version {ver}, expected {ABI_VERSION}")
            _lib = lib
    return _lib


def check(fn: str, status: int) -> None:
    if status != CAB_OK:
        msg = load().cab_last_error().decode(errors="replace")
        if status in (CAB_EINVAL, CAB_EDTYPE, CAB_ESHAPE, CAB_EWORKSPACE):
            raise ValueError(f"{fn}: {msg} (status {status})")
        raise CabError(fn, status, msg)


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return CAB_F32
    if t.dtype == torch.float16:
        return CAB_F16
    if t.dtype == torch.bfloat16:
        return CAB_BF16
    raise TypeError(f"unsupported dtype {t.dtype}; expected float32, float16 or bfloat16")


def require_device(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected a torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise RuntimeError(
                "CAB-Attention kernels run on the GPU only (HIP, gfx950); got a tensor on "
                f"{t.device}. Move inputs to a cuda device.")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def strides4(t: torch.Tensor):
    arr = (ctypes.c_int64 * 4)(*t.stride())
    return arr


def aligned_rows(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` or a contiguous copy so that its last dim is contiguous and
    rows start on 16-byte boundaries (what the kernels' vector loads need)."""
    def ok(x):
        es = x.element_size()
        return (x.stride(-1) == 1 and x.data_ptr() % 16 == 0
                and all((s * es) % 16 == 0 for s in x.stride()[:-1]))
    if ok(t):
        return t
    t = t.contiguous()
    return t if ok(t) else t.clone()


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t):
    return None if t is None else t.data_ptr()

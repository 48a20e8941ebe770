"""Token-level Forman-Ricci curvature on the GPU.

Same names, arguments and return values as the reference's
``cab_attention/kernels/frc_triton.py`` (:166-314): ``compute_frc``,
``compute_frc_triton``, ``compute_frc_pytorch``,
``compute_node_strengths_triton`` and ``compute_triangles_triton``. All of
them run the HIP kernels of ``cab_token_frc`` (the ``_pytorch`` and
``_triton`` names are kept for callers; there is no CPU path).

For an attention graph ``A [N, N]`` (frc_triton.py:79-83, :138-160, :279-291):
``S = A.sum(1)``, ``T = (A @ A).sum(1)``, ``F = 4 S - 2 S + 3 T``. Because
``(A @ A).sum(1) = A @ S``, the kernels make two passes over A instead of
forming ``A @ A``.

``frc_from_keys`` and ``symmetrize_attention`` are the device halves of
``FRCTracker.compute_from_keys`` / ``compute_from_attention``
(scoring/frc.py:36-136).
"""

from __future__ import annotations

import torch

from .. import _native as nat


def token_frc(attention: torch.Tensor, return_parts: bool = False):
    """fp32 curvature ``F [N]`` of ``attention [N, N]`` (fp32, fp16 or bf16,
    last dim contiguous); with ``return_parts``, ``(S, T, F)``."""
    if attention.dim() != 2 or attention.shape[0] != attention.shape[1]:
        raise ValueError(f"attention must be a square [N, N] matrix; got {tuple(attention.shape)}")
    dev = nat.require_device(attention)
    dt = nat.dtype_code(attention)
    n = attention.shape[0]
    a = attention if (attention.stride(1) == 1 and attention.stride(0) >= n) else attention.contiguous()
    s = torch.empty(n, dtype=torch.float32, device=dev)
    t = torch.empty(n, dtype=torch.float32, device=dev)
    f = torch.empty(n, dtype=torch.float32, device=dev)
    lib = nat.load()
    with torch.cuda.device(dev):
        st = lib.cab_token_frc(a.data_ptr(), dt, n, a.stride(0) if n else 0, s.data_ptr(),
                               t.data_ptr(), f.data_ptr(), nat.stream_ptr(dev))
    nat.check("cab_token_frc", st)
    return (s, t, f) if return_parts else f


def compute_node_strengths_triton(attention: torch.Tensor) -> torch.Tensor:
    """``S_i = sum_j A_ij`` in the input dtype (frc_triton.py:167-193)."""
    return token_frc(attention, return_parts=True)[0].to(attention.dtype)


def compute_triangles_triton(attention: torch.Tensor) -> torch.Tensor:
    """``T_i = sum_j sum_k A_ij A_jk`` in the input dtype (frc_triton.py:196-222)."""
    return token_frc(attention, return_parts=True)[1].to(attention.dtype)


def compute_frc_triton(attention: torch.Tensor) -> torch.Tensor:
    """``F = 4 S - 2 S + 3 T`` in the input dtype (frc_triton.py:225-265)."""
    return token_frc(attention).to(attention.dtype)


def compute_frc_pytorch(attention: torch.Tensor) -> torch.Tensor:
    """The reference's torch formulation (frc_triton.py:269-293); here the same
    HIP kernels (GPU tensors only)."""
    return token_frc(attention).to(attention.dtype)


def compute_frc(attention: torch.Tensor, use_triton: bool = True) -> torch.Tensor:
    """Token FRC scores ``[N]`` (frc_triton.py:296-314). ``use_triton`` is
    accepted and ignored; a CPU tensor raises instead of falling back."""
    return token_frc(attention).to(attention.dtype)


def symmetrize_attention(attention: torch.Tensor) -> torch.Tensor:
    """``(agg.T + agg) / 2`` with ``agg = attention.mean(dim=(0, 1))`` for
    ``attention [B, H, N_q, N_k]`` (torch broadcasting: N_q == N_k, or one of
    them 1), as fp32 ``[n, n]`` (``cab_attention_symmetrize``)."""
    if attention.dim() != 4:
        raise ValueError("attention must be [B, H, N_q, N_kv]")
    B, H, nq, nk = attention.shape
    if not (nq == nk or nq == 1 or nk == 1):
        raise ValueError(f"attention_agg.T + attention_agg needs N_q == N_kv or a size-1 dim; "
                         f"got N_q={nq}, N_kv={nk}")
    dev = nat.require_device(attention)
    dt = nat.dtype_code(attention)
    n = max(nq, nk)
    out = torch.empty((n, n), dtype=torch.float32, device=dev)
    lib = nat.load()
    with torch.cuda.device(dev):
        st = lib.cab_attention_symmetrize(attention.data_ptr(), dt, B, H, nq, nk,
                                          nat.strides4(attention), out.data_ptr(), n,
                                          nat.stream_ptr(dev))
    nat.check("cab_attention_symmetrize", st)
    return out


def frc_from_keys(keys: torch.Tensor, return_parts: bool = False):
    """Token curvature of the key-similarity graph of ``keys [B, H, N, D]``
    (D <= 256) without forming it (``cab_token_frc_from_keys``): fp32
    ``F [N]``, or with ``return_parts`` a dict of ``strengths``,
    ``triangles``, ``row_sums`` (sum_j relu(kn_i . kn_j)) and ``frc``."""
    if keys.dim() != 4:
        raise ValueError("keys must be [B, H, N, D]")
    B, H, N, D = keys.shape
    if D > 256:
        raise ValueError(f"head dim {D} above 256")
    dev = nat.require_device(keys)
    dt = nat.dtype_code(keys)
    lib = nat.load()
    f = torch.empty(N, dtype=torch.float32, device=dev)
    parts = None
    if return_parts:
        parts = {k: torch.empty(N, dtype=torch.float32, device=dev)
                 for k in ("strengths", "triangles", "row_sums")}
    if N == 0 or B * H == 0:
        if B * H == 0 and N > 0:
            raise ValueError("keys has no (batch, head) slices to average")
        return ({**parts, "frc": f} if return_parts else f)
    wbytes = int(lib.cab_token_frc_keys_workspace_bytes(N, D))
    ws = torch.empty(wbytes, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        st = lib.cab_token_frc_from_keys(
            keys.data_ptr(), dt, B, H, N, D, nat.strides4(keys),
            nat.ptr(parts and parts["strengths"]), nat.ptr(parts and parts["triangles"]),
            nat.ptr(parts and parts["row_sums"]), f.data_ptr(), ws.data_ptr(), ws.numel(),
            nat.stream_ptr(dev))
    nat.check("cab_token_frc_from_keys", st)
    return {**parts, "frc": f} if return_parts else f

"""C-ABI boundary checks that need no GPU: the library loads, exports every
symbol include/cab_hip.h declares, and rejects bad arguments with the
documented status codes before anything is launched."""

import ctypes
import re
import subprocess

import pytest
import torch

from conftest import PKG, ROOT

from cab_attention import _native as nat

HEADER = ROOT / "include" / "cab_hip.h"


@pytest.fixture(scope="module")
def lib():
    if not nat.LIB_PATH.exists():
        from cab_attention import _build
        _build.build(verbose=False)
    return nat.load()


def declared_symbols():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)  # drop comments
    return sorted(set(re.findall(r"\b(cab_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_hot_path():
    syms = declared_symbols()
    for name in ("cab_abi_version", "cab_last_error", "cab_coarsen_maxl2",
                 "cab_block_frc_workspace_bytes", "cab_block_frc", "cab_block_topk",
                 "cab_block_sparse_attn_workspace_bytes", "cab_block_sparse_attn_fwd",
                 "cab_block_sparse_attn_pack_v", "cab_block_sparse_attn_fwd_packed",
                 "cab_block_topk_hybrid", "cab_flash_attn_workspace_bytes",
                 "cab_flash_attn_fwd", "cab_attn_key_scores", "cab_evict_select",
                 "cab_evict_connectivity", "cab_kv_gather", "cab_token_frc",
                 "cab_evict_select_workspace_bytes",
                 "cab_attention_symmetrize", "cab_token_frc_keys_workspace_bytes",
                 "cab_token_frc_from_keys"):
        assert name in syms
    assert set(syms) == set(nat.SIGNATURES), "ctypes table and header disagree"


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(nat.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s(cab_\w+)$", out, re.M))
    missing = set(declared_symbols()) - exported
    assert not missing, f"not exported: {missing}"
    assert lib.cab_abi_version() == nat.ABI_VERSION


def _s4(*v):
    return (ctypes.c_int64 * 4)(*v)


FAKE = 0x7f0000000000  # 16-byte aligned address that is never dereferenced


def test_coarsen_validation(lib):
    st = _s4(8 * 64 * 128, 64 * 128, 128, 1)
    call = lambda **kw: lib.cab_coarsen_maxl2(
        kw.get("q", FAKE), FAKE, kw.get("dt", nat.CAB_BF16), kw.get("B", 1), 8, 64,
        kw.get("D", 128), kw.get("qs", st), st, kw.get("bs", 64), FAKE, FAKE, None, None, None)
    assert call(dt=7) == nat.CAB_EDTYPE
    assert call(D=12) == nat.CAB_ESHAPE
    assert call(D=1024) == nat.CAB_ESHAPE
    assert call(bs=0) == nat.CAB_EINVAL
    assert call(q=None) == nat.CAB_EINVAL
    assert call(q=FAKE + 2) == nat.CAB_ESHAPE
    assert call(qs=_s4(1, 1, 128, 2)) == nat.CAB_ESHAPE
    assert call(qs=_s4(8 * 64 * 128, 64 * 128, 12, 1)) == nat.CAB_ESHAPE
    assert b"stride" in lib.cab_last_error()
    assert call(B=0) == nat.CAB_OK  # empty batch: nothing to launch


def test_frc_validation(lib):
    need = lib.cab_block_frc_workspace_bytes(2, 8, 2000, 128, 1, 0)
    assert need >= 4 * 16 * 2048 * 2048 * 2
    call = lambda **kw: lib.cab_block_frc(
        FAKE, FAKE, kw.get("dt", nat.CAB_BF16), 1, 1, kw.get("M", 64), kw.get("D", 128), 0.1,
        kw.get("temp", 1.0), 0.5, kw.get("norm", 1), kw.get("form", 0), FAKE, None, None,
        kw.get("ws", FAKE), kw.get("wsb", 1 << 40), None)
    assert call(dt=5) == nat.CAB_EDTYPE
    assert call(D=100) == nat.CAB_ESHAPE
    assert call(norm=2) == nat.CAB_EINVAL
    assert call(form=3) == nat.CAB_EINVAL
    assert call(temp=0.0) == nat.CAB_EINVAL
    assert call(wsb=16) == nat.CAB_EWORKSPACE
    assert call(ws=None) == nat.CAB_EWORKSPACE
    assert call(ws=FAKE + 16) == nat.CAB_EWORKSPACE
    assert call(M=40000) == nat.CAB_ESHAPE
    assert call(M=0) == nat.CAB_OK


def test_topk_validation(lib):
    call = lambda **kw: lib.cab_block_topk(FAKE, 1, 1, kw.get("M", 64), kw.get("k", 3), 0, 1, 0,
                                           FAKE, FAKE, None, None)
    assert call(k=0) == nat.CAB_EINVAL
    assert call(k=65) == nat.CAB_EINVAL
    assert call(M=32769, k=3) == nat.CAB_ESHAPE
    assert call(M=0) == nat.CAB_OK
    hyb = lambda **kw: lib.cab_block_topk_hybrid(FAKE, kw.get("mag", FAKE), 1, 1, 64, 3,
                                                 kw.get("kmag", 1), 1, 1, 0, FAKE, FAKE, None, None)
    assert hyb(kmag=4) == nat.CAB_EINVAL
    assert hyb(kmag=-1) == nat.CAB_EINVAL
    assert hyb(mag=None) == nat.CAB_EINVAL


def test_attention_validation(lib):
    ws = lib.cab_block_sparse_attn_workspace_bytes
    assert ws(nat.CAB_BF16, 1, 8, 65, 128, 64) == 8 * 2 * 16384
    assert ws(nat.CAB_F16, 1, 8, 65, 128, 64) == 8 * 2 * 16384
    assert ws(nat.CAB_F32, 1, 8, 65, 128, 64) == 8 * 2 * 65536  # split K and V^T images
    assert ws(nat.CAB_BF16, 1, 8, 64, 64, 64) == 8 * 8192   # head dim 64: 8 KB tiles
    assert ws(nat.CAB_F32, 1, 8, 64, 64, 64) == 8 * 32768
    assert ws(nat.CAB_BF16, 1, 8, 64, 96, 64) == 0
    assert ws(7, 1, 8, 64, 128, 64) == 0
    st = _s4(8 * 64 * 128, 64 * 128, 128, 1)
    call = lambda **kw: lib.cab_block_sparse_attn_fwd(
        FAKE, FAKE, FAKE, kw.get("dt", nat.CAB_BF16), 1, 8, 64, kw.get("D", 128), st, st, st,
        kw.get("os", st), kw.get("bs", 64), FAKE, FAKE, kw.get("kmax", 3), kw.get("scale", 0.088),
        1, FAKE, None, kw.get("ws", FAKE), kw.get("wsb", 1 << 30), None)
    assert call(dt=nat.CAB_F32 + 9) == nat.CAB_EDTYPE
    # fp32: rows must stay 16-byte aligned at 4 bytes per element and the
    # workspace must hold the 64 KB split images
    st2 = _s4(8 * 64 * 130, 64 * 130, 130, 1)  # 260-byte bf16 rows (ok), 520-byte fp32 rows (not)
    assert call(dt=nat.CAB_F32, os=st2) == nat.CAB_ESHAPE
    assert call(dt=nat.CAB_F32, wsb=8 * 65536 - 1) == nat.CAB_EWORKSPACE
    assert call(D=96) == nat.CAB_ESHAPE
    assert call(bs=48) == nat.CAB_ESHAPE
    assert call(bs=512) == nat.CAB_ESHAPE
    # other block sizes: lists over 64-token tiles in the workspace after the
    # packed V (256-byte aligned parts): idx [BH, M64, K64] int32, counts
    # [BH, M64] int32 and, below 64, sub-tile masks [BH, M64, K64] uint64
    wk = lib.cab_block_sparse_attn_workspace_bytes_k
    base = 8 * 16384  # N = 64: one 64-token block per head
    rup = lambda x: -(-x // 256) * 256
    assert wk(nat.CAB_BF16, 1, 8, 64, 128, 64, 3) == base
    assert wk(nat.CAB_BF16, 1, 8, 64, 128, 128, 3) == base + rup(8 * 6 * 4) + rup(8 * 4)
    assert wk(nat.CAB_BF16, 1, 8, 64, 128, 16, 3) == base + rup(8 * 12 * 4) + rup(8 * 4) + 8 * 12 * 8
    assert wk(nat.CAB_BF16, 1, 8, 64, 128, 48, 3) == 0 and wk(nat.CAB_BF16, 1, 8, 64, 128, 16, 0) == 0
    assert call(bs=16, wsb=wk(nat.CAB_BF16, 1, 8, 64, 128, 16, 3) - 1) == nat.CAB_EWORKSPACE
    assert call(bs=128, wsb=base) == nat.CAB_EWORKSPACE
    assert call(bs=8, kmax=513) == nat.CAB_ESHAPE  # 513 * 8 merged entries > 4096
    assert call(kmax=0) == nat.CAB_EINVAL
    assert call(scale=-0.1) == nat.CAB_EINVAL
    assert call(os=_s4(1, 1, 1, 3)) == nat.CAB_ESHAPE
    assert call(wsb=1024) == nat.CAB_EWORKSPACE
    assert call(ws=None) == nat.CAB_EWORKSPACE
    pack = lambda **kw: lib.cab_block_sparse_attn_pack_v(
        kw.get("v", FAKE), nat.CAB_BF16, 1, 8, 64, kw.get("D", 128), st, 64, FAKE,
        kw.get("wsb", 1 << 30), None)
    assert pack(D=96) == nat.CAB_ESHAPE
    assert pack(v=None) == nat.CAB_EINVAL
    assert pack(wsb=100) == nat.CAB_EWORKSPACE
    assert lib.cab_block_sparse_attn_pack_v(FAKE, nat.CAB_F32, 1, 8, 64, 128, st, 64, FAKE,
                                            1 << 30, None) == nat.CAB_EDTYPE
    packed = lambda **kw: lib.cab_block_sparse_attn_fwd_packed(
        FAKE, FAKE, kw.get("vt", FAKE), nat.CAB_BF16, 1, 8, 64, 128, st, st, st, 64, FAKE, FAKE,
        kw.get("kmax", 3), 0.088, 1, FAKE, None, kw.get("vtb", 1 << 30), None)
    assert packed(kmax=0) == nat.CAB_EINVAL
    assert packed(vt=None) == nat.CAB_EWORKSPACE
    assert packed(vtb=8 * 16384 - 1) == nat.CAB_EWORKSPACE
    assert lib.cab_block_sparse_attn_fwd_packed(
        FAKE, FAKE, FAKE, nat.CAB_F32, 1, 8, 64, 128, st, st, st, 64, FAKE, FAKE, 3, 0.088, 1,
        FAKE, None, 1 << 30, None) == nat.CAB_EDTYPE


def test_python_layer_refuses_cpu_tensors(lib):
    from cab_attention.kernels import (block_sparse_attention, coarsen_qk_max_l2,
                                       compute_block_frc, generate_block_mask)
    x = torch.randn(1, 1, 64, 128)
    with pytest.raises(RuntimeError, match="GPU only"):
        coarsen_qk_max_l2(x, x, 64)
    with pytest.raises(RuntimeError, match="GPU only"):
        compute_block_frc(x, x)
    with pytest.raises(RuntimeError, match="GPU only"):
        generate_block_mask(torch.randn(1, 1, 4, 4), 0.5)
    idx = torch.zeros(1, 1, 1, 1, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU only"):
        block_sparse_attention(x, x, x, idx, idx[..., 0], 64)


def test_missing_library_fails_loudly(tmp_path):
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "import torch\n"
        "from cab_attention import _native as n\n"
        "n.LIB_PATH = n.LIB_PATH.with_name('absent.so')\n"
        "try:\n    n.load()\nexcept RuntimeError as e:\n    print('RAISED', e)\n" % str(PKG))
    out = subprocess.run(["python", "-c", code], capture_output=True, text=True, timeout=300)
    assert "RAISED" in out.stdout and "no fallback" in out.stdout


def test_module_contract_on_host():
    from cab_attention import CABAttention, CoarseCurvaturePredictor
    p = CoarseCurvaturePredictor(block_size=64, sparsity=0.95, lambda_redundancy=0.5,
                                 use_triton=False)
    assert p.block_size == 64 and p.sparsity == 0.95
    f = p.estimate_flops(131072, 128)
    assert f["M"] == 2048 and f["triangles"] == 2 * 2048 ** 3
    assert p.keep_per_row(128000) == 100
    a = CABAttention(dim=512, num_heads=8, block_size=64, sparsity=0.95)
    assert a.num_heads == 8 and a.predictor.block_size == 64
    assert a.predictor.sparsity == 0.95
    with pytest.raises(ValueError):
        CABAttention(dim=500, num_heads=8)
    # the executor runs head dims 64 and 128 and block sizes 8 ... 256: others
    # are rejected at construction, not in forward
    CABAttention(dim=1024, num_heads=8)
    for bs in (8, 16, 32, 128, 256):
        assert CABAttention(dim=512, num_heads=8, block_size=bs).predictor.block_size == bs
    with pytest.raises(ValueError, match="head_dim"):
        CABAttention(dim=768, num_heads=8)
    with pytest.raises(ValueError, match="block_size"):
        CABAttention(dim=512, num_heads=8, block_size=48)
    with pytest.raises(ValueError):
        CoarseCurvaturePredictor(sparsity=1.5)


def test_dense_attention_validation(lib):
    """cab_flash_attn_fwd / cab_attn_key_scores refuse bad shapes, dtypes,
    head groupings, scales and workspaces before any launch."""
    ws = lib.cab_flash_attn_workspace_bytes
    assert ws(nat.CAB_BF16, 1, 2, 65, 128) == 2 * 2 * 16384
    assert ws(nat.CAB_F32, 1, 2, 65, 128) == 2 * 2 * 65536
    assert ws(nat.CAB_BF16, 1, 2, 65, 64) == 2 * 2 * 8192
    assert ws(nat.CAB_BF16, 1, 2, 65, 80) == 0
    st = _s4(8 * 64 * 128, 64 * 128, 128, 1)
    fwd = lambda **kw: lib.cab_flash_attn_fwd(
        FAKE, FAKE, FAKE, kw.get("dt", nat.CAB_BF16), 1, kw.get("H", 8), kw.get("Hkv", 2), 64, 64,
        kw.get("D", 128), st, st, st, kw.get("os", st), kw.get("scale", 0.088), 1, FAKE, None,
        kw.get("ws", FAKE), kw.get("wsb", 1 << 30), None)
    assert fwd(dt=9) == nat.CAB_EDTYPE
    assert fwd(D=80) == nat.CAB_ESHAPE
    assert fwd(H=8, Hkv=3) == nat.CAB_ESHAPE
    assert fwd(scale=0.0) == nat.CAB_EINVAL
    assert fwd(os=_s4(1, 1, 1, 3)) == nat.CAB_ESHAPE
    assert fwd(wsb=2 * 16384 - 1) == nat.CAB_EWORKSPACE
    assert fwd(ws=None) == nat.CAB_EWORKSPACE
    ss = _s4(8 * 64, 64, 1, 0)
    sc = lambda **kw: lib.cab_attn_key_scores(
        FAKE, FAKE, kw.get("lse", FAKE), kw.get("dt", nat.CAB_BF16), 1, 8, 2, 64, 64, 128,
        kw.get("st", st), kw.get("st", st), 0.088, 1, kw.get("scores", FAKE), kw.get("ss", ss), 0, None)
    assert sc(dt=9) == nat.CAB_EDTYPE
    # fp32 is accepted; its rows must stay 16-byte aligned at 4 bytes per
    # element (130-element rows are 260 bytes in bf16, 520 in fp32)
    st130 = _s4(8 * 64 * 130, 64 * 130, 130, 1)
    assert sc(dt=nat.CAB_F32, st=st130) == nat.CAB_ESHAPE
    assert b"16-byte" in lib.cab_last_error()
    assert sc(lse=None) == nat.CAB_EINVAL
    assert sc(scores=None) == nat.CAB_EINVAL
    assert sc(ss=_s4(8 * 64, 64, 2, 0)) == nat.CAB_ESHAPE
    # 16 query rows are staged through one buffer descriptor: a token stride
    # of 2^27 bytes or more (2^26 bf16 elements) is refused
    assert sc(st=_s4(0, 0, 1 << 26, 1)) == nat.CAB_ESHAPE
    assert b"2^27" in lib.cab_last_error()


def test_eviction_validation(lib):
    sel = lambda **kw: lib.cab_evict_select(
        kw.get("scores", FAKE), kw.get("ns", 10), None, kw.get("n", 10), kw.get("local", 2),
        kw.get("imp", 3), kw.get("br", 2), 1, kw.get("mode", 1), kw.get("keep", FAKE), FAKE, None,
        kw.get("ws", None), kw.get("wsb", 0), None)
    big = 1 << 15  # from here on a workspace is required
    wsb = lib.cab_evict_select_workspace_bytes(big)
    assert wsb > 0 and lib.cab_evict_select_workspace_bytes((1 << 20) + 1) == 0
    assert sel(n=big, ns=big) == nat.CAB_EWORKSPACE
    assert sel(n=big, ns=big, ws=FAKE, wsb=wsb - 1) == nat.CAB_EWORKSPACE
    assert sel(n=big, ns=big, ws=FAKE + 16, wsb=wsb) == nat.CAB_EWORKSPACE
    assert sel(n=(1 << 20) + 1) == nat.CAB_ESHAPE
    # the no-allocation variant: same checks, its scratch holds 2^20 positions
    noalloc = lambda **kw: lib.cab_evict_select_noalloc(
        FAKE, 10, None, kw.get("n", 100), kw.get("loc", 1), 2, 3, 1, kw.get("mode", 1), FAKE,
        FAKE, None, None)
    assert noalloc(n=(1 << 20) + 1) == nat.CAB_ESHAPE
    assert b"scratch" in lib.cab_last_error()
    assert noalloc(loc=101) == nat.CAB_EINVAL
    assert noalloc(mode=4) == nat.CAB_EINVAL
    assert sel(local=11) == nat.CAB_EINVAL
    assert sel(imp=-1) == nat.CAB_EINVAL
    assert sel(mode=4) == nat.CAB_EINVAL
    assert sel(mode=2) == nat.CAB_EINVAL  # no bridge scores
    assert sel(scores=None) == nat.CAB_EINVAL
    assert sel(keep=None) == nat.CAB_EINVAL
    assert lib.cab_evict_connectivity(FAKE, 10, 9, FAKE, FAKE, None) == nat.CAB_ESHAPE
    assert lib.cab_evict_connectivity(None, 10, 10, FAKE, FAKE, None) == nat.CAB_EINVAL
    ptrs = (ctypes.c_void_p * 1)(FAKE)
    nulls = (ctypes.c_void_p * 1)(None)
    st = _s4(1 << 20, 1 << 16, 256, 0)
    g = lambda **kw: lib.cab_kv_gather(kw.get("src", ptrs), ptrs, 1, 1, 2, 100,
                                       kw.get("rb", 256), kw.get("ss", st), st, FAKE, 10, None)
    assert g(rb=100) == nat.CAB_ESHAPE
    assert g(ss=_s4(1 << 20, 1 << 16, 8, 0)) == nat.CAB_ESHAPE
    assert g(src=nulls) == nat.CAB_EINVAL


def test_token_frc_validation(lib):
    """Argument checks of the token-FRC entry points (nothing is launched)."""
    tf = lambda **kw: lib.cab_token_frc(kw.get("a", FAKE), kw.get("dt", nat.CAB_F32),
                                        kw.get("n", 10), kw.get("lda", 10), kw.get("s", FAKE),
                                        None, kw.get("f", FAKE), None)
    assert tf(dt=9) == nat.CAB_EDTYPE
    assert tf(n=-1) == nat.CAB_ESHAPE
    assert tf(lda=9) == nat.CAB_ESHAPE
    assert tf(s=None) == nat.CAB_EINVAL
    assert tf(f=None) == nat.CAB_EINVAL
    assert tf(a=None, n=0) == nat.CAB_OK  # empty graph: nothing to do
    st = _s4(600, 100, 10, 1)
    sym = lambda **kw: lib.cab_attention_symmetrize(FAKE, nat.CAB_BF16, 2, 3, kw.get("nq", 10),
                                                    kw.get("nk", 10), st, kw.get("out", FAKE),
                                                    kw.get("ldo", 10), None)
    assert sym(nq=4, nk=10) == nat.CAB_ESHAPE
    assert sym(ldo=9) == nat.CAB_ESHAPE
    assert sym(out=None) == nat.CAB_EINVAL
    ws = lib.cab_token_frc_keys_workspace_bytes(1000, 128)
    assert ws > 0 and lib.cab_token_frc_keys_workspace_bytes(1000, 257) == 0
    assert lib.cab_token_frc_keys_workspace_bytes(2000, 128) > ws
    ks = _s4(8 * 1000 * 128, 1000 * 128, 128, 1)
    fk = lambda **kw: lib.cab_token_frc_from_keys(
        FAKE, nat.CAB_BF16, 1, 8, 1000, kw.get("D", 128), ks, None, None, None, kw.get("f", FAKE),
        kw.get("ws", FAKE), kw.get("wsb", ws), None)
    assert fk(D=300) == nat.CAB_ESHAPE
    assert fk(f=None) == nat.CAB_EINVAL
    assert fk(wsb=ws - 1) == nat.CAB_EWORKSPACE
    assert fk(ws=FAKE + 16) == nat.CAB_EWORKSPACE


def test_visualize_frc_statistics_on_host(tmp_path):
    """visualize_frc_statistics (README.md:106-111) is host-only: its
    summary equals numpy's over the same diagnostics, and with matplotlib
    present it writes the histogram figure."""
    import numpy as np
    from cab_attention.kernels.frc_kernel import visualize_frc_statistics
    from oracle import cab_oracle as O
    rng = np.random.default_rng(12)
    qc = rng.standard_normal((1, 2, 40, 32)).astype(np.float32)
    kc = rng.standard_normal((1, 2, 40, 32)).astype(np.float32)
    f, a, t = O.compute_block_frc(qc, kc, lambda_redundancy=0.5)
    path = tmp_path / "frc.png"
    st = visualize_frc_statistics(torch.from_numpy(f), torch.from_numpy(a), torch.from_numpy(t),
                                  save_path=str(path))
    f32 = f.astype(np.float32).astype(np.float64)
    assert st["frc_mean"] == pytest.approx(f32.mean(), rel=1e-5)
    assert st["frc_std"] == pytest.approx(f32.std(ddof=1), rel=1e-4)
    assert st["frc_min"] == pytest.approx(f32.min()) and st["frc_max"] == pytest.approx(f32.max())
    assert st["frc_negative_fraction"] == pytest.approx((f < 0).mean())
    assert st["affinity_mean"] == pytest.approx(a.mean(), rel=1e-5)
    assert st["triangles_mean"] == pytest.approx(t.mean(), rel=1e-5)
    try:
        import matplotlib  # noqa: F401
    except ImportError:
        return
    assert path.exists() and path.stat().st_size > 1000

"""GPU parity of token-level FRC through the C ABI: cab_token_frc (strengths,
2-hop weights and curvature of an [N, N] graph), cab_attention_symmetrize and
cab_token_frc_from_keys, plus the FRCTracker built on them, against the
float64 oracle on the same seeded inputs."""

import numpy as np
import pytest
import torch

from oracle import cab_oracle as O

pytestmark = pytest.mark.gpu

DTYPES = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


def f64(t):
    return t.detach().double().cpu().numpy()


def rand_graph(n, seed, dt, kind="uniform"):
    g = torch.Generator().manual_seed(seed)
    a = torch.rand((n, n), generator=g)
    if kind == "softmax":
        a = torch.softmax(torch.randn((n, n), generator=g) * 3, dim=-1)
    return a.to(DTYPES[dt])


@pytest.mark.parametrize("dt", ["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("n", [1, 3, 64, 100, 1000, 4099])
def test_token_frc_matches_oracle(cuda, dt, n):
    """S, T, F within rtol 1e-5 (fp32 sums of non-negative terms) of the
    oracle on the same (widened) input values."""
    from cab_attention.kernels import token_frc
    for kind, seed in (("uniform", n), ("softmax", n + 1)):
        a = rand_graph(n, seed, dt, kind)
        s, t, f = token_frc(a.to(cuda), return_parts=True)
        ws, wt, wf = O.token_frc(f64(a))
        for name, got, want in (("S", s, ws), ("T", t, wt), ("F", f, wf)):
            np.testing.assert_allclose(f64(got), want, rtol=1e-5, err_msg=f"{kind} {name}")


def test_token_frc_strided_and_unaligned_rows(cuda):
    """A view with row stride > n (vector loads) and one whose rows are not
    16-byte aligned (scalar loads) give the contiguous result."""
    from cab_attention.kernels import token_frc
    for n, pad in ((257, 7), (300, 4), (64, 1)):
        big = rand_graph(n + pad, 5 + n, "fp32").to(cuda)
        view = big[:n, :n]
        s, t, f = token_frc(view, return_parts=True)
        ws, wt, wf = O.token_frc(f64(view))
        np.testing.assert_allclose(f64(t), wt, rtol=1e-5)
        np.testing.assert_allclose(f64(f), wf, rtol=1e-5)


def test_reference_named_entry_points(cuda):
    """compute_frc / _triton / _pytorch and the strength / triangle helpers
    return the input dtype, as the reference's do (frc_triton.py:181, :210,
    :251)."""
    from cab_attention.kernels import (compute_frc, compute_frc_pytorch, compute_frc_triton,
                                       compute_node_strengths_triton, compute_triangles_triton)
    a = rand_graph(200, 9, "bf16").to(cuda)
    ws, wt, wf = O.token_frc(f64(a))
    for fn in (compute_frc, compute_frc_triton, compute_frc_pytorch):
        out = fn(a)
        assert out.dtype == torch.bfloat16 and out.shape == (200,)
        np.testing.assert_allclose(f64(out), wf, rtol=8e-3)  # bf16 output rounding
    np.testing.assert_allclose(f64(compute_node_strengths_triton(a)), ws, rtol=8e-3)
    np.testing.assert_allclose(f64(compute_triangles_triton(a)), wt, rtol=8e-3)
    with pytest.raises(ValueError):
        compute_frc(a[:, :10])
    with pytest.raises(RuntimeError):
        compute_frc(a.cpu())


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("B,H,nq,nk", [(2, 3, 100, 100), (1, 2, 1, 257), (2, 2, 33, 1),
                                       (1, 1, 1, 1), (3, 4, 300, 300)])
def test_symmetrize_matches_oracle(cuda, dt, B, H, nq, nk):
    from cab_attention.kernels import symmetrize_attention
    g = torch.Generator().manual_seed(B * 1000 + nq + nk)
    att = torch.rand((B, H, nq, nk), generator=g).to(DTYPES[dt])
    got = symmetrize_attention(att.to(cuda))
    np.testing.assert_allclose(f64(got), O.symmetrize_attention(f64(att)), rtol=1e-6, atol=1e-7)
    # a transposed view (non-contiguous strides) gives the same matrix
    view = att.to(cuda).transpose(2, 3).contiguous().transpose(2, 3)
    assert torch.equal(symmetrize_attention(view), got)


def _gram_bound(keys):
    """Per-row bound on |delta r_i| from the bf16 hi/lo split (about 2^-17
    relative per product, summed over |G_ij|) plus fp32 rounding."""
    x = keys.mean(axis=(0, 1))
    kn = x / np.maximum(np.linalg.norm(x, axis=-1, keepdims=True), 1e-12)
    return 2e-5 * np.abs(kn @ kn.T).sum(axis=1) + 1e-6


@pytest.mark.parametrize("dt", ["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("B,H,N,D", [(1, 2, 100, 64), (2, 4, 1000, 128), (1, 3, 517, 80),
                                     (1, 1, 300, 256), (1, 8, 4097, 128), (1, 1, 1, 16)])
def test_frc_from_keys_matches_oracle(cuda, dt, B, H, N, D):
    """The relu row sums r within the split-product bound, then S, T, F;
    the [N, N] graph is never formed on the GPU."""
    from cab_attention.kernels import frc_from_keys
    g = torch.Generator().manual_seed(N * 7 + D)
    keys = torch.randn((B, H, N, D), generator=g).to(DTYPES[dt])
    got = frc_from_keys(keys.to(cuda), return_parts=True)
    kd = f64(keys)
    want = O.frc_from_keys(kd)
    bound = _gram_bound(kd)
    r = f64(got["row_sums"])
    assert np.all(np.abs(r - want["row_sums"]) <= bound), np.max(np.abs(r - want["row_sums"]) / bound)
    np.testing.assert_allclose(f64(got["strengths"]), want["strengths"], atol=1e-6, rtol=0)
    tol_t = 2 * bound / want["row_sums"] + 2e-6
    assert np.all(np.abs(f64(got["triangles"]) - want["triangles"]) <= tol_t)
    assert np.all(np.abs(f64(got["frc"]) - want["frc"]) <= 3 * tol_t + 4e-6)


@pytest.mark.parametrize("dt", ["fp32", "bf16", "fp16"])
def test_frc_from_keys_element_wise_loads(cuda, dt):
    """Layouts the 16-byte load path cannot take run the element-wise prep
    path (keys_prep_kernel<T, false>): D not a multiple of 8, a last-dim
    strided view, and keys starting one element past a 16-byte boundary;
    each is checked against the oracle as the contiguous case is."""
    from cab_attention.kernels import frc_from_keys
    g = torch.Generator().manual_seed(77)
    B, H, N = 1, 2, 301
    cases = []
    k100 = torch.randn((B, H, N, 100), generator=g).to(DTYPES[dt])
    cases.append(("D=100", k100, k100.to(cuda)))
    wide = torch.randn((B, H, N, 2 * 64), generator=g).to(DTYPES[dt])
    strided = wide.to(cuda)[..., ::2]
    assert strided.stride(-1) == 2
    cases.append(("last-dim stride 2", wide[..., ::2], strided))
    flat = torch.randn(B * H * N * 64 + 1, generator=g).to(DTYPES[dt])
    off = flat.to(cuda)[1:].view(B, H, N, 64)
    assert off.data_ptr() % 16 != 0
    cases.append(("offset by one element", flat[1:].view(B, H, N, 64), off))
    for name, host, dev in cases:
        got = frc_from_keys(dev, return_parts=True)
        kd = f64(host)
        want = O.frc_from_keys(kd)
        bound = _gram_bound(kd)
        r = f64(got["row_sums"])
        assert np.all(np.abs(r - want["row_sums"]) <= bound), name
        tol_t = 2 * bound / want["row_sums"] + 2e-6
        assert np.all(np.abs(f64(got["triangles"]) - want["triangles"]) <= tol_t), name
        assert np.all(np.abs(f64(got["frc"]) - want["frc"]) <= 3 * tol_t + 4e-6), name


def test_frc_from_keys_special_inputs(cuda):
    """Zero keys score 0; parallel and antipodal keys give the closed-form
    all-ones and identity graphs; a [B, N, H, D] layout passed as a
    transposed view (arbitrary strides) matches the contiguous keys."""
    from cab_attention.kernels import frc_from_keys
    rng = np.random.default_rng(3)
    k = rng.standard_normal((1, 2, 70, 128)).astype(np.float32)
    k[:, :, [0, 33, 69]] = 0.0
    u = rng.standard_normal(128).astype(np.float32)
    k[:, :, 40:50] = (rng.random(10)[:, None] + 0.5).astype(np.float32) * u
    k[:, :, 50] = -u
    got = frc_from_keys(torch.from_numpy(k).to(cuda), return_parts=True)
    want = O.frc_from_keys(k)
    assert np.all(f64(got["frc"])[[0, 33, 69]] == 0.0)
    np.testing.assert_allclose(f64(got["row_sums"]), want["row_sums"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(f64(got["frc"]), want["frc"], atol=1e-5)
    bnhd = torch.from_numpy(np.ascontiguousarray(k.transpose(0, 2, 1, 3))).to(cuda)
    again = frc_from_keys(bnhd.transpose(1, 2), return_parts=True)
    assert torch.equal(again["row_sums"], got["row_sums"]) and torch.equal(again["frc"], got["frc"])


def test_frc_tracker(cuda):
    """FRCTracker: scores in the keys' dtype; within the update interval the
    cached scores come back extended with zeros; attention input (2-D and
    4-D); bottom-k with exclusions (lowest first, ties in position order);
    pruning."""
    from cab_attention.scoring import FRCTracker
    g = torch.Generator().manual_seed(21)
    keys = torch.randn((1, 4, 200, 64), generator=g).to(cuda)
    tr = FRCTracker(device=cuda)
    f1 = tr.compute_from_keys(keys)
    assert f1.dtype == torch.float32 and f1.shape == (200,) and len(tr) == 200
    np.testing.assert_allclose(f64(f1), O.frc_from_keys(f64(keys))["frc"], atol=1e-5)
    longer = torch.cat([keys, torch.randn((1, 4, 5, 64), generator=g).to(cuda)], dim=2)
    f2 = tr.compute_from_keys(longer)
    assert f2.shape == (205,) and torch.equal(f2[:200], f1) and torch.all(f2[200:] == 0)
    f3 = tr.compute_from_keys(longer, force_update=True)
    np.testing.assert_allclose(f64(f3), O.frc_from_keys(f64(longer))["frc"], atol=1e-5)
    assert tr.compute_from_keys(keys.to(torch.bfloat16), force_update=True).dtype == torch.bfloat16

    att = torch.softmax(torch.randn((2, 3, 150, 150), generator=g), dim=-1).to(cuda)
    f4 = tr.compute_from_attention(att)
    wf = O.token_frc(O.symmetrize_attention(f64(att)))[2]
    np.testing.assert_allclose(f64(f4), wf, rtol=1e-5)
    m = O.symmetrize_attention(f64(att))
    f5 = tr.compute_from_attention(torch.from_numpy(m).float().to(cuda))
    np.testing.assert_allclose(f64(f5), wf, rtol=1e-5)

    sc = f64(f5)
    excl = torch.tensor([int(np.argmin(sc)), 3, 7], device=cuda)
    idx = tr.get_bottom_k_indices(10, exclude_indices=excl).cpu().numpy()
    masked = sc.copy()
    masked[excl.cpu().numpy()] = np.inf
    assert list(idx) == list(np.argsort(masked.astype(np.float32), kind="stable")[:10])
    tr.prune(torch.tensor([5, 1, 149, 400], device=cuda))
    assert len(tr) == 3 and tr.last_update_len == 3
    np.testing.assert_array_equal(f64(tr.get_scores()), sc[[5, 1, 149]])
    tr.reset()
    assert len(tr) == 0 and tr.get_bottom_k_indices(3).numel() == 0

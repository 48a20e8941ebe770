"""GPU parity of the dense attention + per-key totals path (the eviction
path's fused kernel): cab_flash_attn_fwd and cab_attn_key_scores through the
C ABI, against the float64 oracle on the same seeded inputs."""

import numpy as np
import pytest
import torch

from oracle import cab_oracle as O

pytestmark = pytest.mark.gpu

DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}
# Output: bf16 / fp16 rounding of the inputs' products and of P; fp32: the
# north-star tolerance (split bf16 operands). lse: fp32 softmax statistics.
ATOL = {"bf16": 2e-2, "fp16": 5e-3, "fp32": 1e-3}
# lse = m + log(sum P) over the same rounded P the output uses: a bf16 P
# entry carries a relative rounding of up to 2^-9, fp16 2^-11, which a row
# with few keys passes into its lse almost unaveraged.
LSE_ATOL = {"bf16": 2e-3, "fp16": 1e-3, "fp32": 1e-3}


def seeded(shape, seed, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * scale).to(dtype)


def np64(t):
    return t.detach().double().cpu().numpy()


def assert_scores_close(got, want, n_queries):
    """Key totals: relative 5e-3 (the lse of pass 1 sums bf16-rounded P),
    plus an absolute floor for keys that receive almost nothing."""
    got = np64(got)
    np.testing.assert_allclose(got, want, rtol=5e-3, atol=1e-5 * max(1, n_queries))


SHAPES = [  # (H, H_kv, N_q, N_k)
    (2, 2, 300, 300),
    (4, 2, 256, 256),   # grouped K / V
    (2, 1, 1, 777),     # one decode query against a cache
    (2, 2, 100, 700),   # a chunk of queries at the end of the cache
    (2, 2, 130, 60),    # more queries than keys (causal: first rows see nothing)
]


@pytest.mark.parametrize("D", [128, 64])
@pytest.mark.parametrize("dt", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("H,Hkv,Nq,Nk", SHAPES)
def test_flash_attention_and_key_scores(cuda, dt, causal, H, Hkv, Nq, Nk, D):
    from cab_attention.kernels import flash_attention, key_scores
    B = 1
    q = seeded((B, H, Nq, D), 1, DTYPES[dt])
    k = seeded((B, Hkv, Nk, D), 2, DTYPES[dt])
    v = seeded((B, Hkv, Nk, D), 3, DTYPES[dt])
    out, lse = flash_attention(q.to(cuda), k.to(cuda), v.to(cuda), causal=causal, return_lse=True)
    w_out, w_lse, w_sc = O.dense_attention_scores(np64(q), np64(k), np64(v), causal=causal)
    err = np.abs(np64(out) - w_out).max()
    assert err <= ATOL[dt], f"max abs error {err}"
    got_lse = np64(lse)
    fin = np.isfinite(w_lse)
    assert np.array_equal(np.isfinite(got_lse), fin)
    np.testing.assert_allclose(got_lse[fin], w_lse[fin], atol=LSE_ATOL[dt], rtol=1e-4)
    sc = key_scores(q.to(cuda), k.to(cuda), lse, causal=causal)
    assert_scores_close(sc, w_sc, Nq)


@pytest.mark.parametrize("causal", [False, True])
def test_cumulative_scores_accumulate_across_calls(cuda, causal):
    """flash_attention_with_cumulative_scores: a prefill, then one decode step
    with the cache grown by one token, adds to the same totals (extended with
    zeros for the new position), as the reference's wrapper does."""
    from cab_attention.kernels import flash_attention_with_cumulative_scores
    B, H, Hkv, N, D = 1, 4, 2, 200, 128
    q1 = seeded((B, H, N, D), 11, torch.bfloat16)
    k = seeded((B, Hkv, N + 1, D), 12, torch.bfloat16)
    v = seeded((B, Hkv, N + 1, D), 13, torch.bfloat16)
    q2 = seeded((B, H, 1, D), 14, torch.bfloat16)
    out1, sc = flash_attention_with_cumulative_scores(q1.to(cuda), k[:, :, :N].to(cuda),
                                                      v[:, :, :N].to(cuda), causal=causal)
    assert tuple(sc.shape) == (B, H, N)
    out2, sc2 = flash_attention_with_cumulative_scores(q2.to(cuda), k.to(cuda), v.to(cuda), sc,
                                                       causal=causal)
    assert tuple(sc2.shape) == (B, H, N + 1)
    _, _, w1 = O.dense_attention_scores(np64(q1), np64(k[:, :, :N]), np64(v[:, :, :N]), causal=causal)
    w_out2, _, w2 = O.dense_attention_scores(np64(q2), np64(k), np64(v), causal=causal)
    want = np.concatenate([w1, np.zeros((B, H, 1))], axis=2) + w2
    assert_scores_close(sc2, want, N + 1)
    assert np.abs(np64(out2) - w_out2).max() <= ATOL["bf16"]


def test_key_scores_are_deterministic(cuda):
    """Fixed-order sums: two calls give the same bits."""
    from cab_attention.kernels import flash_attention, key_scores
    q = seeded((1, 4, 1000, 128), 21, torch.bfloat16).to(cuda)
    k = seeded((1, 4, 1000, 128), 22, torch.bfloat16).to(cuda)
    v = seeded((1, 4, 1000, 128), 23, torch.bfloat16).to(cuda)
    _, lse = flash_attention(q, k, v, causal=True, return_lse=True)
    a = key_scores(q, k, lse, causal=True)
    b = key_scores(q, k, lse, causal=True)
    assert torch.equal(a, b)


def test_accumulation_module_and_strided_views(cuda):
    """FlashAttentionWithAccumulation on [B, N, H, D] views (the reference's
    layout guess) keeps running totals; the inputs are transposed views, not
    copies."""
    from cab_attention.kernels import FlashAttentionWithAccumulation, get_all_cumulative_scores
    B, N, H, D = 1, 192, 4, 128
    x = seeded((B, N, 3, H, D), 31, torch.bfloat16).to(cuda)
    q, k, v = x[:, :, 0], x[:, :, 1], x[:, :, 2]  # [B, N, H, D] views
    mod = FlashAttentionWithAccumulation(causal=True)
    model = torch.nn.Sequential(mod)
    out, none = mod(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
    assert none is None and tuple(out.shape) == (B, H, N, D)
    out2, _ = mod(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
    assert torch.equal(out, out2)
    _, _, w = O.dense_attention_scores(np64(q.transpose(1, 2)), np64(k.transpose(1, 2)),
                                       np64(v.transpose(1, 2)), causal=True)
    assert_scores_close(mod.get_cumulative_scores(), 2 * w, 2 * N)
    assert set(get_all_cumulative_scores(model)) == {"0"}
    mod.reset_scores()
    assert mod.get_cumulative_scores() is None


@pytest.mark.parametrize("D", [128, 64])
def test_flash_attention_longer_sequence(cuda, D):
    """N = 4096 causal with grouped heads: outputs on sampled rows and every
    key total against the oracle."""
    from cab_attention.kernels import flash_attention_with_cumulative_scores
    B, H, Hkv, N = 1, 2, 1, 4096
    q = seeded((B, H, N, D), 41, torch.bfloat16)
    k = seeded((B, Hkv, N, D), 42, torch.bfloat16)
    v = seeded((B, Hkv, N, D), 43, torch.bfloat16)
    out, sc = flash_attention_with_cumulative_scores(q.to(cuda), k.to(cuda), v.to(cuda), causal=True)
    w_out, _, w_sc = O.dense_attention_scores(np64(q), np64(k), np64(v), causal=True)
    rows = [0, 1, 63, 64, 2047, 4095]
    assert np.abs(np64(out)[:, :, rows] - w_out[:, :, rows]).max() <= ATOL["bf16"]
    assert_scores_close(sc, w_sc, N)
    np.testing.assert_allclose(np64(sc).sum(-1), N, rtol=1e-3)

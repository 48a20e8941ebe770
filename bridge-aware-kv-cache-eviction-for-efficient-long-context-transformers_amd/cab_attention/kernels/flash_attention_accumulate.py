"""Dense attention with per-key attention totals (KV-cache eviction scores).

Same module path, names and call contract as the reference's
``cab_attention/kernels/flash_attention_accumulate.py``:
``flash_attention_with_cumulative_scores`` (:172-261),
``FlashAttentionWithAccumulation`` (:264-363), ``get_all_cumulative_scores``
(:548-598) and ``repeat_kv`` (:470-481). The work runs in two HIP calls:
``cab_flash_attn_fwd`` (attention output and each query's log-sum-exp) and
``cab_attn_key_scores`` (each key's total softmax probability over the
queries).

Two deliberate differences from the reference kernel (:23-169):

* the score of key s is ``sum_t softmax_t(s)``, the attention probability
  it receives, which is what the reference's eager path sums
  (experiments/longbench_qa/runner.py:680-685); the reference's kernel adds
  ``exp(q.k - running max)``, a number that depends on its tile order;
* ``causal`` is available (the reference has the mask commented out,
  :107), aligned so that the N_q queries are the last N_q of the N_k key
  positions, and K / V may have fewer heads than Q (grouped-query
  attention, without materialising ``repeat_kv``).

Scores are summed in a fixed order without atomics, so repeated calls give
identical bits.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from .. import _native as nat


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float | None = None,
                    causal: bool = False, out: torch.Tensor | None = None,
                    return_lse: bool = False):
    """Dense attention ``softmax(q k^T * scale) v`` (``cab_flash_attn_fwd``).

    q: ``[B, H, N_q, D]``; k, v: ``[B, H_kv, N_k, D]`` with ``H % H_kv == 0``
    (query head h reads K / V head ``h // (H // H_kv)``); D = 64 or 128; bf16, fp16
    or fp32. ``causal`` lets query t see keys ``s <= t + N_k - N_q``. Returns
    the output ``[B, H, N_q, D]`` and, with ``return_lse``, the fp32
    natural-log log-sum-exp ``[B, H, N_q]``.
    """
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be [B, H, N, D]")
    if k.shape != v.shape:
        raise ValueError(f"k and v shapes differ: {tuple(k.shape)} vs {tuple(v.shape)}")
    B, H, N_q, D = q.shape
    if k.shape[0] != B or k.shape[3] != D:
        raise ValueError(f"k / v must be [B={B}, H_kv, N_k, D={D}]; got {tuple(k.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k, v dtypes differ")
    H_kv, N_k = k.shape[1], k.shape[2]
    dev = nat.require_device(q, k, v)
    lib = nat.load()
    dt = nat.dtype_code(q)
    q = nat.aligned_rows(q)
    k = nat.aligned_rows(k)
    v = nat.aligned_rows(v)
    if out is None:
        out = torch.empty((B, H, N_q, D), dtype=q.dtype, device=dev)
    elif tuple(out.shape) != (B, H, N_q, D) or out.dtype != q.dtype:
        raise ValueError("out must match q's shape and dtype")
    lse = torch.empty((B, H, N_q), dtype=torch.float32, device=dev) if return_lse else None
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    wbytes = lib.cab_flash_attn_workspace_bytes(dt, B, H_kv, N_k, D)
    ws = torch.empty(max(int(wbytes), 16), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        st = lib.cab_flash_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), dt, B, H, H_kv, N_q,
                                    N_k, D, nat.strides4(q), nat.strides4(k), nat.strides4(v),
                                    nat.strides4(out), float(scale), int(bool(causal)),
                                    out.data_ptr(), nat.ptr(lse), ws.data_ptr(), ws.numel(),
                                    nat.stream_ptr(dev))
    nat.check("cab_flash_attn_fwd", st)
    return (out, lse) if return_lse else out


def key_scores(q: torch.Tensor, k: torch.Tensor, lse: torch.Tensor, scale: float | None = None,
               causal: bool = False, scores: torch.Tensor | None = None,
               accumulate: bool = False) -> torch.Tensor:
    """``scores[b, h, s] (+)= sum_t exp(q_t . k_s * scale - lse[b, h, t])``
    (``cab_attn_key_scores``), with the lse of :func:`flash_attention` on the
    same q, k. bf16, fp16 or fp32."""
    B, H, N_q, D = q.shape
    H_kv, N_k = k.shape[1], k.shape[2]
    if tuple(lse.shape) != (B, H, N_q) or lse.dtype != torch.float32:
        raise ValueError(f"lse must be fp32 [B, H, N_q] = {(B, H, N_q)}")
    dev = nat.require_device(q, k, lse)
    lib = nat.load()
    dt = nat.dtype_code(q)
    if q.dtype != k.dtype:
        raise TypeError("q, k dtypes differ")
    q = nat.aligned_rows(q)
    k = nat.aligned_rows(k)
    lse = lse.contiguous()
    if scores is None:
        scores = torch.empty((B, H, N_k), dtype=torch.float32, device=dev)
        accumulate = False
    elif (tuple(scores.shape) != (B, H, N_k) or scores.dtype != torch.float32
          or scores.stride(-1) != 1):
        raise ValueError(f"scores must be fp32 [B, H, N_k] = {(B, H, N_k)} with a contiguous last dim")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    st3 = nat.strides4(scores)  # [b, h, token] strides (the 4th slot is unused)
    with torch.cuda.device(dev):
        st = lib.cab_attn_key_scores(q.data_ptr(), k.data_ptr(), lse.data_ptr(), dt, B, H, H_kv,
                                     N_q, N_k, D, nat.strides4(q), nat.strides4(k), float(scale),
                                     int(bool(causal)), scores.data_ptr(), st3,
                                     int(bool(accumulate)), nat.stream_ptr(dev))
    nat.check("cab_attn_key_scores", st)
    return scores


def flash_attention_with_cumulative_scores(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cumulative_scores: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    causal: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Attention output and per-key attention totals.

    Args:
        q: ``[B, H, N_q, D]``; k, v: ``[B, H_kv, N_k, D]`` (``H_kv`` divides
            ``H``). bf16, fp16 or fp32, D = 64 or 128.
        cumulative_scores: optional fp32 ``[B, H, N_old]`` running totals. They
            are added to (not reset); when ``N_old < N_k`` they are first
            extended with zeros for the new key positions, as in the
            reference (:222-229).
        scale: defaults to ``1/sqrt(D)``.
        causal: query t sees keys ``s <= t + N_k - N_q``.

    Returns:
        ``(output [B, H, N_q, D], cumulative_scores [B, H, N_k])``.
    """
    B, H, N_q, D = q.shape
    N_k = k.shape[2]
    out, lse = flash_attention(q, k, v, scale=scale, causal=causal, return_lse=True)
    if cumulative_scores is None:
        return out, key_scores(q, k, lse, scale=scale, causal=causal)
    if cumulative_scores.dim() != 3 or tuple(cumulative_scores.shape[:2]) != (B, H):
        raise ValueError(f"cumulative_scores must be [B={B}, H={H}, N]")
    if cumulative_scores.shape[2] < N_k:
        extension = torch.zeros(B, H, N_k - cumulative_scores.shape[2], dtype=torch.float32,
                                device=q.device)
        cumulative_scores = torch.cat([cumulative_scores.float(), extension], dim=2)
    elif cumulative_scores.shape[2] > N_k:
        raise ValueError(f"cumulative_scores has {cumulative_scores.shape[2]} key positions, "
                         f"more than N_k={N_k}")
    if cumulative_scores.dtype != torch.float32 or cumulative_scores.stride(-1) != 1:
        cumulative_scores = cumulative_scores.float().contiguous()
    return out, key_scores(q, k, lse, scale=scale, causal=causal, scores=cumulative_scores,
                           accumulate=True)


class FlashAttentionWithAccumulation(torch.nn.Module):
    """Attention that keeps per-key attention totals across calls
    (reference :264-363). ``forward(query, key, value)`` takes ``[B, H, N, D]``
    (or ``[B, N, H, D]`` when the head counts of query and key differ, as the
    reference guesses) and returns ``(output, None)``."""

    def __init__(self, original_attention: Optional[torch.nn.Module] = None,
                 accumulate_scores: bool = True, causal: bool = False):
        super().__init__()
        self.original_attention = original_attention
        self.accumulate_scores = accumulate_scores
        self.causal = causal
        self.cumulative_scores = None
        self.reset_scores()

    def reset_scores(self):
        """Forget the totals (start of a new sequence)."""
        self.cumulative_scores = None

    def get_cumulative_scores(self) -> Optional[torch.Tensor]:
        """The running totals ``[B, H, N]``, or None."""
        return self.cumulative_scores

    def forward(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, **kwargs):
        transpose_back = query.dim() == 4 and query.shape[1] != key.shape[1]
        if transpose_back:
            query, key, value = (t.transpose(1, 2) for t in (query, key, value))
        if self.accumulate_scores:
            output, self.cumulative_scores = flash_attention_with_cumulative_scores(
                query, key, value, self.cumulative_scores, causal=self.causal)
        else:
            output = flash_attention(query, key, value, causal=self.causal)
        if transpose_back:
            output = output.transpose(1, 2)
        return output, None


def repeat_kv(hidden_states: torch.Tensor, n_rep: int) -> torch.Tensor:
    """``[B, H_kv, N, D] -> [B, H_kv * n_rep, N, D]`` (each head repeated
    n_rep times in place), for callers that need per-query-head K / V. The
    kernels above take the grouped K / V directly."""
    batch, num_kv_heads, slen, head_dim = hidden_states.shape
    if n_rep == 1:
        return hidden_states
    hidden_states = hidden_states[:, :, None, :, :].expand(batch, num_kv_heads, n_rep, slen,
                                                           head_dim)
    return hidden_states.reshape(batch, num_kv_heads * n_rep, slen, head_dim)


def get_all_cumulative_scores(model: torch.nn.Module) -> dict:
    """Map module name -> running totals for every
    :class:`FlashAttentionWithAccumulation` in ``model`` (and every module
    carrying a ``_flash_cumulative_scores`` attribute)."""
    scores = {}
    for name, module in model.named_modules():
        s = getattr(module, "_flash_cumulative_scores", None)
        if s is None and isinstance(module, FlashAttentionWithAccumulation):
            s = module.get_cumulative_scores()
        if s is not None:
            scores[name] = s
    return scores

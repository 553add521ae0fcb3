"""CPU oracle for the FlashAttention path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module,
and only as the checker (or the timed CPU baseline). The product path
(myk_llm_amd.flash_attn) never calls it and fails loudly without the HIP library.

Restated from the reference (never imported):
  * reference()            tests/test_flash_attn.py:13-28  — fp32 masked softmax attention
  * reference_with_lse()   adds the base-2 LSE of flash_attn.py:147-153 ((heads, rows),
                           +inf and O = 0 for rows that see no key)
  * reference_varlen()     per-document split, tests/test_flash_attn.py:79-81
  * kvcache_reference()    flash_attn_with_kvcache semantics, flash_attn.py:467-490
  * window()               flash_attn.py:435-439
  * visible_mask()         flash_attn.py:14-18 / tests/test_flash_attn.py:19-26
  * block_ranges()         flash_attn.py:58-68 (integer tile skipping)
  * visible_pairs()        the pair count behind the FLOP convention,
                           scripts/benchmark_attention.py:49-50

How each function is pinned (tests/test_oracle.py):
  * reference / reference_with_lse: against the independent float64 C brute force
    (oracle/attn_ref.c), against torch's scaled_dot_product_attention on causal and
    full cases, and closed forms (one visible key -> O = v_j; q = 0 -> mean of visible v,
    LSE = log2(count); empty rows -> O = 0, LSE = +inf); committed golden fixtures.
  * gradients (autograd of reference): against the C brute-force backward and a float64
    finite-difference gradcheck; delta = rowsum(dO*O) against sum_j P dP.
  * visible_mask / window: explicit loops over the formula; per-row counts against the
    closed form min(i+1, w).
  * block_ranges: exhaustive invariants on small inputs.
  * visible_pairs: closed form P(n, w) = w(w+1)/2 + (n-w) w and brute force.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

UNBOUNDED = 1 << 30  # flash_attn.py:32
LOG2E = 1.4426950408889634  # flash_attn.py:33


def window(causal: bool, window_size: tuple[int, int]) -> tuple[int, int]:
    """(left, right) offsets, -1 -> unbounded, causal forces right = 0 (flash_attn.py:435-439)."""
    left, right = window_size
    left = UNBOUNDED if left < 0 else left
    right = 0 if causal else (UNBOUNDED if right < 0 else right)
    return left, right


def visible_mask(seqlen_q: int, seqlen_k: int, causal: bool, window_size: tuple[int, int]) -> torch.Tensor:
    """(Lq, Lk) bool: query i sees key j iff i + Lk - Lq - left <= j <= i + Lk - Lq + right
    (tests/test_flash_attn.py:19-26; flash_attn.py:14-18)."""
    pos = torch.arange(seqlen_q)[:, None] + seqlen_k - seqlen_q
    key = torch.arange(seqlen_k)[None, :]
    left, right = window_size[0], 0 if causal else window_size[1]
    vis = torch.ones(seqlen_q, seqlen_k, dtype=torch.bool)
    if left >= 0:
        vis &= key >= pos - left
    if right >= 0:
        vis &= key <= pos + right
    return vis


def reference(q, k, v, causal, window_size, softmax_scale: Optional[float] = None):
    """fp32 attention with flash-attn masking (tests/test_flash_attn.py:13-28).
    q (B, Lq, H, D), k/v (B, Lk, Hkv, D); returns O (B, Lq, H, D) fp32. Differentiable."""
    seqlen_q, seqlen_k, heads = q.shape[1], k.shape[1], q.shape[2]
    k = k.float().repeat_interleave(heads // k.shape[2], 2)
    v = v.float().repeat_interleave(heads // v.shape[2], 2)
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    scores = torch.einsum("bqhd,bkhd->bhqk", q.float(), k) * scale
    vis = visible_mask(seqlen_q, seqlen_k, causal, window_size).to(q.device)
    probs = torch.softmax(scores.masked_fill(~vis, float("-inf")), -1).nan_to_num(0.0)
    return torch.einsum("bhqk,bkhd->bqhd", probs, v)


def reference_with_lse(q, k, v, causal, window_size, softmax_scale: Optional[float] = None):
    """(O, LSE): LSE is base 2 of the scaled scores, shape (H, B * Lq), +inf for rows that see
    no key, whose O is 0 (flash_attn.py:147-153, :363)."""
    seqlen_q, seqlen_k, heads = q.shape[1], k.shape[1], q.shape[2]
    kk = k.float().repeat_interleave(heads // k.shape[2], 2)
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    scores = torch.einsum("bqhd,bkhd->bhqk", q.float(), kk) * scale
    vis = visible_mask(seqlen_q, seqlen_k, causal, window_size).to(q.device)
    lse_e = torch.logsumexp(scores.masked_fill(~vis, float("-inf")), -1)  # (B, H, Lq)
    lse2 = lse_e * LOG2E
    lse2 = torch.where(torch.isneginf(lse2), torch.full_like(lse2, float("inf")), lse2)
    lse2 = lse2.permute(1, 0, 2).reshape(heads, -1)  # (H, B * Lq)
    return reference(q, k, v, causal, window_size, softmax_scale), lse2


def reference_varlen(q, k, v, cu_seqlens, causal, window_size, softmax_scale: Optional[float] = None,
                     with_lse: bool = False):
    """Packed q (T, H, D), k/v (T, Hkv, D): each document attends within itself
    (tests/test_flash_attn.py:79-81). Returns O (T, H, D) fp32 [and LSE (H, T)]."""
    bounds = [int(x) for x in cu_seqlens.tolist()]
    outs, lses = [], []
    for a, b in zip(bounds, bounds[1:]):
        if with_lse:
            o, l2 = reference_with_lse(q[None, a:b], k[None, a:b], v[None, a:b], causal, window_size, softmax_scale)
            outs.append(o[0])
            lses.append(l2)
        else:
            outs.append(reference(q[None, a:b], k[None, a:b], v[None, a:b], causal, window_size, softmax_scale)[0])
    out = torch.cat(outs) if outs else q.float().new_zeros(q.shape)
    if with_lse:
        return out, (torch.cat(lses, 1) if lses else q.float().new_zeros((q.shape[1], 0)))
    return out


def kvcache_reference(q, k_cache, v_cache, k_new, v_new, cache_seqlens, causal, window_size,
                      softmax_scale: Optional[float] = None):
    """flash_attn_with_kvcache (flash_attn.py:467-490) on CPU copies: returns
    (O fp32 (B, Lq, H, D), LSE (H, B * Lq), k_cache', v_cache'), the caches after the write."""
    kc, vc = k_cache.clone(), v_cache.clone()
    lens = [int(x) for x in cache_seqlens.tolist()]
    new = 0
    if k_new is not None and v_new is not None:
        new = k_new.shape[1]
        for b, n in enumerate(lens):
            for t in range(new):
                if n + t < kc.shape[1]:
                    kc[b, n + t] = k_new[b, t]
                    vc[b, n + t] = v_new[b, t]
    outs, lses = [], []
    for b, n in enumerate(lens):
        used = min(n + new, kc.shape[1])
        o, l2 = reference_with_lse(q[b:b + 1], kc[b:b + 1, :used], vc[b:b + 1, :used], causal, window_size,
                                   softmax_scale)
        outs.append(o)
        lses.append(l2)
    return torch.cat(outs), torch.cat(lses, 1), kc, vc


def block_ranges(s0: int, block_s: int, lo_off: int, hi_off: int, t_len: int, block_t: int):
    """flash_attn.py:58-68: for self indices [s0, s0 + block_s) seeing other indices t with
    lo_off <= t - s <= hi_off, 0 <= t < t_len, the block_t-aligned [lo, hi) to visit, split
    as [lo, mid_lo) masked, [mid_lo, mid_hi) unmasked, [mid_hi, hi) masked."""
    lo = max(s0 + lo_off, 0) // block_t * block_t
    hi = max(min(s0 + block_s + hi_off, t_len), lo)
    mid_lo = min(-(-max(s0 + block_s - 1 + lo_off, lo) // block_t) * block_t, hi)
    mid_hi = max(min(s0 + hi_off + 1, t_len), 0) // block_t * block_t
    return lo, mid_lo, max(mid_hi, mid_lo), hi


def visible_pairs(lengths, window_size: int | None = None) -> int:
    """Visible (query, key) pairs of causal documents with an optional model-convention
    window w (each query sees min(i + 1, w) keys) — scripts/benchmark_attention.py:49."""
    total = 0
    for n in lengths:
        if window_size is None or window_size >= n:
            total += n * (n + 1) // 2
        else:
            w = window_size
            total += w * (w + 1) // 2 + (n - w) * w
    return total


def backward_reference(q, k, v, dout, causal, window_size, softmax_scale: Optional[float] = None):
    """dQ, dK, dV (fp32) by autograd through reference(), as tests/test_flash_attn.py:61-64."""
    qf, kf, vf = (x.detach().float().requires_grad_() for x in (q, k, v))
    out = reference(qf, kf, vf, causal, window_size, softmax_scale)
    return torch.autograd.grad(out, (qf, kf, vf), dout.float())


def backward_reference_varlen(q, k, v, dout, cu_seqlens, causal, window_size, softmax_scale: Optional[float] = None):
    qf, kf, vf = (x.detach().float().requires_grad_() for x in (q, k, v))
    out = reference_varlen(qf, kf, vf, cu_seqlens, causal, window_size, softmax_scale)
    return torch.autograd.grad(out, (qf, kf, vf), dout.float())

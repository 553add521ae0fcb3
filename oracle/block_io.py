"""CPU oracle for the attention block's prologue and epilogue — TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py's cpu_baseline leg may import this module, as the checker. The
product path (myk_llm_amd.block_io) never calls it and fails loudly without the HIP library.

Restated from the reference (never imported), with the rounding points of its bf16-autocast
training default (train/config.py:101-104; trainer.py:234):
  * rope_tables()   RotaryEmbedding._build, model/layers.py:80-85 (fp32 angles
                    pos * base^(-2i/D), repeated per pair, cos and sin)
  * rms_norm()      RMSNorm.forward, layers.py:22-25 (x * rsqrt(mean(x^2) + eps) * w; under
                    autocast pow/rsqrt run in fp32 and the fp32 weight promotes the product)
  * rotate_half()   layers.py:66-70 (interleaved pairs: (x0, x1) -> (-x1, x0))
  * rope()          RotaryEmbedding.rotate, layers.py:93-98 (x*cos + rotate_half(x)*sin in
                    fp32, cast back)
  * qk_norm_rope()  Attention.forward, mixers.py:85-89 (norm, `.to(v.dtype)`, then RoPE)
  * output_gate()   mixers.py:116-117 (out * sigmoid(gate); under autocast sigmoid keeps the
                    bf16 input type, so it is rounded before the product)
Gradients are autograd of these functions with the same casts (a cast's backward rounds the
gradient to the source type, the rounding points of the reference's backward).

`acc` selects the arithmetic type (float32 as in the reference; float64 for the pins) and
`store` the rounding type between steps (None: no rounding).

How each function is pinned (tests/test_block_io_oracle.py):
  * rope / rotate_half: against complex multiplication (x[2i] + i x[2i+1]) e^{i p theta_i} in
    float64 numpy with theta_i = base^(-2i/D) computed independently; position 0 is the
    identity; pair norms are preserved; q.k after rotation depends only on the position
    difference.
  * rope_tables: against numpy float64 cos/sin of the same angles (fp32 table error bound).
  * rms_norm: mean(y^2) = ms / (ms + eps) for unit weights (closed form); scale invariance;
    the weight multiplies per column.
  * output_gate: gate = 0 halves x exactly; large |gate| passes or blocks x; the gradient
    against the closed form sigmoid(g) dy and dy x sigmoid(g) (1 - sigmoid(g)).
  * gradients: float64 central finite differences of the whole prologue and of the gate.
  * planted mistakes (a sign flip in rotate_half, a pair-order swap, a mean over D - 1, a
    gate derivative without the sigmoid factor) fail these pins.
"""

from __future__ import annotations

from typing import Optional

import torch


def rope_tables(head_dim: int, length: int, base: float, dtype=torch.float32):
    """layers.py:80-85."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=dtype) / head_dim))
    angles = torch.outer(torch.arange(length, dtype=dtype), inv_freq)
    angles = torch.repeat_interleave(angles, repeats=2, dim=-1)
    return angles.cos(), angles.sin()


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float, acc=torch.float32) -> torch.Tensor:
    """layers.py:22-25 under autocast: fp32 statistics and product."""
    xa = x.to(acc)
    return xa * torch.rsqrt(xa.pow(2).mean(dim=-1, keepdim=True) + eps) * w.to(acc)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """layers.py:66-70: dims (2i, 2i+1) -> (-x[2i+1], x[2i])."""
    x1 = x[..., ::2]
    x2 = x[..., 1::2]
    return torch.stack((-x2, x1), dim=-1).flatten(start_dim=-2)


def rope(x: torch.Tensor, position_ids: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
         acc=torch.float32) -> torch.Tensor:
    """layers.py:93-98 without the final cast: x (batch, seq, heads, D), position_ids
    (batch, seq)."""
    c = cos.to(acc)[position_ids].unsqueeze(2)
    s = sin.to(acc)[position_ids].unsqueeze(2)
    xa = x.to(acc)
    return xa * c + rotate_half(xa) * s


def qk_norm_rope(q, k, position_ids, cos, sin, q_weight=None, k_weight=None, eps: float = 1e-6,
                 acc=torch.float32, store: Optional[torch.dtype] = "input"):
    """mixers.py:85-89. q/k (batch, seq, heads, D); returns (q, k) in `store` (default: the
    input type; None keeps `acc`)."""
    st = q.dtype if store == "input" else store

    def cast(t):
        return t if st is None else t.to(st)

    if q_weight is not None:
        q, k = cast(rms_norm(q, q_weight, eps, acc)), cast(rms_norm(k, k_weight, eps, acc))
    if cos is not None:
        q, k = cast(rope(q, position_ids, cos, sin, acc)), cast(rope(k, position_ids, cos, sin, acc))
    return q, k


class _Sigmoid16(torch.autograd.Function):
    """torch.sigmoid on a 16-bit tensor as the reference's GPU runs it: fp32 inside, output
    rounded; backward grad * (1 - s) * s in fp32 from the rounded s, rounded (the GPU's opmath
    sigmoid_backward; torch's CPU fp16 kernel rounds after every operation instead)."""

    @staticmethod
    def forward(ctx, g):  # pyright: ignore[reportIncompatibleMethodOverride]
        s = torch.sigmoid(g.float()).to(g.dtype)
        ctx.save_for_backward(s)
        return s

    @staticmethod
    def backward(ctx, grad):  # pyright: ignore[reportIncompatibleMethodOverride]
        (s,) = ctx.saved_tensors
        sf = s.float()
        return (grad.float() * (1.0 - sf) * sf).to(s.dtype)


def output_gate(out: torch.Tensor, gate: torch.Tensor, acc=torch.float32,
                store: Optional[torch.dtype] = "input") -> torch.Tensor:
    """mixers.py:116-117 under autocast: sigmoid in the input type, then the product."""
    st = out.dtype if store == "input" else store
    if st is None:
        return out.to(acc) * torch.sigmoid(gate.to(acc))
    # sigmoid of the 16-bit gate: fp32 inside, rounded; its backward uses that rounded output
    s = _Sigmoid16.apply(gate.to(st))
    return (out.to(acc) * s.to(acc)).to(st)

"""The attention block's elementwise prologue and epilogue on MI355X (gfx950), the steps either
side of the FlashAttention path in every attention block of myk-llm (mixers.py:72-118):

    qk_norm_rope(q, k, position_ids, cos, sin, q_weight=None, k_weight=None, eps=1e-6)
        -> (q, k)      q/k RMSNorm cast back to the input type, then RoPE (mixers.py:85-89)
    qkv_norm_rope(qkv, num_heads, num_kv_heads, head_dim, position_ids, cos, sin,
                  q_weight=None, k_weight=None, eps=1e-6)
        -> (q, k, v)   the same on the fused projection output (mixers.py:81-84): v is a view
                       of qkv, and the backward writes the whole d(qkv) in one launch
    output_gate(out, gate) -> out * sigmoid(gate)           (mixers.py:116-117)
    rope_tables(head_dim, length, base, device)  -> (cos, sin)  (layers.py:80-85)

Semantics follow the reference modules under bf16 autocast, its training default
(train/config.py:101-104): RMSNorm (layers.py:15-25) in fp32 with fp32 weights, rounded to
the input type (`.to(v.dtype)`, mixers.py:87); RotaryEmbedding.rotate (layers.py:93-98) on
interleaved pairs in fp32, rounded back; the gate's sigmoid rounded to the input type, then
the product. position_ids index the cos/sin tables row-wise like `cos_cached[position_ids]`
(positions outside the table read its nearest row instead of raising).

Every element is computed by the kernels of libmykfa.so (csrc/block_io.hip) through its C
ABI on torch's current stream; Python validates, allocates outputs with torch's caching
allocator and passes pointers. There is no CPU or PyTorch fallback.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch
from torch import Tensor

from . import _lib
from .flash_attn import _DeviceGuard, _dtype_code, _ptr, _stream

_HEAD_DIMS = (16, 32, 64, 128, 256)


# --- helpers ---------------------------------------------------------------------------------


def _ready(x: Tensor) -> Tensor:
    """16-byte aligned base and strides that are multiples of 8 elements along a contiguous
    last dimension (the kernels' 16-byte accesses); anything else is copied once."""
    if x.stride(-1) == 1 and x.data_ptr() % 16 == 0 and all(s % 8 == 0 for s in x.stride()[:-1]):
        return x
    return x.contiguous()


def _bshd(x: Tensor) -> Tensor:
    """(batch, seq, heads, D) view of a 4-D tensor or of a packed (tokens, heads, D) one."""
    return x if x.dim() == 4 else x.unsqueeze(0)


def _strides3(x: Tensor) -> tuple[int, int, int]:
    return x.stride(0), x.stride(1), x.stride(2)


def _check_qk(q: Tensor, k: Tensor) -> None:
    if not (q.is_cuda and k.is_cuda):
        raise RuntimeError("the q/k prologue is CUDA-only: q and k must be GPU (HIP) tensors")
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype:
        raise TypeError(f"the q/k prologue needs matching bf16/fp16 q and k; got {q.dtype}, {k.dtype}")
    if q.dim() not in (3, 4) or k.dim() != q.dim():
        raise ValueError("q and k must both be (batch, seq, heads, head_dim) or (tokens, heads, head_dim)")
    if q.shape[-1] not in _HEAD_DIMS or k.shape[-1] != q.shape[-1]:
        raise ValueError(f"head_dim must be one of {list(_HEAD_DIMS)} for q and k; got {q.shape[-1]}, {k.shape[-1]}")
    if q.shape[:-2] != k.shape[:-2]:
        raise ValueError(f"q and k must have the same leading (batch, seq) shape; got {tuple(q.shape)}, {tuple(k.shape)}")


def _positions(position_ids: Tensor, batch: int, seqlen: int, device) -> Tensor:
    """int64 positions viewed as (batch, seqlen) (broadcast like cos_cached[position_ids])."""
    if position_ids.device != device:
        raise ValueError("position_ids must be on the same device as q and k")
    pos = position_ids.to(torch.int64)
    if pos.dim() == 1:
        pos = pos.unsqueeze(0)
    if pos.dim() != 2:
        raise ValueError(f"position_ids must be (batch, seq) or (seq,); got {tuple(position_ids.shape)}")
    return pos.expand(batch, seqlen)


def _table(t: Tensor, head_dim: int, device) -> Tensor:
    if t.dim() != 2 or t.shape[1] != head_dim:
        raise ValueError(f"cos/sin tables must be (positions, head_dim={head_dim}); got {tuple(t.shape)}")
    t = t.to(device=device, dtype=torch.float32)
    if t.stride(1) != 1 or t.stride(0) % 4 or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def _weight(w: Tensor, head_dim: int, device) -> Tensor:
    if w.shape != (head_dim,):
        raise ValueError(f"RMSNorm weights must be ({head_dim},); got {tuple(w.shape)}")
    w = w.to(device=device, dtype=torch.float32)
    return w if w.is_contiguous() and w.data_ptr() % 16 == 0 else w.contiguous()


def _prologue_params(q_in, k_in, q_out, k_out, pos, cos, sin, qw, kw, eps) -> _lib.QkPrologueParams:
    """q_in/k_in/q_out/k_out are 4-D (batch, seq, heads, D)."""
    p = _lib.QkPrologueParams()
    p.q_in, p.k_in, p.q_out, p.k_out = _ptr(q_in), _ptr(k_in), _ptr(q_out), _ptr(k_out)
    p.qi_batch_stride, p.qi_token_stride, p.qi_head_stride = _strides3(q_in)
    p.ki_batch_stride, p.ki_token_stride, p.ki_head_stride = _strides3(k_in)
    if q_out is not None:
        p.qo_batch_stride, p.qo_token_stride, p.qo_head_stride = _strides3(q_out)
        p.ko_batch_stride, p.ko_token_stride, p.ko_head_stride = _strides3(k_out)
    if cos is not None:
        p.position_ids = pos.data_ptr()
        p.pos_batch_stride, p.pos_token_stride = pos.stride(0), pos.stride(1)
        p.cos, p.sin = cos.data_ptr(), sin.data_ptr()
        if sin.stride(0) != cos.stride(0):
            raise ValueError("cos and sin tables must share one row stride")
        p.table_stride, p.table_rows = cos.stride(0), min(cos.shape[0], sin.shape[0])
    p.q_weight, p.k_weight = _ptr(qw), _ptr(kw)
    p.eps = float(eps)
    p.batch, p.seqlen = q_in.shape[0], q_in.shape[1]
    p.num_heads, p.num_kv_heads, p.head_dim = q_in.shape[2], k_in.shape[2], q_in.shape[3]
    p.dtype = _dtype_code(q_in.dtype)
    return p


def _launch_prologue(q_in, k_in, pos, cos, sin, qw, kw, eps):
    q_out = torch.empty(q_in.shape, dtype=q_in.dtype, device=q_in.device)
    k_out = torch.empty(k_in.shape, dtype=k_in.dtype, device=k_in.device)
    p = _prologue_params(q_in, k_in, q_out, k_out, pos, cos, sin, qw, kw, eps)
    with _DeviceGuard(q_in.device):
        _lib.check(_lib.lib().mykfa_qk_prologue_fwd(ctypes.byref(p), _stream(q_in.device)))
    return q_out, k_out


def _launch_prologue_bwd(q_in, k_in, pos, cos, sin, qw, kw, eps, dq_out, dk_out, dq_in, dk_in,
                         dv_src=None, dv_dst=None):
    """Writes dq_in/dk_in (and dv_dst); returns the weight gradients (or None, None)."""
    L = _lib.lib()
    f = _prologue_params(q_in, k_in, None, None, pos, cos, sin, qw, kw, eps)
    b = _lib.QkPrologueBwdParams()
    b.fwd = f
    b.dq_out, b.dk_out, b.dq_in, b.dk_in = dq_out.data_ptr(), dk_out.data_ptr(), dq_in.data_ptr(), dk_in.data_ptr()
    b.dqo_batch_stride, b.dqo_token_stride, b.dqo_head_stride = _strides3(dq_out)
    b.dko_batch_stride, b.dko_token_stride, b.dko_head_stride = _strides3(dk_out)
    b.dqi_batch_stride, b.dqi_token_stride, b.dqi_head_stride = _strides3(dq_in)
    b.dki_batch_stride, b.dki_token_stride, b.dki_head_stride = _strides3(dk_in)
    if dv_src is not None:
        b.dv_src, b.dv_dst = dv_src.data_ptr(), dv_dst.data_ptr()
        b.dvs_batch_stride, b.dvs_token_stride, b.dvs_head_stride = _strides3(dv_src)
        b.dvd_batch_stride, b.dvd_token_stride, b.dvd_head_stride = _strides3(dv_dst)
    dqw = dkw = ws = None
    nbytes = 0
    if qw is not None:
        d = q_in.shape[-1]
        dqw = torch.empty(d, dtype=torch.float32, device=q_in.device)
        dkw = torch.empty(d, dtype=torch.float32, device=q_in.device)
        b.dq_weight, b.dk_weight = dqw.data_ptr(), dkw.data_ptr()
        nbytes = L.mykfa_qk_prologue_bwd_workspace_size(f.batch, f.seqlen, f.num_heads, f.num_kv_heads, f.head_dim)
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q_in.device)
    with _DeviceGuard(q_in.device):
        _lib.check(L.mykfa_qk_prologue_bwd(ctypes.byref(b), _ptr(ws), nbytes, _stream(q_in.device)))
    return dqw, dkw


def _grad_or_zeros(g: Optional[Tensor], like: Tensor) -> Tensor:
    return torch.zeros_like(like) if g is None else _ready(_bshd(g))


# --- autograd ----------------------------------------------------------------------------------


class _QkNormRope(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, q_weight, k_weight, pos, cos, sin, eps):  # pyright: ignore[reportIncompatibleMethodOverride]
        q4, k4 = _ready(_bshd(q)), _ready(_bshd(k))
        q_out, k_out = _launch_prologue(q4, k4, pos, cos, sin, q_weight, k_weight, eps)
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(q4, k4, q_weight, k_weight, pos, cos, sin)
        ctx.eps, ctx.packed = eps, q.dim() == 3
        if ctx.packed:
            return q_out[0], k_out[0]
        return q_out, k_out

    @staticmethod
    def backward(ctx, dq, dk):  # pyright: ignore[reportIncompatibleMethodOverride]
        q4, k4, qw, kw, pos, cos, sin = ctx.saved_tensors
        dq4, dk4 = _grad_or_zeros(dq, q4), _grad_or_zeros(dk, k4)
        dq_in, dk_in = torch.empty_like(q4), torch.empty_like(k4)
        dqw, dkw = _launch_prologue_bwd(q4, k4, pos, cos, sin, qw, kw, ctx.eps, dq4, dk4, dq_in, dk_in)
        if ctx.packed:
            dq_in, dk_in = dq_in[0], dk_in[0]
        return dq_in, dk_in, dqw, dkw, None, None, None, None


class _QkvNormRope(torch.autograd.Function):
    @staticmethod
    def forward(ctx, qkv, q_weight, k_weight, pos, cos, sin, eps, num_heads, num_kv_heads, head_dim):  # pyright: ignore[reportIncompatibleMethodOverride]
        lead = qkv.shape[:-1]
        x = qkv if qkv.dim() == 3 else qkv.unsqueeze(0)
        b, s = x.shape[0], x.shape[1]
        qs, ks = num_heads * head_dim, num_kv_heads * head_dim
        q_in = x[..., :qs].view(b, s, num_heads, head_dim)
        k_in = x[..., qs:qs + ks].view(b, s, num_kv_heads, head_dim)
        q_out, k_out = _launch_prologue(q_in, k_in, pos, cos, sin, q_weight, k_weight, eps)
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(qkv, q_weight, k_weight, pos, cos, sin)
        ctx.meta = (eps, num_heads, num_kv_heads, head_dim)
        v = qkv[..., qs + ks:].view(*lead, num_kv_heads, head_dim)
        if qkv.dim() == 2:
            return q_out[0], k_out[0], v
        return q_out, k_out, v

    @staticmethod
    def backward(ctx, dq, dk, dv):  # pyright: ignore[reportIncompatibleMethodOverride]
        qkv, qw, kw, pos, cos, sin = ctx.saved_tensors
        eps, hq, hkv, d = ctx.meta
        x = qkv if qkv.dim() == 3 else qkv.unsqueeze(0)
        b, s = x.shape[0], x.shape[1]
        qs, ks = hq * d, hkv * d
        q_in = x[..., :qs].view(b, s, hq, d)
        k_in = x[..., qs:qs + ks].view(b, s, hkv, d)
        dqkv = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        dq_in = dqkv[..., :qs].view(b, s, hq, d)
        dk_in = dqkv[..., qs:qs + ks].view(b, s, hkv, d)
        dv_dst = dqkv[..., qs + ks:].view(b, s, hkv, d)
        dq4, dk4 = _grad_or_zeros(dq, q_in), _grad_or_zeros(dk, k_in)
        if dv is None:
            dv_dst.zero_()
            dv_src = None
        else:
            dv_src = _ready(_bshd(dv))
        dqw, dkw = _launch_prologue_bwd(q_in, k_in, pos, cos, sin, qw, kw, eps, dq4, dk4, dq_in, dk_in,
                                        dv_src, None if dv_src is None else dv_dst)
        return dqkv.view(qkv.shape), dqw, dkw, None, None, None, None, None, None, None


class _OutputGate(torch.autograd.Function):
    @staticmethod
    def forward(ctx, out, gate):  # pyright: ignore[reportIncompatibleMethodOverride]
        x2, g2 = _rows(out), _rows(gate)
        y = torch.empty(out.shape, dtype=out.dtype, device=out.device)
        p = _gate_params(x2, g2, y.view(-1, out.shape[-1]))
        with _DeviceGuard(out.device):
            _lib.check(_lib.lib().mykfa_gate_fwd(ctypes.byref(p), _stream(out.device)))
        ctx.save_for_backward(x2, g2)
        ctx.shape = out.shape
        return y

    @staticmethod
    def backward(ctx, dy):  # pyright: ignore[reportIncompatibleMethodOverride]
        x2, g2 = ctx.saved_tensors
        dy2 = _rows(dy)
        dx = torch.empty(ctx.shape, dtype=x2.dtype, device=x2.device)
        dg = torch.empty(ctx.shape, dtype=x2.dtype, device=x2.device)
        w = x2.shape[1]
        p = _gate_params(x2, g2, None, dy2, dx.view(-1, w), dg.view(-1, w))
        with _DeviceGuard(x2.device):
            _lib.check(_lib.lib().mykfa_gate_bwd(ctypes.byref(p), _stream(x2.device)))
        return dx, dg


def _rows(x: Tensor) -> Tensor:
    """(rows, width) view with a 16-byte aligned base and a row stride of 8k elements."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(1) != 1 or x2.data_ptr() % 16 or x2.stride(0) % 8:
        x2 = x2.contiguous()
    return x2


def _gate_params(x2, g2, y2, dy2=None, dx2=None, dg2=None) -> _lib.GateParams:
    p = _lib.GateParams()
    p.x, p.gate, p.y = x2.data_ptr(), g2.data_ptr(), _ptr(y2)
    p.dy, p.dx, p.dgate = _ptr(dy2), _ptr(dx2), _ptr(dg2)
    p.x_row_stride, p.gate_row_stride = x2.stride(0), g2.stride(0)
    p.y_row_stride = 0 if y2 is None else y2.stride(0)
    p.dy_row_stride = 0 if dy2 is None else dy2.stride(0)
    p.dx_row_stride = 0 if dx2 is None else dx2.stride(0)
    p.dgate_row_stride = 0 if dg2 is None else dg2.stride(0)
    p.rows, p.width = x2.shape[0], x2.shape[1]
    p.dtype = _dtype_code(x2.dtype)
    return p


# --- public API --------------------------------------------------------------------------------


def rope_tables(head_dim: int, length: int, base: float, device=None) -> tuple[Tensor, Tensor]:
    """RotaryEmbedding's fp32 cos/sin tables (layers.py:80-85): angles pos * base^(-2i/D),
    each repeated for the two elements of pair i, so row p holds (cos, cos, ...) per pair."""
    if head_dim % 2:
        raise ValueError("head_dim must be even for RoPE")
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim))
    angles = torch.outer(torch.arange(length, dtype=torch.float32, device=device), inv_freq)
    angles = torch.repeat_interleave(angles, repeats=2, dim=-1)
    return angles.cos(), angles.sin()


def _prep(q, k, position_ids, cos, sin, q_weight, k_weight):
    d = q.shape[-1]
    if (q_weight is None) != (k_weight is None):
        raise ValueError("q_weight and k_weight must both be given or both be None")
    if (cos is None) != (sin is None):
        raise ValueError("cos and sin must both be given or both be None")
    q4 = _bshd(q)
    pos = None
    if cos is not None:
        if position_ids is None:
            raise ValueError("position_ids are required with cos/sin tables")
        pos = _positions(position_ids, q4.shape[0], q4.shape[1], q.device)
        cos, sin = _table(cos, d, q.device), _table(sin, d, q.device)
    if q_weight is not None:
        q_weight, k_weight = _weight(q_weight, d, q.device), _weight(k_weight, d, q.device)
    return pos, cos, sin, q_weight, k_weight


def qk_norm_rope(q: Tensor, k: Tensor, position_ids: Optional[Tensor], cos: Optional[Tensor], sin: Optional[Tensor],
                 q_weight: Optional[Tensor] = None, k_weight: Optional[Tensor] = None,
                 eps: float = 1e-6) -> tuple[Tensor, Tensor]:
    """q/k RMSNorm (when weights are given) then RoPE (when tables are given), fused
    (mixers.py:85-89). q (batch, seq, Hq, D) or packed (tokens, Hq, D); k likewise with Hkv
    heads; any strides with a contiguous last dimension (views of a fused projection work).
    Returns new contiguous q, k in the input type; differentiable in q, k and the weights."""
    _check_qk(q, k)
    pos, cos, sin, qw, kw = _prep(q, k, position_ids, cos, sin, q_weight, k_weight)
    return _QkNormRope.apply(q, k, qw, kw, pos, cos, sin, float(eps))


def qkv_norm_rope(qkv: Tensor, num_heads: int, num_kv_heads: int, head_dim: int, position_ids: Optional[Tensor],
                  cos: Optional[Tensor], sin: Optional[Tensor], q_weight: Optional[Tensor] = None,
                  k_weight: Optional[Tensor] = None, eps: float = 1e-6) -> tuple[Tensor, Tensor, Tensor]:
    """The prologue on the fused projection output qkv (batch, seq, (Hq + 2 Hkv) D) or packed
    (tokens, ...), split as q | k | v like mixers.py:81-84. Returns new q, k and v as a view of
    qkv. The backward writes d(qkv) — the q and k gradients and a copy of v's — in one launch
    instead of a gradient per slice and a concatenation."""
    if not qkv.is_cuda:
        raise RuntimeError("the q/k prologue is CUDA-only: qkv must be a GPU (HIP) tensor")
    if qkv.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"the q/k prologue needs a bf16/fp16 qkv; got {qkv.dtype}")
    if head_dim not in _HEAD_DIMS:
        raise ValueError(f"head_dim must be one of {list(_HEAD_DIMS)}; got {head_dim}")
    if qkv.dim() not in (2, 3) or qkv.shape[-1] != (num_heads + 2 * num_kv_heads) * head_dim:
        raise ValueError(f"qkv must be (batch, seq, (Hq + 2 Hkv) * D) or (tokens, ...); got {tuple(qkv.shape)}")
    if qkv.stride(-1) != 1 or qkv.data_ptr() % 16 or any(st % 8 for st in qkv.stride()[:-1]):
        qkv = qkv.contiguous()
    x = qkv if qkv.dim() == 3 else qkv.unsqueeze(0)
    q_view = x[..., : num_heads * head_dim].view(x.shape[0], x.shape[1], num_heads, head_dim)
    pos, cos, sin, qw, kw = _prep(q_view, None, position_ids, cos, sin, q_weight, k_weight)
    return _QkvNormRope.apply(qkv, qw, kw, pos, cos, sin, float(eps), num_heads, num_kv_heads, head_dim)


def output_gate(out: Tensor, gate: Tensor) -> Tensor:
    """out * sigmoid(gate) (mixers.py:116-117), same shapes, last dimension a multiple of 8;
    the sigmoid is rounded to the input type before the product, as under autocast."""
    if not (out.is_cuda and gate.is_cuda):
        raise RuntimeError("the output gate is CUDA-only: out and gate must be GPU (HIP) tensors")
    if out.dtype not in (torch.bfloat16, torch.float16) or gate.dtype != out.dtype:
        raise TypeError(f"the output gate needs matching bf16/fp16 tensors; got {out.dtype}, {gate.dtype}")
    if out.shape != gate.shape:
        raise ValueError(f"out and gate must have the same shape; got {tuple(out.shape)}, {tuple(gate.shape)}")
    if out.dim() == 0 or out.shape[-1] % 8:
        raise ValueError(f"the last dimension must be a multiple of 8; got {tuple(out.shape)}")
    return _OutputGate.apply(out, gate)

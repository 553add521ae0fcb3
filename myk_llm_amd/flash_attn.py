"""Host side of the MI355X FlashAttention that stands in for myk-llm's
src/myk_llm/ops/flash_attn.py.

Entry points. Their names, positional arguments, defaults and exception types are the
reference's (flash_attn.py:442-490), so Attention.forward, generate() and the decode
benchmark call them unchanged:

    flash_attn_func          dense batches, q (B, Sq, Hq, D) against k / v (B, Sk, Hkv, D)
    flash_attn_varlen_func   documents packed along the token axis and delimited by int32
                             cu_seqlens offsets
    flash_attn_with_kvcache  stores this step's keys / values in a preallocated per-sequence
                             cache and attends over the grown cache; no gradient, and safe
                             to capture in a HIP graph

Keyword-only ``return_softmax_lse=False`` is this build's one addition: with True the call
also hands back the fp32 log-sum-exp in base 2, one row per query head ``(Hq, rows)``, which is
what the backward consumes.

Masking. Queries line up with the END of their keys. With Lq queries and Lk keys in a
sequence, query i may attend to key j exactly when j - i lies in
[Lk - Lq - left, Lk - Lq + right]; ``window_size = (left, right)`` with -1 meaning no limit on
that side, and ``causal=True`` pins right to 0. GQA maps query head h to key/value head
h // (Hq / Hkv). Inputs are bf16 or fp16 with head_dim 16, 32, 64, 128 or 256.

Every FLOP runs in libmykfa.so's gfx950 kernels, reached through its C ABI (include/mykfa.h)
on torch's current stream. This module checks arguments, allocates outputs from torch's
caching allocator and passes pointers; when the library is missing every call raises, as
nothing here can compute attention on its own.
"""

from __future__ import annotations

import ctypes
import math
import os
from typing import Optional

import torch
from torch import Tensor

from . import _lib

_UNBOUNDED = _lib.UNBOUNDED  # flash_attn.py:32
_HEAD_DIMS = (16, 32, 64, 128, 256)  # flash_attn.py:322-323
_DECODE_MAX_Q = 16  # few queries per sequence use the split-K decode kernel (flash_attn.py:364)


def _ds_budget_bytes() -> int:
    """Most device memory the backward may take for its stored dS (bf16, one 32 x 32 block per
    (query tile, key block) pair of the band, bounded per query tile by the band width): 4 GiB
    unless MYKFA_BWD_DS_MAX_MB says otherwise (0 turns the stored-dS backward off)."""
    mb = os.environ.get("MYKFA_BWD_DS_MAX_MB")
    return (4 << 30) if mb is None else int(mb) << 20


# Requests above this size are also checked against the device's free memory first.
_DS_CHECK_FREE_ABOVE = 256 << 20


def _available_bytes(device: torch.device) -> int:
    """Device memory a new allocation can take without evicting anything: the driver's free
    memory plus what torch's caching allocator holds unused."""
    free, _ = torch.cuda.mem_get_info(device)
    return free + max(torch.cuda.memory_reserved(device) - torch.cuda.memory_allocated(device), 0)


def _plan_ds_workspace(per_head: int, kv_heads: int, budget: int, alloc, available=None):
    """The stored-dS workspace of the backward: (KV heads per pass, buffer), or (0, None) for
    the recomputing backward. Which backward runs depends on the shape alone (one KV head's
    workspace within the budget); how many KV heads share a pass may also depend on free
    memory, which changes no result bit (KV heads are independent). Takes as many KV heads
    per pass as the budget allows (at most every head); a request above _DS_CHECK_FREE_ABOVE
    is capped at 80 % of `available()` bytes, but never below one head, and an allocation that
    still fails (torch.OutOfMemoryError) is retried with half as many heads. Only when one head's
    workspace cannot be allocated at all does the call take the recomputing backward (results
    within the same tolerance of the reference, not bitwise those of the stored-dS one)."""
    heads = min(kv_heads, budget // per_head) if per_head > 0 else 0
    if heads > 1 and available is not None and heads * per_head > _DS_CHECK_FREE_ABOVE:
        heads = max(1, min(heads, int(0.8 * available()) // per_head))
    while heads > 0:
        try:
            return heads, alloc(heads * per_head)
        except torch.OutOfMemoryError:
            heads //= 2
    return 0, None


# --- validation (flash_attn.py:331-350) ---------------------------------------------------


def _check_meta(q: Tensor, k: Tensor, v: Tensor) -> None:
    """dtype / head_dim / head-ratio checks of _check (flash_attn.py:340-346)."""
    head_dim = q.shape[-1]
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError(f"flash attention needs matching bf16/fp16 q, k, v; got {q.dtype}, {k.dtype}, {v.dtype}")
    if head_dim not in _HEAD_DIMS or k.shape[-1] != head_dim or v.shape[-1] != head_dim:
        raise ValueError(f"head_dim must be one of {list(_HEAD_DIMS)} for q, k and v; got "
                         f"{q.shape[-1]}, {k.shape[-1]}, {v.shape[-1]}")
    if q.shape[-2] % k.shape[-2] or k.shape[-2] != v.shape[-2]:
        raise ValueError(f"query heads ({q.shape[-2]}) must be a multiple of key/value heads ({k.shape[-2]})")


def _check(q: Tensor, k: Tensor, v: Tensor) -> None:
    """flash_attn.py:336-346, same order and exception types."""
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("flash attention is CUDA-only: q, k and v must be GPU (HIP) tensors")
    _check_meta(q, k, v)
    _same_device(q.device, k=k, v=v)


def _same_device(device: torch.device, **tensors: Optional[Tensor]) -> None:
    """Every tensor the kernels dereference must live on q's GPU. A host tensor (or one on
    another GPU) would hand the kernel a pointer it cannot read; the reference fails the
    same calls with a RuntimeError (a device mismatch in torch, or Triton refusing a host
    pointer), and so does this, before anything is launched."""
    for name, t in tensors.items():
        if t is not None and t.device != device:
            raise RuntimeError(f"every tensor must be on the same GPU: {name} is on {t.device}, expected {device}")


def _last_dim_contiguous(x: Tensor) -> Tensor:
    return x if x.stride(-1) == 1 else x.contiguous()


def _strides(x: Tensor) -> tuple[int, int, int]:
    """(batch, token, head) strides in elements; batch is 0 for packed varlen tensors."""
    s = x.stride()
    return (s[0], s[1], s[2]) if len(s) == 4 else (0, s[0], s[1])


def _kernel_ready(x: Tensor) -> Tensor:
    """The kernels read 16 bytes at a time along head_dim: a 16-byte aligned base and
    strides that are multiples of 8 elements. Anything else is copied once."""
    s = x.stride()
    odd = 0
    for v in s[:-1]:
        odd |= v
    if s[-1] == 1 and not (odd & 7) and not (x.data_ptr() & 15):
        return x
    return x.contiguous()


def _window(causal: bool, window_size: tuple[int, int]) -> tuple[int, int]:
    """flash_attn.py:435-439."""
    left, right = window_size
    left = _UNBOUNDED if left < 0 else left
    right = 0 if causal else (_UNBOUNDED if right < 0 else right)
    return left, right


def _dtype_code(dtype: torch.dtype) -> int:
    return _lib.DTYPE_BF16 if dtype == torch.bfloat16 else _lib.DTYPE_FP16


def _stream(device: torch.device) -> int:
    """The raw hipStream_t of torch's current stream on device (no Stream object is built:
    this runs on every launch)."""
    return torch._C._cuda_getCurrentRawStream(device.index if device.index is not None
                                               else torch.cuda.current_device())


def _ptr(x: Optional[Tensor]) -> Optional[int]:
    return None if x is None else x.data_ptr()


class _DeviceGuard:
    """Makes x's device current for the launch when it is not already."""

    def __init__(self, device: torch.device):
        self.device = device
        self.guard = None

    def __enter__(self):
        if self.device.index is not None and self.device.index != torch.cuda.current_device():
            self.guard = torch.cuda.device(self.device)
            self.guard.__enter__()

    def __exit__(self, *exc):
        if self.guard is not None:
            self.guard.__exit__(*exc)


def _fwd_values(q, k, v, out, lse, cu_q, cu_k, seqused_k, max_q, max_k, scale, wl, wr) -> tuple:
    """The fields of mykfa_fwd_params, in declaration order (NULL pointers as 0)."""
    varlen = cu_q is not None
    return (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
            *_strides(q), *_strides(k), *_strides(v), *_strides(out), lse.stride(0),
            0 if cu_q is None else cu_q.data_ptr(), 0 if cu_k is None else cu_k.data_ptr(),
            0 if seqused_k is None else seqused_k.data_ptr(),
            cu_q.numel() - 1 if varlen else q.shape[0], q.shape[-2], k.shape[-2], q.shape[-1],
            max_q, max_k, wl, wr, scale, _dtype_code(q.dtype))


def _bwd_values(fwd_values: tuple, dout, dq, dk, dv, delta) -> tuple:
    """The fields of mykfa_bwd_params, in declaration order, after those of its fwd member."""
    return (*fwd_values, dout.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), delta.data_ptr(),
            *_strides(dout), *_strides(dq), *_strides(dk), *_strides(dv))


def _packed(packer, values):
    """A parameter block (bytes laid out as the C struct) filled in one call."""
    buf = bytearray(packer.size)
    packer.pack_into(buf, 0, *values)
    return buf


def _fwd_params(q, k, v, out, lse, cu_q, cu_k, seqused_k, max_q, max_k, scale, wl, wr) -> _lib.FwdParams:
    return _lib.FwdParams.from_buffer(_packed(_lib.FWD_PACK, _fwd_values(q, k, v, out, lse, cu_q, cu_k, seqused_k,
                                                                         max_q, max_k, scale, wl, wr)))


def _int32(x: Optional[Tensor]) -> Optional[Tensor]:
    if x is None:
        return None
    return x if (x.dtype == torch.int32 and x.is_contiguous()) else x.to(torch.int32).contiguous()


# --- launchers (flash_attn.py:353-406) ----------------------------------------------------


def _forward(q: Tensor, k: Tensor, v: Tensor, cu_seqlens_q: Optional[Tensor], cu_seqlens_k: Optional[Tensor],
             seqused_k: Optional[Tensor], max_seqlen_q: int, max_seqlen_k: int, softmax_scale: float,
             window_left: int, window_right: int) -> tuple[Tensor, Tensor]:
    """O and the base-2 LSE (num_heads, rows), fp32 (flash_attn.py:353-373)."""
    dev = q.device
    _same_device(dev, k=k, v=v, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k, seqused_k=seqused_k)
    varlen = cu_seqlens_q is not None
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    cu_q, cu_k, seqused = _int32(cu_seqlens_q), _int32(cu_seqlens_k), _int32(seqused_k)
    shape = q.shape
    out = torch.empty_like(q, memory_format=torch.contiguous_format)
    lse = q.new_empty((shape[-2], shape[0] if varlen else shape[0] * shape[1]), dtype=torch.float32)
    p = _lib.FwdParams.from_buffer(_packed(_lib.FWD_PACK, _fwd_values(
        q, k, v, out, lse, cu_q, cu_k, seqused, max_seqlen_q, max_seqlen_k, softmax_scale, window_left,
        window_right)))
    L = _lib.lib()
    with _DeviceGuard(dev):
        if not varlen and 0 < max_seqlen_q <= _DECODE_MAX_Q:
            _decode_launch(L, p, dev)
        else:
            _lib.check(L.mykfa_fwd(ctypes.byref(p), _stream(dev)))
    return out, lse


def _decode_launch(L, p: _lib.FwdParams, device: torch.device, k_new: Optional[Tensor] = None,
                   v_new: Optional[Tensor] = None) -> None:
    """Split-K decode with its LSE merge; the workspace comes from torch's allocator. With
    k_new / v_new the decode first writes them into the caches after seqused_k[b]."""
    d = _lib.DecodeParams()
    d.fwd = p
    splits = L.mykfa_decode_num_splits(p.batch, p.num_heads, p.num_kv_heads, p.max_seqlen_q, p.max_seqlen_k)
    d.num_splits = splits
    if k_new is not None:
        d.seqlen_new = k_new.shape[1]
        d.k_new, d.v_new = k_new.data_ptr(), v_new.data_ptr()
        d.kn_batch_stride, d.kn_token_stride, d.kn_head_stride = _strides(k_new)
        d.vn_batch_stride, d.vn_token_stride, d.vn_head_stride = _strides(v_new)
    nbytes = L.mykfa_decode_workspace_size(p.batch, p.num_heads, p.max_seqlen_q, p.head_dim, splits)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)
    _lib.check(L.mykfa_decode(ctypes.byref(d), ws.data_ptr(), ws.numel(), _stream(device)))


def _decode_append(q: Tensor, k_cache: Tensor, v_cache: Tensor, k: Tensor, v: Tensor, cache_seqlens: Tensor,
                   softmax_scale: float, window_left: int, window_right: int) -> tuple[Tensor, Tensor]:
    """flash_attn_with_kvcache for decode-sized q in one split-K launch plus its merge: the
    decode writes k / v into the caches itself (flash_attn.py:480-488)."""
    k, v = _kernel_ready(k), _kernel_ready(v)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty((q.shape[-2], q.shape[0] * q.shape[1]), dtype=torch.float32, device=q.device)
    p = _fwd_params(q, k_cache, v_cache, out, lse, None, None, cache_seqlens, q.shape[1], k_cache.shape[1],
                    softmax_scale, window_left, window_right)
    with _DeviceGuard(q.device):
        _decode_launch(_lib.lib(), p, q.device, k, v)
    return out, lse


def _backward(dout: Tensor, q: Tensor, k: Tensor, v: Tensor, out: Tensor, lse: Tensor,
              cu_seqlens_q: Optional[Tensor], cu_seqlens_k: Optional[Tensor], max_seqlen_q: int,
              max_seqlen_k: int, softmax_scale: float, window_left: int,
              window_right: int) -> tuple[Tensor, Tensor, Tensor]:
    """dQ, dK, dV (flash_attn.py:376-406)."""
    _same_device(q.device, dout=dout, k=k, v=v, out=out, lse=lse, cu_seqlens_q=cu_seqlens_q,
                 cu_seqlens_k=cu_seqlens_k)
    return _backward_launch(dout, q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                            softmax_scale, window_left, window_right)


def _backward_launch(dout, q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                     softmax_scale, window_left, window_right):
    """_backward once every tensor is known to be on q's GPU (the autograd node's saved tensors
    were checked by its forward; the incoming gradient is on the output's device)."""
    dev = q.device
    dout = _kernel_ready(dout)
    q, k, v, out = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v), _kernel_ready(out)
    cu_q, cu_k = _int32(cu_seqlens_q), _int32(cu_seqlens_k)
    fmt = torch.contiguous_format
    dq = torch.empty_like(q, memory_format=fmt)
    dk = torch.empty_like(k, memory_format=fmt)
    dv = torch.empty_like(v, memory_format=fmt)
    delta = torch.empty_like(lse)
    p = _lib.BwdParams.from_buffer(_packed(_lib.BWD_PACK, _bwd_values(_fwd_values(
        q, k, v, out, lse, cu_q, cu_k, None, max_seqlen_q, max_seqlen_k, softmax_scale, window_left, window_right),
        dout, dq, dk, dv, delta)))
    L = _lib.lib()
    with _DeviceGuard(dev):
        # dK/dV store dS and dQ is formed from it (five products per block pair instead of
        # seven) when at least one KV head's dS fits the budget; KV heads then go in passes.
        # Under graph capture the free-memory query is skipped (the budget alone sizes the
        # passes; the graph's memory pool serves the allocation).
        per_head = L.mykfa_bwd_workspace_per_kv_head(ctypes.byref(p))
        available = None if torch.cuda.is_current_stream_capturing() else (lambda: _available_bytes(dev))
        heads, ws = (_plan_ds_workspace(per_head, k.shape[-2], _ds_budget_bytes(),
                                        lambda n: torch.empty(n, dtype=torch.uint8, device=dev),
                                        available) if per_head else (0, None))
        if heads > 0:
            _lib.check(L.mykfa_bwd_ws(ctypes.byref(p), ws.data_ptr(), ws.numel(), _stream(dev)))
        else:
            _lib.check(L.mykfa_bwd(ctypes.byref(p), _stream(dev)))
    return dq, dk, dv


def _check_append(k_cache: Tensor, v_cache: Tensor, k: Tensor, v: Tensor, cache_seqlens: Tensor) -> None:
    """The cache write copies 16-bit elements as they are: the new keys / values must have
    the caches' dtype (the reference's index write raises on a mismatch too) and live on
    the caches' GPU."""
    if not (k.dtype == v.dtype == k_cache.dtype == v_cache.dtype):
        raise TypeError(f"new keys/values ({k.dtype}, {v.dtype}) must match the caches' dtype "
                        f"({k_cache.dtype}, {v_cache.dtype})")
    _same_device(k_cache.device, v_cache=v_cache, k=k, v=v, cache_seqlens=cache_seqlens)


def _kv_append(k_cache: Tensor, v_cache: Tensor, k: Tensor, v: Tensor, cache_seqlens: Tensor) -> None:
    """cache[b, cache_seqlens[b] + t] = new[b, t] (flash_attn.py:480-485)."""
    _check_append(k_cache, v_cache, k, v, cache_seqlens)
    k, v = _kernel_ready(k), _kernel_ready(v)
    seqlens = _int32(cache_seqlens)
    p = _lib.KvAppendParams()
    p.k_cache, p.v_cache, p.k_new, p.v_new = k_cache.data_ptr(), v_cache.data_ptr(), k.data_ptr(), v.data_ptr()
    p.cache_seqlens = seqlens.data_ptr()
    p.kc_batch_stride, p.kc_token_stride, p.kc_head_stride = _strides(k_cache)
    p.vc_batch_stride, p.vc_token_stride, p.vc_head_stride = _strides(v_cache)
    p.kn_batch_stride, p.kn_token_stride, p.kn_head_stride = _strides(k)
    p.vn_batch_stride, p.vn_token_stride, p.vn_head_stride = _strides(v)
    p.batch, p.seqlen_new, p.capacity = k.shape[0], k.shape[1], k_cache.shape[1]
    p.num_kv_heads, p.head_dim, p.dtype = k.shape[2], k.shape[3], _dtype_code(k.dtype)
    L = _lib.lib()
    with _DeviceGuard(k_cache.device):
        _lib.check(L.mykfa_kv_append(ctypes.byref(p), _stream(k_cache.device)))


# --- torch.library ops: opaque to torch.compile, so fullgraph tracing needs no break ------


@torch.library.custom_op("mykfa::fwd", mutates_args=())
def _fwd_op(q: Tensor, k: Tensor, v: Tensor, cu_seqlens_q: Optional[Tensor], cu_seqlens_k: Optional[Tensor],
            seqused_k: Optional[Tensor], max_seqlen_q: int, max_seqlen_k: int, softmax_scale: float,
            window_left: int, window_right: int) -> tuple[Tensor, Tensor]:
    return _forward(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, max_seqlen_q, max_seqlen_k, softmax_scale,
                    window_left, window_right)


@_fwd_op.register_fake
def _(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, max_seqlen_q, max_seqlen_k, softmax_scale, window_left,
      window_right):
    rows = q.shape[0] if cu_seqlens_q is not None else q.shape[0] * q.shape[1]
    return torch.empty_like(q, memory_format=torch.contiguous_format), q.new_empty((q.shape[-2], rows),
                                                                                   dtype=torch.float32)


@torch.library.custom_op("mykfa::bwd", mutates_args=())
def _bwd_op(dout: Tensor, q: Tensor, k: Tensor, v: Tensor, out: Tensor, lse: Tensor,
            cu_seqlens_q: Optional[Tensor], cu_seqlens_k: Optional[Tensor], max_seqlen_q: int, max_seqlen_k: int,
            softmax_scale: float, window_left: int, window_right: int) -> tuple[Tensor, Tensor, Tensor]:
    return _backward(dout, q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                     softmax_scale, window_left, window_right)


@_bwd_op.register_fake
def _(dout, q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale,
      window_left, window_right):
    fmt = torch.contiguous_format
    return (torch.empty_like(q, memory_format=fmt), torch.empty_like(k, memory_format=fmt),
            torch.empty_like(v, memory_format=fmt))


@torch.library.custom_op("mykfa::kv_append", mutates_args=("k_cache", "v_cache"))
def _kv_append_op(k_cache: Tensor, v_cache: Tensor, k: Tensor, v: Tensor, cache_seqlens: Tensor) -> None:
    _kv_append(k_cache, v_cache, k, v, cache_seqlens)


@_kv_append_op.register_fake
def _(k_cache, v_cache, k, v, cache_seqlens):
    return None


def _compiling() -> bool:
    return torch.compiler.is_compiling()


def _fwd(*args):
    return _fwd_op(*args) if _compiling() else _forward(*args)



# --- autograd (flash_attn.py:412-429) ------------------------------------------------------


class _FlashAttn(torch.autograd.Function):
    """The autograd node (flash_attn.py:412-429). With with_lse the LSE is a second,
    non-differentiable output; without it (the common call) the node has one output, which
    spares the autograd engine an output edge per call."""

    @staticmethod
    def forward(ctx, q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale,
                window_left, window_right, with_lse):
        out, lse = _fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, None, max_seqlen_q, max_seqlen_k, softmax_scale,
                        window_left, window_right)
        ctx.save_for_backward(q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k)
        ctx.args = (max_seqlen_q, max_seqlen_k, softmax_scale, window_left, window_right)
        ctx.set_materialize_grads(False)  # an unused output gets no zero-filled gradient
        if with_lse:
            ctx.mark_non_differentiable(lse)
            return out, lse
        return out

    @staticmethod
    def backward(ctx, dout, *_):  # pyright: ignore[reportIncompatibleMethodOverride]
        if dout is None:
            return (None,) * 11
        q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k = ctx.saved_tensors
        if _compiling():
            dq, dk, dv = _bwd_op(dout, q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k, *ctx.args)
        else:
            dq, dk, dv = _backward_launch(dout, q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k, *ctx.args)
        return dq, dk, dv, None, None, None, None, None, None, None, None


# --- public API (flash_attn.py:442-490) ----------------------------------------------------


def flash_attn_func(
    q: Tensor, k: Tensor, v: Tensor, causal: bool = False, window_size: tuple[int, int] = (-1, -1),
    softmax_scale: float | None = None, *, return_softmax_lse: bool = False,
):
    """Attention over a dense batch: q is (B, Sq, Hq, D) and k, v are (B, Sk, Hkv, D) with Hq a
    multiple of Hkv. Returns O shaped like q (and the base-2 LSE with return_softmax_lse)."""
    _check(q, k, v)
    q, k, v = (_last_dim_contiguous(x) for x in (q, k, v))
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    wl, wr = _window(causal, window_size)
    return _FlashAttn.apply(q, k, v, None, None, q.shape[1], k.shape[1], scale, wl, wr, return_softmax_lse)


def flash_attn_varlen_func(
    q: Tensor, k: Tensor, v: Tensor, cu_seqlens_q: Tensor, cu_seqlens_k: Tensor, max_seqlen_q: int,
    max_seqlen_k: int, causal: bool = False, window_size: tuple[int, int] = (-1, -1),
    softmax_scale: float | None = None, *, return_softmax_lse: bool = False,
):
    """Attention over packed documents: q is (Tq, Hq, D) and k, v are (Tk, Hkv, D); document b
    owns query rows [cu_seqlens_q[b], cu_seqlens_q[b + 1]) and key rows likewise from
    cu_seqlens_k (int32 offsets on q's GPU). max_seqlen_q / max_seqlen_k bound the longest
    document and only size the launch grid."""
    _check(q, k, v)
    _same_device(q.device, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k)
    q, k, v = (_last_dim_contiguous(x) for x in (q, k, v))
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    wl, wr = _window(causal, window_size)
    return _FlashAttn.apply(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, scale, wl, wr,
                            return_softmax_lse)


def flash_attn_with_kvcache(
    q: Tensor, k_cache: Tensor, v_cache: Tensor, k: Tensor | None = None, v: Tensor | None = None, *,
    cache_seqlens: Tensor, causal: bool = False, window_size: tuple[int, int] = (-1, -1),
    softmax_scale: float | None = None, return_softmax_lse: bool = False,
):
    """Decoding (or chunked prefill) against static caches k_cache / v_cache of shape
    (B, capacity, Hkv, D). Given k and v of shape (B, new, Hkv, D), sequence b's rows are first
    stored at cache positions cache_seqlens[b] + t; q then attends over the first
    cache_seqlens[b] + new positions of its sequence. Advancing cache_seqlens is left to the
    caller, and no gradient flows. A position at or past the capacity is not written (the
    reference's index write would fault there) and the attended length is clipped to the
    capacity."""
    _check(q, k_cache, v_cache)
    if k_cache.stride(-1) != 1 or v_cache.stride(-1) != 1:
        raise ValueError("the caches need a contiguous last dimension")
    _same_device(q.device, cache_seqlens=cache_seqlens)
    if k is not None and v is not None:
        _check_append(k_cache, v_cache, k, v, cache_seqlens)
    q = _last_dim_contiguous(q)
    seqused = cache_seqlens.to(torch.int32)
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    if k is not None and v is not None:
        # The reference's index writes (flash_attn.py:480-485) raise on a shape that does not
        # match (batch, new, kv_heads, head_dim) of the caches; so does this.
        want = (q.shape[0], k.shape[1], k_cache.shape[2], k_cache.shape[3])
        if tuple(k.shape) != want or tuple(v.shape) != want:
            raise RuntimeError(f"new keys/values of shapes {tuple(k.shape)}, {tuple(v.shape)} do not match "
                               f"the caches: expected {want}")
    if (k is not None and v is not None and not _compiling() and 0 < q.shape[1] <= _DECODE_MAX_Q
            and _kernel_ready(q) is q and _kernel_ready(k_cache) is k_cache and _kernel_ready(v_cache) is v_cache):
        _check_meta(q, k, v)
        out, lse = _decode_append(q, k_cache, v_cache, k, v, _int32(seqused), scale, *_window(causal, window_size))
        return (out, lse) if return_softmax_lse else out
    if k is not None and v is not None:
        if _compiling():
            _kv_append_op(k_cache, v_cache, k, v, seqused)
        else:
            _kv_append(k_cache, v_cache, k, v, seqused)
        seqused = seqused + k.shape[1]
    out, lse = _fwd(q, k_cache, v_cache, None, None, seqused, q.shape[1], k_cache.shape[1], scale,
                    *_window(causal, window_size))
    return (out, lse) if return_softmax_lse else out

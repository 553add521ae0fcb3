"""Fused linear + cross-entropy on MI355X (gfx950): the drop-in for myk-llm's
src/myk_llm/ops/fused_ce.py (exported by ops/__init__.py:2), same name, signature, defaults
and return values:

    fused_linear_cross_entropy(hidden, weight, targets, normalizer, z_loss=0.0,
                               ignore_index=-100, chunk_size=2048) -> (loss, ce_sum, z_sum)

loss = (sum of per-token CE + z_loss * sum of lse^2) / normalizer over supervised tokens;
ce_sum / z_sum are detached sums for logging (fused_ce.py:111-132). The (tokens, vocab)
logits are never materialized whole: tokens are processed in chunks, each chunk's logits
(hidden_chunk @ weight^T, bf16 GEMM with fp32 accumulation) are overwritten in place by the
gfx950 CE row kernel (csrc/fused_ce.hip, through the C ABI) with d loss / d logits, which the
next two GEMMs fold into the hidden and weight gradients at once. As in the reference the
gradient is computed during the forward pass, so the loss is backpropagated exactly once.

The three products per chunk are plain library GEMMs (torch.matmul on ROCm = hipBLASLt). The
weight gradient accumulates in fp32 inside the GEMM (beta = 1, fp32 output) instead of rounding
each chunk's bf16 product before an fp32 add (fused_ce.py:89): one pass over the fp32
gradient per chunk instead of three, and no bf16 rounding of the partial sums.
"""

from __future__ import annotations

import ctypes
from typing import cast

import torch
from torch import Tensor

from . import _lib
from .flash_attn import _DeviceGuard, _dtype_code, _same_device, _stream


def _ce_rows(logits: Tensor, targets: Tensor, ce: Tensor, lse: Tensor, scale: float, z_coef: float,
             ignore_index: int) -> None:
    """The row kernel on one chunk: lse, ce, and logits := d loss / d logits, in place."""
    p = _lib.CeParams()
    p.logits, p.targets, p.ce, p.lse = logits.data_ptr(), targets.data_ptr(), ce.data_ptr(), lse.data_ptr()
    p.row_stride, p.rows, p.vocab = logits.stride(0), logits.shape[0], logits.shape[1]
    p.ignore_index = int(ignore_index)
    p.scale, p.z_coef = float(scale), float(z_coef)
    p.dtype = _dtype_code(logits.dtype)
    _lib.check(_lib.lib().mykfa_ce_rows(ctypes.byref(p), _stream(logits.device)))


def _accumulate_fp32(acc: Tensor, a: Tensor, b: Tensor) -> None:
    """acc (fp32) += a @ b with bf16 operands, accumulated in fp32 by the GEMM itself."""
    torch.ops.aten.addmm.dtype_out(acc, a, b, torch.float32, beta=1, alpha=1, out=acc)


def _chunk_spans(n: int, size: int) -> list[tuple[int, int]]:
    return [(lo, min(lo + size, n)) for lo in range(0, n, size)]


def _loss_and_gradients(hidden: Tensor, weight: Tensor, targets: Tensor, scale: float, z_coef: float,
                        ignore_index: int, chunk_size: int) -> tuple[Tensor, Tensor, Tensor]:
    """One pass over the tokens in chunks. Returns (row_stats, d_hidden, d_weight):
    row_stats[0] / row_stats[1] are every token's cross-entropy and natural-log LSE (fp32),
    d_hidden (bf16) and d_weight (fp32) the gradients of the loss for an upstream gradient of 1.

    Per chunk: the logits GEMM writes a (rows, vocab) bf16 block, the gfx950 row kernel turns
    that block into d loss / d logits in place while producing the row statistics, and the
    same block then feeds the two gradient GEMMs. d_weight is accumulated in fp32 by the
    GEMM (beta = 1) so no partial sum is ever rounded to bf16."""
    dev = hidden.device
    tokens, width = hidden.shape
    w16 = weight if weight.dtype == torch.bfloat16 else weight.to(torch.bfloat16)
    row_stats = torch.empty((2, tokens), dtype=torch.float32, device=dev)
    d_hidden = torch.empty((tokens, width), dtype=torch.bfloat16, device=dev)
    d_weight = torch.zeros(weight.shape, dtype=torch.float32, device=dev)
    tgt = targets if targets.dtype == torch.int64 else targets.to(torch.int64)
    for lo, hi in _chunk_spans(tokens, chunk_size):
        h16 = hidden[lo:hi]
        if h16.dtype != torch.bfloat16:
            h16 = h16.to(torch.bfloat16)
        block = torch.mm(h16, w16.t())
        _ce_rows(block, tgt[lo:hi], row_stats[0, lo:hi], row_stats[1, lo:hi], scale, z_coef, ignore_index)
        torch.mm(block, w16, out=d_hidden[lo:hi])
        _accumulate_fp32(d_weight, block.t(), h16)
    return row_stats, d_hidden, d_weight


class _LinearCrossEntropy(torch.autograd.Function):
    """The loss and both gradients come out of the forward (the reference's scheme,
    fused_ce.py:70-108): the backward only multiplies the stored gradients by the upstream
    gradient of the loss and casts them to the parameters' dtypes."""

    @staticmethod
    def forward(ctx, hidden, weight, targets, normalizer, z_coef, ignore_index, chunk_size):  # pyright: ignore[reportIncompatibleMethodOverride]
        scale = 1.0 / normalizer
        with torch.autocast(device_type="cuda", enabled=False), _DeviceGuard(hidden.device):
            row_stats, d_hidden, d_weight = _loss_and_gradients(hidden, weight, targets, scale, z_coef,
                                                                ignore_index, chunk_size)
        ce_sum = row_stats[0].sum()
        z_sum = torch.dot(row_stats[1], row_stats[1])
        ctx.save_for_backward(d_hidden, d_weight)
        ctx.grad_dtypes = (hidden.dtype, weight.dtype)
        ctx.mark_non_differentiable(ce_sum, z_sum)
        return torch.add(ce_sum, z_sum, alpha=z_coef) * scale, ce_sum, z_sum

    @staticmethod
    def backward(ctx, upstream, _unused_ce, _unused_z):  # pyright: ignore[reportIncompatibleMethodOverride]
        d_hidden, d_weight = ctx.saved_tensors
        hidden_dtype, weight_dtype = ctx.grad_dtypes
        return (d_hidden.mul(upstream).to(hidden_dtype), d_weight.mul(upstream).to(weight_dtype),
                None, None, None, None, None)


def fused_linear_cross_entropy(hidden: Tensor, weight: Tensor, targets: Tensor, normalizer: float,
                               z_loss: float = 0.0, ignore_index: int = -100,
                               chunk_size: int = 2048) -> tuple[Tensor, Tensor, Tensor]:
    """Returns (loss, ce_sum, z_sum): loss = (sum CE + z_loss * sum lse^2) / normalizer
    (fused_ce.py:111-132). hidden (..., H), weight (V, H), targets (...) integer class ids
    with ignore_index marking unsupervised tokens."""
    if not hidden.is_cuda:
        raise RuntimeError("fused cross entropy is CUDA-only")
    _same_device(hidden.device, weight=weight, targets=targets)
    if chunk_size <= 0:
        raise ValueError(f"chunk_size must be positive; got {chunk_size}")
    result = _LinearCrossEntropy.apply(hidden.reshape(-1, hidden.size(-1)), weight, targets.reshape(-1),
                                       float(normalizer), float(z_loss), ignore_index, chunk_size)
    return cast(tuple[Tensor, Tensor, Tensor], result)

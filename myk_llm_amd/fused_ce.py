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
from .flash_attn import _DeviceGuard, _dtype_code, _stream


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


class _FusedLinearCE(torch.autograd.Function):
    """fused_ce.py:70-108: gradients computed in the forward, scaled in the backward."""

    @staticmethod
    def forward(ctx, hidden, weight, targets, normalizer, z_coef, ignore_index, chunk_size):  # pyright: ignore[reportIncompatibleMethodOverride]
        num_tokens, hidden_size = hidden.shape
        vocab_size = weight.shape[0]
        scale = 1.0 / normalizer
        compute_dtype = torch.bfloat16  # GEMMs in bf16 (fp32 accumulate); softmax in fp32
        weight_c = weight.to(compute_dtype)
        grad_hidden = torch.empty(num_tokens, hidden_size, device=hidden.device, dtype=compute_dtype)
        grad_weight = torch.zeros(vocab_size, hidden_size, device=hidden.device, dtype=torch.float32)
        ce = torch.empty(num_tokens, device=hidden.device, dtype=torch.float32)
        lse = torch.empty(num_tokens, device=hidden.device, dtype=torch.float32)
        tgt = targets.to(torch.int64)
        with torch.autocast(device_type="cuda", enabled=False), _DeviceGuard(hidden.device):
            for start in range(0, num_tokens, chunk_size):
                end = min(start + chunk_size, num_tokens)
                hidden_chunk = hidden[start:end].to(compute_dtype)
                logits = hidden_chunk @ weight_c.t()
                _ce_rows(logits, tgt[start:end], ce[start:end], lse[start:end], scale, z_coef, ignore_index)
                torch.mm(logits, weight_c, out=grad_hidden[start:end])
                _accumulate_fp32(grad_weight, logits.t(), hidden_chunk)
        ctx.save_for_backward(grad_hidden, grad_weight)
        ctx.hidden_dtype, ctx.weight_dtype = hidden.dtype, weight.dtype
        ce_sum, z_sum = ce.sum(), lse.square().sum()
        loss = (ce_sum + z_coef * z_sum) * scale
        ctx.mark_non_differentiable(ce_sum, z_sum)
        return loss, ce_sum, z_sum

    @staticmethod
    def backward(ctx, grad_loss, _grad_ce, _grad_z):  # pyright: ignore[reportIncompatibleMethodOverride]
        grad_hidden, grad_weight = ctx.saved_tensors
        return ((grad_hidden * grad_loss).to(ctx.hidden_dtype), (grad_weight * grad_loss).to(ctx.weight_dtype),
                None, None, None, None, None)


def fused_linear_cross_entropy(hidden: Tensor, weight: Tensor, targets: Tensor, normalizer: float,
                               z_loss: float = 0.0, ignore_index: int = -100,
                               chunk_size: int = 2048) -> tuple[Tensor, Tensor, Tensor]:
    """Returns (loss, ce_sum, z_sum): loss = (sum CE + z_loss * sum lse^2) / normalizer
    (fused_ce.py:111-132). hidden (..., H), weight (V, H), targets (...) integer class ids
    with ignore_index marking unsupervised tokens."""
    if not hidden.is_cuda:
        raise RuntimeError("fused cross entropy is CUDA-only")
    if chunk_size <= 0:
        raise ValueError(f"chunk_size must be positive; got {chunk_size}")
    result = _FusedLinearCE.apply(hidden.reshape(-1, hidden.size(-1)), weight, targets.reshape(-1),
                                  float(normalizer), float(z_loss), ignore_index, chunk_size)
    return cast(tuple[Tensor, Tensor, Tensor], result)

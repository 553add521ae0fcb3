"""Muon's batched Gram products on MI355X (gfx950): the drop-in for the batched SYRK of
myk-llm's src/myk_llm/ops/muon.py (exported by ops/__init__.py), same names and arguments:

    batched_syrk(x, bias=None, alpha=1.0, beta=0.0, out=None) -> out
        out[b] = alpha * x[b] @ x[b]^T + beta * bias[b] in bf16, computing only the
        lower-triangular tiles and mirroring them (ops/muon.py:28-143)
    batched_newton_schulz_orthogonalize(packed, steps, transposed=None, norm_sq=None, eps=1e-7)
        the quintic Newton-Schulz iteration on a batch of matrices (ops/muon.py:218-268):
        per step G = X X^T and G2 = b G + c G G through batched_syrk, X' = a X + G2 X

The SYRK runs in the hand-written gfx950 kernel of libmykfa.so (csrc/syrk.hip) through its C
ABI; the third product of each step (a general matrix product) is a library GEMM
(torch.baddbmm = hipBLASLt), as in the reference (cuBLAS baddbmm).

Differences from the reference's layout handling: the kernel reads k-contiguous rows whose
length is a multiple of 64, so transposed or strided x and unaligned k are copied once
(zero-padded) before the call; the Newton-Schulz driver transposes tall matrices with one
contiguous copy instead of iterating on transposed views (batched bf16 products on transposed
views are avoided on this platform).
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch
from torch import Tensor

from . import _lib
from .flash_attn import _DeviceGuard, _same_device, _stream

NS_COEFFICIENTS = (3.4445, -4.7750, 2.0315)  # ops/muon.py:25


def _kernel_x(x: Tensor) -> Tensor:
    """x as (B, M, Kp) bf16 rows with Kp a multiple of 64, 16-byte aligned, row stride 8k."""
    b, m, k = x.shape
    kp = (k + 63) // 64 * 64
    ok = (x.stride(2) == 1 and kp == k and x.data_ptr() % 16 == 0 and x.stride(1) % 8 == 0
          and x.stride(1) >= k and x.stride(0) >= 0)
    if ok:
        return x
    xp = torch.zeros((b, m, kp), dtype=torch.bfloat16, device=x.device)
    xp[..., :k] = x
    return xp


def batched_syrk(x: Tensor, bias: Optional[Tensor] = None, alpha: float = 1.0, beta: float = 0.0,
                 out: Optional[Tensor] = None) -> Tensor:
    """alpha * (x @ x.transpose(-2, -1)) + beta * bias for bf16 x of shape (B, M, K)
    (ops/muon.py:107-143). Only the lower-triangular tiles are evaluated and mirrored, so a
    given bias is assumed symmetric (as in the reference)."""
    if not x.is_cuda:
        raise RuntimeError("batched SYRK is CUDA-only: x must be a GPU (HIP) tensor")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"batched SYRK needs bf16 x; got {x.dtype}")
    if x.dim() != 3:
        raise ValueError(f"x must be (batch, m, k); got {tuple(x.shape)}")
    B, M, _ = x.shape
    _same_device(x.device, bias=bias, out=out)
    if out is None:
        out = torch.empty((B, M, M), device=x.device, dtype=torch.bfloat16)
    if out.shape != (B, M, M) or out.dtype != torch.bfloat16:
        raise ValueError(f"out must be bf16 ({B}, {M}, {M}); got {out.dtype} {tuple(out.shape)}")
    if bias is not None and (bias.shape != (B, M, M) or bias.dtype != torch.bfloat16):
        raise ValueError(f"bias must be bf16 ({B}, {M}, {M}); got {bias.dtype} {tuple(bias.shape)}")
    xk = _kernel_x(x)
    o = out
    if not (o.stride(2) == 1 and o.stride(1) % 4 == 0 and o.data_ptr() % 8 == 0 and o.stride(1) >= M):
        # the kernel's mirrored stores are 8 bytes wide: rows padded to a multiple of 4
        o = torch.empty((B, M, (M + 3) // 4 * 4), device=x.device, dtype=torch.bfloat16)[:, :, :M]
    if bias is not None and (bias.stride(2) != 1 or bias.data_ptr() % 2):
        bias = bias.contiguous()
    p = _lib.SyrkParams()
    p.x, p.out = xk.data_ptr(), o.data_ptr()
    p.x_batch_stride, p.x_row_stride = xk.stride(0), xk.stride(1)
    p.out_batch_stride, p.out_row_stride = o.stride(0), o.stride(1)
    if bias is not None:
        p.bias = bias.data_ptr()
        p.bias_batch_stride, p.bias_row_stride = bias.stride(0), bias.stride(1)
    p.batch, p.m, p.k = B, M, xk.shape[2]
    p.alpha, p.beta = float(alpha), float(beta)
    p.dtype = _lib.DTYPE_BF16
    with _DeviceGuard(x.device):
        _lib.check(_lib.lib().mykfa_syrk(ctypes.byref(p), _stream(x.device)))
    if o is not out:
        out.copy_(o)
    return out


def _frobenius_norm(packed: Tensor) -> Tensor:
    """Per-matrix Frobenius norm in fp32 of contiguous (B, rows, cols), as
    torch.linalg.vector_norm(packed, dim=(-2, -1), dtype=torch.float32) (ops/muon.py:241) but
    reduced in two levels (256 partial norms per matrix, then their root sum of squares): a
    single reduction with only B outputs runs on a handful of workgroups on this platform
    (measured 688 us for 9 x 1024 x 4096 bf16)."""
    B = packed.shape[0]
    flat = packed.view(B, -1)
    parts = 256 if flat.shape[1] % 256 == 0 and flat.shape[1] >= 256 * 1024 else 1
    partial = torch.linalg.vector_norm(flat.view(B, parts, -1), dim=-1, dtype=torch.float32)
    return partial.square().sum(-1).sqrt() if parts > 1 else partial[:, 0]


def batched_newton_schulz_orthogonalize(packed: Tensor, steps: int, transposed: Optional[bool] = None,
                                        norm_sq: Optional[Tensor] = None, eps: float = 1e-7) -> Tensor:
    """Batched quintic Newton-Schulz on packed (B, rows, cols) in bf16 (ops/muon.py:218-268).

    With norm_sq (per-matrix squared Frobenius norm of packed) the input is scaled by
    1 / max(sqrt(norm_sq), eps) in place, as the reference's _scale_bf16_kernel does;
    otherwise its norm is computed first. Returns a contiguous (B, rows, cols) tensor."""
    a, b, c = NS_COEFFICIENTS
    if packed.dtype != torch.bfloat16:
        packed = packed.bfloat16()
    if not packed.is_contiguous():
        packed = packed.contiguous()
    B, rows, cols = packed.shape
    if transposed is None:
        transposed = rows > cols
    if norm_sq is not None:
        inv = 1.0 / torch.clamp(norm_sq.reshape(B, 1, 1).float().sqrt(), min=eps)
        packed.copy_((packed.float() * inv).bfloat16())
    else:
        norm = _frobenius_norm(packed).reshape(B, 1, 1).clamp_(min=eps)
        packed = (packed / norm).bfloat16()
    x = packed.transpose(-2, -1).contiguous() if transposed else packed
    M = x.size(1)
    gram = torch.empty((B, M, M), device=x.device, dtype=torch.bfloat16)
    gram2 = torch.empty((B, M, M), device=x.device, dtype=torch.bfloat16)
    x_next = torch.empty_like(x)
    for _ in range(steps):
        batched_syrk(x, out=gram)
        batched_syrk(gram, bias=gram, alpha=c, beta=b, out=gram2)
        torch.baddbmm(x, gram2, x, beta=a, alpha=1.0, out=x_next)
        x, x_next = x_next, x
    return x.transpose(-2, -1).contiguous() if transposed else x

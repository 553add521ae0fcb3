"""CPU oracle for Muon's batched SYRK and Newton-Schulz iteration — TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py's cpu_baseline leg may import this module, as the checker. The
product path (myk_llm_amd.muon) never calls it and fails loudly without the HIP library.

Restated from the reference (never imported):
  * syrk_reference()          _batched_syrk_kernel / batched_syrk, ops/muon.py:28-143:
                              alpha * x x^T + beta * bias (bias symmetric), in float64
  * newton_schulz_reference() newton_schulz_orthogonalize, train/optim.py:20-32: x / ||x||,
                              then `steps` times x <- a x + (b G + c G G) x with G = x x^T,
                              on the transpose when rows > cols; bf16 rounding of x after the
                              normalization and after every step (the reference runs in bf16)
How each is pinned (tests/test_muon_oracle.py): syrk against numpy's product, symmetry and
the diagonal = squared row norms; Newton-Schulz against the SVD: the result keeps the input's
singular vectors and maps its singular values into the quintic's band, NS(G^T) = NS(G)^T, and
a planted wrong coefficient or a dropped normalization fails those checks.
"""

from __future__ import annotations

import numpy as np
import torch

NS_COEFFICIENTS = (3.4445, -4.7750, 2.0315)  # ops/muon.py:25


def syrk_reference(x, bias=None, alpha=1.0, beta=0.0):
    """x (B, M, K) -> (B, M, M) float64."""
    x64 = torch.as_tensor(x).double()
    out = alpha * (x64 @ x64.transpose(-2, -1))
    if bias is not None:
        out = out + beta * torch.as_tensor(bias).double()
    return out


def newton_schulz_reference(g: torch.Tensor, steps: int, eps: float = 1e-7, store=torch.bfloat16,
                            coeffs=NS_COEFFICIENTS) -> torch.Tensor:
    """train/optim.py:20-32 with fp32 arithmetic and rounding to `store` where the reference's
    bf16 tensors are (None: no rounding)."""
    a, b, c = coeffs
    rnd = (lambda t: t.to(store).float()) if store is not None else (lambda t: t)
    x = rnd(g.float())
    transposed = g.size(0) > g.size(1)
    if transposed:
        x = x.T
    x = rnd(x / x.norm().clamp(min=eps))
    for _ in range(steps):
        gram = rnd(x @ x.T)
        gram2 = rnd(b * gram + c * (gram @ gram))
        x = rnd(a * x + gram2 @ x)
    return x.T if transposed else x

"""CPU oracle for the fused linear + cross-entropy — TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py's cpu_baseline leg may import this module, as the checker. The
product path (myk_llm_amd.fused_ce) never calls it and fails loudly without the HIP library.

Restated from the reference (never imported):
  * ce_rows()        _ce_kernel, ops/fused_ce.py:20-67: per row lse = logsumexp, ce = lse -
                     logit[target], gradient softmax * scale * (1 + 2 z lse) - scale * onehot;
                     ignored rows -> zeros, ce = lse = 0
  * loss_reference() the reference's own test formula, tests/test_fused_ce.py:27-33: bf16
                     operands, fp32 logits, F.cross_entropy(sum, ignore_index), lse of the
                     supervised rows, (ce + z * sum lse^2) / normalizer; gradients by autograd

How each is pinned (tests/test_fused_ce_oracle.py): ce/lse against torch's
F.cross_entropy / logsumexp; closed forms (constant rows: lse = c + log V, ce = log V;
gradient rows sum to scale * 2 z lse); the gradient against float64 central finite
differences of scale * (ce + z lse^2); ignored rows; planted mistakes (a dropped factor 2 in
the z-loss term, the onehot at the wrong column) fail the pins.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def ce_rows(logits: np.ndarray, targets: np.ndarray, scale: float, z_coef: float, ignore_index: int = -100):
    """float64 restatement of _ce_kernel (fused_ce.py:20-67) on a (rows, V) array.
    Returns (grad, ce, lse)."""
    x = np.asarray(logits, dtype=np.float64)
    t = np.asarray(targets, dtype=np.int64)
    rows, v = x.shape
    m = x.max(axis=1, keepdims=True)
    lse = (m + np.log(np.exp(x - m).sum(axis=1, keepdims=True)))[:, 0]
    ign = t == ignore_index
    tc = np.where(ign, 0, t)
    ce = lse - x[np.arange(rows), tc]
    grad = np.exp(x - lse[:, None]) * (scale * (1.0 + 2.0 * z_coef * lse))[:, None]
    grad[np.arange(rows), tc] -= scale
    grad[ign] = 0.0
    ce[ign] = 0.0
    lse = np.where(ign, 0.0, lse)
    return grad, ce, lse


def loss_reference(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor, normalizer: float,
                   z_loss: float = 0.0, ignore_index: int = -100):
    """tests/test_fused_ce.py:27-33 (fp32 logits of bf16 operands). Returns (loss, ce_sum)."""
    logits = (hidden.bfloat16().float() @ weight.bfloat16().float().t())
    valid = targets != ignore_index
    ce = F.cross_entropy(logits, targets, ignore_index=ignore_index, reduction="sum")
    lse = torch.logsumexp(logits, -1)[valid]
    return (ce + z_loss * lse.square().sum()) / normalizer, ce

"""Pins of the fused cross-entropy oracle (oracle/fused_ce.py) and host-side checks of the
CE row entry point (no GPU)."""

import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from myk_llm_amd import _lib
from oracle import fused_ce as oc


def _rows(n, v, seed=0, scale=3.0):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((n, v)) * scale, rng.integers(0, v, n)


@pytest.mark.parametrize("z", [0.0, 1e-3, 0.5])
def test_ce_and_lse_match_torch(z):
    x, t = _rows(7, 333)
    t[2] = -100
    grad, ce, lse = oc.ce_rows(x, t, 0.25, z)
    xt = torch.tensor(x)
    ref_ce = F.cross_entropy(xt, torch.tensor(t), ignore_index=-100, reduction="none").numpy()
    ref_lse = torch.logsumexp(xt, -1).numpy()
    valid = t != -100
    np.testing.assert_allclose(ce[valid], ref_ce[valid], rtol=1e-12)
    np.testing.assert_allclose(lse[valid], ref_lse[valid], rtol=1e-12)
    assert ce[2] == 0 and lse[2] == 0 and not grad[2].any()


def test_closed_forms():
    v, c = 1000, 2.5
    x = np.full((3, v), c)
    grad, ce, lse = oc.ce_rows(x, np.array([0, 5, 999]), 1.0, 0.1)
    np.testing.assert_allclose(lse, c + np.log(v), rtol=1e-14)
    np.testing.assert_allclose(ce, np.log(v), rtol=1e-14)
    # softmax sums to one: sum(grad) = scale (1 + 2 z lse) - scale = 2 z lse scale
    x, t = _rows(5, 257, seed=1)
    grad, ce, lse = oc.ce_rows(x, t, 0.5, 0.01)
    np.testing.assert_allclose(grad.sum(axis=1), 2 * 0.01 * lse * 0.5, rtol=1e-10, atol=1e-14)


def test_gradient_matches_finite_differences():
    x, t = _rows(2, 11, seed=2, scale=1.0)
    scale, z = 0.7, 0.05
    grad, _, _ = oc.ce_rows(x, t, scale, z)

    def loss(xx):
        _, ce, lse = oc.ce_rows(xx, t, scale, z)
        return scale * (ce + z * lse ** 2).sum()

    h = 1e-6
    num = np.zeros_like(x)
    for i in range(x.shape[0]):
        for j in range(x.shape[1]):
            xp, xm = x.copy(), x.copy()
            xp[i, j] += h
            xm[i, j] -= h
            num[i, j] = (loss(xp) - loss(xm)) / (2 * h)
    np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-8)


def test_loss_reference_matches_the_row_oracle():
    g = torch.Generator().manual_seed(3)
    hidden, weight = torch.randn(40, 16, generator=g), 0.3 * torch.randn(50, 16, generator=g)
    targets = torch.randint(0, 50, (40,), generator=g)
    targets[::5] = -100
    loss, ce_sum = oc.loss_reference(hidden, weight, targets, 17.0, 1e-3)
    logits = (hidden.bfloat16().float() @ weight.bfloat16().float().t()).double().numpy()
    _, ce, lse = oc.ce_rows(logits, targets.numpy(), 1.0, 0.0)
    assert abs(ce_sum.item() - ce.sum()) < 1e-3
    assert abs(loss.item() - (ce.sum() + 1e-3 * (lse ** 2).sum()) / 17.0) < 1e-4


def test_planted_mistakes_fail_the_pins(monkeypatch):
    x, t = _rows(2, 11, seed=4, scale=1.0)
    scale, z = 0.7, 0.05
    good, _, lse = oc.ce_rows(x, t, scale, z)
    # z-loss derivative without its factor 2
    bad = np.exp(x - lse[:, None]) * (scale * (1.0 + z * lse))[:, None]
    bad[np.arange(2), t] -= scale
    assert np.abs(bad - good).max() > 1e-4
    # onehot subtracted one column to the right
    bad2 = good.copy()
    bad2[np.arange(2), t] += scale
    bad2[np.arange(2), (t + 1) % 11] -= scale
    assert np.abs(bad2.sum(axis=1) - good.sum(axis=1)).max() < 1e-12  # row sums cannot see it
    _, ce, _ = oc.ce_rows(x, t, scale, z)
    ref_ce = F.cross_entropy(torch.tensor(x), torch.tensor(t), reduction="none").numpy()
    _, ce_shift, _ = oc.ce_rows(x, (t + 1) % 11, scale, z)
    assert np.abs(ce_shift - ref_ce).max() > 1e-3 and np.abs(ce - ref_ce).max() < 1e-12


# --- host-only checks of the C entry point ------------------------------------------------------


def _good():
    p = _lib.CeParams()
    p.logits, p.targets, p.ce, p.lse = 0x10000, 0x20000, 0x30000, 0x40000
    p.row_stride, p.rows, p.vocab, p.ignore_index = 65536, 2048, 65536, -100
    p.scale, p.z_coef, p.dtype = 1e-3, 0.0, _lib.DTYPE_BF16
    return p


@pytest.mark.parametrize("field,value,text", [
    ("dtype", 5, "bf16/fp16"),
    ("vocab", 0, "vocab"),
    ("rows", -1, "rows"),
    ("row_stride", 100, "row_stride"),
    ("targets", 0, "non-NULL"),
    ("targets", 0x20004, "misaligned"),
    ("scale", float("nan"), "NaN"),
])
def test_ce_validation(field, value, text):
    L = _lib.lib()
    assert L.mykfa_validate_ce(ctypes.byref(_good())) == _lib.OK
    p = _good()
    setattr(p, field, value)
    assert L.mykfa_validate_ce(ctypes.byref(p)) != _lib.OK
    assert text in L.mykfa_last_error().decode()
    q = _good()
    q.rows = 0
    q.logits = 0
    assert L.mykfa_ce_rows(ctypes.byref(q), None) == _lib.OK  # nothing to do: no launch


def test_cpu_tensors_are_rejected():
    from myk_llm_amd.fused_ce import fused_linear_cross_entropy

    with pytest.raises(RuntimeError, match="CUDA-only"):
        fused_linear_cross_entropy(torch.zeros(4, 8), torch.zeros(16, 8), torch.zeros(4, dtype=torch.long), 1.0)

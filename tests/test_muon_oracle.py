"""Pins of the Muon oracle (oracle/muon.py) and host-side checks of the SYRK entry point."""

import ctypes

import numpy as np
import pytest
import torch

from myk_llm_amd import _lib
from oracle import muon as om


def test_syrk_reference_against_numpy():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 17, 23))
    got = om.syrk_reference(x, alpha=0.5).numpy()
    want = 0.5 * np.einsum("bmk,bnk->bmn", x, x)
    np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-12)
    np.testing.assert_allclose(got, got.transpose(0, 2, 1), rtol=0, atol=1e-12)
    np.testing.assert_allclose(np.diagonal(got, axis1=1, axis2=2), 0.5 * (x ** 2).sum(-1), rtol=1e-12)
    bias = rng.standard_normal((3, 17, 17))
    bias = bias + bias.transpose(0, 2, 1)
    np.testing.assert_allclose(om.syrk_reference(x, bias, 2.0, -3.0).numpy(), 2.0 * want / 0.5 - 3.0 * bias, rtol=1e-12)


def _with_spectrum(rows, cols, s, seed=0):
    g = torch.Generator().manual_seed(seed)
    u, _ = torch.linalg.qr(torch.randn(rows, rows, generator=g, dtype=torch.float64))
    v, _ = torch.linalg.qr(torch.randn(cols, cols, generator=g, dtype=torch.float64))
    k = min(rows, cols)
    return u[:, :k] @ torch.diag(torch.as_tensor(s, dtype=torch.float64)) @ v[:, :k].T, u[:, :k], v[:, :k]


@pytest.mark.parametrize("rows,cols", [(48, 96), (96, 48)])
def test_newton_schulz_against_the_svd(rows, cols):
    k = min(rows, cols)
    s = np.geomspace(0.05, 1.0, k)
    g, u, v = _with_spectrum(rows, cols, s)
    out = om.newton_schulz_reference(g.float(), 5, store=None).double()
    core = u.T @ out @ v  # ~diagonal in the input's singular bases
    off = core - torch.diag(torch.diagonal(core))
    assert off.abs().max().item() < 1e-3 * core.abs().max().item() + 1e-4
    sv = torch.diagonal(core)
    # 5 quintic steps map singular values >= 0.05 (of a unit-norm input) into a band around 1
    assert sv.min().item() > 0.6 and sv.max().item() < 1.3, (sv.min().item(), sv.max().item())
    # NS of the transpose is the transpose of NS
    out_t = om.newton_schulz_reference(g.T.float(), 5, store=None).double()
    torch.testing.assert_close(out_t, out.T, rtol=1e-5, atol=1e-5)


def test_planted_mistakes_fail_the_pins():
    k = 48
    g, u, v = _with_spectrum(48, 96, np.geomspace(0.05, 1.0, k))
    bad = om.newton_schulz_reference(g.float(), 5, store=None, coeffs=(3.4445, -4.7750, 0.5)).double()
    sv = torch.diagonal(u.T @ bad @ v)
    assert sv.min().item() <= 0.6 or sv.max().item() >= 1.3
    unnormalized = om.newton_schulz_reference(4.0 * g.float(), 0, store=None).double()
    assert abs(torch.linalg.matrix_norm(unnormalized).item() - 1.0) < 1e-6  # the normalization is there


def _good():
    p = _lib.SyrkParams()
    p.x, p.out = 0x10000, 0x20000
    p.x_batch_stride, p.x_row_stride = 1024 * 4096, 4096
    p.out_batch_stride, p.out_row_stride = 1024 * 1024, 1024
    p.batch, p.m, p.k, p.alpha, p.beta, p.dtype = 9, 1024, 4096, 1.0, 0.0, _lib.DTYPE_BF16
    return p


@pytest.mark.parametrize("field,value,text", [
    ("dtype", 1, "bf16"),
    ("k", 4000, "multiple of 64"),
    ("m", -1, "negative"),
    ("x", 0x10008, "16-byte aligned"),
    ("x_row_stride", 4100, "multiple of 8"),
    ("out", 0x20004, "8-byte aligned"),
    ("out_row_stride", 1022, "row stride"),
    ("alpha", float("nan"), "NaN"),
    ("batch", 1 << 26, "grid limit"),  # 2^26 matrices x 36 tiles > 2^31 workgroups
])
def test_syrk_validation(field, value, text):
    L = _lib.lib()
    assert L.mykfa_validate_syrk(ctypes.byref(_good())) == _lib.OK
    p = _good()
    setattr(p, field, value)
    assert L.mykfa_validate_syrk(ctypes.byref(p)) != _lib.OK
    assert text in L.mykfa_last_error().decode()
    q = _good()
    q.m = 0
    q.x = q.out = 0
    assert L.mykfa_syrk(ctypes.byref(q), None) == _lib.OK  # nothing to do: no launch


def test_cpu_tensors_are_rejected():
    from myk_llm_amd.muon import batched_syrk

    with pytest.raises(RuntimeError, match="CUDA-only"):
        batched_syrk(torch.zeros(2, 8, 32, dtype=torch.bfloat16))


@pytest.mark.parametrize("shape", [(3, 1024, 512), (2, 100, 52)])
def test_frobenius_norm_matches_float64(shape):
    """The driver's two-level fp32 norm (host logic, runs on CPU tensors) against the float64
    root sum of squares of the same bf16 values."""
    from myk_llm_amd.muon import _frobenius_norm

    x = torch.randn(*shape, generator=torch.Generator().manual_seed(5)).bfloat16()
    exact = x.double().square().sum((-2, -1)).sqrt()
    got = _frobenius_norm(x)
    assert got.dtype == torch.float32 and got.shape == (shape[0],)
    assert ((got.double() - exact).abs() <= 1e-6 * exact).all()

"""Pins of the prologue / epilogue oracle (oracle/block_io.py) on the CPU: independent
formulas (complex rotation, numpy tables), closed forms, invariants and float64 finite
differences, each chosen so that a plausible slip in the restatement fails it (the planted
mistakes at the end)."""

import math

import numpy as np
import pytest
import torch

from oracle import block_io as ob


def _complex_rope(x, pos, base):
    """(x[2i] + i x[2i+1]) * exp(i pos theta_i), theta_i = base^(-2i/D), in float64 numpy."""
    x = np.asarray(x, dtype=np.float64)
    d = x.shape[-1]
    theta = base ** (-np.arange(0, d, 2, dtype=np.float64) / d)
    ang = np.asarray(pos, dtype=np.float64)[..., None] * theta  # (B, S, D/2)
    z = (x[..., 0::2] + 1j * x[..., 1::2]) * np.exp(1j * ang)[:, :, None, :]
    out = np.empty_like(x)
    out[..., 0::2], out[..., 1::2] = z.real, z.imag
    return out


def _rand(*shape, seed=0, dtype=torch.float64):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=dtype)


@pytest.mark.parametrize("d,base", [(16, 10000.0), (64, 10000.0), (128, 500000.0)])
def test_rope_is_complex_rotation(d, base):
    x = _rand(2, 7, 3, d)
    pos = torch.tensor([[0, 1, 2, 3, 100, 1000, 4095], [5, 5, 9, 0, 17, 2047, 3]])
    cos, sin = ob.rope_tables(d, 4096, base, dtype=torch.float64)
    got = ob.rope(x, pos, cos, sin, acc=torch.float64).numpy()
    np.testing.assert_allclose(got, _complex_rope(x.numpy(), pos.numpy(), base), rtol=0, atol=1e-9)


def test_rope_tables_against_numpy():
    d, n, base = 64, 8192, 10000.0
    cos, sin = ob.rope_tables(d, n, base)  # fp32, as the reference module builds them
    theta = base ** (-np.arange(0, d, 2, dtype=np.float64) / d)
    ang = np.repeat(np.arange(n, dtype=np.float64)[:, None] * theta, 2, axis=1)
    # fp32 angles: fl(pos * fl(1 / fl(base^x))) carries a few units of 2^-24 relative error,
    # plus the cos/sin rounding
    bound = np.abs(ang) * 2.0 ** -21 + 2e-7
    assert (np.abs(cos.double().numpy() - np.cos(ang)) <= bound).all()
    assert (np.abs(sin.double().numpy() - np.sin(ang)) <= bound).all()
    assert torch.equal(cos[:, 0::2], cos[:, 1::2]) and torch.equal(sin[:, 0::2], sin[:, 1::2])


def test_rope_identity_norms_and_relative_positions():
    d = 64
    cos, sin = ob.rope_tables(d, 512, 10000.0)
    x = _rand(1, 4, 2, d, dtype=torch.float32)
    zero = torch.zeros(1, 4, dtype=torch.long)
    assert torch.equal(ob.rope(x, zero, cos, sin), x)  # cos(0) = 1, sin(0) = 0 exactly
    pos = torch.tensor([[3, 50, 200, 511]])
    y = ob.rope(x.double(), pos, cos, sin, acc=torch.float64)
    pair = lambda t: t[..., 0::2] ** 2 + t[..., 1::2] ** 2  # noqa: E731
    torch.testing.assert_close(pair(y), pair(x.double()), rtol=1e-6, atol=1e-6)
    # <R(p) q, R(p') k> depends only on p - p'
    q, k = _rand(1, 1, 1, d, seed=1), _rand(1, 1, 1, d, seed=2)
    c64, s64 = ob.rope_tables(d, 512, 10000.0, dtype=torch.float64)

    def dot(pq, pk):
        a = ob.rope(q, torch.tensor([[pq]]), c64, s64, acc=torch.float64)
        b = ob.rope(k, torch.tensor([[pk]]), c64, s64, acc=torch.float64)
        return (a * b).sum().item()

    assert abs(dot(10, 3) - dot(107, 100)) < 1e-9
    assert abs(dot(10, 3) - dot(10, 4)) > 1e-3


def test_rms_norm_closed_forms():
    d, eps = 64, 1e-6
    x = _rand(3, 5, 2, d)
    ones = torch.ones(d, dtype=torch.float64)
    y = ob.rms_norm(x, ones, eps, acc=torch.float64)
    ms = x.pow(2).mean(-1)
    torch.testing.assert_close(y.pow(2).mean(-1), ms / (ms + eps), rtol=1e-12, atol=0)
    torch.testing.assert_close(ob.rms_norm(7.5 * x, ones, 0.0, torch.float64), ob.rms_norm(x, ones, 0.0, torch.float64))
    w = _rand(d, seed=3)
    torch.testing.assert_close(ob.rms_norm(x, w, eps, torch.float64), y * w)


def test_output_gate_closed_forms():
    x = _rand(4, 32, dtype=torch.float32).to(torch.bfloat16)
    assert torch.equal(ob.output_gate(x, torch.zeros_like(x)), x / 2)  # sigmoid(0) = 1/2 exactly
    big = torch.full_like(x, 40.0)
    assert torch.equal(ob.output_gate(x, big), x)
    assert (ob.output_gate(x, -big).float().abs() <= x.float().abs() * 1e-17).all()
    # gradient against the closed form in float64
    xo, g, dy = _rand(3, 16, seed=1), _rand(3, 16, seed=2), _rand(3, 16, seed=3)
    xo.requires_grad_(True)
    g.requires_grad_(True)
    y = ob.output_gate(xo, g, acc=torch.float64, store=None)
    dx, dg = torch.autograd.grad(y, (xo, g), dy)
    s = 1.0 / (1.0 + torch.exp(-g.detach()))
    torch.testing.assert_close(dx, dy * s, rtol=1e-12, atol=0)
    torch.testing.assert_close(dg, dy * xo.detach() * s * (1 - s), rtol=1e-12, atol=1e-15)


def test_output_gate_rounding_points():
    """Under autocast the sigmoid is a bf16 op: the product uses the rounded sigmoid."""
    x = _rand(64, 64, dtype=torch.float32).to(torch.bfloat16)
    g = _rand(64, 64, seed=1, dtype=torch.float32).to(torch.bfloat16)
    s = torch.sigmoid(g.float()).to(torch.bfloat16).float()
    assert torch.equal(ob.output_gate(x, g), (x.float() * s).to(torch.bfloat16))


def test_prologue_gradients_match_finite_differences():
    torch.manual_seed(0)
    b, s, hq, hkv, d = 1, 3, 2, 1, 16
    cos, sin = ob.rope_tables(d, 64, 10000.0, dtype=torch.float64)
    pos = torch.tensor([[0, 5, 33]])
    q, k = _rand(b, s, hq, d, seed=1), _rand(b, s, hkv, d, seed=2)
    qw, kw = 1 + 0.1 * _rand(d, seed=3), 1 + 0.1 * _rand(d, seed=4)
    args = [t.clone().requires_grad_(True) for t in (q, k, qw, kw)]

    def f(q_, k_, qw_, kw_):
        return ob.qk_norm_rope(q_, k_, pos, cos, sin, qw_, kw_, 1e-6, acc=torch.float64, store=None)

    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-8)


def test_kernel_rounding_points_are_the_modules():
    """With store = bf16 the oracle rounds after the norm and after the rotation, exactly as
    `q_norm(q).to(v.dtype)` then `rope` (whose result `.to(x.dtype)`) do."""
    d = 32
    cos, sin = ob.rope_tables(d, 128, 10000.0)
    q = _rand(2, 9, 4, d, dtype=torch.float32).to(torch.bfloat16)
    k = _rand(2, 9, 2, d, seed=1, dtype=torch.float32).to(torch.bfloat16)
    w = (1 + 0.1 * _rand(d, seed=2, dtype=torch.float32))
    pos = torch.arange(9).expand(2, -1)
    oq, ok = ob.qk_norm_rope(q, k, pos, cos, sin, w, w, 1e-6)
    assert oq.dtype == torch.bfloat16
    nq = ob.rms_norm(q, w, 1e-6).to(torch.bfloat16)
    assert torch.equal(oq, ob.rope(nq, pos, cos, sin).to(torch.bfloat16))


# --- planted mistakes: each variant must fail one of the pins above --------------------------


def _bad_rotate_sign(x):
    x1, x2 = x[..., ::2], x[..., 1::2]
    return torch.stack((x2, x1), dim=-1).flatten(start_dim=-2)  # lost minus sign


def _bad_rotate_pairs(x):
    h = x.shape[-1] // 2  # half-split convention instead of interleaved pairs
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def test_planted_mistakes_fail_the_pins(monkeypatch):
    d, base = 16, 10000.0
    x = _rand(1, 3, 1, d)
    pos = torch.tensor([[1, 7, 30]])
    cos, sin = ob.rope_tables(d, 64, base, dtype=torch.float64)
    want = _complex_rope(x.numpy(), pos.numpy(), base)
    for bad in (_bad_rotate_sign, _bad_rotate_pairs):
        monkeypatch.setattr(ob, "rotate_half", bad)
        got = ob.rope(x, pos, cos, sin, acc=torch.float64).numpy()
        assert np.abs(got - want).max() > 1e-3, bad.__name__
    monkeypatch.undo()

    # RMS over D - 1 instead of the mean breaks the closed form mean(y^2) = ms / (ms + eps)
    xx = _rand(4, d)
    y = xx * torch.rsqrt(xx.pow(2).sum(-1, keepdim=True) / (d - 1) + 1e-6)
    ms = xx.pow(2).mean(-1)
    assert (y.pow(2).mean(-1) - ms / (ms + 1e-6)).abs().max() > 1e-3

    # a gate derivative without the sigmoid factor breaks the closed-form gradient
    g, dy, xo = _rand(8, seed=1), _rand(8, seed=2), _rand(8, seed=3)
    s = torch.sigmoid(g)
    assert (dy * xo * (1 - s) - dy * xo * s * (1 - s)).abs().max() > 1e-3
    assert math.isfinite(float(s.sum()))

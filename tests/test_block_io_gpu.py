"""Parity of the prologue / epilogue kernels (csrc/block_io.hip) with the CPU oracle
(oracle/block_io.py) on identical seeded inputs.

Bars:
- forward outputs within one storage ulp of the oracle, which rounds at the reference's
  points (the rotation is computed op for op, so almost every element is bit-identical; the
  norm's fp32 sum order and rsqrt may move a rounding by one ulp);
- input gradients within the reference's tolerance (2e-2 * max|ref| + 1e-3,
  tests/test_flash_attn.py:37-40) and the north-star mean-abs bound; norm-weight gradients
  (fp32 sums over every token and head) within 1e-3 relative of the oracle's;
- the fused-projection variant's d(qkv) bit-identical to the per-slice path's;
- weight gradients bitwise repeatable (fixed-order reduction).
"""

import sys

import pytest
import torch

from _util import assert_close, assert_north_star, storage_ulp
from myk_llm_amd import block_io as bio
from oracle import block_io as ob

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _within_ulps(actual, expected, ulps=1, what="", pairs=False):
    """Every element within `ulps` storage ulps of the oracle's. With `pairs` (rotated
    outputs) one more ulp of the element's pair magnitude is allowed: a one-ulp difference in
    the rounded norm output feeds the rotation, which moves it into both elements of the pair
    at the pair's scale, not at the (possibly much smaller) element's."""
    a, e = actual.float().cpu(), expected.float().cpu()
    d = (a - e).abs()
    bound = ulps * storage_ulp(e, actual.dtype) + 1e-30
    if pairs:
        mag = (e[..., 0::2] ** 2 + e[..., 1::2] ** 2).sqrt().repeat_interleave(2, dim=-1)
        bound = bound + storage_ulp(mag, actual.dtype)
    bad = (d > bound).sum().item()
    exact = (d == 0).float().mean().item()
    _say(f"  {what}: max-abs {d.max().item():.3e}, exact {100 * exact:.2f}%")
    assert bad == 0, f"{what}: {bad} elements beyond {ulps} ulp (max-abs {d.max().item():.3e})"
    return exact


def _inputs(b, s, hq, hkv, d, dtype, seed=0, table=4096, theta=10000.0):
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(b, s, (hq + 2 * hkv) * d, generator=g) * 1.5).to(dtype)
    pos = torch.randint(0, table, (b, s), generator=g)
    qw = 1.0 + 0.2 * torch.randn(d, generator=g)
    kw = 1.0 + 0.2 * torch.randn(d, generator=g)
    dq = torch.randn(b, s, hq, d, generator=g).to(dtype)
    dk = torch.randn(b, s, hkv, d, generator=g).to(dtype)
    dv = torch.randn(b, s, hkv, d, generator=g).to(dtype)
    cos, sin = ob.rope_tables(d, table, theta)
    return qkv, pos, qw, kw, cos, sin, dq, dk, dv


def _split(qkv, hq, hkv, d):
    b, s = qkv.shape[:2]
    q, k, v = qkv.split((hq * d, hkv * d, hkv * d), -1)
    return q.view(b, s, hq, d), k.view(b, s, hkv, d), v.view(b, s, hkv, d)


CASES = [
    # (batch, seq, Hq, Hkv, D, dtype, norm, rope)
    (2, 37, 8, 2, 64, torch.bfloat16, True, True),
    (1, 129, 16, 4, 128, torch.bfloat16, True, True),
    (3, 20, 4, 4, 32, torch.bfloat16, True, True),
    (2, 9, 4, 1, 16, torch.bfloat16, True, True),
    (1, 33, 4, 2, 256, torch.bfloat16, True, True),
    (2, 40, 8, 2, 64, torch.float16, True, True),
    (2, 40, 8, 2, 64, torch.bfloat16, False, True),
    (2, 40, 8, 2, 64, torch.bfloat16, True, False),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}S{c[1]}H{c[2]}/{c[3]}D{c[4]}{str(c[5])[-4:]}n{int(c[6])}r{int(c[7])}")
def test_prologue_matches_oracle(case):
    b, s, hq, hkv, d, dtype, norm, rope = case
    _say(f"prologue case {case}")
    qkv, pos, qw, kw, cos, sin, dq, dk, dv = _inputs(b, s, hq, hkv, d, dtype)
    args = dict(q_weight=qw if norm else None, k_weight=kw if norm else None)
    tables = (cos, sin) if rope else (None, None)

    # kernel: q/k as strided views of the fused projection, as Attention.forward passes them
    x = qkv.cuda().requires_grad_(True)
    qv, kv, _ = _split(x, hq, hkv, d)
    qw_g = qw.cuda().requires_grad_(norm)
    kw_g = kw.cuda().requires_grad_(norm)
    oq, ok = bio.qk_norm_rope(qv, kv, pos.cuda(), *(t.cuda() if t is not None else None for t in tables),
                              q_weight=qw_g if norm else None, k_weight=kw_g if norm else None)
    grads = torch.autograd.grad((oq, ok), (x, qw_g, kw_g) if norm else (x,), (dq.cuda(), dk.cuda()))
    torch.cuda.synchronize()

    # oracle on the CPU, the reference's rounding points
    xc = qkv.clone().requires_grad_(True)
    qc, kc, _ = _split(xc, hq, hkv, d)
    qwc, kwc = qw.clone().requires_grad_(norm), kw.clone().requires_grad_(norm)
    rq, rk = ob.qk_norm_rope(qc, kc, pos, *tables, qwc if norm else None, kwc if norm else None, 1e-6)
    rgrads = torch.autograd.grad((rq, rk), (xc, qwc, kwc) if norm else (xc,), (dq, dk))

    _within_ulps(oq, rq, 1, "q", pairs=norm and rope)
    _within_ulps(ok, rk, 1, "k", pairs=norm and rope)
    dx, rdx = grads[0].float().cpu(), rgrads[0].float()
    nqk = (hq + hkv) * d
    assert torch.equal(dx[..., nqk:], torch.zeros_like(dx[..., nqk:])), "v slice gradient must be zero"
    assert_close(dx[..., :nqk], rdx[..., :nqk])
    assert_north_star(grads[0][..., :nqk], rdx[..., :nqk], what="d(q,k)_in")
    if norm:
        for got, ref, name in ((grads[1], rgrads[1], "dq_weight"), (grads[2], rgrads[2], "dk_weight")):
            err = (got.cpu() - ref).abs().max().item()
            _say(f"  {name}: max-abs {err:.3e} of {ref.abs().max().item():.3e}")
            assert err <= 1e-3 * ref.abs().max().item() + 1e-5, name


def test_packed_tokens_and_expanded_positions():
    """(tokens, heads, D) packed inputs with one position row broadcast over the batch
    (position_ids = arange(S).expand(B, -1) in the reference's model, transformer.py:305-306)."""
    t, hq, hkv, d = 300, 8, 2, 64
    qkv, _, qw, kw, cos, sin, dq, dk, _ = _inputs(1, t, hq, hkv, d, torch.bfloat16, seed=3)
    pos = torch.arange(t)
    q, k, _ = _split(qkv, hq, hkv, d)
    oq, ok = bio.qk_norm_rope(q[0].cuda(), k[0].cuda(), pos.cuda(), cos.cuda(), sin.cuda(), qw.cuda(), kw.cuda())
    assert oq.shape == (t, hq, d) and ok.shape == (t, hkv, d)
    rq, rk = ob.qk_norm_rope(q, k, pos[None], cos, sin, qw, kw, 1e-6)
    _within_ulps(oq, rq[0], 1, "q packed", pairs=True)
    _within_ulps(ok, rk[0], 1, "k packed", pairs=True)


@pytest.mark.parametrize("packed", [False, True])
def test_fused_qkv_gradient_is_the_per_slice_one(packed):
    b, s, hq, hkv, d = 2, 50, 8, 2, 64
    qkv, pos, qw, kw, cos, sin, dq, dk, dv = _inputs(b, s, hq, hkv, d, torch.bfloat16, seed=1)
    if packed:
        qkv, pos, dq, dk, dv = qkv[0], pos[0], dq[0], dk[0], dv[0]
    dev = [t.cuda() for t in (pos, cos, sin)]

    x1 = qkv.cuda().requires_grad_(True)
    w1 = [qw.cuda().requires_grad_(True), kw.cuda().requires_grad_(True)]
    q1, k1, v1 = bio.qkv_norm_rope(x1, hq, hkv, d, *dev, *w1)
    assert v1.data_ptr() == x1.data_ptr() + (hq + hkv) * d * 2, "v must be a view of qkv"
    g1 = torch.autograd.grad((q1, k1, v1), (x1, *w1), (dq.cuda(), dk.cuda(), dv.cuda()))

    x2 = qkv.cuda().requires_grad_(True)
    w2 = [qw.cuda().requires_grad_(True), kw.cuda().requires_grad_(True)]
    lead = x2.shape[:-1]
    q2, k2, v2 = (t.view(*lead, -1, d) for t in x2.split((hq * d, hkv * d, hkv * d), -1))
    oq, ok = bio.qk_norm_rope(q2, k2, *dev, *w2)
    g2 = torch.autograd.grad((oq, ok, v2), (x2, *w2), (dq.cuda(), dk.cuda(), dv.cuda()))
    torch.cuda.synchronize()
    assert torch.equal(q1, oq) and torch.equal(k1, ok) and torch.equal(v1, v2)
    for a, e in zip(g1, g2):
        assert torch.equal(a, e)


def test_fused_qkv_without_value_gradient():
    b, s, hq, hkv, d = 1, 16, 4, 2, 32
    qkv, pos, qw, kw, cos, sin, dq, dk, _ = _inputs(b, s, hq, hkv, d, torch.bfloat16, seed=2)
    x = qkv.cuda().requires_grad_(True)
    q, k, v = bio.qkv_norm_rope(x, hq, hkv, d, pos.cuda(), cos.cuda(), sin.cuda(), qw.cuda(), kw.cuda())
    (gx,) = torch.autograd.grad((q, k), (x,), (dq.cuda(), dk.cuda()))
    assert torch.equal(gx[..., (hq + hkv) * d:], torch.zeros_like(gx[..., (hq + hkv) * d:]))


def test_weight_gradients_are_deterministic():
    b, s, hq, hkv, d = 2, 700, 16, 4, 128
    qkv, pos, qw, kw, cos, sin, dq, dk, dv = _inputs(b, s, hq, hkv, d, torch.bfloat16, seed=4)
    outs = []
    for _ in range(3):
        x = qkv.cuda().requires_grad_(True)
        w = [qw.cuda().requires_grad_(True), kw.cuda().requires_grad_(True)]
        q, k, v = bio.qkv_norm_rope(x, hq, hkv, d, pos.cuda(), cos.cuda(), sin.cuda(), *w)
        outs.append(torch.autograd.grad((q, k, v), (x, *w), (dq.cuda(), dk.cuda(), dv.cuda())))
    for g in outs[1:]:
        for a, e in zip(g, outs[0]):
            assert torch.equal(a, e)


def test_full_size_cfg3_shape():
    """BASELINE config 3's projection shape: 16384 packed tokens, Hq=16, Hkv=4, D=128."""
    t, hq, hkv, d = 16384, 16, 4, 128
    _say("prologue full size (16384, 16+4+4, 128)")
    qkv, _, qw, kw, cos, sin, dq, dk, dv = _inputs(1, t, hq, hkv, d, torch.bfloat16, seed=5, table=16384,
                                                    theta=500000.0)
    qkv, dq, dk, dv = qkv[0], dq[0], dk[0], dv[0]
    # positions restart at every document, as a packed varlen batch's do
    lens = [711, 2660, 98, 121, 284, 1387, 690, 4956, 583, 1375, 347, 449, 71, 145, 266, 792, 1449]
    pos = torch.cat([torch.arange(n) for n in lens])
    x = qkv.cuda().requires_grad_(True)
    w = [qw.cuda().requires_grad_(True), kw.cuda().requires_grad_(True)]
    q, k, v = bio.qkv_norm_rope(x, hq, hkv, d, pos.cuda(), cos.cuda(), sin.cuda(), *w)
    g = torch.autograd.grad((q, k, v), (x, *w), (dq.cuda(), dk.cuda(), dv.cuda()))
    torch.cuda.synchronize()

    xc = qkv.clone().requires_grad_(True)
    qc, kc, vc = (u.view(t, -1, d) for u in xc.split((hq * d, hkv * d, hkv * d), -1))
    wc = [qw.clone().requires_grad_(True), kw.clone().requires_grad_(True)]
    rq, rk = ob.qk_norm_rope(qc[None], kc[None], pos[None], cos, sin, *wc, 1e-6)
    rg = torch.autograd.grad((rq, rk, vc), (xc, *wc), (dq[None], dk[None], dv))
    _within_ulps(q, rq[0], 1, "q", pairs=True)
    _within_ulps(k, rk[0], 1, "k", pairs=True)
    assert_close(g[0], rg[0])
    assert_north_star(g[0], rg[0], what="d(qkv)")
    for got, ref in zip(g[1:], rg[1:]):
        assert (got.cpu() - ref).abs().max().item() <= 1e-3 * ref.abs().max().item() + 1e-5


@pytest.mark.parametrize("shape,dtype", [((2, 37, 512), torch.bfloat16), ((300, 64), torch.bfloat16),
                                         ((4, 8, 128), torch.float16), ((16384, 2048), torch.bfloat16)])
def test_output_gate_matches_oracle(shape, dtype):
    _say(f"gate {shape} {dtype}")
    g = torch.Generator().manual_seed(7)
    x = torch.randn(*shape, generator=g).to(dtype)
    gate = (torch.randn(*shape, generator=g) * 3).to(dtype)
    dy = torch.randn(*shape, generator=g).to(dtype)
    xd, gd = x.cuda().requires_grad_(True), gate.cuda().requires_grad_(True)
    y = bio.output_gate(xd, gd)
    dx, dg = torch.autograd.grad(y, (xd, gd), dy.cuda())
    xc, gc = x.clone().requires_grad_(True), gate.clone().requires_grad_(True)
    ry = ob.output_gate(xc, gc)
    rdx, rdg = torch.autograd.grad(ry, (xc, gc), dy)
    _within_ulps(y, ry, 1, "y")
    _within_ulps(dx, rdx, 1, "dx")
    _within_ulps(dg, rdg, 1, "dgate")


def test_output_gate_strided_input():
    """A gate that is a column slice of a wider projection (non-contiguous rows)."""
    g = torch.Generator().manual_seed(8)
    wide = torch.randn(64, 3 * 256, generator=g).to(torch.bfloat16)
    x = torch.randn(64, 256, generator=g).to(torch.bfloat16)
    y = bio.output_gate(x.cuda(), wide.cuda()[:, 256:512])
    _within_ulps(y, ob.output_gate(x, wide[:, 256:512]), 1, "y strided")


def test_errors_match_the_conventions():
    x = torch.zeros(2, 4, 2, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(TypeError):
        bio.qk_norm_rope(x.float(), x.float(), None, None, None)
    with pytest.raises(ValueError, match="head_dim"):
        bio.qk_norm_rope(x[..., :48], x[..., :48], None, None, None)
    with pytest.raises(ValueError, match="both be given"):
        bio.qk_norm_rope(x, x, None, None, None, q_weight=torch.ones(64, device="cuda"))
    with pytest.raises(ValueError, match="position_ids"):
        c = torch.ones(16, 64, device="cuda")
        bio.qk_norm_rope(x, x, None, c, c)
    with pytest.raises(ValueError, match="multiple of 8"):
        bio.output_gate(x[..., :12], x[..., :12])

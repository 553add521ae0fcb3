"""Pins of the CPU oracle (oracle/attention.py), run on the CPU.

Each oracle function is checked against something that does not share its code: the
independent float64 C brute force (oracle/attn_ref.c), torch's scaled_dot_product_attention,
closed forms, finite differences, explicit loops over the mask formula and exhaustive
invariants. Planted-mistake tests show that plausible slips in the oracle (a shifted mask
bound, a dropped scale, a wrong GQA head map, a natural-log LSE) fail these pins.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as A
from oracle.cref import UNBOUNDED, attn_ref


def _rand(*shape, seed=0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed))


CASES = [
    # (B, Lq, Lk, H, Hkv, D, causal, window)
    (2, 16, 16, 4, 2, 16, True, (-1, -1)),
    (1, 23, 23, 2, 1, 32, True, (5, 0)),
    (2, 9, 17, 4, 4, 16, True, (-1, -1)),     # queries at the end of the keys
    (1, 20, 7, 3, 1, 16, True, (-1, -1)),     # Lq > Lk: empty rows
    (1, 19, 19, 2, 2, 32, False, (-1, -1)),
    (1, 19, 25, 4, 2, 16, False, (4, 3)),     # asymmetric bidirectional window
    (1, 12, 30, 8, 2, 16, True, (0, 0)),      # each row sees exactly one key
]


def _resolved(causal, window):
    return A.window(causal, window)


def _c_oracle(q, k, v, causal, window, dout=None, scale=None):
    wl, wr = _resolved(causal, window)
    return attn_ref(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                    None if dout is None else dout.double().numpy(), window_left=wl, window_right=wr, scale=scale)


@pytest.mark.parametrize("case", CASES)
def test_forward_and_lse_match_float64_bruteforce(case):
    b, lq, lk, h, hk, d, causal, window = case
    q, k, v = _rand(b, lq, h, d, seed=1), _rand(b, lk, hk, d, seed=2), _rand(b, lk, hk, d, seed=3)
    o, lse = A.reference_with_lse(q, k, v, causal, window)
    ref = _c_oracle(q, k, v, causal, window)
    np.testing.assert_allclose(o.numpy(), ref["o"], rtol=0, atol=2e-5)
    inf = np.isinf(ref["lse2"])
    assert np.array_equal(np.isinf(lse.numpy()), inf)
    np.testing.assert_allclose(lse.numpy()[~inf], ref["lse2"][~inf], rtol=0, atol=2e-5)


@pytest.mark.parametrize("case", CASES)
def test_gradients_match_float64_bruteforce(case):
    b, lq, lk, h, hk, d, causal, window = case
    q, k, v = _rand(b, lq, h, d, seed=4), _rand(b, lk, hk, d, seed=5), _rand(b, lk, hk, d, seed=6)
    dout = _rand(b, lq, h, d, seed=7)
    dq, dk, dv = A.backward_reference(q, k, v, dout, causal, window)
    ref = _c_oracle(q, k, v, causal, window, dout)
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        np.testing.assert_allclose(got.numpy(), ref[key], rtol=0, atol=5e-5)


def test_bruteforce_backward_matches_finite_differences():
    """Pins the C backward (and through it the autograd oracle) by central differences."""
    rng = np.random.default_rng(0)
    b, lq, lk, h, hk, d = 1, 5, 7, 2, 1, 4
    q, k, v = rng.standard_normal((b, lq, h, d)), rng.standard_normal((b, lk, hk, d)), rng.standard_normal((b, lk, hk, d))
    dout = rng.standard_normal((b, lq, h, d))
    wl, wr = 3, 0
    res = attn_ref(q, k, v, dout, window_left=wl, window_right=wr)

    def loss(q_, k_, v_):
        return float((attn_ref(q_, k_, v_, window_left=wl, window_right=wr)["o"] * dout).sum())

    eps = 1e-6
    for name, x, g in (("q", q, res["dq"]), ("k", k, res["dk"]), ("v", v, res["dv"])):
        num = np.zeros_like(x)
        it = np.nditer(x, flags=["multi_index"])
        for _ in it:
            i = it.multi_index
            xp, xm = x.copy(), x.copy()
            xp[i] += eps
            xm[i] -= eps
            args_p = {"q": (xp, k, v), "k": (q, xp, v), "v": (q, k, xp)}[name]
            args_m = {"q": (xm, k, v), "k": (q, xm, v), "v": (q, k, xm)}[name]
            num[i] = (loss(*args_p) - loss(*args_m)) / (2 * eps)
        np.testing.assert_allclose(g, num, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("lq, lk, hq, hk", [(64, 64, 4, 2), (33, 33, 8, 8), (17, 17, 4, 1)])
def test_causal_matches_torch_sdpa(lq, lk, hq, hk):
    """A library routine fixes the causal / full cases (Lq == Lk: top-left = bottom-right)."""
    q, k, v = _rand(2, lq, hq, 32, seed=8), _rand(2, lk, hk, 32, seed=9), _rand(2, lk, hk, 32, seed=10)
    for causal in (True, False):
        got = A.reference(q, k, v, causal, (-1, -1))
        exp = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                             is_causal=causal, enable_gqa=True).transpose(1, 2)
        torch.testing.assert_close(got, exp, rtol=1e-5, atol=1e-5)


def test_closed_forms():
    # One visible key (window (0, 0)): O = v_j, LSE = scale * q.k_j * log2(e).
    q, k, v = _rand(1, 6, 2, 16, seed=11), _rand(1, 10, 2, 16, seed=12), _rand(1, 10, 2, 16, seed=13)
    o, lse = A.reference_with_lse(q, k, v, False, (0, 0))
    j = torch.arange(6) + 4
    torch.testing.assert_close(o[0], v[0, j], rtol=0, atol=1e-6)
    s = (q[0] * k[0, j]).sum(-1) / 4.0 * A.LOG2E  # (6, 2)
    torch.testing.assert_close(lse, s.T, rtol=0, atol=1e-5)
    # q = 0: uniform weights over the visible keys, LSE = log2(count).
    qz = torch.zeros(1, 8, 2, 16)
    o, lse = A.reference_with_lse(qz, k[:, :8], v[:, :8], True, (2, 0))
    for i in range(8):
        vis = list(range(max(0, i - 2), i + 1))
        torch.testing.assert_close(o[0, i], v[0, vis].mean(0), rtol=0, atol=1e-6)
        assert abs(lse[0, i].item() - math.log2(len(vis))) < 1e-6
    # Lq > Lk, causal: the first Lq - Lk rows see nothing -> O = 0, LSE = +inf.
    o, lse = A.reference_with_lse(_rand(1, 9, 2, 16), k[:, :4], v[:, :4], True, (-1, -1))
    assert torch.all(o[0, :5] == 0) and torch.all(torch.isinf(lse[:, :5])) and torch.all(lse[:, :5] > 0)
    assert torch.all(torch.isfinite(lse[:, 5:]))


def test_delta_identity():
    """delta = rowsum(dO * O) (flash_attn.py:215) equals sum_j P_ij dP_ij."""
    q, k, v, do = _rand(1, 12, 2, 16, seed=14), _rand(1, 12, 2, 16, seed=15), _rand(1, 12, 2, 16, seed=16), \
        _rand(1, 12, 2, 16, seed=17)
    o = A.reference(q, k, v, True, (4, 0))
    delta = (o * do).sum(-1)  # (1, Lq, H)
    vis = A.visible_mask(12, 12, True, (4, 0))
    s = torch.einsum("bqhd,bkhd->bhqk", q, k) / 4.0
    p = torch.softmax(s.masked_fill(~vis, float("-inf")), -1)
    dp = torch.einsum("bqhd,bkhd->bhqk", do, v)
    torch.testing.assert_close(delta, (p * dp).sum(-1).permute(0, 2, 1), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("lq, lk", [(7, 7), (5, 11), (11, 5), (1, 9), (9, 1)])
@pytest.mark.parametrize("causal, window", [(True, (-1, -1)), (True, (2, 0)), (False, (-1, -1)), (False, (3, 1)),
                                            (False, (0, 4)), (True, (0, 7))])
def test_mask_matches_formula_loops(lq, lk, causal, window):
    """flash_attn.py:14-18, written as explicit loops."""
    wl, wr = A.window(causal, window)
    m = A.visible_mask(lq, lk, causal, window)
    for i in range(lq):
        for j in range(lk):
            assert bool(m[i, j]) == (i + lk - lq - wl <= j <= i + lk - lq + wr), (i, j)


@pytest.mark.parametrize("n, w", [(1, None), (10, None), (10, 3), (10, 10), (10, 40), (257, 64)])
def test_pair_count_closed_form(n, w):
    """P(n, w) = w(w+1)/2 + (n-w) w (each query sees min(i+1, w) keys) vs the mask."""
    brute = int(A.visible_mask(n, n, True, ((w - 1) if w else -1, 0)).sum())
    assert A.visible_pairs([n], w) == brute == sum(min(i + 1, w or n) for i in range(n))


def _block_ranges_invariants(fn):
    """Exhaustive small-case invariants of a block-range function; returns the first failure."""
    for bt in (1, 2, 4, 8):
        for bs in (1, 3, 4, 8):
            for t_len in (0, 1, 5, 8, 13):
                for s0 in range(0, 12, 3):
                    for lo_off in (-UNBOUNDED, -9, -4, -1, 0, 2, 5):
                        for hi_off in (-3, 0, 1, 4, 9, UNBOUNDED):
                            lo, mid_lo, mid_hi, hi = fn(s0, bs, lo_off, hi_off, t_len, bt)
                            selfs = range(s0, s0 + bs)
                            vis = {t for s in selfs for t in range(t_len) if lo_off <= t - s <= hi_off}
                            args = (s0, bs, lo_off, hi_off, t_len, bt)
                            if lo % bt or not (lo <= mid_lo <= mid_hi <= hi) and hi > lo:
                                return args, "ordering/alignment"
                            if any(not (lo <= t < hi) for t in vis):
                                return args, "visible element outside [lo, hi)"
                            for t in range(mid_lo, mid_hi):
                                if any(not (lo_off <= t - s <= hi_off and t < t_len) for s in selfs):
                                    return args, "masked element inside [mid_lo, mid_hi)"
    return None


def test_block_ranges_invariants():
    assert _block_ranges_invariants(A.block_ranges) is None


def test_planted_mistakes_fail_the_pins():
    """Plant plausible mistakes in the oracle and show that the pins above catch them."""
    b, lq, lk, h, hk, d = 1, 9, 13, 4, 2, 16
    q, k, v = _rand(b, lq, h, d, seed=20), _rand(b, lk, hk, d, seed=21), _rand(b, lk, hk, d, seed=22)
    ref = _c_oracle(q, k, v, True, (3, 0))

    orig_mask = A.visible_mask

    def shifted_mask(lq_, lk_, causal, window):  # off-by-one right bound
        m = orig_mask(lq_, lk_, causal, window)
        return m | torch.roll(m, 1, dims=1)

    def wrong_gqa(q_, k_, v_, causal, window, scale=None):  # h % Hkv instead of h // group
        rep = q_.shape[2] // k_.shape[2]
        return A.reference(q_, k_.repeat(1, 1, rep, 1), v_.repeat(1, 1, rep, 1), causal, window, scale)

    try:
        A.visible_mask = shifted_mask
        bad = A.reference(q, k, v, True, (3, 0))
    finally:
        A.visible_mask = orig_mask
    assert np.abs(bad.numpy() - ref["o"]).max() > 1e-3
    assert np.abs(wrong_gqa(q, k, v, True, (3, 0)).numpy() - ref["o"]).max() > 1e-3
    no_scale = A.reference(q, k, v, True, (3, 0), softmax_scale=1.0)
    assert np.abs(no_scale.numpy() - ref["o"]).max() > 1e-3
    _, lse = A.reference_with_lse(q, k, v, True, (3, 0))
    fin = ~np.isinf(ref["lse2"])
    assert np.abs(lse.numpy()[fin] / A.LOG2E - ref["lse2"][fin]).max() > 1e-3  # natural-log LSE is caught

    def bad_ranges(s0, bs, lo_off, hi_off, t_len, bt):  # mid_hi without the +1
        lo, mid_lo, mid_hi, hi = A.block_ranges(s0, bs, lo_off, hi_off, t_len, bt)
        mh = max(min(s0 + hi_off + 2, t_len), 0) // bt * bt
        return lo, mid_lo, max(mh, mid_lo), hi

    assert _block_ranges_invariants(bad_ranges) is not None


def test_varlen_documents_are_independent():
    """Changing one document's tokens leaves every other document's output unchanged."""
    lengths = [5, 9, 3]
    cu = torch.tensor([0, 5, 14, 17], dtype=torch.int32)
    q, k, v = _rand(17, 4, 16, seed=30), _rand(17, 2, 16, seed=31), _rand(17, 2, 16, seed=32)
    o1 = A.reference_varlen(q, k, v, cu, True, (-1, -1))
    k2 = k.clone()
    k2[5:14] = _rand(9, 2, 16, seed=33)
    o2 = A.reference_varlen(q, k2, v, cu, True, (-1, -1))
    assert torch.equal(o1[:5], o2[:5]) and torch.equal(o1[14:], o2[14:])
    assert not torch.allclose(o1[5:14], o2[5:14])
    assert o1.shape[0] == sum(lengths)


def test_kvcache_reference_writes_and_attends():
    b, cap, hk, d = 2, 12, 2, 16
    kc, vc = torch.zeros(b, cap, hk, d), torch.zeros(b, cap, hk, d)
    kn, vn = _rand(b, 3, hk, d, seed=40), _rand(b, 3, hk, d, seed=41)
    lens = torch.tensor([4, 10])
    q = _rand(b, 3, 4, d, seed=42)
    o, lse, kc2, vc2 = A.kvcache_reference(q, kc, vc, kn, vn, lens, True, (-1, -1))
    assert torch.equal(kc2[0, 4:7], kn[0]) and torch.equal(kc2[1, 10:12], kn[1, :2])  # beyond capacity dropped
    exp = A.reference(q[1:2], kc2[1:2, :12], vc2[1:2, :12], True, (-1, -1))
    torch.testing.assert_close(o[1:2], exp)

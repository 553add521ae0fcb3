"""The compact row layout of the stored dS (ds_band / ds_row_off / ds_seq_blocks / ds_head_blocks
in myk_llm_amd/csrc/bwd.hip), restated and checked on the CPU against the attention mask itself
(flash_attn.py:11-22): query tile i of a sequence owns row_off(i + 1) - row_off(i) slots starting
at its first key block max(i + floor(lo_f / 32), 0); every 32-key block holding a visible
(query, key) pair of the tile must get a slot, rows must not overlap, and the host's size bound
must cover every packed batch it admits. A planted mistake in the closed form is caught."""

import random

import pytest

UNBOUNDED = 1 << 30


def band(k_len, q_len, wl, wr):
    return k_len - q_len - wl, min(k_len - q_len + wr, UNBOUNDED)


def ds_band(q_len, k_len, wl, wr, c_hi_extra=1):
    lo_f, hi_f = band(k_len, q_len, wl, wr)
    return lo_f >> 5, c_hi_extra - ((-hi_f) >> 5), (k_len + 31) >> 5


def clamp_sum(c, i, n):
    lo = min(max(-c, 0), i)
    hi = min(max(n - c, 0), i)
    return (hi - lo) * c + (hi * (hi - 1) - lo * (lo - 1)) // 2 + (i - hi) * n


def row_off(bd, i):
    c_lo, c_hi, n = bd
    return clamp_sum(c_hi, i, n) - clamp_sum(c_lo, i, n)


def seq_blocks(q_len, k_len, wl, wr, **kw):
    if q_len <= 0 or k_len <= 0:
        return 0
    return row_off(ds_band(q_len, k_len, wl, wr, **kw), (q_len + 31) >> 5)


def visible_blocks(q_len, k_len, wl, wr, i):
    """Key blocks with a visible pair in query tile i, straight from the mask."""
    lo_f, hi_f = band(k_len, q_len, wl, wr)
    out = set()
    for q in range(32 * i, min(32 * i + 32, q_len)):
        lo, hi = max(q + lo_f, 0), min(q + hi_f, k_len - 1)
        for k in range(lo, hi + 1):
            out.add(k >> 5)
    return out


def check_sequence(q_len, k_len, wl, wr, **kw):
    bd = ds_band(q_len, k_len, wl, wr, **kw)
    lo_f, _ = band(k_len, q_len, wl, wr)
    nt = (q_len + 31) >> 5
    for i in range(nt):
        w = row_off(bd, i + 1) - row_off(bd, i)
        assert w >= 0
        vis = visible_blocks(q_len, k_len, wl, wr, i)
        if vis:
            first = max(i + (lo_f >> 5), 0)
            assert min(vis) >= first, (q_len, k_len, wl, wr, i)
            assert max(vis) - first < w, (q_len, k_len, wl, wr, i, sorted(vis), first, w)
    return row_off(bd, nt)


CASES = [(q, k, wl, wr) for q, k in [(1, 1), (31, 31), (32, 32), (33, 33), (100, 100), (257, 257), (64, 200),
                                     (200, 64), (5, 300), (300, 5)]
         for wl, wr in [(UNBOUNDED, 0), (0, 0), (31, 0), (32, 0), (100, 0), (UNBOUNDED, UNBOUNDED), (10, 40),
                        (UNBOUNDED, 7)]]


@pytest.mark.parametrize("q_len, k_len, wl, wr", CASES)
def test_every_visible_block_has_a_slot(q_len, k_len, wl, wr):
    total = check_sequence(q_len, k_len, wl, wr)
    assert total == seq_blocks(q_len, k_len, wl, wr)


def test_causal_rows_are_a_triangle():
    # Causal self-attention of n tiles: rows of 1, 2, ..., n blocks.
    for n in (1, 5, 40):
        assert seq_blocks(32 * n, 32 * n, UNBOUNDED, 0) == n * (n + 1) // 2
    # A 1024-key window (w - 1 = 1023 left): rows grow to 33 blocks and stay there.
    bd = ds_band(8192, 8192, 1023, 0)
    widths = [row_off(bd, i + 1) - row_off(bd, i) for i in range(256)]
    assert widths[:33] == list(range(1, 34)) and set(widths[33:]) == {33}


def head_blocks_bound(rows, batch, max_q, max_k, wl, wr, same_cu=True):
    tiles = (rows + 31 * batch) // 32
    rect = tiles * min((max_k + 31) // 32, (32 + wl + wr + 31) // 32 + 1)
    if not same_cu or wr != 0:
        return rect
    m = min(max_q, max_k)
    ntm = (m + 31) // 32
    if ntm <= 0:
        return rect
    return min(rect, -(-tiles * seq_blocks(m, m, wl, wr) // ntm))


def test_packed_bound_covers_every_batch():
    """For packed causal self-attention the host sizes the dS by (rows, batch, max_seqlen) alone;
    random batches (including empty and maximal documents) never need more."""
    rng = random.Random(0)
    for _ in range(3000):
        batch = rng.randint(1, 20)
        max_len = rng.choice([1, 31, 33, 200, 1000, 4956])
        lens = [rng.choice([0, max_len, rng.randint(0, max_len)]) for _ in range(batch)]
        wl, wr = rng.choice([(UNBOUNDED, 0), (0, 0), (255, 0), (1023, 0), (UNBOUNDED, 5), (40, 40)])
        rows = sum(lens)
        need = sum(seq_blocks(n, n, wl, wr) for n in lens)
        assert need <= head_blocks_bound(rows, batch, max(lens), max(lens), wl, wr), (lens, wl, wr)


def test_planted_mistake_fails():
    """Dropping the one-block allowance of c_hi (a band end rounded as if it were aligned)
    leaves visible blocks without a slot."""
    with pytest.raises(AssertionError):
        for q, k, wl, wr in CASES:
            check_sequence(q, k, wl, wr, c_hi_extra=0)

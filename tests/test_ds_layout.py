"""The stored-dS block layout shared by the dK/dV and dQ-from-dS kernels (ds_chunk and
lds_tr_block32 in myk_llm_amd/csrc/bwd.hip), restated and checked on the CPU: a dK/dV wave's two
stores each cover 1 KB of the block exactly once, the dQ pass's transpose reads hand every lane
the MFMA operand it needs (keys 16 kb + 8 g + 0..7 of query l32), and each 32-lane half of a
transpose read touches all 64 LDS banks once (no bank conflicts)."""

import numpy as np


def ds_chunk(kb, g, key):
    return 64 * kb + 32 * g + (key ^ (4 * (2 * kb + g)))


def _stored_block():
    """Element index -> (key, query) code of a 32 x 32 block written by the dK/dV wave: lane
    (key l32, g) holds queries 16 kb + 8 g + 0..7 of its key in register group kb."""
    blk = -np.ones(1024, dtype=np.int64)
    for kb in range(2):
        for lane in range(64):
            l32, g = lane & 31, lane >> 5
            for i in range(8):
                blk[ds_chunk(kb, g, l32) * 8 + i] = l32 * 32 + 16 * kb + 8 * g + i
    return blk


def _tr_read(blk, addr):
    """ds_read_b64_tr_b16: within each 16-lane group, lane j receives element j % 4 of the
    4-element vector addressed by lane 4 i + j // 4, for i = 0..3."""
    out = np.zeros((64, 4), dtype=np.int64)
    for grp in range(4):
        for j in range(16):
            for i in range(4):
                out[16 * grp + j, i] = blk[addr[16 * grp + 4 * i + j // 4] + j % 4]
    return out


def _tr_addresses(kbp):
    a0, a1 = [], []
    for lane in range(64):
        grp, jj = lane >> 4, lane & 15
        key = 16 * kbp + 8 * (grp >> 1) + (jj >> 2)
        qk, qg, half = grp & 1, (jj >> 1) & 1, 4 * (jj & 1)
        a0.append(ds_chunk(qk, qg, key) * 8 + half)
        a1.append(ds_chunk(qk, qg, key + 4) * 8 + half)
    return a0, a1


def test_stores_cover_each_half_once():
    for kb in range(2):
        chunks = sorted(ds_chunk(kb, lane >> 5, lane & 31) for lane in range(64))
        assert chunks == list(range(64 * kb, 64 * kb + 64))
    assert (_stored_block() >= 0).all()


def test_transpose_reads_form_the_operand():
    blk = _stored_block()
    for kbp in range(2):
        a0, a1 = _tr_addresses(kbp)
        got = np.concatenate([_tr_read(blk, a0), _tr_read(blk, a1)], axis=1)
        for lane in range(64):
            l32, g = lane & 31, lane >> 5
            assert list(got[lane]) == [(16 * kbp + 8 * g + i) * 32 + l32 for i in range(8)]


def test_transpose_reads_are_conflict_free():
    for kbp in range(2):
        for addr in _tr_addresses(kbp):
            for half in range(2):
                banks = []
                for lane in range(32 * half, 32 * half + 32):
                    b0 = (addr[lane] * 2 // 4) % 64
                    banks += [b0, (b0 + 1) % 64]
                assert sorted(banks) == list(range(64))


def test_planted_layout_mistake_fails():
    """Without the XOR (the plain lane-major layout) the reads still form the operand but hit
    each bank twice: the conflict check is what pins the swizzle."""
    def plain(kb, g, key):
        return 64 * kb + 32 * g + key
    addr = []
    for lane in range(32):
        grp, jj = lane >> 4, lane & 15
        key = 8 * (grp >> 1) + (jj >> 2)
        addr.append(plain(grp & 1, (jj >> 1) & 1, key) * 8 + 4 * (jj & 1))
    banks = sorted(((a * 2 // 4) % 64 + d) % 64 for a in addr for d in (0, 1))
    assert banks != list(range(64))

"""mykfa_decode_noalloc (the allocation-free decode: split-K partials in a static device
array) against mykfa_decode with a caller workspace, through the C ABI: bit-identical results
for the same split count on consecutive calls (the second smaller, so stale scratch contents
from the first would show), the library's split count cut to the 16 MiB scratch when its own
choice does not fit, and an explicit split count that does not fit rejected before launch."""

import ctypes
import sys

import pytest
import torch

from _util import assert_close, assert_lse
from myk_llm_amd import _lib
from myk_llm_amd import flash_attn as fa
from oracle.attention import kvcache_reference

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _inputs(batch, cap, lens, nq, heads, kv_heads, d, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)  # noqa: E731
    kc, vc = mk(batch, cap, kv_heads, d), mk(batch, cap, kv_heads, d)
    q, kn, vn = mk(batch, nq, heads, d), mk(batch, nq, kv_heads, d), mk(batch, nq, kv_heads, d)
    return q, kc, vc, kn, vn, torch.tensor(lens, dtype=torch.int32)


def _params(q, kc, vc, cl, kn, vn, splits):
    out = torch.empty_like(q)
    lse = torch.full((q.shape[2], q.shape[0] * q.shape[1]), float("nan"), dtype=torch.float32, device="cuda")
    p = _lib.DecodeParams()
    p.fwd = fa._fwd_params(q, kc, vc, out, lse, None, None, cl, q.shape[1], kc.shape[1], q.shape[-1] ** -0.5,
                           _lib.UNBOUNDED, 0)
    p.num_splits = splits
    p.seqlen_new = kn.shape[1]
    p.k_new, p.v_new = kn.data_ptr(), vn.data_ptr()
    p.kn_batch_stride, p.kn_token_stride, p.kn_head_stride = fa._strides(kn)
    p.vn_batch_stride, p.vn_token_stride, p.vn_head_stride = fa._strides(vn)
    return p, out, lse


def _run(noalloc, q, kc, vc, cl, kn, vn, splits):
    """One decode step (append + split-K + merge) on copies of the caches; returns (O, LSE, K, V)."""
    kc, vc = kc.clone(), vc.clone()
    p, out, lse = _params(q, kc, vc, cl, kn, vn, splits)
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        _lib.check(L.mykfa_decode_noalloc(ctypes.byref(p), stream))
    else:
        n = splits if splits > 0 else L.mykfa_decode_num_splits(p.fwd.batch, p.fwd.num_heads, p.fwd.num_kv_heads,
                                                                 p.fwd.max_seqlen_q, p.fwd.max_seqlen_k)
        p.num_splits = n
        nbytes = L.mykfa_decode_workspace_size(p.fwd.batch, p.fwd.num_heads, p.fwd.max_seqlen_q, q.shape[-1], n)
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device="cuda")
        _lib.check(L.mykfa_decode(ctypes.byref(p), ws.data_ptr(), ws.numel(), stream))
    torch.cuda.synchronize()
    return out, lse, kc, vc


def _gpu(*xs):
    return [x.cuda() for x in xs]


def test_noalloc_matches_the_workspace_entry_point_on_consecutive_calls():
    # cfg5's shape class (one query, Hq 16 / Hkv 4, D 64) at 64 sequences, then a smaller batch
    # with shorter caches: the second call must not see the first call's partials.
    cases = [(64, 4100, 1, 64, 11), (5, 1500, 4, 64, 12)]
    for batch, cap, nq, d, seed in cases:
        g = torch.Generator().manual_seed(seed)
        lens = torch.randint(0, cap - nq, (batch,), generator=g).tolist()
        q, kc, vc, kn, vn, cl = _gpu(*_inputs(batch, cap, lens, nq, 16, 4, d, seed))
        _say(f"noalloc batch={batch} cap={cap} nq={nq} D={d}")
        L = _lib.lib()
        splits = L.mykfa_decode_num_splits(batch, 16, 4, nq, cap)
        assert splits > 1
        assert L.mykfa_decode_workspace_size(batch, 16, nq, d, splits) <= _lib.DECODE_SCRATCH_BYTES
        got = _run(True, q, kc, vc, cl, kn, vn, 0)
        ref = _run(False, q, kc, vc, cl, kn, vn, splits)
        for a, b in zip(got, ref):
            assert torch.equal(a, b)
        exp, exp_lse, ekc, evc = kvcache_reference(q.float().cpu(), kc.float().cpu(), vc.float().cpu(),
                                                   kn.float().cpu(), vn.float().cpu(), cl.cpu(), True, (-1, -1))
        assert torch.equal(got[2].cpu().float(), ekc) and torch.equal(got[3].cpu().float(), evc)
        assert_close(got[0], exp)
        assert_lse(got[1], exp_lse)


def test_noalloc_cuts_its_split_count_to_the_scratch():
    """16 sequences x 16 query rows x D = 256: the library's choice (9 split slots per sequence,
    19 MB of 16-bit partials) does not fit 16 MiB; the allocation-free call runs the largest count
    that does (7) and equals the workspace entry point at that count."""
    batch, cap, nq, d = 16, 8192, 16, 256
    g = torch.Generator().manual_seed(21)
    lens = torch.randint(0, cap - nq, (batch,), generator=g).tolist()
    q, kc, vc, kn, vn, cl = _gpu(*_inputs(batch, cap, lens, nq, 16, 4, d, 21))
    L = _lib.lib()
    default = L.mykfa_decode_num_splits(batch, 16, 4, nq, cap)
    per_split = L.mykfa_decode_workspace_size(batch, 16, nq, d, 2) // 2
    assert default * per_split > _lib.DECODE_SCRATCH_BYTES
    fit = _lib.DECODE_SCRATCH_BYTES // per_split
    fit = fit - 1 if fit > 1 and fit % 8 == 0 else fit
    _say(f"noalloc cut: default {default} splits, {fit} fit")
    got = _run(True, q, kc, vc, cl, kn, vn, 0)
    ref = _run(False, q, kc, vc, cl, kn, vn, fit)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    exp, exp_lse, _, _ = kvcache_reference(q.float().cpu(), kc.float().cpu(), vc.float().cpu(), kn.float().cpu(),
                                           vn.float().cpu(), cl.cpu(), True, (-1, -1))
    assert_close(got[0], exp)
    assert_lse(got[1], exp_lse)


def test_noalloc_rejects_an_explicit_split_count_beyond_the_scratch():
    # 12 split slots of 16 sequences x 16 query rows x D = 256: 25 MB of partials > 16 MiB.
    batch, cap, nq, d = 16, 8192, 16, 256
    q, kc, vc, kn, vn, cl = _gpu(*_inputs(batch, cap, [100] * batch, nq, 16, 4, d, 22))
    kc0 = kc.clone()
    p, out, lse = _params(q, kc, vc, cl, kn, vn, 12)
    rc = _lib.lib().mykfa_decode_noalloc(ctypes.byref(p), torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.ERR_WORKSPACE
    assert b"scratch" in _lib.lib().mykfa_last_error()
    torch.cuda.synchronize()
    assert torch.equal(kc, kc0)  # rejected before any launch: the caches are untouched

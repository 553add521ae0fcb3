"""Split-K decode and KV append on the GPU: every split count agrees with the oracle, the
cache write is bit-exact (tests/test_flash_attn.py:102), writes beyond the capacity are
dropped, and a HIP-graph capture of flash_attn_with_kvcache replays to the eager result
(the static-cache decode caller captures one step, scripts/benchmark_decode.py:149-151)."""

import ctypes
import sys

import pytest
import torch

from _util import assert_close, assert_lse
from myk_llm_amd import _lib, flash_attn_with_kvcache
from myk_llm_amd import flash_attn as fa
from oracle.attention import kvcache_reference

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _make(batch, cap, lens, nq, heads, kv_heads, d, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    kc = torch.randn(batch, cap, kv_heads, d, generator=g).to(dtype)
    vc = torch.randn(batch, cap, kv_heads, d, generator=g).to(dtype)
    q = torch.randn(batch, nq, heads, d, generator=g).to(dtype)
    kn = torch.randn(batch, nq, kv_heads, d, generator=g).to(dtype)
    vn = torch.randn(batch, nq, kv_heads, d, generator=g).to(dtype)
    return q, kc, vc, kn, vn, torch.tensor(lens, dtype=torch.int32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("nq", [1, 2, 4, 16])
@pytest.mark.parametrize("heads, kv_heads", [(16, 4), (8, 8), (8, 1)])
@pytest.mark.parametrize("window", [(-1, -1), (100, 0)])
def test_decode_matches_oracle(nq, heads, kv_heads, window, dtype):
    _say(f"decode nq={nq} H={heads}/{kv_heads} window={window} {dtype}")
    lens = [0, 1, 31, 32, 33, 500, 1000, 2047]
    q, kc, vc, kn, vn, cl = _make(len(lens), 2100, lens, nq, heads, kv_heads, 64, dtype=dtype)
    exp, exp_lse, ekc, evc = kvcache_reference(q.float(), kc.float(), vc.float(), kn.float(), vn.float(), cl, True,
                                               window)
    kcg, vcg = kc.cuda(), vc.cuda()
    out, lse = flash_attn_with_kvcache(q.cuda(), kcg, vcg, kn.cuda(), vn.cuda(), cache_seqlens=cl.cuda(),
                                       causal=True, window_size=window, return_softmax_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(kcg.cpu().float(), ekc) and torch.equal(vcg.cpu().float(), evc)
    assert_close(out, exp)
    assert_lse(lse, exp_lse)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [16, 32, 64, 128, 256])
def test_decode_head_dims(d, dtype):
    _say(f"decode D={d} {dtype}")
    lens = [7, 300, 129]
    q, kc, vc, kn, vn, cl = _make(3, 400, lens, 4, 8, 2, d, seed=1, dtype=dtype)
    exp, exp_lse, _, _ = kvcache_reference(q.float(), kc.float(), vc.float(), kn.float(), vn.float(), cl, True,
                                           (-1, -1))
    out, lse = flash_attn_with_kvcache(q.cuda(), kc.cuda(), vc.cuda(), kn.cuda(), vn.cuda(), cache_seqlens=cl.cuda(),
                                       causal=True, return_softmax_lse=True)
    assert_close(out, exp)
    assert_lse(lse, exp_lse)


@pytest.mark.parametrize("batch, heads, kv_heads, nq", [(300, 16, 4, 1), (300, 16, 4, 4), (9, 3, 1, 1), (9, 6, 2, 3)])
def test_decode_large_batches_and_row_counts(batch, heads, kv_heads, nq):
    """More sequences than the split plan's 256 threads take in one pass (every workgroup
    computes the plan in two passes over the lengths), and sequences whose rows (query heads x
    queries) are not a multiple of four, which the merge takes one row per wave instead of four."""
    _say(f"decode batch={batch} H={heads}/{kv_heads} nq={nq}")
    g = torch.Generator().manual_seed(batch + heads + nq)
    lens = torch.randint(0, 300, (batch,), generator=g).tolist()
    lens[0], lens[-1] = 0, 299
    q, kc, vc, kn, vn, cl = _make(batch, 320, lens, nq, heads, kv_heads, 64, seed=batch + nq)
    exp, exp_lse, ekc, evc = kvcache_reference(q.float(), kc.float(), vc.float(), kn.float(), vn.float(), cl, True,
                                               (-1, -1))
    kcg, vcg = kc.cuda(), vc.cuda()
    out, lse = flash_attn_with_kvcache(q.cuda(), kcg, vcg, kn.cuda(), vn.cuda(), cache_seqlens=cl.cuda(),
                                       causal=True, return_softmax_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(kcg.cpu().float(), ekc) and torch.equal(vcg.cpu().float(), evc)
    assert_close(out, exp)
    assert_lse(lse, exp_lse)


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 16, 64, 128])
def test_every_split_count_agrees(splits):
    """The C ABI with an explicit split count: split-K + merge is independent of the split.
    128 splits of 32 keys give rows with up to 125 partials: the merge's 64-split chunks and
    the rescale between them."""
    _say(f"splits={splits}")
    lens = [1000, 17, 4000, 2500]
    q, kc, vc, _, _, cl = _make(len(lens), 4096, lens, 4, 16, 4, 64, seed=2)
    exp, exp_lse, _, _ = kvcache_reference(q.float(), kc.float(), vc.float(), None, None, cl, True, (-1, -1))
    qg, kcg, vcg, clg = q.cuda(), kc.cuda(), vc.cuda(), cl.cuda()
    out = torch.empty_like(qg)
    lse = torch.empty((qg.shape[2], qg.shape[0] * qg.shape[1]), dtype=torch.float32, device="cuda")
    p = _lib.DecodeParams()
    p.fwd = fa._fwd_params(qg, kcg, vcg, out, lse, None, None, clg, q.shape[1], kc.shape[1], 0.125,
                           _lib.UNBOUNDED, 0)
    p.num_splits = splits
    L = _lib.lib()
    nbytes = L.mykfa_decode_workspace_size(p.fwd.batch, p.fwd.num_heads, p.fwd.max_seqlen_q, 64, splits)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(L.mykfa_decode(ctypes.byref(p), ws.data_ptr(), ws.numel(), stream))
    torch.cuda.synchronize()
    assert_close(out, exp)
    assert_lse(lse, exp_lse)
    # Too small a workspace is rejected before any launch.
    if nbytes > 0:
        assert L.mykfa_decode(ctypes.byref(p), ws.data_ptr(), nbytes - 1, stream) == _lib.ERR_WORKSPACE


def test_append_beyond_capacity_is_dropped():
    b, cap, hk, d = 2, 10, 2, 64
    kc = torch.zeros(b, cap, hk, d, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    kn = torch.randn(b, 4, hk, d).to(torch.bfloat16).cuda()
    vn = torch.randn(b, 4, hk, d).to(torch.bfloat16).cuda()
    q = torch.randn(b, 4, 4, d).to(torch.bfloat16).cuda()
    cl = torch.tensor([2, 8], dtype=torch.int32, device="cuda")
    flash_attn_with_kvcache(q, kc, vc, kn, vn, cache_seqlens=cl, causal=True)
    assert torch.equal(kc[0, 2:6], kn[0]) and torch.equal(kc[1, 8:10], kn[1, :2])
    assert torch.all(kc[0, 6:] == 0) and torch.all(kc[0, :2] == 0)


def test_graph_capture_replays_match_eager():
    """Capture one decode step (append + split-K + merge) in a HIP graph; several replays with
    eager work and syncs in between all reproduce the eager result bit for bit."""
    lens = [100, 900, 33]
    q, kc, vc, kn, vn, cl = _make(3, 1024, lens, 4, 16, 4, 64, seed=3)
    q, kn, vn, cl = q.cuda(), kn.cuda(), vn.cuda(), cl.cuda()
    kc_e, vc_e = kc.cuda(), vc.cuda()
    eager = flash_attn_with_kvcache(q, kc_e, vc_e, kn, vn, cache_seqlens=cl, causal=True).clone()
    kc_g, vc_g = kc.cuda(), vc.cuda()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        flash_attn_with_kvcache(q, kc_g, vc_g, kn, vn, cache_seqlens=cl, causal=True)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = flash_attn_with_kvcache(q, kc_g, vc_g, kn, vn, cache_seqlens=cl, causal=True)
    for i in range(4):
        out.zero_()
        torch.randn(1000, device="cuda").sum()  # unrelated eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
    assert torch.equal(kc_g, kc_e)


def _decode_abi(q, kc, vc, cl, splits, kn=None, vn=None, n_new=0):
    """mykfa_decode through the C ABI; kn / vn (or n_new pre-appended rows) are this step's keys."""
    out = torch.empty_like(q)
    lse = torch.empty((q.shape[2], q.shape[0] * q.shape[1]), dtype=torch.float32, device="cuda")
    p = _lib.DecodeParams()
    p.fwd = fa._fwd_params(q, kc, vc, out, lse, None, None, cl, q.shape[1], kc.shape[1], 0.125, _lib.UNBOUNDED, 0)
    p.num_splits = splits
    p.seqlen_new = kn.shape[1] if kn is not None else n_new
    if kn is not None:
        p.k_new, p.v_new = kn.data_ptr(), vn.data_ptr()
        p.kn_batch_stride, p.kn_token_stride, p.kn_head_stride = fa._strides(kn)
        p.vn_batch_stride, p.vn_token_stride, p.vn_head_stride = fa._strides(vn)
    L = _lib.lib()
    nbytes = L.mykfa_decode_workspace_size(p.fwd.batch, p.fwd.num_heads, p.fwd.max_seqlen_q, q.shape[-1], splits)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device="cuda")
    _lib.check(L.mykfa_decode(ctypes.byref(p), ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return out, lse


@pytest.mark.parametrize("splits", [1, 3, 7, 16])
def test_decode_appends_new_keys_itself(splits):
    """k_new / v_new in the decode params: the split-K kernel writes them into the caches
    (flash_attn.py:480-485) before attending. New rows straddle split boundaries (7 splits of
    608 keys over 4096 rows: 606..609, 1214..1217) and the capacity (4093..4096: row 4096 is
    dropped); caches must equal the reference's bit for bit and outputs match the oracle."""
    _say(f"fused append splits={splits}")
    lens = [606, 1214, 0, 4093, 2000]
    q, kc, vc, kn, vn, cl = _make(len(lens), 4096, lens, 4, 16, 4, 64, seed=5)
    exp, exp_lse, ekc, evc = kvcache_reference(q.float(), kc.float(), vc.float(), kn.float(), vn.float(), cl, True,
                                               (-1, -1))
    kcg, vcg = kc.cuda(), vc.cuda()
    out, lse = _decode_abi(q.cuda(), kcg, vcg, cl.cuda(), splits, kn.cuda(), vn.cuda())
    assert torch.equal(kcg.cpu().float(), ekc) and torch.equal(vcg.cpu().float(), evc)
    assert_close(out, exp)
    assert_lse(lse, exp_lse)


def test_decode_counts_preappended_keys():
    """seqlen_new without k_new / v_new: the rows are already in the caches (mykfa_kv_append)
    and the decode attends over seqused_k[b] + seqlen_new keys."""
    lens = [10, 700, 1500]
    q, kc, vc, kn, vn, cl = _make(len(lens), 2048, lens, 2, 8, 2, 64, seed=6)
    exp, exp_lse, ekc, evc = kvcache_reference(q.float(), kc.float(), vc.float(), kn.float(), vn.float(), cl, True,
                                               (-1, -1))
    out, lse = _decode_abi(q.cuda(), ekc.to(torch.bfloat16).cuda(), evc.to(torch.bfloat16).cuda(), cl.cuda(), 5,
                           n_new=kn.shape[1])
    assert_close(out, exp)
    assert_lse(lse, exp_lse)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_append_then_attend_path(dtype):
    """More than 16 new queries take the separate append kernel, then the prefill forward over
    cache_seqlens + new keys (flash_attn.py:480-488); the cache write is bit-exact."""
    _say(f"append path {dtype}")
    lens = [0, 40, 300]
    q, kc, vc, kn, vn, cl = _make(len(lens), 512, lens, 24, 8, 2, 64, seed=7, dtype=dtype)
    exp, exp_lse, ekc, evc = kvcache_reference(q.float(), kc.float(), vc.float(), kn.float(), vn.float(), cl, True,
                                               (-1, -1))
    kcg, vcg = kc.cuda(), vc.cuda()
    out, lse = flash_attn_with_kvcache(q.cuda(), kcg, vcg, kn.cuda(), vn.cuda(), cache_seqlens=cl.cuda(),
                                       causal=True, return_softmax_lse=True)
    assert torch.equal(kcg.cpu().float(), ekc) and torch.equal(vcg.cpu().float(), evc)
    assert_close(out, exp)
    assert_lse(lse, exp_lse)


def test_mismatched_new_keys_raise_before_any_launch():
    """New keys/values must share the caches' dtype and GPU, and cache_seqlens must be on the
    GPU: each mismatch raises and leaves the caches untouched (on both the fused decode path
    and the separate append path)."""
    q, kc, vc, kn, vn, cl = _make(2, 64, [3, 5], 1, 4, 2, 64)
    q, kc, vc, cl = q.cuda(), kc.cuda(), vc.cuda(), cl.cuda()
    kc0 = kc.clone()
    for nq in (1, 20):
        qq = q.expand(2, nq, 4, 64).contiguous()
        knn, vnn = kn.expand(2, nq, 2, 64).contiguous(), vn.expand(2, nq, 2, 64).contiguous()
        with pytest.raises(TypeError):
            flash_attn_with_kvcache(qq, kc, vc, knn.cuda().half(), vnn.cuda().half(), cache_seqlens=cl, causal=True)
        with pytest.raises(TypeError):
            flash_attn_with_kvcache(qq, kc, vc, knn.cuda().float(), vnn.cuda().float(), cache_seqlens=cl, causal=True)
        with pytest.raises(RuntimeError):
            flash_attn_with_kvcache(qq, kc, vc, knn, vnn, cache_seqlens=cl, causal=True)  # new keys on the host
        with pytest.raises(RuntimeError):
            flash_attn_with_kvcache(qq, kc, vc, knn.cuda(), vnn.cuda(), cache_seqlens=cl.cpu(), causal=True)
    torch.cuda.synchronize()
    assert torch.equal(kc, kc0)


def test_new_keys_of_the_wrong_shape_raise():
    q, kc, vc, kn, vn, cl = _make(2, 64, [3, 5], 1, 4, 2, 64)
    q, kc, vc, cl = q.cuda(), kc.cuda(), vc.cuda(), cl.cuda()
    with pytest.raises(RuntimeError):
        flash_attn_with_kvcache(q, kc, vc, kn[:, :, :1].cuda(), vn[:, :, :1].cuda(), cache_seqlens=cl, causal=True)
    with pytest.raises(RuntimeError):
        flash_attn_with_kvcache(q, kc, vc, kn.cuda(), vn[:, :, :1].cuda(), cache_seqlens=cl, causal=True)

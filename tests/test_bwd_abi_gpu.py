"""The backward entry points of the C ABI on the GPU: mykfa_bwd_dq computes delta =
rowsum(dO * O) itself (the preprocess fused into _bwd_dq_kernel, flash_attn.py:215-216) and
writes the same values mykfa_bwd_preprocess does, so dK/dV may follow either; mykfa_bwd is
dQ then dK/dV."""

import ctypes
import sys

import pytest
import torch

from myk_llm_amd import _lib
from myk_llm_amd import flash_attn as fa

pytestmark = pytest.mark.gpu


def _params(q, k, v, out, lse, dout, delta, cu, max_q, max_k, scale, wl, wr):
    p = _lib.BwdParams()
    p.fwd = fa._fwd_params(q, k, v, out, lse, cu, cu, None, max_q, max_k, scale, wl, wr)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    p.dout, p.dq, p.dk, p.dv, p.delta = dout.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), delta.data_ptr()
    p.do_batch_stride, p.do_token_stride, p.do_head_stride = fa._strides(dout)
    p.dq_batch_stride, p.dq_token_stride, p.dq_head_stride = fa._strides(dq)
    p.dk_batch_stride, p.dk_token_stride, p.dk_head_stride = fa._strides(dk)
    p.dv_batch_stride, p.dv_token_stride, p.dv_head_stride = fa._strides(dv)
    return p, dq, dk, dv


@pytest.mark.parametrize("d", [64, 128])
def test_dq_writes_the_preprocess_delta(d):
    print(f"bwd abi D={d}", flush=True)
    sys.stdout.flush()
    g = torch.Generator().manual_seed(11)
    lens = [300, 1, 77, 512]
    tot, h, hk = sum(lens), 8, 2
    q, k, v, do = (torch.randn(tot, n, d, generator=g).to(torch.bfloat16).cuda() for n in (h, hk, hk, h))
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32).cuda()
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    out = torch.empty_like(q)
    lse = torch.empty((h, tot), dtype=torch.float32, device="cuda")
    scale = d ** -0.5
    wl, wr = fa._window(True, (-1, -1))
    fp = fa._fwd_params(q, k, v, out, lse, cu, cu, None, max(lens), max(lens), scale, wl, wr)
    _lib.check(L.mykfa_fwd(ctypes.byref(fp), stream))
    d_pre = torch.full_like(lse, float("nan"))
    d_dq = torch.full_like(lse, float("nan"))
    p1, _, dk1, dv1 = _params(q, k, v, out, lse, do, d_pre, cu, max(lens), max(lens), scale, wl, wr)
    p2, dq2, dk2, dv2 = _params(q, k, v, out, lse, do, d_dq, cu, max(lens), max(lens), scale, wl, wr)
    _lib.check(L.mykfa_bwd_preprocess(ctypes.byref(p1), stream))
    _lib.check(L.mykfa_bwd_dkdv(ctypes.byref(p1), stream))
    _lib.check(L.mykfa_bwd_dq(ctypes.byref(p2), stream))
    _lib.check(L.mykfa_bwd_dkdv(ctypes.byref(p2), stream))
    torch.cuda.synchronize()
    ref = (do.float() * out.float()).sum(-1).t()  # (heads, rows)
    torch.testing.assert_close(d_pre, ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(d_dq, ref, rtol=1e-5, atol=1e-5)
    # dK/dV from either delta agree to bf16 rounding of nearly identical fp32 sums.
    torch.testing.assert_close(dk1.float(), dk2.float(), rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(dv1.float(), dv2.float(), rtol=0, atol=0)
    # mykfa_bwd (dQ then dK/dV) reproduces the two separate calls bit for bit.
    d3 = torch.full_like(lse, float("nan"))
    p3, dq3, dk3, dv3 = _params(q, k, v, out, lse, do, d3, cu, max(lens), max(lens), scale, wl, wr)
    _lib.check(L.mykfa_bwd(ctypes.byref(p3), stream))
    torch.cuda.synchronize()
    assert torch.equal(dq3, dq2) and torch.equal(dk3, dk2) and torch.equal(dv3, dv2)

"""Parity at BASELINE.json's full sizes: the kernels against the fp32 oracle on identical
seeded inputs (myk_llm_amd.bench_configs recipes), with the north-star bounds:
O, dQ, dK, dV within max-abs 2e-2 / mean-abs 2e-3 of the fp32 reference and LSE within
1e-3. For the large configs the oracle's fp32 torch math runs on the GPU (per document /
per batch element); for config 1 it runs on the CPU."""

import sys

import pytest
import torch

from _util import assert_close, assert_lse, assert_north_star, north_star_errors
from myk_llm_amd import flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache
from myk_llm_amd.bench_configs import make_inputs, workloads
from oracle.attention import kvcache_reference, reference, reference_varlen, reference_with_lse

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _report(name, got, exp):
    mx, mn = north_star_errors(got, exp)
    floor_mx, floor_mn = north_star_errors(exp.to(got.dtype).float(), exp)
    _say(f"  {name}: max-abs {mx:.3e} mean-abs {mn:.3e} (bf16 storage floor: {floor_mx:.3e} / {floor_mn:.3e})")


def test_cfg1_cpu_oracle_plumbing():
    """Config 1: B=1, T=512, Hq=Hkv=8, D=64, causal; oracle fp32 on the CPU, kernel on a bf16 copy."""
    _say("cfg1")
    w = workloads()["cfg1"]
    inp = make_inputs(w, device="cpu")
    q, k, v = inp["q"], inp["k"], inp["v"]
    exp_o, exp_lse = reference_with_lse(q, k, v, True, (-1, -1))
    qb, kb, vb = (x.to(torch.bfloat16) for x in (q, k, v))
    exp_b, exp_lse_b = reference_with_lse(qb, kb, vb, True, (-1, -1))
    out, lse = flash_attn_func(qb.cuda(), kb.cuda(), vb.cuda(), causal=True, return_softmax_lse=True)
    _report("O vs oracle(bf16 inputs)", out, exp_b.cuda())
    _report("O vs oracle(fp32 inputs)", out, exp_o.cuda())
    assert_north_star(out, exp_b.cuda(), what="O")
    assert_lse(lse, exp_lse_b)
    assert_close(out, exp_o)  # against the fp32 original too, at the reference's tolerance
    assert_lse(lse, exp_lse, tol=2e-2)


def _varlen_check(w, backward):
    inp = make_inputs(w, device="cuda", with_grad_out=backward)
    q, k, v = (inp[n].requires_grad_(backward) for n in ("q", "k", "v"))
    cu, mx = inp["cu_seqlens"], inp["max_seqlen"]
    out, lse = flash_attn_varlen_func(q, k, v, cu, cu, mx, mx, causal=True, return_softmax_lse=True)
    grads = torch.autograd.grad(out, (q, k, v), inp["dout"]) if backward else None
    qf, kf, vf = (x.detach().float().requires_grad_(backward) for x in (q, k, v))
    exp, exp_lse = reference_varlen(qf, kf, vf, cu.cpu(), True, (-1, -1), with_lse=True)
    _report("O", out, exp)
    assert_north_star(out, exp, what="O")
    assert_lse(lse, exp_lse)
    if backward:
        eg = torch.autograd.grad(exp, (qf, kf, vf), inp["dout"].float())
        for name, g, e in zip(("dQ", "dK", "dV"), grads, eg):
            _report(name, g, e)
        for name, g, e in zip(("dQ", "dK", "dV"), grads, eg):
            assert_north_star(g, e, what=name)


def test_cfg2_varlen_gqa_forward():
    """Config 2: 8 docs, 8248 tokens, Hq=16, Hkv=4, D=64 (forward, and backward for the
    north-star fwd+bwd target on this shape)."""
    _say("cfg2")
    _varlen_check(workloads()["cfg2"], backward=True)


def test_cfg3_varlen_gqa_fwd_bwd():
    """Config 3: 17 log-uniform docs, 16384 tokens, Hq=16, Hkv=4, D=128, fwd+bwd."""
    _say("cfg3")
    _varlen_check(workloads()["cfg3"], backward=True)


def test_cfg4_sliding_window_fwd_bwd():
    """Config 4: B=4, T=8192, window (1023, 0), Hq=16, Hkv=4, D=128, fwd+bwd; the oracle runs
    per batch element."""
    _say("cfg4")
    w = workloads()["cfg4"]
    inp = make_inputs(w, device="cuda")
    q, k, v = (inp[n].requires_grad_() for n in ("q", "k", "v"))
    out, lse = flash_attn_func(q, k, v, causal=True, window_size=w.window_size, return_softmax_lse=True)
    grads = torch.autograd.grad(out, (q, k, v), inp["dout"])
    errs = {n: [] for n in ("O", "dQ", "dK", "dV")}
    for b in range(w.batch):
        qf, kf, vf = (x[b:b + 1].detach().float().requires_grad_() for x in (q, k, v))
        exp, exp_lse = reference_with_lse(qf, kf, vf, True, w.window_size)
        eg = torch.autograd.grad(exp, (qf, kf, vf), inp["dout"][b:b + 1].float())
        assert_lse(lse[:, b * w.seqlen:(b + 1) * w.seqlen], exp_lse)
        for n, got, e in zip(("O", "dQ", "dK", "dV"), (out, *grads), (exp, *eg)):
            errs[n].append(north_star_errors(got[b:b + 1], e))
            assert_north_star(got[b:b + 1], e, what=f"{n}[b={b}]")
        del exp, eg, qf, kf, vf
    for n, e in errs.items():
        _say(f"  {n}: max-abs {max(x[0] for x in e):.3e} mean-abs {max(x[1] for x in e):.3e}")


@pytest.mark.parametrize("name", ["cfg5", "cfg5_mtp"])
def test_cfg5_decode(name):
    """Config 5: B=64, caches up to 16384 (+ nq appended), Hq=16, Hkv=4, D=64, nq = 1 / 4."""
    _say(name)
    w = workloads()[name]
    inp = make_inputs(w, device="cuda")
    kc, vc = inp["k"].clone(), inp["v"].clone()
    out, lse = flash_attn_with_kvcache(inp["q"], kc, vc, inp["k_new"], inp["v_new"],
                                       cache_seqlens=inp["cache_seqlens"], causal=True, return_softmax_lse=True)
    exp, exp_lse, ekc, evc = kvcache_reference(inp["q"].float(), inp["k"].float(), inp["v"].float(),
                                               inp["k_new"].float(), inp["v_new"].float(), inp["cache_seqlens"],
                                               True, (-1, -1))
    assert torch.equal(kc.float(), ekc) and torch.equal(vc.float(), evc)
    _report("O", out, exp)
    assert_north_star(out, exp, what="O")
    assert_lse(lse, exp_lse)

"""Parity at BASELINE.json's full sizes: the kernels against the fp32 oracle on identical
seeded inputs (myk_llm_amd.bench_configs recipes), with the north-star bounds:
O, dQ, dK, dV within max-abs 2e-2 / mean-abs 2e-3 of the fp32 reference and LSE within
1e-3. For the large configs the oracle's fp32 torch math runs on the GPU (per document /
per batch element); for config 1 it runs on the CPU."""

import sys

import pytest
import torch

from _util import assert_close, assert_lse, assert_north_star, north_star_errors, record_parity
from myk_llm_amd import flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache
from myk_llm_amd.bench_configs import make_inputs, workloads
from oracle.attention import kvcache_reference, reference, reference_varlen, reference_with_lse

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _report(config, name, got, exp):
    """Checks the north-star bounds and records the raw errors beside the storage floor (the
    fp32 reference rounded to the output type, measured against itself)."""
    mx, mn, excess = assert_north_star(got, exp, what=f"{config} {name}")
    floor_mx, floor_mn = north_star_errors(exp.to(got.device).to(got.dtype).float(), exp)
    _say(f"  {name}: max-abs {mx:.3e} mean-abs {mn:.3e} beyond-half-ulp {excess:.3e} "
         f"(storage floor: {floor_mx:.3e} / {floor_mn:.3e})")
    record_parity(config, name, max_abs=mx, mean_abs=mn, max_abs_beyond_half_ulp=excess,
                  floor_max_abs=floor_mx, floor_mean_abs=floor_mn)


def _report_lse(config, got, exp, what="LSE"):
    assert_lse(got, exp, what=f"{config} {what}")
    a, e = got.float().cpu(), exp.float().cpu()
    fin = ~torch.isinf(e)
    mx = (a[fin] - e[fin]).abs().max().item() if fin.any() else 0.0
    _say(f"  {what}: max-abs {mx:.3e}")
    record_parity(config, what, max_abs=mx)


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
    _report("cfg1", "O", out, exp_b.cuda())
    _report_lse("cfg1", lse, exp_lse_b)
    # Against the fp32 original (before the bf16 cast of the inputs), at the reference's own
    # tolerance (tests/test_flash_attn.py:37-40).
    mx, mn = north_star_errors(out, exp_o.cuda())
    _say(f"  O vs oracle on the fp32 inputs: max-abs {mx:.3e} mean-abs {mn:.3e}")
    record_parity("cfg1", "O vs fp32 inputs", max_abs=mx, mean_abs=mn)
    assert_close(out, exp_o)
    assert_lse(lse, exp_lse, tol=2e-2)


def _varlen_check(config, w, backward):
    inp = make_inputs(w, device="cuda", with_grad_out=backward)
    q, k, v = (inp[n].requires_grad_(backward) for n in ("q", "k", "v"))
    cu, mx = inp["cu_seqlens"], inp["max_seqlen"]
    out, lse = flash_attn_varlen_func(q, k, v, cu, cu, mx, mx, causal=True, return_softmax_lse=True)
    grads = torch.autograd.grad(out, (q, k, v), inp["dout"]) if backward else None
    qf, kf, vf = (x.detach().float().requires_grad_(backward) for x in (q, k, v))
    exp, exp_lse = reference_varlen(qf, kf, vf, cu.cpu(), True, (-1, -1), with_lse=True)
    _report(config, "O", out, exp)
    _report_lse(config, lse, exp_lse)
    if backward:
        eg = torch.autograd.grad(exp, (qf, kf, vf), inp["dout"].float())
        for name, g, e in zip(("dQ", "dK", "dV"), grads, eg):
            _report(config, name, g, e)


def test_cfg2_varlen_gqa_forward():
    """Config 2: 8 docs, 8248 tokens, Hq=16, Hkv=4, D=64 (forward, and backward for the
    north-star fwd+bwd target on this shape)."""
    _say("cfg2")
    _varlen_check("cfg2", workloads()["cfg2"], backward=True)


def test_cfg3_varlen_gqa_fwd_bwd():
    """Config 3: 17 log-uniform docs, 16384 tokens, Hq=16, Hkv=4, D=128, fwd+bwd."""
    _say("cfg3")
    _varlen_check("cfg3", workloads()["cfg3"], backward=True)


def test_cfg4_sliding_window_fwd_bwd():
    """Config 4: B=4, T=8192, window (1023, 0), Hq=16, Hkv=4, D=128, fwd+bwd; the oracle runs
    per batch element, and each tensor's errors are gathered over the four elements."""
    _say("cfg4")
    w = workloads()["cfg4"]
    inp = make_inputs(w, device="cuda")
    q, k, v = (inp[n].requires_grad_() for n in ("q", "k", "v"))
    out, lse = flash_attn_func(q, k, v, causal=True, window_size=w.window_size, return_softmax_lse=True)
    grads = torch.autograd.grad(out, (q, k, v), inp["dout"])
    names = ("O", "dQ", "dK", "dV")
    stats = {n: [] for n in (*names, "LSE")}
    for b in range(w.batch):
        qf, kf, vf = (x[b:b + 1].detach().float().requires_grad_() for x in (q, k, v))
        exp, exp_lse = reference_with_lse(qf, kf, vf, True, w.window_size)
        eg = torch.autograd.grad(exp, (qf, kf, vf), inp["dout"][b:b + 1].float())
        got_lse = lse[:, b * w.seqlen:(b + 1) * w.seqlen]
        assert_lse(got_lse, exp_lse, what=f"cfg4 LSE[b={b}]")
        stats["LSE"].append(((got_lse.float().cpu() - exp_lse.float().cpu()).abs().max().item(),))
        for n, got, e in zip(names, (out, *grads), (exp, *eg)):
            mx, mn, excess = assert_north_star(got[b:b + 1], e, what=f"cfg4 {n}[b={b}]")
            floor_mx, floor_mn = north_star_errors(e.to(got.dtype).float(), e)
            stats[n].append((mx, mn, excess, floor_mx, floor_mn))
        del exp, eg, qf, kf, vf
    for n in names:
        rows = stats[n]
        mx, excess, floor_mx = (max(r[i] for r in rows) for i in (0, 2, 3))
        mn, floor_mn = (sum(r[i] for r in rows) / len(rows) for i in (1, 4))
        _say(f"  {n}: max-abs {mx:.3e} mean-abs {mn:.3e} beyond-half-ulp {excess:.3e} "
             f"(storage floor: {floor_mx:.3e} / {floor_mn:.3e})")
        record_parity("cfg4", n, max_abs=mx, mean_abs=mn, max_abs_beyond_half_ulp=excess,
                      floor_max_abs=floor_mx, floor_mean_abs=floor_mn)
    lse_mx = max(r[0] for r in stats["LSE"])
    _say(f"  LSE: max-abs {lse_mx:.3e}")
    record_parity("cfg4", "LSE", max_abs=lse_mx)


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
    _report(name, "O", out, exp)
    _report_lse(name, lse, exp_lse)

"""Benchmark of the MI355X FlashAttention path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload cfg2] [--quick]

One "step" is one pass of the hot path over one batch of synthetic input. The headline
workload is BASELINE config 2 (GQA varlen causal, 8 packed documents, 8248 tokens, Hq=16,
Hkv=4, D=64, bf16), run as forward + backward through the public API (the north-star
target is fwd+bwd on this 8K-token GQA varlen shape). Prefill steps are timed as the
reference times them (scripts/benchmark_attention.py:31-40): eager public-API calls back to
back with HIP events around them, here split into 5 consecutive blocks and reported as the
median block's time per step; the host enqueues a step (~160 us) faster than the GPU runs it,
so the GPU never waits. --graph replays a captured HIP graph instead (ROCm 7 adds ~7 us
between graph kernel nodes, which back-to-back eager launches do not). Decode steps are
graph replays, as in the reference's scripts/benchmark_decode.py:122-157, which captures a
whole model decode step (every layer's attention and the rest) in one graph: here one graph
holds the attention decode of DECODE_LAYERS layers, each with its own caches, and a layer's
time is the replay time over DECODE_LAYERS. A graph of a single call is timed as well
("ms_single_call_graph"): each replay carries ~5 us of fixed cost that a model step pays
once, not once per layer. Every timed region
follows the W warmup steps and a further ~0.3 s of untimed steps (settle()), so that the
GPU's clocks have ramped up: the first ~0.2 s of load runs up to 15% slower.
FLOPs follow the reference's convention (scripts/benchmark_attention.py:49-50, 86):
F_fwd = 4 * visible pairs * Hq * D, F_fwd+bwd = 3.5 * F_fwd.

Printed: ONE JSON line with the headline value, a "roofline" object for the step's
dominant kernel (its algorithmic FLOPs / its average duration measured with HIP events on
its launch stream), a "cpu_baseline" object (the oracle's fp32 CPU attention on a bounded
sample, timed on this host's cores), and a "configs" object with every other BASELINE
config (fwd / fwd+bwd TFLOP/s with a roofline object per fwd+bwd config, decode GB/s,
fractions of peak) and the reference benchmark's six shapes beside its published times.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from myk_llm_amd import _lib, flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache  # noqa: E402
from myk_llm_amd import flash_attn as fa  # noqa: E402
from myk_llm_amd.bench_configs import BF16_PEAK_TFLOPS, HBM_PEAK_GBS, make_inputs, workloads  # noqa: E402


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# --- timing helpers -------------------------------------------------------------------------


def settle(fn, seconds: float = 0.3) -> None:
    """Run fn untimed for about `seconds` of wall time. The GPU's clocks ramp up over the first
    ~0.1-0.2 s of sustained load: measured on the box, the cfg2 step takes 195 us in its first
    50 repeats and 170 us afterwards. Steady-state throughput is what a training run sees."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


def time_events(fn, reps: int, warmup: int = 2, blocks: int = 5) -> float:
    """ms per call of fn (launches on torch's current stream): after `warmup` untimed calls and
    a settle() of the clocks, exactly `reps` calls back to back, split into `blocks`
    consecutive blocks with a HIP event between blocks (no synchronization inside the timed
    region); the median over the blocks of each block's time per call."""
    for _ in range(warmup):
        fn()
    settle(fn)
    nb = max(1, min(blocks, reps))
    sizes = [reps // nb + (1 if i < reps % nb else 0) for i in range(nb)]
    events = [torch.cuda.Event(enable_timing=True) for _ in range(nb + 1)]
    torch.cuda.synchronize()
    events[0].record()
    for i, n in enumerate(sizes):
        for _ in range(n):
            fn()
        events[i + 1].record()
    torch.cuda.synchronize()
    return statistics.median(events[i].elapsed_time(events[i + 1]) / sizes[i] for i in range(nb))


def capture(fn, warmup: int = 3):
    """Capture fn into a HIP graph (warm-up on a side stream first, as torch requires)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warmup):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


# --- direct C-ABI launches of single kernels (for per-kernel durations) -------------------------


class KernelCalls:
    """Prepared C-ABI calls of each kernel of the attention step on fixed buffers."""

    def __init__(self, q, k, v, cu, max_q, max_k, scale, wl, wr, dout=None):
        self.L = _lib.lib()
        q, k, v = fa._kernel_ready(q), fa._kernel_ready(k), fa._kernel_ready(v)
        varlen = cu is not None
        rows = q.shape[0] if varlen else q.shape[0] * q.shape[1]
        self.out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        self.lse = torch.empty((q.shape[-2], rows), dtype=torch.float32, device=q.device)
        self.fp = fa._fwd_params(q, k, v, self.out, self.lse, cu, cu, None, max_q, max_k, scale, wl, wr)
        self.keep = [q, k, v, cu]
        self.stream = torch.cuda.current_stream().cuda_stream
        _lib.check(self.L.mykfa_fwd(ctypes.byref(self.fp), self.stream))
        if dout is not None:
            dout = fa._kernel_ready(dout)
            self.dq, self.dk, self.dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
            self.delta = torch.empty_like(self.lse)
            p = _lib.BwdParams()
            p.fwd = self.fp
            p.dout, p.dq, p.dk, p.dv = dout.data_ptr(), self.dq.data_ptr(), self.dk.data_ptr(), self.dv.data_ptr()
            p.delta = self.delta.data_ptr()
            p.do_batch_stride, p.do_token_stride, p.do_head_stride = fa._strides(dout)
            p.dq_batch_stride, p.dq_token_stride, p.dq_head_stride = fa._strides(self.dq)
            p.dk_batch_stride, p.dk_token_stride, p.dk_head_stride = fa._strides(self.dk)
            p.dv_batch_stride, p.dv_token_stride, p.dv_head_stride = fa._strides(self.dv)
            self.bp = p
            self.keep.append(dout)
            # The schedule that the autograd backward takes for this shape, by the same rule
            # (fa._plan_ds_workspace): stored dS (delta, dK/dV storing dS, dQ from dS) when at
            # least one KV head's workspace fits, else the recomputing dQ and dK/dV;
            # `ds_passes` = the passes of KV heads the stored-dS backward takes (0: recomputing).
            per = self.L.mykfa_bwd_workspace_per_kv_head(ctypes.byref(p))
            heads, ws = fa._plan_ds_workspace(per, k.shape[-2], fa._ds_budget_bytes(),
                                              lambda n: torch.empty(n, dtype=torch.uint8, device=q.device),
                                              lambda: fa._available_bytes(q.device))
            self.ws = ws
            self.ds_passes = (k.shape[-2] + heads - 1) // heads if heads > 0 else 0

    def fwd(self):
        _lib.check(self.L.mykfa_fwd(ctypes.byref(self.fp), self.stream))

    def dkdv(self):
        _lib.check(self.L.mykfa_bwd_dkdv(ctypes.byref(self.bp), self.stream))

    def dq_(self):
        _lib.check(self.L.mykfa_bwd_dq(ctypes.byref(self.bp), self.stream))

    def delta_(self):
        _lib.check(self.L.mykfa_bwd_preprocess(ctypes.byref(self.bp), self.stream))

    def dkdv_ds(self):
        _lib.check(self.L.mykfa_bwd_dkdv_ws(ctypes.byref(self.bp), self.ws.data_ptr(), self.ws.numel(), self.stream))

    def dq_ds(self):
        _lib.check(self.L.mykfa_bwd_dq_ws(ctypes.byref(self.bp), self.ws.data_ptr(), self.ws.numel(), self.stream))

    def bwd_ws(self):
        _lib.check(self.L.mykfa_bwd_ws(ctypes.byref(self.bp), self.ws.data_ptr(), self.ws.numel(), self.stream))


class DecodeCalls:
    """Prepared C-ABI calls of the split-K decode and its merge on one cache set."""

    def __init__(self, q, kc, vc, lens, scale):
        self.L = _lib.lib()
        b, nq, h, d = q.shape
        self.out = torch.empty_like(q)
        self.lse = torch.empty((h, b * nq), dtype=torch.float32, device=q.device)
        wl, wr = fa._window(True, (-1, -1))
        fp = fa._fwd_params(q, kc, vc, self.out, self.lse, None, None, lens, nq, kc.shape[1], scale, wl, wr)
        self.dp = _lib.DecodeParams()
        self.dp.fwd = fp
        self.dp.num_splits = self.L.mykfa_decode_num_splits(b, h, kc.shape[2], nq, kc.shape[1])
        n = self.L.mykfa_decode_workspace_size(b, h, nq, d, self.dp.num_splits)
        self.ws = torch.empty(max(n, 16), dtype=torch.uint8, device=q.device)
        self.keep = [q, kc, vc, lens]
        self.stream = torch.cuda.current_stream().cuda_stream

    def splitk(self):
        _lib.check(self.L.mykfa_decode_splitk(ctypes.byref(self.dp), self.ws.data_ptr(), self.ws.numel(), self.stream))

    def merge(self):
        _lib.check(self.L.mykfa_decode_merge(ctypes.byref(self.dp), self.ws.data_ptr(), self.ws.numel(), self.stream))


# --- workloads ----------------------------------------------------------------------------------


def attention_step(w, inp, backward: bool):
    """The public-API call of workload w (+ autograd backward)."""
    if w.kind == "varlen":
        q, k, v = (inp[n].requires_grad_(backward) for n in ("q", "k", "v"))
        cu, mx = inp["cu_seqlens"], inp["max_seqlen"]

        def fwd():
            return flash_attn_varlen_func(q, k, v, cu, cu, mx, mx, causal=True, window_size=w.window_size)
    else:
        q, k, v = (inp[n].requires_grad_(backward) for n in ("q", "k", "v"))

        def fwd():
            return flash_attn_func(q, k, v, causal=True, window_size=w.window_size)

    if not backward:
        return fwd
    dout = inp["dout"]

    def step():
        out = fwd()
        return torch.autograd.grad(out, (q, k, v), dout)

    return step


def measure_prefill(w, steps: int, warmup: int, backward: bool, use_graph: bool = False):
    inp = make_inputs(w, device="cuda", with_grad_out=backward)
    step = attention_step(w, inp, backward)
    if use_graph:
        g = capture(step, warmup)
        ms = time_events(g.replay, steps, warmup=1)
    else:
        ms = time_events(step, steps, warmup)
    flops = w.fwd_flops * (3.5 if backward else 1.0)
    # Per-kernel durations on the same inputs, through the C ABI on torch's current stream.
    scale = 1.0 / (w.head_dim ** 0.5)
    wl, wr = fa._window(True, w.window_size)
    cu = inp.get("cu_seqlens")
    mq = inp["max_seqlen"] if cu is not None else w.seqlen
    kc = KernelCalls(inp["q"].detach(), inp["k"].detach(), inp["v"].detach(), cu, mq, mq, scale, wl, wr,
                     inp["dout"] if backward else None)
    reps = max(steps, 10)
    kern = {"fwd": time_events(kc.fwd, reps)}
    if backward and kc.ws is not None and kc.ds_passes == 1:
        # Stored-dS backward: delta, dK/dV (also storing dS), dQ from dS.
        kern["bwd_delta"] = time_events(kc.delta_, reps)
        kern["bwd_dkdv"] = time_events(kc.dkdv_ds, reps)
        kern["bwd_dq"] = time_events(kc.dq_ds, reps)
    elif backward and kc.ws is not None:
        # Stored dS over several passes of KV heads (the half entry points need every head's
        # workspace at once): the whole backward as one entry.
        kern["bwd_ws_passes"] = time_events(kc.bwd_ws, reps)
    elif backward:
        # Recomputing backward: dQ (which also computes delta = rowsum(dO * O)) then dK/dV.
        kern["bwd_dq"] = time_events(kc.dq_, reps)
        kern["bwd_dkdv"] = time_events(kc.dkdv, reps)
    # Algorithmic FLOPs per launch (convention split: fwd = 2 products; of the 5 backward
    # products, dK/dV's kernel owns S, dP, dV, dK = 2.0 F_fwd and dQ's owns dQ = 0.5 F_fwd;
    # delta is HBM-bound streaming, no credited FLOPs).
    algo = {"fwd": w.fwd_flops, "bwd_dkdv": 2.0 * w.fwd_flops, "bwd_dq": 0.5 * w.fwd_flops,
            "bwd_ws_passes": 2.5 * w.fwd_flops}
    del inp, step, kc
    return ms, flops, kern, algo


def roofline_of(kern, algo, profile=None):
    """The roofline object of the dominant kernel among those with credited FLOPs: its
    algorithmic FLOPs / its duration, against the bf16 dense peak; traffic from the committed
    copy-calibrated counter summary of `profile`, when there is one."""
    dom = max((k for k in kern if algo.get(k, 0) > 0), key=lambda k: kern[k])
    achieved = algo[dom] / (kern[dom] * 1e-3) / 1e12
    return {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 2), "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
            "traffic": profiled_traffic(dom, profile) if profile else None, "kernel_ms": round(kern[dom], 5)}


# The reference's own benchmark shapes (scripts/benchmark_attention.py:21-29) and its published
# times, fwd / fwd+bwd in ms, of its Triton kernels on its development GPU (an sm_120 part;
# notes/flash-attn.md:62-67): context for the MI355X numbers, not a target.
REFERENCE_SHAPES = [
    # (batch, seq_len, heads, kv_heads, head_dim, window or None, documents or None, published)
    (8, 2048, 8, 2, 128, None, None, (0.385, 1.706)),
    (8, 2048, 8, 2, 128, 512, None, (0.198, 0.783)),
    (8, 2048, 8, 2, 128, None, [300, 700, 48, 1000], (0.199, 0.804)),
    (2, 8192, 8, 2, 128, None, None, (1.387, 6.035)),
    (16, 1024, 4, 4, 64, None, None, (0.058, 0.236)),
    (16, 1024, 4, 4, 64, 256, None, (0.029, 0.113)),
]


def measure_reference_shapes(reps: int = 30):
    """Forward and forward + backward at the reference benchmark's shapes, set up as it sets
    them up (scripts/benchmark_attention.py:44-62: N(0,1) bf16 inputs, windows as
    (window - 1, 0), documents packed with cu_seqlens, the backward as autograd.grad of the
    forward), timed by time_events. FLOPs: 4 * visible pairs * heads * head_dim, x 3.5 for
    forward + backward (:49-50, :86)."""
    out = []
    g = torch.Generator(device="cuda").manual_seed(0)
    for batch, seq, h, hk, d, window, docs, published in REFERENCE_SHAPES:
        make = lambda n: torch.randn(batch, seq, n, d, device="cuda", generator=g).to(torch.bfloat16)
        q, k, v, do = make(h), make(hk), make(hk), make(h)
        lengths = docs or [seq]
        pairs = batch * sum(min(i + 1, window or seq) for n in lengths for i in range(n))
        flops = 4.0 * pairs * h * d
        ws = (window - 1, 0) if window else (-1, -1)
        if docs is None:
            inputs = tuple(x.requires_grad_() for x in (q, k, v))
            grad = do
            fwd = lambda: flash_attn_func(*inputs, causal=True, window_size=ws)
        else:
            cu = torch.tensor([0] + list(torch.tensor(docs * batch).cumsum(0)), dtype=torch.int32, device="cuda")
            inputs = tuple(x.flatten(0, 1).requires_grad_() for x in (q, k, v))
            grad = do.flatten(0, 1)
            fwd = lambda: flash_attn_varlen_func(*inputs, cu, cu, seq, seq, causal=True, window_size=ws)
        ms_f = time_events(fwd, reps, warmup=3)
        ms_b = time_events(lambda: torch.autograd.grad(fwd(), inputs, grad), reps, warmup=3)
        out.append({"shape": {"batch": batch, "seq_len": seq, "heads": h, "kv_heads": hk, "head_dim": d,
                              "window": window, "documents": docs},
                    "fwd_ms": round(ms_f, 4), "fwd_TFLOP/s": round(flops / (ms_f * 1e-3) / 1e12, 1),
                    "fwdbwd_ms": round(ms_b, 4), "fwdbwd_TFLOP/s": round(3.5 * flops / (ms_b * 1e-3) / 1e12, 1),
                    "reference_published_ms": {"fwd": published[0], "fwdbwd": published[1]}})
        del q, k, v, do, inputs, grad
    return out


DECODE_LAYERS = 4


def measure_decode(w, steps: int, warmup: int):
    """flash_attn_with_kvcache (append + split-K decode + merge) for DECODE_LAYERS layers, each
    with its own caches (> 4 GB in all, so the 256 MB Infinity Cache cannot hold them),
    captured in one graph as a model's decode step is; returns the time per layer, the time of
    a one-call graph (alternating two layers' caches), per-kernel times and the split count."""
    g0 = torch.Generator(device="cuda").manual_seed(0)
    b = len(w.cache_seqlens)
    layers = []
    for _ in range(DECODE_LAYERS):
        kc = torch.randn(b, w.capacity, w.kv_heads, w.head_dim, device="cuda", generator=g0).to(torch.bfloat16)
        vc = torch.randn(b, w.capacity, w.kv_heads, w.head_dim, device="cuda", generator=g0).to(torch.bfloat16)
        q = torch.randn(b, w.nq, w.heads, w.head_dim, device="cuda", generator=g0).to(torch.bfloat16)
        kn = torch.randn(b, w.nq, w.kv_heads, w.head_dim, device="cuda", generator=g0).to(torch.bfloat16)
        vn = torch.randn(b, w.nq, w.kv_heads, w.head_dim, device="cuda", generator=g0).to(torch.bfloat16)
        layers.append((q, kc, vc, kn, vn))
    lens = torch.tensor(w.cache_seqlens, dtype=torch.int32, device="cuda")

    def call(layer):
        q, kc, vc, kn, vn = layer
        return flash_attn_with_kvcache(q, kc, vc, kn, vn, cache_seqlens=lens, causal=True)

    def model_step():
        return [call(layer) for layer in layers]

    g_step = capture(model_step, warmup)
    ms = time_events(g_step.replay, steps, warmup=1) / DECODE_LAYERS
    singles = [capture(lambda layer=layer: call(layer), warmup) for layer in layers[:2]]
    it = [0]

    def replay():
        singles[it[0] % 2].replay()
        it[0] += 1

    ms_single = time_events(replay, steps * 2, warmup=2)
    sets = [(kc, vc) for _, kc, vc, _, _ in layers[:2]]
    q = layers[0][0]
    nsets = 2
    # Per-kernel durations through the C ABI, alternating the cache sets as above (the lengths
    # already include the appended tokens).
    scale = 1.0 / (w.head_dim ** 0.5)
    calls = [DecodeCalls(q, kc, vc, lens, scale) for kc, vc in sets]
    it2 = [0]

    def one(name):
        def f():
            getattr(calls[it2[0] % nsets], name)()
            it2[0] += 1
        return f

    kern = {"decode_splitk": time_events(one("splitk"), steps * nsets, warmup=nsets),
            "decode_merge": time_events(one("merge"), steps * nsets, warmup=nsets)}
    splits = calls[0].dp.num_splits
    del sets, g_step, singles, calls, layers
    return ms, ms_single, kern, splits


def measure_block_io(w, steps: int):
    """The attention block's prologue (q/k RMSNorm + RoPE on the fused projection, forward and
    backward with the value-gradient copy) and epilogue (output gate, forward and backward) at
    workload w's shape (positions restart at every document), as direct C-ABI launches on
    prepared buffers (two sets, alternated). Algorithmic bytes: every tensor element read or written once, plus each
    distinct cos/sin table row once. Beside them, the reference's composed PyTorch chain
    (mixers.py:85-89, :116-117 under autocast: separate elementwise kernels) on the same GPU."""
    from myk_llm_amd import block_io as bio

    t, hq, hkv, d = sum(w.lengths), w.heads, w.kv_heads, w.head_dim
    pos = torch.cat([torch.arange(n, device="cuda") for n in w.lengths])
    table_rows = max(w.lengths)
    cos, sin = bio.rope_tables(d, table_rows, 500000.0, device="cuda")
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    pos2 = pos.unsqueeze(0)
    width = hq * d

    def make_set(seed):
        """Every buffer of the four kernels, and their parameter blocks."""
        g = torch.Generator(device="cuda").manual_seed(seed)
        bs = {}
        qkv = torch.randn(t, (hq + 2 * hkv) * d, device="cuda", generator=g).to(torch.bfloat16)
        bs["qw"] = 1 + 0.1 * torch.randn(d, device="cuda", generator=g)
        bs["kw"] = 1 + 0.1 * torch.randn(d, device="cuda", generator=g)
        dq = torch.randn(t, hq, d, device="cuda", generator=g).to(torch.bfloat16)
        dk = torch.randn(t, hkv, d, device="cuda", generator=g).to(torch.bfloat16)
        dv = torch.randn(t, hkv, d, device="cuda", generator=g).to(torch.bfloat16)
        x = qkv.unsqueeze(0)
        q_in = x[..., :hq * d].view(1, t, hq, d)
        k_in = x[..., hq * d:(hq + hkv) * d].view(1, t, hkv, d)
        q_out = torch.empty_like(q_in, memory_format=torch.contiguous_format)
        k_out = torch.empty(1, t, hkv, d, dtype=qkv.dtype, device="cuda")
        fp = bio._prologue_params(q_in, k_in, q_out, k_out, pos2, cos, sin, bs["qw"], bs["kw"], 1e-6)
        dqkv = torch.empty_like(x)
        bp = _lib.QkPrologueBwdParams()
        bp.fwd = fp
        dq4, dk4, dv4 = dq.unsqueeze(0), dk.unsqueeze(0), dv.unsqueeze(0)
        dq_in = dqkv[..., :hq * d].view(1, t, hq, d)
        dk_in = dqkv[..., hq * d:(hq + hkv) * d].view(1, t, hkv, d)
        dv_dst = dqkv[..., (hq + hkv) * d:].view(1, t, hkv, d)
        bp.dq_out, bp.dk_out, bp.dq_in, bp.dk_in = dq4.data_ptr(), dk4.data_ptr(), dq_in.data_ptr(), dk_in.data_ptr()
        bp.dqo_batch_stride, bp.dqo_token_stride, bp.dqo_head_stride = bio._strides3(dq4)
        bp.dko_batch_stride, bp.dko_token_stride, bp.dko_head_stride = bio._strides3(dk4)
        bp.dqi_batch_stride, bp.dqi_token_stride, bp.dqi_head_stride = bio._strides3(dq_in)
        bp.dki_batch_stride, bp.dki_token_stride, bp.dki_head_stride = bio._strides3(dk_in)
        bp.dv_src, bp.dv_dst = dv4.data_ptr(), dv_dst.data_ptr()
        bp.dvs_batch_stride, bp.dvs_token_stride, bp.dvs_head_stride = bio._strides3(dv4)
        bp.dvd_batch_stride, bp.dvd_token_stride, bp.dvd_head_stride = bio._strides3(dv_dst)
        dqw, dkw = torch.empty(d, device="cuda"), torch.empty(d, device="cuda")
        bp.dq_weight, bp.dk_weight = dqw.data_ptr(), dkw.data_ptr()
        nws = L.mykfa_qk_prologue_bwd_workspace_size(1, t, hq, hkv, d)
        ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
        og = torch.randn(t, width, device="cuda", generator=g).to(torch.bfloat16)
        gg = torch.randn(t, width, device="cuda", generator=g).to(torch.bfloat16)
        dy = torch.randn(t, width, device="cuda", generator=g).to(torch.bfloat16)
        y, dx, dg = torch.empty_like(og), torch.empty_like(og), torch.empty_like(og)
        gp = bio._gate_params(og, gg, y, dy, dx, dg)
        bs.update(x=x, q_out=q_out, k_out=k_out, dqkv=dqkv, dq4=dq4, dk4=dk4, dv4=dv4, dqw=dqw, dkw=dkw,
                  ws=ws, og=og, gg=gg, dy=dy, y=y, dx=dx, dg=dg, fp=fp, bp=bp, gp=gp, nws=nws)
        return bs

    # Two sets of buffers, alternated call by call: a call touches 168 MB (prologue forward),
    # 285 MB (its backward), 201 MB (gate forward) or 335 MB (gate backward) of one set, so the
    # two sets together exceed the 256 MB Infinity Cache and every call reads its inputs from
    # HBM, as the decode timing does.
    sets = [make_set(1), make_set(11)]
    turn = [0]

    def alternating(launch):
        def f():
            launch(sets[turn[0] % 2])
            turn[0] += 1
        return f

    calls = {
        "prologue_fwd": alternating(lambda b: _lib.check(L.mykfa_qk_prologue_fwd(ctypes.byref(b["fp"]), stream))),
        "prologue_bwd": alternating(lambda b: _lib.check(
            L.mykfa_qk_prologue_bwd(ctypes.byref(b["bp"]), b["ws"].data_ptr(), b["nws"], stream))),
        "gate_fwd": alternating(lambda b: _lib.check(L.mykfa_gate_fwd(ctypes.byref(b["gp"]), stream))),
        "gate_bwd": alternating(lambda b: _lib.check(L.mykfa_gate_bwd(ctypes.byref(b["gp"]), stream))),
    }
    s0 = sets[0]
    x, qw, kw, dq4, dk4, dv4 = s0["x"], s0["qw"], s0["kw"], s0["dq4"], s0["dk4"], s0["dv4"]
    og, gg, dy = s0["og"], s0["gg"], s0["dy"]
    e = 2  # bytes per element
    qk = t * (hq + hkv) * d * e
    tables = 2 * table_rows * d * 4
    algo = {
        "prologue_fwd": 2 * qk + t * 8 + tables + 2 * d * 4,
        "prologue_bwd": 3 * qk + 2 * t * hkv * d * e + t * 8 + tables + 4 * d * 4,
        "gate_fwd": 3 * t * width * e,
        "gate_bwd": 5 * t * width * e,
    }
    out = {}
    reps = max(steps, 20)
    for name, fn in calls.items():
        ms = time_events(fn, reps)
        gbs = algo[name] / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 2), "bytes": int(algo[name]), "GB/s": round(gbs, 1),
                     "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}

    # The reference's chain on the same GPU, forward and forward + backward (autocast rounding
    # points written out: fp32 norm, cast, fp32 rotation, cast; bf16 sigmoid, bf16 product).
    cos_t, sin_t = cos, sin

    def rot_half(u):
        return torch.stack((-u[..., 1::2], u[..., ::2]), dim=-1).flatten(start_dim=-2)

    def torch_prologue(xq, xk, wq, wk):
        def norm(u, wt):
            u32 = u.float()
            return (u32 * torch.rsqrt(u32.pow(2).mean(-1, keepdim=True) + 1e-6) * wt).to(u.dtype)

        c, s_ = cos_t[pos2].unsqueeze(2), sin_t[pos2].unsqueeze(2)

        def rope(u):
            u32 = u.float()
            return (u32 * c + rot_half(u32) * s_).to(u.dtype)

        return rope(norm(xq, wq)), rope(norm(xk, wk))

    xr = x.detach().requires_grad_(True)
    wq_r, wk_r = qw.clone().requires_grad_(True), kw.clone().requires_grad_(True)

    def torch_fwd():
        return torch_prologue(xr[..., :hq * d].view(1, t, hq, d), xr[..., hq * d:(hq + hkv) * d].view(1, t, hkv, d),
                              wq_r, wk_r)

    def torch_fwdbwd():
        a, b = torch_fwd()
        return torch.autograd.grad((a, b, xr[..., (hq + hkv) * d:].view(1, t, hkv, d)), (xr, wq_r, wk_r),
                                   (dq4, dk4, dv4))

    ogr, ggr = og.detach().requires_grad_(True), gg.detach().requires_grad_(True)

    def torch_gate_fwdbwd():
        yy = ogr * torch.sigmoid(ggr)
        return torch.autograd.grad(yy, (ogr, ggr), dy)

    out["torch_chain_us"] = {"prologue_fwd": round(time_events(torch_fwd, 20) * 1e3, 1),
                             "prologue_fwd+bwd": round(time_events(torch_fwdbwd, 20) * 1e3, 1),
                             "gate_fwd": round(time_events(lambda: og * torch.sigmoid(gg), 20) * 1e3, 1),
                             "gate_fwd+bwd": round(time_events(torch_gate_fwdbwd, 20) * 1e3, 1)}
    out["shape"] = {"tokens": t, "heads": hq, "kv_heads": hkv, "head_dim": d, "gate_width": width}
    return out


def measure_fused_ce(steps: int, tokens: int = 16384, hidden: int = 1024, vocab: int = 65536, chunk: int = 2048):
    """fused_linear_cross_entropy at the reference model's head (hidden 1024, tied 64K
    vocabulary: configs/model/200m.yaml; 2048-token chunks: train/config.py:79) over 16384
    tokens, bf16 hidden and fp32 weight as under autocast with fp32 master weights. The whole
    op (3 GEMMs per chunk + the CE row kernel; its backward only scales) and the CE row kernel
    alone on one chunk (algorithmic bytes: the logits read once and written once). Beside
    them, the same chunk loop with the CE rows as torch ops (no row kernel)."""
    from myk_llm_amd.fused_ce import _ce_rows, fused_linear_cross_entropy

    g = torch.Generator(device="cuda").manual_seed(2)
    h = torch.randn(tokens, hidden, device="cuda", generator=g).to(torch.bfloat16)
    w = 0.05 * torch.randn(vocab, hidden, device="cuda", generator=g)
    t = torch.randint(0, vocab, (tokens,), device="cuda", generator=g)
    t[::9] = -100
    norm = float((t != -100).sum().item())

    def op():
        loss, _, _ = fused_linear_cross_entropy(h, w, t, norm, 1e-4, chunk_size=chunk)
        return loss

    ms = time_events(op, max(5, steps // 5))
    flops = 6.0 * tokens * hidden * vocab

    logits = (h[:chunk] @ w.to(torch.bfloat16).t()).contiguous()
    work = logits.clone()
    ce, lse = torch.empty(chunk, device="cuda"), torch.empty(chunk, device="cuda")
    tc = t[:chunk]

    def rows():  # rewrites `work` in place each call: same bytes, same work per call
        _ce_rows(work, tc, ce, lse, 1.0 / norm, 1e-4, -100)

    ms_rows = time_events(rows, max(20, steps))
    row_bytes = 2 * chunk * vocab * 2

    wb = w.to(torch.bfloat16)

    def torch_chain():
        gh = torch.empty(tokens, hidden, device="cuda", dtype=torch.bfloat16)
        gw = torch.zeros(vocab, hidden, device="cuda")
        total = torch.zeros((), device="cuda")
        for s0 in range(0, tokens, chunk):
            hc = h[s0:s0 + chunk]
            lg = (hc @ wb.t()).float()
            tt = t[s0:s0 + chunk]
            valid = tt != -100
            ls = torch.logsumexp(lg, -1)
            total += torch.where(valid, ls - lg.gather(1, tt.clamp_min(0)[:, None])[:, 0], 0.0).sum()
            p = torch.softmax(lg, -1) * ((1 + 2e-4 * ls) / norm)[:, None]
            p.scatter_add_(1, tt.clamp_min(0)[:, None], torch.where(valid, -1.0 / norm, 0.0)[:, None])
            p = (p * valid[:, None]).to(torch.bfloat16)
            torch.mm(p, wb, out=gh[s0:s0 + chunk])
            gw.add_(p.t() @ hc)
        return total

    ms_torch = time_events(torch_chain, max(3, steps // 10))
    return {"shape": {"tokens": tokens, "hidden": hidden, "vocab": vocab, "chunk": chunk},
            "ms": round(ms, 4), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1),
            "frac_of_bf16_peak": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "ce_rows_us": round(ms_rows * 1e3, 2), "ce_rows_bytes": row_bytes,
            "ce_rows_GB/s": round(row_bytes / (ms_rows * 1e-3) / 1e9, 1),
            "ce_rows_frac_of_hbm_peak": round(row_bytes / (ms_rows * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "torch_ce_rows_chain_ms": round(ms_torch, 4)}


def measure_syrk(steps: int):
    """Muon's batched SYRK (x x^T over lower-triangular 128 x 128 tiles) and one 5-step
    Newton-Schulz orthogonalization at buckets of the reference model (9 matrices of
    1024 x 4096 and 1024 x 1024; configs/model/200m.yaml), beside torch's full batched product
    (hipBLASLt bmm of x with a contiguous x^T) on the same GPU. TFLOP/s count the products
    the kernel executes (2 M'^2 K per lower tile, M' = 128), the MFMA roofline's work; the
    full-GEMM-equivalent rate (2 M^2 K) is given too."""
    from myk_llm_amd.muon import batched_newton_schulz_orthogonalize, batched_syrk

    out = {}
    for b, m, k in ((9, 1024, 4096), (9, 1024, 1024)):
        g = torch.Generator(device="cuda").manual_seed(3)
        x = (torch.randn(b, m, k, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        gram = torch.empty(b, m, m, device="cuda", dtype=torch.bfloat16)
        ms = time_events(lambda: batched_syrk(x, out=gram), max(20, steps // 4))
        xt = x.transpose(-2, -1).contiguous()
        ms_bmm = time_events(lambda: torch.bmm(x, xt), max(20, steps // 4))
        t = (m + 127) // 128
        executed = 2.0 * b * (t * (t + 1) // 2) * 128 * 128 * k
        full = 2.0 * b * m * m * k
        key = f"b{b}_m{m}_k{k}"
        out[key] = {"us": round(ms * 1e3, 2), "TFLOP/s_executed": round(executed / (ms * 1e-3) / 1e12, 1),
                    "frac_of_bf16_peak": round(executed / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                    "TFLOP/s_full_gemm_equivalent": round(full / (ms * 1e-3) / 1e12, 1),
                    "torch_bmm_full_us": round(ms_bmm * 1e3, 2)}
        if k == 4096:
            mats = (torch.randn(b, m, k, device="cuda", generator=g)).to(torch.bfloat16)
            out[key]["newton_schulz_5_steps_ms"] = round(
                time_events(lambda: batched_newton_schulz_orthogonalize(mats.clone(), 5), 10), 4)
    return out


# --- CPU baseline ---------------------------------------------------------------------------------


def cpu_baseline(w, budget_s: float = 12.0, reps: int = 3):
    """The reference's CPU attention path (fp32 einsum reference(), restated in oracle/) with
    CPU autograd for the backward, looping per document, on this host's cores. The sample is
    the leading documents of the workload, taken in order by a first (warm-up) pass until
    budget_s / (reps + 1) of CPU work has been spent; that sample is then timed `reps` more
    times and the median repetition is reported (1 warm-up + reps repetitions)."""
    from oracle.attention import reference

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    inp = make_inputs(w, device="cpu", with_grad_out=True)
    cu = inp["cu_seqlens"].tolist()

    def run_doc(a, b):
        q, k, v = (inp[n][a:b][None].float().requires_grad_() for n in ("q", "k", "v"))
        do = inp["dout"][a:b][None].float()
        t0 = time.perf_counter()
        out = reference(q, k, v, True, w.window_size)
        torch.autograd.grad(out, (q, k, v), do)
        return time.perf_counter() - t0

    # Warm-up pass: fixes the sample.
    done_pairs, t_warm, docs = 0, 0.0, 0
    for a, b in zip(cu, cu[1:]):
        t_warm += run_doc(a, b)
        done_pairs += (b - a) * (b - a + 1) // 2
        docs += 1
        if t_warm >= budget_s / (reps + 1):
            break
    times = [sum(run_doc(a, b) for a, b in zip(cu[:docs], cu[1:docs + 1])) for _ in range(reps)]
    t_total = statistics.median(times)
    flops = 3.5 * 4.0 * done_pairs * w.heads * w.head_dim
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return {"value": round(flops / t_total / 1e12, 6), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"fwd+bwd fp32 oracle (reference() restated, CPU autograd) over the first {docs} of "
                      f"{len(cu) - 1} {w.name} documents ({done_pairs} visible pairs); 1 warm-up + {reps} "
                      f"repetitions, median {t_total:.3f} s (repetitions {', '.join(f'{t:.3f}' for t in times)} s); "
                      f"{model}",
            "seconds": round(t_total, 3), "repetitions": reps}


# --- HBM traffic from the committed rocprofv3 summary -------------------------------------------------

def profiled_traffic(kernel: str, profile: str = "cfg2_fwdbwd"):
    """HBM bytes per dispatch of `kernel` (a kernels_ms key) as measured by the two
    copy-calibrated rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) summarized in
    profiles/<profile>_hbm_traffic.txt, whose 'traffic_bytes <kernel> <bytes>' lines carry the
    figures; None when the summary is absent."""
    try:
        with open(os.path.join(ROOT, "profiles", f"{profile}_hbm_traffic.txt")) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic_bytes" and parts[1] == kernel:
                    return int(parts[2])
    except OSError:
        pass
    return None


# --- main -------------------------------------------------------------------------------------------


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="cfg2")
    ap.add_argument("--quick", action="store_true", help="headline only: no other configs, no CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-only", action="store_true", help="only the decode configs (for profiling)")
    ap.add_argument("--syrk-only", action="store_true", help="only Muon's batched SYRK (for profiling)")
    ap.add_argument("--fused-ce-only", action="store_true",
                    help="only the fused linear + cross-entropy at the reference model's head (for profiling)")
    ap.add_argument("--block-io-only", action="store_true",
                    help="only the attention-block prologue / epilogue kernels at the cfg3 shape (for profiling)")
    ap.add_argument("--reference-shapes-only", action="store_true",
                    help="only the reference benchmark's six shapes, eager fwd and fwd+bwd (for profiling)")
    ap.add_argument("--graph", action="store_true", help="time prefill steps as HIP graph replays instead of eager calls")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run a plain 256 MiB fp32 copy kernel 3 times (reads and writes 2^28 bytes "
                         "each), the reference dispatch for scaling FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    _lib.lib()
    if args.copy_calibration:
        src = torch.randn(1 << 26, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)  # one elementwise kernel: 256 MiB read, 256 MiB written
        torch.cuda.synchronize()
        del src, dst
    W = workloads()
    if args.decode_only:
        # The decode workloads alone (for profiling their kernels); not the contract line.
        out = {}
        for name in ("cfg5", "cfg5_mtp"):
            wk = W[name]
            m, m1, kk, splits = measure_decode(wk, args.steps, args.warmup)
            out[name] = {"ms": round(m, 5), "GB/s": round(wk.decode_bytes / (m * 1e-3) / 1e9, 1),
                         "ms_single_call_graph": round(m1, 5), "splits": splits,
                         "kernel_ms": {k: round(v, 5) for k, v in kk.items()}}
        print(json.dumps({"decode_only": out}), flush=True)
        return
    if args.syrk_only:
        print(json.dumps({"muon_syrk": measure_syrk(args.steps)}), flush=True)
        return
    if args.fused_ce_only:
        print(json.dumps({"fused_ce_200m_head": measure_fused_ce(args.steps)}), flush=True)
        return
    if args.block_io_only:
        print(json.dumps({"block_io_cfg3": measure_block_io(W["cfg3"], args.steps)}), flush=True)
        return
    if args.reference_shapes_only:
        print(json.dumps({"reference_shapes": measure_reference_shapes(max(10, min(args.steps, 30)))}), flush=True)
        return
    w = W[args.workload]
    log(f"headline {w.name}: fwd+bwd, steps={args.steps} warmup={args.warmup}")
    torch.cuda.synchronize()
    ms, flops, kern, algo = measure_prefill(w, args.steps, args.warmup, backward=True, use_graph=args.graph)
    value = flops / (ms * 1e-3) / 1e12
    roof = roofline_of(kern, algo, f"{args.workload}_fwdbwd")
    log(f"  {ms:.4f} ms/step, {value:.1f} TFLOP/s; kernels (ms): " + ", ".join(f"{k}={v:.4f}" for k, v in kern.items()))
    configs = {}
    if not args.quick:
        for name in ("cfg2", "cfg3", "cfg4"):
            wk = W[name]
            for bwd in ((False, True) if name != "cfg2" else (False,)):
                log(f"config {wk.name} {'fwd+bwd' if bwd else 'fwd'}")
                m, f, kk, algo_k = measure_prefill(wk, max(10, args.steps // 2), 3, backward=bwd, use_graph=args.graph)
                t = f / (m * 1e-3) / 1e12
                key = f"{name}_{'fwdbwd' if bwd else 'fwd'}"
                configs[key] = {
                    "workload": wk.name, "ms": round(m, 5), "TFLOP/s": round(t, 2),
                    "frac_of_bf16_peak": round(t / BF16_PEAK_TFLOPS, 4),
                    "kernel_ms": {k: round(v, 5) for k, v in kk.items()},
                    "roofline": roofline_of(kk, algo_k, key if bwd else None)}
                log(f"  {m:.4f} ms, {t:.1f} TFLOP/s")
        for name in ("cfg5", "cfg5_mtp"):
            wk = W[name]
            log(f"config {wk.name} decode")
            m, m1, kk, splits = measure_decode(wk, max(10, args.steps // 2), 3)
            gbs = wk.decode_bytes / (m * 1e-3) / 1e9
            # Roofline of the split-K kernel: the step's algorithmic bytes (each K/V byte once per
            # GQA group, q, O, LSE) over its own average duration.
            kgbs = wk.decode_bytes / (kk["decode_splitk"] * 1e-3) / 1e9
            configs[name] = {"workload": wk.name, "ms": round(m, 5), "GB/s": round(gbs, 1),
                             "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "bytes": int(wk.decode_bytes),
                             "layers_per_graph": DECODE_LAYERS, "ms_single_call_graph": round(m1, 5),
                             "GB/s_single_call_graph": round(wk.decode_bytes / (m1 * 1e-3) / 1e9, 1),
                             "splits": splits, "kernel_ms": {k: round(v, 5) for k, v in kk.items()},
                             "roofline": {"kernel": "decode_splitk", "bound": "hbm", "achieved": round(kgbs, 1),
                                          "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(kgbs / HBM_PEAK_GBS, 4),
                                          "traffic": profiled_traffic("decode_splitk", "cfg5_decode")
                                          if name == "cfg5" else None}}
            log(f"  {m * 1e3:.1f} us per layer ({m1 * 1e3:.1f} us as a one-call graph), {gbs:.0f} GB/s; kernels (ms): " + ", ".join(f"{k}={v:.4f}" for k, v in kk.items()))
        log("fused linear + cross-entropy at the reference model's head")
        configs["fused_ce_200m_head"] = measure_fused_ce(args.steps)
        log("  " + json.dumps(configs["fused_ce_200m_head"]))
        log("Muon batched SYRK and Newton-Schulz")
        configs["muon_syrk"] = measure_syrk(args.steps)
        log("  " + json.dumps(configs["muon_syrk"]))
        log("the reference benchmark's shapes")
        configs["reference_shapes"] = measure_reference_shapes()
        for r in configs["reference_shapes"]:
            log(f"  {r['shape']}: fwd {r['fwd_ms']} ms {r['fwd_TFLOP/s']} TFLOP/s, fwd+bwd {r['fwdbwd_ms']} ms "
                f"{r['fwdbwd_TFLOP/s']} TFLOP/s (reference, its GPU: {r['reference_published_ms']})")
        log("attention-block prologue / epilogue at the cfg3 shape")
        configs["block_io_cfg3"] = measure_block_io(W["cfg3"], args.steps)
        log("  " + json.dumps(configs["block_io_cfg3"]))
    cpu = None
    if not (args.quick or args.no_cpu):
        log("cpu baseline")
        cpu = cpu_baseline(w)
        log(f"  {cpu}")
    line = {
        "metric": "attn fwd/fwd+bwd TFLOP/s + decode GB/s, % of MI355X peak, 1 GPU",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v/dO, BASELINE config recipes)",
        "config": {"workload": w.name, "pass": "fwd+bwd", "tokens": sum(w.lengths), "docs": len(w.lengths),
                   "heads": w.heads, "kv_heads": w.kv_heads, "head_dim": w.head_dim,
                   "timing": "hipgraph replay" if args.graph else "eager calls, HIP events", "parallelism": "none (1 GPU)"},
        "frac_of_bf16_peak": round(value / BF16_PEAK_TFLOPS, 4),
        "roofline": roof,
        "kernels_ms": {k: round(v, 5) for k, v in kern.items()},
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

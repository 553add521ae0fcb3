"""Model-level parity harness: the kernels driven through an Attention-shaped caller.

The caller mirrors the reference's attention block (mixers.py:72-118): one fused q/k/v
projection viewed per head (non-contiguous head strides), q/k RMSNorm cast back to bf16,
interleaved-pair RoPE applied in fp32 (model/layers.py:66-101), a sliding-window or global
causal attention, an output gate out * sigmoid(gate_proj(x)) and the output projection. Two
such blocks (one local, one global) form a small residual stack. The checks follow the
reference's model tests (tests/test_model.py:64-96, :121-141):

- a full causal pass equals prefill + token-by-token decode, both with the reference's
  concatenated cache (flash_attn_func with one query) and with a static cache written by
  flash_attn_with_kvcache (the decode benchmark's caller, scripts/benchmark_decode.py:52-93);
- a packed varlen batch equals each document run alone;
- a decode step captured in a HIP graph replays to the eager result, bit for bit, over
  several replays with eager work in between;
- the whole stack agrees with the same stack on the fp32 oracle attention.
"""

import sys

import pytest
import torch
import torch.nn.functional as F

from _util import assert_close
from myk_llm_amd import flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache
from myk_llm_amd.block_io import output_gate, qkv_norm_rope, rope_tables
from oracle.attention import reference, reference_varlen

pytestmark = pytest.mark.gpu

HIDDEN, HEADS, KV_HEADS, HEAD_DIM = 128, 4, 2, 32
WINDOW = 48  # the local layer's window (the reference passes window_size = (w - 1, 0))


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _rms(x, w, eps=1e-6):
    x32 = x.float()
    return x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps) * w


def _rope(x, pos, theta):
    """Interleaved pairs (2i, 2i+1) rotated by pos * theta^(-2i / D), in fp32."""
    d = x.shape[-1]
    inv = theta ** (-torch.arange(0, d, 2, device=x.device, dtype=torch.float32) / d)
    ang = pos.float()[..., None] * inv  # (B, S, D/2)
    c, s = ang.cos()[:, :, None, :], ang.sin()[:, :, None, :]
    x2 = x.float().unflatten(-1, (d // 2, 2))
    a, b = x2[..., 0], x2[..., 1]
    return torch.stack((a * c - b * s, a * s + b * c), -1).flatten(-2).to(x.dtype)


def _linear(x, w):
    """x (..., in) @ w^T as a 2-D product."""
    return F.linear(x.reshape(-1, x.shape[-1]), w).reshape(*x.shape[:-1], w.shape[0])


class Block:
    """One attention block; `attend(q, k, v)` is supplied per pass (full, cached, packed)."""

    def __init__(self, gen, local, fused=False):
        def p(*shape, scale=0.08):
            return (torch.randn(*shape, generator=gen) * scale).to(torch.bfloat16).cuda()

        self.local = local
        self.window = (WINDOW - 1, 0) if local else (-1, -1)
        self.theta = 10000.0 if local else 500000.0
        self.w_qkv = p((HEADS + 2 * KV_HEADS) * HEAD_DIM, HIDDEN)
        self.w_o = p(HIDDEN, HEADS * HEAD_DIM)
        self.w_gate = p(HEADS * HEAD_DIM, HIDDEN)
        self.qn = (1.0 + 0.1 * torch.randn(HEAD_DIM, generator=gen)).cuda()
        self.kn = (1.0 + 0.1 * torch.randn(HEAD_DIM, generator=gen)).cuda()
        # fused: the prologue / epilogue kernels (myk_llm_amd.block_io) instead of torch ops
        self.fused = fused
        self.cos, self.sin = rope_tables(HEAD_DIM, 1024, self.theta, device="cuda")

    def params(self):
        return [self.w_qkv, self.w_o, self.w_gate, self.qn, self.kn]

    def qkv(self, x, pos):
        b, s, _ = x.shape
        if self.fused:
            return qkv_norm_rope(_linear(x, self.w_qkv), HEADS, KV_HEADS, HEAD_DIM, pos, self.cos, self.sin,
                                 self.qn, self.kn)
        q, k, v = _linear(x, self.w_qkv).split((HEADS * HEAD_DIM, KV_HEADS * HEAD_DIM, KV_HEADS * HEAD_DIM), -1)
        q, k, v = (t.view(b, s, -1, HEAD_DIM) for t in (q, k, v))  # strided views of the fused output
        q, k = _rms(q, self.qn).to(v.dtype), _rms(k, self.kn).to(v.dtype)
        return _rope(q, pos, self.theta), _rope(k, pos, self.theta), v

    def out(self, x, o):
        b, s, _ = x.shape
        if self.fused:
            o = output_gate(o.reshape(b, s, -1), _linear(x, self.w_gate))
        else:
            o = o.reshape(b, s, -1) * torch.sigmoid(_linear(x, self.w_gate))
        return _linear(o, self.w_o)


def _model(seed=0, fused=False):
    g = torch.Generator().manual_seed(seed)
    emb = (torch.randn(500, HIDDEN, generator=g) * 0.5).to(torch.bfloat16).cuda()
    return emb, [Block(g, local=True, fused=fused), Block(g, local=False, fused=fused)]


def _full(emb, blocks, ids, attn="kernel"):
    x = emb[ids]
    b, s = ids.shape
    pos = torch.arange(s, device="cuda").expand(b, -1)
    for blk in blocks:
        q, k, v = blk.qkv(x, pos)
        if attn == "kernel":
            o = flash_attn_func(q, k, v, causal=True, window_size=blk.window)
        else:
            o = reference(q.float(), k.float(), v.float(), True, blk.window).to(q.dtype)
        x = x + blk.out(x, o)
    return x


def _incremental_concat(emb, blocks, ids, prompt):
    """Prefill, then one token at a time over caches grown by concatenation (the reference's
    dense path, mixers.py:106-115: flash_attn_func with Sq = 1 runs the split-K decode)."""
    b, s = ids.shape
    caches = [None] * len(blocks)
    outs = []
    for t0, t1 in [(0, prompt)] + [(t, t + 1) for t in range(prompt, s)]:
        x = emb[ids[:, t0:t1]]
        pos = torch.arange(t0, t1, device="cuda").expand(b, -1)
        for i, blk in enumerate(blocks):
            q, k, v = blk.qkv(x, pos)
            if caches[i] is not None:
                k, v = torch.cat([caches[i][0], k], 1), torch.cat([caches[i][1], v], 1)
            caches[i] = (k, v)
            o = flash_attn_func(q, k, v, causal=True, window_size=blk.window)
            x = x + blk.out(x, o)
        outs.append(x)
    return torch.cat(outs, 1)


class StaticDecoder:
    """Static caches (batch, capacity, kv_heads, head_dim) written by flash_attn_with_kvcache
    itself, as the decode benchmark's caller does; the caller advances cache_seqlens."""

    def __init__(self, emb, blocks, batch, capacity):
        self.emb, self.blocks = emb, blocks
        z = lambda: torch.zeros(batch, capacity, KV_HEADS, HEAD_DIM, dtype=torch.bfloat16, device="cuda")
        self.caches = [(z(), z()) for _ in blocks]
        self.seqlens = torch.zeros(batch, dtype=torch.int32, device="cuda")

    def step(self, x, pos):
        for blk, (kc, vc) in zip(self.blocks, self.caches):
            q, k, v = blk.qkv(x, pos)
            o = flash_attn_with_kvcache(q, kc, vc, k, v, cache_seqlens=self.seqlens, causal=True,
                                        window_size=blk.window)
            x = x + blk.out(x, o)
        return x


def _incremental_static(emb, blocks, ids, prompt):
    b, s = ids.shape
    dec = StaticDecoder(emb, blocks, b, s + 8)
    outs = []
    for t0, t1 in [(0, prompt)] + [(t, t + 1) for t in range(prompt, s)]:
        pos = torch.arange(t0, t1, device="cuda").expand(b, -1)
        outs.append(dec.step(emb[ids[:, t0:t1]], pos))
        dec.seqlens += t1 - t0
    return torch.cat(outs, 1)


@torch.no_grad()
def test_incremental_decoding_matches_full_forward():
    """Prefill longer than the sliding window, then token-by-token decode == one full pass
    (tests/test_model.py:64-83), with both cache styles."""
    _say("harness: incremental vs full")
    emb, blocks = _model()
    ids = torch.randint(0, 500, (2, 200), generator=torch.Generator().manual_seed(1)).cuda()
    full = _full(emb, blocks, ids)
    assert_close(_incremental_concat(emb, blocks, ids, 150), full)
    assert_close(_incremental_static(emb, blocks, ids, 150), full)


@torch.no_grad()
def test_document_masking_isolates_documents():
    """A packed row with document masking == each document run on its own
    (tests/test_model.py:86-96), through flash_attn_varlen_func with cu_q = cu_k."""
    _say("harness: packed vs alone")
    emb, blocks = _model()
    ids = torch.randint(0, 500, (1, 256), generator=torch.Generator().manual_seed(2)).cuda()
    cu = torch.tensor([0, 100, 256], dtype=torch.int32, device="cuda")
    x = emb[ids]
    pos = torch.cat([torch.arange(100), torch.arange(156)]).cuda()[None]
    for blk in blocks:
        q, k, v = blk.qkv(x, pos)
        o = flash_attn_varlen_func(q[0], k[0], v[0], cu, cu, 156, 156, causal=True, window_size=blk.window)
        x = x + blk.out(x, o[None])
    alone = torch.cat([_full(emb, blocks, ids[:, :100]), _full(emb, blocks, ids[:, 100:])], 1)
    assert_close(x, alone)


@torch.no_grad()
def test_stack_matches_the_fp32_oracle_attention():
    """The two-block stack on the kernels == the same stack on the fp32 oracle attention."""
    _say("harness: kernels vs oracle")
    emb, blocks = _model()
    ids = torch.randint(0, 500, (2, 160), generator=torch.Generator().manual_seed(3)).cuda()
    assert_close(_full(emb, blocks, ids), _full(emb, blocks, ids, attn="oracle"))
    # The packed path against the oracle's per-document reference as well.
    cu = torch.tensor([0, 70, 160], dtype=torch.int32, device="cuda")
    blk = blocks[1]
    x = emb[ids[:1]]
    q, k, v = blk.qkv(x, torch.cat([torch.arange(70), torch.arange(90)]).cuda()[None])
    o = flash_attn_varlen_func(q[0], k[0], v[0], cu, cu, 90, 90, causal=True)
    ref = reference_varlen(q[0].float(), k[0].float(), v[0].float(), cu.cpu(), True, (-1, -1))
    assert_close(o, ref)


@pytest.mark.parametrize("fused", [False, True])
@torch.no_grad()
def test_decode_step_replays_from_a_graph(fused):
    """A decode step (both blocks, static caches written by the kernel) captured in a HIP
    graph: every replay equals the eager step on the same state, bit for bit
    (tests/test_model.py:121-141), with eager work and synchronizations between replays;
    also with the fused prologue / epilogue kernels in the captured step."""
    _say(f"harness: graph replay (fused={fused})")
    emb, blocks = _model(fused=fused)
    b, prompt, steps = 2, 64, 6
    ids = torch.randint(0, 500, (b, prompt + steps), generator=torch.Generator().manual_seed(4)).cuda()
    eager, graphed = StaticDecoder(emb, blocks, b, 128), StaticDecoder(emb, blocks, b, 128)
    pos0 = torch.arange(prompt, device="cuda").expand(b, -1)
    for dec in (eager, graphed):
        dec.step(emb[ids[:, :prompt]], pos0)
        dec.seqlens += prompt
    x_in = torch.zeros(b, 1, HIDDEN, dtype=torch.bfloat16, device="cuda")
    pos_in = torch.zeros(b, 1, dtype=torch.long, device="cuda")
    # Warm up on a side stream (allocator, library handles), then capture one step.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        scratch = StaticDecoder(emb, blocks, b, 128)
        scratch.step(x_in, pos_in)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_graph = graphed.step(x_in, pos_in)
    for t in range(prompt, prompt + steps):
        x_in.copy_(emb[ids[:, t:t + 1]])
        pos_in.fill_(t)
        graph.replay()
        torch.cuda.synchronize()
        y_eager = eager.step(emb[ids[:, t:t + 1]], torch.full((b, 1), t, device="cuda"))
        torch.cuda.synchronize()
        assert torch.equal(y_graph, y_eager), f"replay at position {t} differs from the eager step"
        eager.seqlens += 1
        graphed.seqlens += 1


def test_fused_prologue_epilogue_training_step():
    """The stack with the fused prologue / epilogue kernels == the stack with the reference's
    torch ops (mixers.py:85-89, :116-117): outputs, and the gradients of every block parameter
    and of the input through a fwd+bwd step (the reference's tolerance)."""
    _say("harness: fused vs composed training step")
    ids = torch.randint(0, 500, (2, 192), generator=torch.Generator().manual_seed(5)).cuda()
    results = []
    for fused in (False, True):
        emb, blocks = _model(seed=6, fused=fused)
        leaves = [t.requires_grad_(True) for blk in blocks for t in blk.params()]
        x0 = emb[ids].detach().requires_grad_(True)
        b, s = ids.shape
        pos = torch.arange(s, device="cuda").expand(b, -1)
        x = x0
        for blk in blocks:
            q, k, v = blk.qkv(x, pos)
            o = flash_attn_func(q, k, v, causal=True, window_size=blk.window)
            x = x + blk.out(x, o)
        dy = torch.randn(x.shape, generator=torch.Generator().manual_seed(7)).to(x.dtype).cuda()
        grads = torch.autograd.grad(x, [x0, *leaves], dy)
        results.append((x.detach(), grads))
    (y0, g0), (y1, g1) = results
    assert_close(y1, y0)
    names = ["x"] + [f"{n}[{i}]" for i in range(2) for n in ("w_qkv", "w_o", "w_gate", "q_norm", "k_norm")]
    for name, a, e in zip(names, g1, g0):
        _say(f"  d{name}: max-abs {(a.float() - e.float()).abs().max().item():.3e} of {e.float().abs().max().item():.3e}")
        assert_close(a, e)

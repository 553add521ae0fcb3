"""The five synthetic workloads of the benchmark (shapes, seeded lengths and inputs).

Every tensor is N(0, 1) drawn on the CPU from ``torch.Generator().manual_seed(seed)`` in
the order q, k, v, dO, then cast and moved; the scale is 1/sqrt(D) and every config is
causal. The FLOP convention is the reference's (scripts/benchmark_attention.py:49-50, 86):
F_fwd = 4 * visible pairs * Hq * D and F_fwd+bwd = 3.5 * F_fwd; decode is priced by the
bytes it must read (each K/V byte once per GQA group) plus what it writes.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
BF16_PEAK_TFLOPS = 2516.6  # MI355X dense bf16 MFMA: 256 CUs x 2.4 GHz x 4096 FLOP/clk


def cfg2_lengths() -> list[int]:
    """First seed s >= 0 whose randint(128, 2049, (8,)) lengths total within [7900, 8500]."""
    s = 0
    while True:
        lens = torch.randint(128, 2049, (8,), generator=torch.Generator().manual_seed(s)).tolist()
        if 7900 <= sum(lens) <= 8500:
            return lens
        s += 1


def cfg3_lengths(total: int = 16384, lo: int = 64, hi: int = 8192) -> list[int]:
    """Log-uniform document lengths in [lo, hi] until the sum reaches total, last one trimmed."""
    g = torch.Generator().manual_seed(0)
    lens: list[int] = []
    while sum(lens) < total:
        u = torch.rand((), generator=g).item()
        lens.append(int(math.exp(math.log(lo) + u * (math.log(hi) - math.log(lo)))))
    lens[-1] -= sum(lens) - total
    return lens


def cfg5_cache_seqlens(batch: int = 64) -> list[int]:
    return torch.randint(256, 16385, (batch,), generator=torch.Generator().manual_seed(0)).tolist()


def causal_pairs(lengths, window: int | None = None) -> int:
    """Visible pairs of causal documents; window w (model convention) -> min(i + 1, w) keys."""
    total = 0
    for n in lengths:
        if window is None or window >= n:
            total += n * (n + 1) // 2
        else:
            total += window * (window + 1) // 2 + (n - window) * window
    return total


@dataclass
class Workload:
    name: str
    kind: str  # "varlen", "dense", "decode"
    heads: int
    kv_heads: int
    head_dim: int
    lengths: list[int] = field(default_factory=list)  # varlen documents or dense batch lengths
    batch: int = 1
    seqlen: int = 0
    window: int | None = None  # model convention (mixers.py:90): window_size = (w - 1, 0)
    backward: bool = False
    nq: int = 1  # decode queries per sequence
    cache_seqlens: list[int] = field(default_factory=list)
    capacity: int = 0
    dtype: torch.dtype = torch.bfloat16

    @property
    def window_size(self) -> tuple[int, int]:
        return (self.window - 1, 0) if self.window else (-1, -1)

    @property
    def pairs(self) -> int:
        if self.kind == "varlen":
            return causal_pairs(self.lengths, self.window)
        if self.kind == "dense":
            return self.batch * causal_pairs([self.seqlen], self.window)
        return sum((n + self.nq) * self.nq - self.nq * (self.nq - 1) // 2 for n in self.cache_seqlens)

    @property
    def fwd_flops(self) -> float:
        return 4.0 * self.pairs * self.heads * self.head_dim

    @property
    def decode_bytes(self) -> float:
        """K and V rows read once per GQA group + q read + O written (bf16) + LSE written (fp32)."""
        kv = sum(n + self.nq for n in self.cache_seqlens) * self.kv_heads * self.head_dim * 2 * 2
        rows = len(self.cache_seqlens) * self.nq * self.heads
        return kv + rows * self.head_dim * 2 * 2 + rows * 4


def workloads() -> dict[str, Workload]:
    c5 = cfg5_cache_seqlens()
    cap = max(c5) + 4
    return {
        "cfg1": Workload("cfg1_cpu_fp32_causal_B1_T512_H8_D64", "dense", 8, 8, 64, batch=1, seqlen=512,
                         dtype=torch.float32),
        "cfg2": Workload("cfg2_varlen_gqa_fwd_8docs_H16_KV4_D64", "varlen", 16, 4, 64, lengths=cfg2_lengths()),
        "cfg3": Workload("cfg3_varlen_gqa_fwdbwd_16k_H16_KV4_D128", "varlen", 16, 4, 128, lengths=cfg3_lengths(),
                         backward=True),
        "cfg4": Workload("cfg4_swa1024_fwdbwd_B4_T8192_H16_KV4_D128", "dense", 16, 4, 128, batch=4, seqlen=8192,
                         window=1024, backward=True),
        "cfg5": Workload("cfg5_decode_B64_H16_KV4_D64_nq1", "decode", 16, 4, 64, batch=64, nq=1,
                         cache_seqlens=c5, capacity=cap),
        "cfg5_mtp": Workload("cfg5_decode_B64_H16_KV4_D64_nq4", "decode", 16, 4, 64, batch=64, nq=4,
                             cache_seqlens=c5, capacity=cap),
    }


def make_inputs(w: Workload, device="cuda", seed: int = 0, with_grad_out: bool | None = None):
    """Seeded inputs of workload w on device: dict with q, k, v[, dout][, cu_seqlens].
    Decode: q (B, nq, H, D), caches (B, capacity, Hkv, D) with rows beyond each length
    zero, new k/v (B, nq, Hkv, D), cache_seqlens (B,) int32."""
    g = torch.Generator().manual_seed(seed)
    dt = w.dtype
    out: dict = {}
    if w.kind == "varlen":
        total = sum(w.lengths)
        shapes = [(total, w.heads, w.head_dim), (total, w.kv_heads, w.head_dim), (total, w.kv_heads, w.head_dim)]
    elif w.kind == "dense":
        shapes = [(w.batch, w.seqlen, w.heads, w.head_dim), (w.batch, w.seqlen, w.kv_heads, w.head_dim),
                  (w.batch, w.seqlen, w.kv_heads, w.head_dim)]
    else:
        b = len(w.cache_seqlens)
        shapes = [(b, w.nq, w.heads, w.head_dim), (b, w.capacity, w.kv_heads, w.head_dim),
                  (b, w.capacity, w.kv_heads, w.head_dim)]
    for name, shape in zip(("q", "k", "v"), shapes):
        out[name] = torch.randn(*shape, generator=g).to(dt).to(device)
    if with_grad_out if with_grad_out is not None else w.backward:
        out["dout"] = torch.randn(*shapes[0], generator=g).to(dt).to(device)
    if w.kind == "varlen":
        cu = torch.tensor([0] + list(torch.tensor(w.lengths).cumsum(0).tolist()), dtype=torch.int32)
        out["cu_seqlens"] = cu.to(device)
        out["max_seqlen"] = max(w.lengths)
    if w.kind == "decode":
        b = len(w.cache_seqlens)
        lens = torch.tensor(w.cache_seqlens, dtype=torch.int32)
        pos = torch.arange(w.capacity)[None, :]
        keep = (pos < lens[:, None])[:, :, None, None].to(device)
        out["k"] = out["k"] * keep
        out["v"] = out["v"] * keep
        out["k_new"] = torch.randn(b, w.nq, w.kv_heads, w.head_dim, generator=g).to(dt).to(device)
        out["v_new"] = torch.randn(b, w.nq, w.kv_heads, w.head_dim, generator=g).to(dt).to(device)
        out["cache_seqlens"] = lens.to(device)
    return out

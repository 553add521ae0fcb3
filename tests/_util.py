"""Shared helpers for the parity tests."""

from __future__ import annotations

import torch


def assert_close(actual, expected):
    """The reference's tolerance (tests/test_flash_attn.py:37-40): relative to the largest
    reference value, bf16 inputs/outputs."""
    tol = 2e-2 * expected.abs().max().item() + 1e-3
    torch.testing.assert_close(actual.float().cpu(), expected.float().cpu(), rtol=0, atol=tol)


def north_star_errors(actual, expected):
    """(max-abs, mean-abs) error against an fp32 reference."""
    d = (actual.float() - expected.float().to(actual.device)).abs()
    return d.max().item(), d.mean().item()


def storage_ulp(x, dtype):
    """One unit in the last place of |x| in the 16-bit storage type (bf16: 8 significant bits,
    fp16: 11)."""
    bits = 8 if dtype == torch.bfloat16 else 11
    _, e = torch.frexp(x.float().abs().clamp_min(1e-30))
    return torch.ldexp(torch.ones_like(x, dtype=torch.float32), (e - bits).to(torch.int32))


def assert_north_star(actual, expected, max_abs=2e-2, mean_abs=2e-3, what=""):
    """The north-star bounds against the fp32 reference: mean-abs <= 2e-3, and max-abs <= 2e-2
    beyond the storage floor of each element. A 16-bit result cannot be closer to an fp32 value
    than its own rounding, which is at most half an ulp (round to nearest): for |x| in [8, 16)
    a bf16 ulp is 2^-4, so even the fp32 reference rounded to bf16 misses it by up to
    2^-5 = 0.031 > 2e-2. The half-ulp term admits exactly that representation error and
    nothing more. Returns (max-abs, mean-abs, max-abs beyond the floor)."""
    exp = expected.float().to(actual.device)
    d = (actual.float() - exp).abs()
    mx, mn = d.max().item(), d.mean().item()
    excess = (d - 0.5 * storage_ulp(exp, actual.dtype)).max().item()
    assert mn <= mean_abs and excess <= max_abs, (
        f"{what}: max-abs {mx:.3e}, beyond half a storage ulp {excess:.3e} (<= {max_abs}), "
        f"mean-abs {mn:.3e} (<= {mean_abs})")
    return mx, mn, excess


def assert_lse(actual, expected, tol=1e-3, what="lse"):
    a, e = actual.float().cpu(), expected.float().cpu()
    inf_a, inf_e = torch.isinf(a), torch.isinf(e)
    assert torch.equal(inf_a, inf_e), f"{what}: +inf rows differ"
    d = (a[~inf_a] - e[~inf_e]).abs()
    mx = d.max().item() if d.numel() else 0.0
    assert mx <= tol, f"{what}: max-abs {mx:.3e} > {tol}"


def random_qkv(batch, seqlen_q, seqlen_k, heads, kv_heads, head_dim, packed=False, dtype=torch.bfloat16,
               device="cuda", requires_grad=True):
    """tests/test_flash_attn.py:31-34, drawn on the CPU from the global seed so the GPU box
    and any torch build agree, then moved."""
    lead_q, lead_k = ((seqlen_q,), (seqlen_k,)) if packed else ((batch, seqlen_q), (batch, seqlen_k))

    def make(*shape):
        return torch.randn(*shape).to(dtype).to(device).requires_grad_(requires_grad)

    return make(*lead_q, heads, head_dim), make(*lead_k, kv_heads, head_dim), make(*lead_k, kv_heads, head_dim)


def record_parity(config, name, **fields):
    """Appends one JSON line of measured errors to the file named by MYKFA_PARITY_LOG (nothing
    when unset), so a run's raw parity numbers can be kept beside its log."""
    import json
    import os

    path = os.environ.get("MYKFA_PARITY_LOG")
    if not path:
        return
    with open(path, "a") as f:
        f.write(json.dumps({"config": config, "tensor": name, **fields}) + "\n")

"""Parity of the batched SYRK kernel (csrc/syrk.hip) and the Newton-Schulz driver
(myk_llm_amd.muon) with the CPU oracle (oracle/muon.py).

- SYRK against the float64 product of the same bf16 inputs: every element within one bf16
  ulp of the exact value plus 1e-5 of the row scale (the kernel accumulates in fp32 and
  rounds once), on the reference test's shapes (tests/test_muon.py:12-26: aligned,
  unaligned and transposed-view inputs, and the biased form with a symmetric bias) and at a
  Muon shape of the reference model; the result is exactly symmetric.
- Newton-Schulz against the oracle's per-matrix iteration with the same bf16 rounding
  points, at the reference test's tolerance (tests/test_muon.py:74-79: rtol 2e-2, atol 1e-2).
"""

import sys

import pytest
import torch

from _util import storage_ulp
from myk_llm_amd.muon import batched_newton_schulz_orthogonalize, batched_syrk
from oracle import muon as om

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _check_syrk(got, x, bias=None, alpha=1.0, beta=0.0, what=""):
    ref = om.syrk_reference(x.cpu().float(), None if bias is None else bias.cpu().float(), alpha, beta)
    g = got.cpu().double()
    scale = (x.cpu().double() ** 2).sum(-1).max().item() * abs(alpha) + (0 if bias is None else abs(beta) * bias.abs().max().item())
    bound = storage_ulp(ref.float(), torch.bfloat16).double() + 1e-5 * scale
    err = (g - ref).abs()
    _say(f"  {what}: max-abs {err.max().item():.3e}, exact-in-bf16 {(g == ref.to(torch.bfloat16).double()).double().mean().item() * 100:.1f}%")
    assert (err <= bound).all(), f"{what}: {(err > bound).sum().item()} elements beyond one ulp"
    assert torch.equal(got, got.transpose(-2, -1)), f"{what}: not symmetric"


@pytest.mark.parametrize(("m", "k", "transposed"), [(100, 150, False), (256, 512, False), (192, 320, True),
                                                    (130, 192, False)])  # m not a multiple of 4: padded out rows
def test_batched_syrk_matches_the_product(m, k, transposed):
    _say(f"syrk m={m} k={k} transposed={transposed}")
    g = torch.Generator().manual_seed(0)
    raw = torch.randn((5, k, m) if transposed else (5, m, k), generator=g).to(torch.bfloat16).cuda()
    x = raw.transpose(-2, -1) if transposed else raw
    gram = batched_syrk(x)
    torch.cuda.synchronize()
    _check_syrk(gram, x, what="x x^T")
    bias = ((gram.float() + gram.float().transpose(-2, -1)) * 0.5).to(torch.bfloat16)
    out = batched_syrk(gram, bias=bias, alpha=2.0315, beta=-4.775)
    torch.cuda.synchronize()
    _check_syrk(out, gram, bias, 2.0315, -4.775, what="2.0315 G G - 4.775 G")


def test_out_argument_and_strided_out():
    x = torch.randn(3, 160, 96).to(torch.bfloat16).cuda()
    big = torch.zeros(3, 160, 200, dtype=torch.bfloat16, device="cuda")
    view = big[:, :, :160]  # row stride 200 (a multiple of 4), last dimension contiguous
    res = batched_syrk(x, out=view)
    assert res.data_ptr() == view.data_ptr()
    _check_syrk(view, x, what="strided out")
    assert torch.equal(big[:, :, 160:], torch.zeros_like(big[:, :, 160:]))


def test_model_shape_and_determinism():
    """A Muon bucket of the reference model (hidden 1024, 9 layers, configs/model/200m.yaml)."""
    _say("syrk (9, 1024, 4096)")
    x = (torch.randn(9, 1024, 4096, generator=torch.Generator().manual_seed(1)) * 0.02).to(torch.bfloat16).cuda()
    a = batched_syrk(x)
    b = batched_syrk(x)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    ref = (x.float() @ x.float().transpose(-2, -1).contiguous())  # fp32 on the GPU, contiguous operands
    err = (a.float() - ref).abs()
    bound = storage_ulp(ref, torch.bfloat16) + 1e-5 * (x.float() ** 2).sum(-1).max()
    _say(f"  max-abs {err.max().item():.3e}")
    assert (err <= bound).all()


@pytest.mark.parametrize("shape", [(4, 320, 192), (3, 128, 384), (2, 256, 256)])
def test_batched_newton_schulz_matches_the_iteration(shape):
    """tests/test_muon.py:74-79 (batched against per-matrix), against the oracle's iteration."""
    _say(f"newton-schulz {shape}")
    mats = torch.randn(*shape, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    got = batched_newton_schulz_orthogonalize(mats.cuda().clone(), steps=5)
    torch.cuda.synchronize()
    assert got.shape == mats.shape and got.is_contiguous()
    ref = torch.stack([om.newton_schulz_reference(mats[i], 5) for i in range(shape[0])])
    err = (got.float().cpu() - ref).abs().max().item()
    _say(f"  max-abs {err:.3e}")
    torch.testing.assert_close(got.float().cpu(), ref, rtol=2e-2, atol=1e-2)


def test_newton_schulz_with_norm_sq():
    mats = torch.randn(4, 192, 320, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).cuda()
    norm_sq = mats.float().pow(2).sum(dim=(-2, -1))
    a = batched_newton_schulz_orthogonalize(mats.clone(), 5, norm_sq=norm_sq)
    b = batched_newton_schulz_orthogonalize(mats.clone(), 5)
    torch.testing.assert_close(a.float(), b.float(), rtol=2e-2, atol=1e-2)

"""One 32768-token causal document, the longest rows a long-context run has: the forward's
rows (the first 64 and the last 256 queries of every head) against fp32 math on the same GPU,
at head_dim 64 and 128 with GQA 4; and the backward of that document (its stored dS would
exceed the default budget, so it takes the recomputing backward) free of unwritten values."""

import math
import sys

import pytest
import torch

from _util import assert_close, assert_lse
from myk_llm_amd import flash_attn_varlen_func

pytestmark = pytest.mark.gpu

LOG2E = 1.0 / math.log(2.0)


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("d", [64, 128])
def test_long_document_forward_rows(d):
    _say(f"32768-token document, head_dim {d}")
    n, hq, hkv = 32768, 16, 4
    g = torch.Generator().manual_seed(d)
    q = torch.randn(n, hq, d, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16).cuda()
    cu = torch.tensor([0, n], dtype=torch.int32).cuda()
    out, lse = flash_attn_varlen_func(q, k, v, cu, cu, n, n, causal=True, return_softmax_lse=True)
    torch.cuda.synchronize()
    rows = torch.cat([torch.arange(64), torch.arange(n - 256, n)]).cuda()
    visible = torch.arange(n, device="cuda")[None, :] <= rows[:, None]
    scale = 1.0 / math.sqrt(d)
    for h in range(hq):
        kv = h // (hq // hkv)
        kt = k[:, kv].float().t().contiguous()
        s = (q[rows, h].float().contiguous() @ kt) * scale
        s = s.masked_fill(~visible, float("-inf"))
        lse_e = torch.logsumexp(s, -1)
        o = torch.softmax(s, -1) @ v[:, kv].float().contiguous()
        assert_close(out[rows, h], o)
        assert_lse(lse[h, rows], lse_e * LOG2E, what=f"head {h} lse")


def test_long_document_backward_is_complete():
    _say("32768-token document, head_dim 128, backward")
    n, hq, hkv, d = 32768, 16, 4, 128
    g = torch.Generator().manual_seed(7)
    q = torch.randn(n, hq, d, generator=g).to(torch.bfloat16).cuda().requires_grad_()
    k = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16).cuda().requires_grad_()
    v = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16).cuda().requires_grad_()
    do = torch.randn(n, hq, d, generator=g).to(torch.bfloat16).cuda()
    cu = torch.tensor([0, n], dtype=torch.int32).cuda()
    out = flash_attn_varlen_func(q, k, v, cu, cu, n, n, causal=True)
    dq, dk, dv = torch.autograd.grad(out, (q, k, v), do)
    torch.cuda.synchronize()
    for x in (dq, dk, dv):
        assert torch.isfinite(x).all()
    # The first query sees only key 0, and a softmax over one key does not depend on its score:
    # query 0's gradient is zero up to the rounding of dP - delta.
    assert dq[0].float().abs().max().item() < 1e-2

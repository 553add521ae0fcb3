"""GPU parity of the gfx950 kernels against the CPU oracle, mirroring the reference's
tests/test_flash_attn.py case by case, plus LSE, fp16, every head_dim, GQA ratios,
strided inputs, empty rows and bitwise determinism."""

import sys

import pytest
import torch
import torch.nn.functional as F

from _util import assert_close, assert_lse, random_qkv
from myk_llm_amd import flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache
from oracle.attention import backward_reference, backward_reference_varlen, reference, reference_varlen, \
    reference_with_lse

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _cpu(*xs):
    return [x.detach().cpu() for x in xs]


@pytest.mark.parametrize(
    "seqlen_q, seqlen_k, heads, kv_heads, head_dim, causal, window",
    [
        (128, 128, 4, 4, 64, True, (-1, -1)),
        (200, 200, 4, 2, 64, True, (-1, -1)),  # partial blocks, GQA
        (300, 300, 8, 2, 128, True, (63, 0)),  # sliding window
        (257, 257, 2, 1, 64, False, (-1, -1)),
        (257, 257, 2, 1, 64, False, (31, 17)),
        (5, 300, 4, 2, 128, True, (63, 0)),  # cached decoding: queries at the end of the keys
        (100, 37, 4, 2, 64, True, (-1, -1)),  # more queries than keys: early rows see nothing
        (130, 130, 2, 1, 256, True, (-1, -1)),
        (130, 130, 2, 1, 16, True, (7, 0)),
    ],
)
def test_matches_reference_output_and_gradients(seqlen_q, seqlen_k, heads, kv_heads, head_dim, causal, window):
    """tests/test_flash_attn.py:43-67."""
    _say(f"case Lq={seqlen_q} Lk={seqlen_k} H={heads}/{kv_heads} D={head_dim} causal={causal} window={window}")
    torch.manual_seed(0)
    q, k, v = random_qkv(2, seqlen_q, seqlen_k, heads, kv_heads, head_dim)
    out, lse = flash_attn_func(q, k, v, causal=causal, window_size=window, return_softmax_lse=True)
    grad_out = torch.randn(out.shape).to(out.dtype).to(out.device)
    grads = torch.autograd.grad(out, (q, k, v), grad_out)
    torch.cuda.synchronize()
    qc, kc, vc, goc = _cpu(q, k, v, grad_out)
    expected, expected_lse = reference_with_lse(qc, kc, vc, causal, window)
    expected_grads = backward_reference(qc, kc, vc, goc, causal, window)
    assert_close(out, expected)
    assert_lse(lse, expected_lse)
    for grad, expected_grad in zip(grads, expected_grads):
        assert_close(grad, expected_grad)


@pytest.mark.parametrize("window", [(-1, -1), (15, 0)])
def test_varlen_keeps_documents_separate(window):
    """tests/test_flash_attn.py:70-85."""
    _say(f"varlen window={window}")
    torch.manual_seed(0)
    lengths = [1, 17, 128, 300, 5, 64, 3]
    cu_seqlens = F.pad(torch.tensor(lengths).cumsum(0), (1, 0)).to(torch.int32).cuda()
    q, k, v = random_qkv(1, sum(lengths), sum(lengths), 4, 2, 64, packed=True)
    out, lse = flash_attn_varlen_func(q, k, v, cu_seqlens, cu_seqlens, 512, 512, causal=True, window_size=window,
                                      return_softmax_lse=True)
    grad_out = torch.randn(out.shape).to(out.dtype).to(out.device)
    grads = torch.autograd.grad(out, (q, k, v), grad_out)
    torch.cuda.synchronize()
    qc, kc, vc, goc = _cpu(q, k, v, grad_out)
    cu = cu_seqlens.cpu()
    expected, expected_lse = reference_varlen(qc, kc, vc, cu, True, window, with_lse=True)
    expected_grads = backward_reference_varlen(qc, kc, vc, goc, cu, True, window)
    assert_close(out, expected)
    assert_lse(lse, expected_lse)
    for grad, expected_grad in zip(grads, expected_grads):
        assert_close(grad, expected_grad)


@pytest.mark.parametrize("window", [(-1, -1), (15, 0)])
def test_kvcache_matches_full_attention(window):
    """tests/test_flash_attn.py:88-112."""
    _say(f"kvcache window={window}")
    torch.manual_seed(0)
    batch, heads, kv_heads, head_dim = 3, 8, 2, 128
    with torch.no_grad():
        q, k, v = random_qkv(batch, 41, 41, heads, kv_heads, head_dim, requires_grad=False)
        k_cache = torch.zeros(batch, 64, kv_heads, head_dim, device="cuda", dtype=torch.bfloat16)
        v_cache = torch.zeros_like(k_cache)
        cache_seqlens = torch.zeros(batch, dtype=torch.int32, device="cuda")
        outs = []
        for a, b in [(0, 37), (37, 38), (38, 41)]:  # prefill, then steps of 1 and 3 tokens
            outs.append(flash_attn_with_kvcache(q[:, a:b], k_cache, v_cache, k[:, a:b], v[:, a:b],
                                                cache_seqlens=cache_seqlens, causal=True, window_size=window))
            cache_seqlens += b - a
        torch.testing.assert_close(k_cache[:, :41], k, rtol=0, atol=0)
        torch.testing.assert_close(v_cache[:, :41], v, rtol=0, atol=0)
        qc, kc, vc = _cpu(q, k, v)
        assert_close(torch.cat(outs, 1), reference(qc, kc, vc, True, window))

        # Ragged caches: each sequence attends over its own length only.
        cache_seqlens = torch.tensor([5, 20, 37], dtype=torch.int32, device="cuda")
        q_new, k_new, v_new = random_qkv(batch, 2, 2, heads, kv_heads, head_dim, requires_grad=False)
        out = flash_attn_with_kvcache(q_new, k_cache, v_cache, k_new, v_new, cache_seqlens=cache_seqlens,
                                      causal=True, window_size=window)
        kcc, vcc, qn = _cpu(k_cache, v_cache, q_new)
        for i, length in enumerate((cache_seqlens + 2).tolist()):
            assert_close(out[i:i + 1], reference(qn[i:i + 1], kcc[i:i + 1, :length], vcc[i:i + 1, :length], True,
                                                 window))


def test_compiles_without_graph_breaks():
    """tests/test_flash_attn.py:115-129."""
    _say("compile fullgraph")
    torch.manual_seed(0)
    q, k, v = random_qkv(2, 96, 96, 4, 2, 64)

    def attend(q, k, v):
        return flash_attn_func(q * 1.0, k, v, causal=True, window_size=(31, 0)).float().square().sum()

    compiled = torch.compile(attend, fullgraph=True)
    loss = compiled(q, k, v)
    grads = torch.autograd.grad(loss, (q, k, v))
    expected = attend(q, k, v)
    expected_grads = torch.autograd.grad(expected, (q, k, v))
    torch.testing.assert_close(loss, expected)
    for grad, expected_grad in zip(grads, expected_grads):
        torch.testing.assert_close(grad, expected_grad)


def test_rejects_unsupported_inputs():
    """tests/test_flash_attn.py:132-137."""
    q = torch.randn(1, 8, 2, 48, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="head_dim"):
        flash_attn_func(q, q, q)
    with pytest.raises(TypeError, match="bf16"):
        flash_attn_func(q.float(), q.float(), q.float())
    q = torch.randn(1, 8, 3, 64, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(1, 8, 2, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="multiple"):
        flash_attn_func(q, k, k)
    q = torch.randn(1, 1, 4, 64, device="cuda", dtype=torch.bfloat16)
    cache = torch.zeros(1, 16, 64, 2, device="cuda", dtype=torch.bfloat16).transpose(2, 3)
    with pytest.raises(ValueError, match="contiguous last dimension"):
        flash_attn_with_kvcache(q, cache, cache, cache_seqlens=torch.zeros(1, dtype=torch.int32, device="cuda"))


@pytest.mark.parametrize("head_dim", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("heads, kv_heads", [(4, 4), (8, 2), (8, 1), (6, 2), (16, 2)])
def test_head_dims_and_gqa_ratios(head_dim, heads, kv_heads):
    """Every supported head_dim (flash_attn.py:322-323) x GQA group sizes 1, 4, 8, 3."""
    _say(f"D={head_dim} H={heads}/{kv_heads}")
    torch.manual_seed(1)
    q, k, v = random_qkv(1, 150, 150, heads, kv_heads, head_dim)
    out, lse = flash_attn_func(q, k, v, causal=True, return_softmax_lse=True)
    grad_out = torch.randn(out.shape).to(out.dtype).to(out.device)
    grads = torch.autograd.grad(out, (q, k, v), grad_out)
    torch.cuda.synchronize()
    qc, kc, vc, goc = _cpu(q, k, v, grad_out)
    expected, expected_lse = reference_with_lse(qc, kc, vc, True, (-1, -1))
    assert_close(out, expected)
    assert_lse(lse, expected_lse)
    for grad, eg in zip(grads, backward_reference(qc, kc, vc, goc, True, (-1, -1))):
        assert_close(grad, eg)


def test_fp16_inputs():
    """fp16 is accepted like bf16 (flash_attn.py:340-341)."""
    torch.manual_seed(2)
    q, k, v = random_qkv(2, 200, 200, 8, 2, 128, dtype=torch.float16)
    out = flash_attn_func(q, k, v, causal=True, window_size=(63, 0))
    assert out.dtype == torch.float16
    grad_out = torch.randn(out.shape).to(out.dtype).to(out.device)
    grads = torch.autograd.grad(out, (q, k, v), grad_out)
    qc, kc, vc, goc = _cpu(q, k, v, grad_out)
    assert_close(out, reference(qc, kc, vc, True, (63, 0)))
    for grad, eg in zip(grads, backward_reference(qc, kc, vc, goc, True, (63, 0))):
        assert_close(grad, eg)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("seqlen_q", [1, 4, 16])
def test_short_queries_take_the_decode_kernels(dtype, seqlen_q):
    """flash_attn_func with at most 16 queries runs the split-K decode kernels (the reference's
    decode config, flash_attn.py:364), in both input types."""
    _say(f"short queries Lq={seqlen_q} {dtype}")
    torch.manual_seed(7)
    q, k, v = random_qkv(3, seqlen_q, 700, 8, 2, 64, dtype=dtype, requires_grad=False)
    out, lse = flash_attn_func(q, k, v, causal=True, return_softmax_lse=True)
    assert out.dtype == dtype
    qc, kc, vc = _cpu(q, k, v)
    expected, expected_lse = reference_with_lse(qc, kc, vc, True, (-1, -1))
    assert_close(out, expected)
    assert_lse(lse, expected_lse)


def test_auxiliary_tensors_on_the_host_are_rejected():
    """cu_seqlens on the host would hand the kernel a host pointer: rejected before launch, like
    the reference (a device mismatch)."""
    q, k, v = random_qkv(1, 64, 64, 4, 2, 64, packed=True, requires_grad=False)
    cu = torch.tensor([0, 30, 64], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="same GPU"):
        flash_attn_varlen_func(q, k, v, cu, cu.cuda(), 34, 34, causal=True)
    with pytest.raises(RuntimeError, match="same GPU"):
        flash_attn_varlen_func(q, k, v, cu.cuda(), cu, 34, 34, causal=True)


def test_strided_views_of_a_fused_projection():
    """q/k/v as views of one fused qkv tensor (mixers.py:81-84): non-contiguous head strides."""
    torch.manual_seed(3)
    b, t, h, hk, d = 2, 96, 8, 2, 64
    qkv = torch.randn(b, t, (h + 2 * hk) * d).to(torch.bfloat16).cuda().requires_grad_()
    q, k, v = qkv.split([h * d, hk * d, hk * d], dim=-1)
    q, k, v = q.view(b, t, h, d), k.view(b, t, hk, d), v.view(b, t, hk, d)
    out = flash_attn_func(q, k, v, causal=True)
    grad_out = torch.randn(out.shape).to(out.dtype).to(out.device)
    (g,) = torch.autograd.grad(out, (qkv,), grad_out)
    qc, kc, vc, goc = _cpu(q, k, v, grad_out)
    assert_close(out, reference(qc, kc, vc, True, (-1, -1)))
    eg = torch.cat([x.reshape(b, t, -1) for x in backward_reference(qc, kc, vc, goc, True, (-1, -1))], -1)
    assert_close(g, eg)


def test_rows_that_see_no_key():
    """Lq > Lk: the first Lq - Lk rows see nothing: O = 0, LSE = +inf (flash_attn.py:147-151)."""
    torch.manual_seed(4)
    q, k, v = random_qkv(1, 100, 37, 4, 2, 64)
    out, lse = flash_attn_func(q, k, v, causal=True, return_softmax_lse=True)
    assert torch.all(out[:, :63] == 0)
    assert torch.all(torch.isinf(lse[:, :63])) and torch.all(lse[:, :63] > 0)
    assert torch.all(torch.isfinite(lse[:, 63:]))
    dq, dk, dv = torch.autograd.grad(out, (q, k, v), torch.ones_like(out))
    assert torch.all(dq[:, :63] == 0)
    assert torch.isfinite(dk).all() and torch.isfinite(dv).all()


def test_backward_is_bitwise_deterministic():
    """No atomics: repeated backward passes are bit-identical (flash_attn.py:20-21)."""
    torch.manual_seed(5)
    lengths = [700, 33, 1200, 90]
    cu = F.pad(torch.tensor(lengths).cumsum(0), (1, 0)).to(torch.int32).cuda()
    q, k, v = random_qkv(1, sum(lengths), sum(lengths), 8, 2, 128, packed=True)
    grad_out = torch.randn(q.shape).to(q.dtype).cuda()
    runs = []
    for _ in range(3):
        out = flash_attn_varlen_func(q, k, v, cu, cu, 1200, 1200, causal=True)
        runs.append([out.detach().clone()] + [g.clone() for g in torch.autograd.grad(out, (q, k, v), grad_out)])
    for r in runs[1:]:
        for a, b in zip(runs[0], r):
            assert torch.equal(a, b)


def test_softmax_scale_and_bidirectional_window():
    torch.manual_seed(6)
    q, k, v = random_qkv(2, 190, 230, 4, 4, 64)
    out = flash_attn_func(q, k, v, causal=False, window_size=(40, 9), softmax_scale=0.3)
    grad_out = torch.randn(out.shape).to(out.dtype).to(out.device)
    grads = torch.autograd.grad(out, (q, k, v), grad_out)
    qc, kc, vc, goc = _cpu(q, k, v, grad_out)
    assert_close(out, reference(qc, kc, vc, False, (40, 9), 0.3))
    for grad, eg in zip(grads, backward_reference(qc, kc, vc, goc, False, (40, 9), 0.3)):
        assert_close(grad, eg)

"""Host-side API contract on the CPU: the reference's signatures, defaults and exception
types (flash_attn.py:336-346, :435-490), the window mapping, and the torch.library ops'
shape functions (used by torch.compile) — no GPU needed."""

import inspect

import pytest
import torch

import myk_llm_amd
from myk_llm_amd import flash_attn as fa


def test_public_signatures_match_the_reference():
    """flash_attn.py:442-490: same parameters, order and defaults; the only addition is a
    keyword-only return_softmax_lse=False."""
    sig = inspect.signature(myk_llm_amd.flash_attn_func)
    assert list(sig.parameters)[:6] == ["q", "k", "v", "causal", "window_size", "softmax_scale"]
    assert sig.parameters["causal"].default is False
    assert sig.parameters["window_size"].default == (-1, -1)
    assert sig.parameters["softmax_scale"].default is None
    assert sig.parameters["return_softmax_lse"].kind is inspect.Parameter.KEYWORD_ONLY
    sig = inspect.signature(myk_llm_amd.flash_attn_varlen_func)
    assert list(sig.parameters)[:10] == ["q", "k", "v", "cu_seqlens_q", "cu_seqlens_k", "max_seqlen_q",
                                         "max_seqlen_k", "causal", "window_size", "softmax_scale"]
    sig = inspect.signature(myk_llm_amd.flash_attn_with_kvcache)
    assert list(sig.parameters)[:5] == ["q", "k_cache", "v_cache", "k", "v"]
    for name in ("cache_seqlens", "causal", "window_size", "softmax_scale", "return_softmax_lse"):
        assert sig.parameters[name].kind is inspect.Parameter.KEYWORD_ONLY
    assert sig.parameters["k"].default is None and sig.parameters["v"].default is None


def test_cpu_tensors_are_rejected_first():
    """flash_attn.py:338-339: the device check comes before the dtype / head_dim checks."""
    q = torch.randn(1, 8, 2, 48)
    with pytest.raises(RuntimeError, match="CUDA-only"):
        myk_llm_amd.flash_attn_func(q, q, q)
    with pytest.raises(RuntimeError, match="CUDA-only"):
        myk_llm_amd.flash_attn_varlen_func(q[0], q[0], q[0], None, None, 8, 8)


@pytest.mark.parametrize("qd, kd, qdim, kdim, qh, kh, exc, text", [
    (torch.float32, torch.float32, 64, 64, 4, 2, TypeError, "bf16"),
    (torch.bfloat16, torch.float16, 64, 64, 4, 2, TypeError, "bf16"),
    (torch.bfloat16, torch.bfloat16, 48, 48, 4, 2, ValueError, "head_dim"),
    (torch.bfloat16, torch.bfloat16, 64, 32, 4, 2, ValueError, "head_dim"),
    (torch.bfloat16, torch.bfloat16, 64, 64, 3, 2, ValueError, "multiple"),
    (torch.float16, torch.float16, 256, 256, 8, 8, None, None),
])
def test_dtype_headdim_ratio_checks(qd, kd, qdim, kdim, qh, kh, exc, text):
    q = torch.zeros(1, 4, qh, qdim, dtype=qd)
    k = torch.zeros(1, 4, kh, kdim, dtype=kd)
    if exc is None:
        fa._check_meta(q, k, k)
    else:
        with pytest.raises(exc, match=text):
            fa._check_meta(q, k, k)


@pytest.mark.parametrize("causal, window, expected", [
    (True, (-1, -1), (1 << 30, 0)),
    (False, (-1, -1), (1 << 30, 1 << 30)),
    (True, (63, 0), (63, 0)),
    (False, (31, 17), (31, 17)),
    (True, (31, 17), (31, 0)),  # causal forces window_right = 0
])
def test_window_mapping(causal, window, expected):
    """flash_attn.py:435-439."""
    assert fa._window(causal, window) == expected


def test_strides_helper():
    """(batch, token, head) in elements; batch = 0 for packed tensors (flash_attn.py:331-333)."""
    x = torch.zeros(2, 5, 3, 16)
    assert fa._strides(x) == (5 * 3 * 16, 3 * 16, 16)
    assert fa._strides(x[0]) == (0, 3 * 16, 16)


def test_custom_op_shape_functions():
    """The fake (meta) implementations give torch.compile the output shapes without a GPU."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(2, 7, 8, 64, dtype=torch.bfloat16)
        k = torch.empty(2, 9, 2, 64, dtype=torch.bfloat16)
        out, lse = torch.ops.mykfa.fwd(q, k, k, None, None, None, 7, 9, 0.125, 1 << 30, 0)
        assert out.shape == q.shape and out.dtype == q.dtype
        assert lse.shape == (8, 14) and lse.dtype == torch.float32
        qp = torch.empty(11, 8, 64, dtype=torch.bfloat16)
        cu = torch.empty(3, dtype=torch.int32)
        out, lse = torch.ops.mykfa.fwd(qp, qp[:, :2], qp[:, :2], cu, cu, None, 6, 6, 0.125, 1 << 30, 0)
        assert lse.shape == (8, 11)
        dq, dk, dv = torch.ops.mykfa.bwd(q, q, k, k, q, torch.empty(8, 14), None, None, 7, 9, 0.125, 1 << 30, 0)
        assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == k.shape


def test_device_and_dtype_guards_raise_on_the_host():
    """The guards run before any launch and need no GPU: a tensor on another device, or new
    keys of another dtype than the caches, raise."""
    from myk_llm_amd.flash_attn import _check_append, _same_device

    gpu = torch.device("cuda", 0)
    x = torch.zeros(4)
    _same_device(gpu, a=None)
    with pytest.raises(RuntimeError, match="same GPU"):
        _same_device(gpu, cu_seqlens_q=x)
    with pytest.raises(RuntimeError, match="cache_seqlens"):
        _same_device(gpu, k=None, cache_seqlens=x.int())
    cache = torch.zeros(1, 8, 2, 16, dtype=torch.bfloat16)
    new = torch.zeros(1, 1, 2, 16, dtype=torch.bfloat16)
    _check_append(cache, cache, new, new, torch.zeros(1, dtype=torch.int32))  # all on the host: consistent
    with pytest.raises(TypeError):
        _check_append(cache, cache, new.half(), new.half(), torch.zeros(1, dtype=torch.int32))
    with pytest.raises(TypeError):
        _check_append(cache, cache, new.float(), new, torch.zeros(1, dtype=torch.int32))


def test_ds_workspace_plan_caps_and_falls_back():
    """The backward's stored-dS workspace: as many KV heads per pass as the budget allows,
    capped by the device's available memory above a size threshold, halved on an allocation
    failure, and none (the recomputing backward) when even one head cannot be allocated."""
    import torch

    from myk_llm_amd.flash_attn import _DS_CHECK_FREE_ABOVE, _plan_ds_workspace

    got = []

    def alloc(n):
        got.append(n)
        return n

    per = 300 << 20
    assert _plan_ds_workspace(per, 4, 4 << 30, alloc) == (4, 4 * per)
    assert _plan_ds_workspace(per, 4, 2 * per + 5, alloc) == (2, 2 * per)
    assert _plan_ds_workspace(0, 4, 4 << 30, alloc) == (0, None)
    assert _plan_ds_workspace(per, 4, per - 1, alloc) == (0, None)
    # Available memory caps a large request at 80 %, but never below one head: the choice of
    # backward depends on the shape only.
    assert _plan_ds_workspace(per, 4, 4 << 30, alloc, lambda: 3 * per)[0] == 2
    assert _plan_ds_workspace(per, 4, 4 << 30, alloc, lambda: 0)[0] == 1
    # Small requests skip the query.
    small = _DS_CHECK_FREE_ABOVE // 4
    assert _plan_ds_workspace(small, 4, 4 << 30, alloc, lambda: 0)[0] == 4

    calls = []

    def oom_above(limit):
        def f(n):
            calls.append(n)
            if n > limit:
                raise torch.OutOfMemoryError("planted")
            return n
        return f

    assert _plan_ds_workspace(per, 4, 4 << 30, oom_above(per)) == (1, per)
    assert calls == [4 * per, 2 * per, per]
    calls.clear()
    assert _plan_ds_workspace(per, 4, 4 << 30, oom_above(0)) == (0, None)
    assert calls == [4 * per, 2 * per, per]

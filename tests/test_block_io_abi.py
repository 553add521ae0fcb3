"""Host-only validation of the prologue / epilogue entry points (csrc/api.hip): every
documented status code without touching a device (validation never dereferences)."""

import ctypes

import pytest

from myk_llm_amd import _lib


@pytest.fixture(scope="module")
def L():
    return _lib.lib()


def good_prologue(b=2, s=64, hq=8, hkv=2, d=64):
    p = _lib.QkPrologueParams()
    p.q_in = p.k_in = p.q_out = p.k_out = 0x10000
    w = (hq + 2 * hkv) * d  # views of a fused projection
    p.qi_batch_stride, p.qi_token_stride, p.qi_head_stride = s * w, w, d
    p.ki_batch_stride, p.ki_token_stride, p.ki_head_stride = s * w, w, d
    p.qo_batch_stride, p.qo_token_stride, p.qo_head_stride = s * hq * d, hq * d, d
    p.ko_batch_stride, p.ko_token_stride, p.ko_head_stride = s * hkv * d, hkv * d, d
    p.position_ids = 0x20000
    p.pos_batch_stride, p.pos_token_stride = 0, 1
    p.cos, p.sin = 0x30000, 0x40000
    p.table_stride, p.table_rows = d, 4096
    p.q_weight, p.k_weight = 0x50000, 0x60000
    p.eps = 1e-6
    p.batch, p.seqlen, p.num_heads, p.num_kv_heads, p.head_dim = b, s, hq, hkv, d
    p.dtype = _lib.DTYPE_BF16
    return p


def good_bwd():
    b = _lib.QkPrologueBwdParams()
    b.fwd = good_prologue()
    b.dq_out = b.dk_out = b.dq_in = b.dk_in = 0x70000
    for pre in ("dqo", "dqi"):
        setattr(b, f"{pre}_batch_stride", 64 * 8 * 64)
        setattr(b, f"{pre}_token_stride", 8 * 64)
        setattr(b, f"{pre}_head_stride", 64)
    for pre in ("dko", "dki"):
        setattr(b, f"{pre}_batch_stride", 64 * 2 * 64)
        setattr(b, f"{pre}_token_stride", 2 * 64)
        setattr(b, f"{pre}_head_stride", 64)
    b.dq_weight, b.dk_weight = 0x80000, 0x90000
    return b


def good_gate():
    g = _lib.GateParams()
    g.x = g.gate = g.y = g.dy = g.dx = g.dgate = 0x10000
    g.x_row_stride = g.gate_row_stride = g.y_row_stride = 1024
    g.dy_row_stride = g.dx_row_stride = g.dgate_row_stride = 1024
    g.rows, g.width, g.dtype = 100, 1024, _lib.DTYPE_BF16
    return g


def test_valid_params_pass(L):
    assert L.mykfa_validate_qk_prologue(ctypes.byref(good_prologue())) == _lib.OK
    assert L.mykfa_validate_qk_prologue_bwd(ctypes.byref(good_bwd())) == _lib.OK
    assert L.mykfa_validate_gate(ctypes.byref(good_gate()), 0) == _lib.OK
    assert L.mykfa_validate_gate(ctypes.byref(good_gate()), 1) == _lib.OK


@pytest.mark.parametrize("field,value,code,text", [
    ("dtype", 7, _lib.ERR_UNSUPPORTED, "bf16/fp16"),
    ("head_dim", 48, _lib.ERR_UNSUPPORTED, "head_dim"),
    ("q_in", 0, _lib.ERR_INVALID, "q_in is NULL"),
    ("k_out", 0x10008, _lib.ERR_INVALID, "16-byte aligned"),
    ("qi_token_stride", 100, _lib.ERR_INVALID, "multiples of 8"),
    ("k_weight", 0, _lib.ERR_INVALID, "both be given"),
    ("sin", 0, _lib.ERR_INVALID, "both be given"),
    ("position_ids", 0, _lib.ERR_INVALID, "position_ids is NULL"),
    ("position_ids", 0x20004, _lib.ERR_INVALID, "8-byte aligned"),
    ("table_rows", 0, _lib.ERR_INVALID, "table_rows"),
    ("table_stride", 32, _lib.ERR_INVALID, "table_stride"),
    ("table_stride", 66, _lib.ERR_INVALID, "table_stride"),
    ("eps", float("nan"), _lib.ERR_INVALID, "eps"),
    ("batch", -1, _lib.ERR_INVALID, "negative shape"),
])
def test_prologue_validation_errors(L, field, value, code, text):
    p = good_prologue()
    setattr(p, field, value)
    assert L.mykfa_validate_qk_prologue(ctypes.byref(p)) == code
    assert text in L.mykfa_last_error().decode()


def test_prologue_options_and_empty(L):
    p = good_prologue()
    p.q_weight = p.k_weight = 0  # no norm: eps unchecked
    p.eps = float("nan")
    assert L.mykfa_validate_qk_prologue(ctypes.byref(p)) == _lib.OK
    p = good_prologue()
    p.cos = p.sin = 0
    p.position_ids = 0  # no rope: positions unused
    assert L.mykfa_validate_qk_prologue(ctypes.byref(p)) == _lib.OK
    p = good_prologue()
    p.seqlen = 0
    p.q_in = 0  # nothing to do: pointers unchecked, and the call launches nothing
    assert L.mykfa_validate_qk_prologue(ctypes.byref(p)) == _lib.OK
    p.q_weight = p.k_weight = 0
    assert L.mykfa_qk_prologue_fwd(ctypes.byref(p), None) == _lib.OK


def test_prologue_bwd_validation(L):
    b = good_bwd()
    b.fwd.q_out = b.fwd.k_out = 0  # the backward ignores the forward's outputs
    assert L.mykfa_validate_qk_prologue_bwd(ctypes.byref(b)) == _lib.OK
    b = good_bwd()
    b.dk_weight = 0
    assert L.mykfa_validate_qk_prologue_bwd(ctypes.byref(b)) == _lib.ERR_INVALID
    assert "dq_weight and dk_weight" in L.mykfa_last_error().decode()
    b = good_bwd()
    b.dv_src = 0x10000
    assert L.mykfa_validate_qk_prologue_bwd(ctypes.byref(b)) == _lib.ERR_INVALID
    assert "dv_src and dv_dst" in L.mykfa_last_error().decode()
    b = good_bwd()
    b.dki_head_stride = 3
    assert L.mykfa_validate_qk_prologue_bwd(ctypes.byref(b)) == _lib.ERR_INVALID
    b = good_bwd()
    # a workspace smaller than any (2, D) partial is refused before any launch (the dummy
    # pointers are never dereferenced)
    assert L.mykfa_qk_prologue_bwd(ctypes.byref(b), 0x100000, 8, None) == _lib.ERR_WORKSPACE
    assert "workspace needs" in L.mykfa_last_error().decode()


def test_prologue_bwd_workspace_size(L):
    # one (2, D) fp32 partial per workgroup, at most 1024 workgroups; 0 for invalid shapes
    assert L.mykfa_qk_prologue_bwd_workspace_size(2, 64, 8, 2, 64) % (2 * 64 * 4) == 0
    assert L.mykfa_qk_prologue_bwd_workspace_size(64, 8192, 16, 4, 128) == 1024 * 2 * 128 * 4
    assert L.mykfa_qk_prologue_bwd_workspace_size(1, 1, 1, 1, 48) == 0
    assert L.mykfa_qk_prologue_bwd_workspace_size(0, 0, 8, 2, 64) == 2 * 64 * 4


@pytest.mark.parametrize("field,value,backward,text", [
    ("width", 12, 0, "multiple of 8"),
    ("width", 0, 0, "multiple of 8"),
    ("rows", -1, 0, "rows"),
    ("dtype", 3, 0, "bf16/fp16"),
    ("y", 0, 0, "y is NULL"),
    ("gate", 0x10004, 0, "16-byte aligned"),
    ("x_row_stride", 1020, 0, "multiples of 8"),
    ("dgate", 0, 1, "dgate is NULL"),
    ("dy_row_stride", 9, 1, "multiples of 8"),
])
def test_gate_validation_errors(L, field, value, backward, text):
    g = good_gate()
    setattr(g, field, value)
    code = L.mykfa_validate_gate(ctypes.byref(g), backward)
    assert code in (_lib.ERR_INVALID, _lib.ERR_UNSUPPORTED)
    assert text in L.mykfa_last_error().decode()


def test_gate_forward_ignores_backward_fields(L):
    g = good_gate()
    g.dy = g.dx = g.dgate = 0
    assert L.mykfa_validate_gate(ctypes.byref(g), 0) == _lib.OK
    g.rows = 0
    assert L.mykfa_gate_bwd(ctypes.byref(g), None) == _lib.OK  # no rows: nothing launched


def test_host_api_rejects_cpu_tensors_first():
    import torch

    from myk_llm_amd import block_io as bio

    x = torch.zeros(2, 4, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="CUDA-only"):
        bio.qk_norm_rope(x, x, None, None, None)
    with pytest.raises(RuntimeError, match="CUDA-only"):
        bio.qkv_norm_rope(torch.zeros(2, 4, 6 * 64, dtype=torch.bfloat16), 4, 1, 64, None, None, None)
    with pytest.raises(RuntimeError, match="CUDA-only"):
        bio.output_gate(x, x)
    with pytest.raises(ValueError, match="even"):
        bio.rope_tables(63, 8, 10000.0)
    cos, sin = bio.rope_tables(64, 8, 10000.0)
    assert cos.shape == (8, 64) and cos.dtype == torch.float32

"""The C-ABI library on the CPU: it loads without a GPU, exports every symbol include/mykfa.h
declares, its struct layouts match the ctypes mirror, and its host-only validation returns
each documented status code (flash_attn.py:336-346, :476-477) without touching a device."""

import ctypes
import re
from pathlib import Path

import pytest

from myk_llm_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "mykfa.h"


@pytest.fixture(scope="module")
def L():
    return _lib.lib()


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(mykfa_\w+)\s*\(", text, re.M)))


def test_every_declared_symbol_is_exported_and_bound(L):
    names = declared_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(L, name), f"{name} missing from libmykfa.so"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_version_and_struct_sizes(L):
    assert L.mykfa_abi_version() == _lib.ABI_VERSION == 7
    assert b"gfx950" in L.mykfa_version()
    assert L.mykfa_sizeof_fwd_params() == ctypes.sizeof(_lib.FwdParams)
    assert L.mykfa_sizeof_bwd_params() == ctypes.sizeof(_lib.BwdParams)
    assert L.mykfa_sizeof_decode_params() == ctypes.sizeof(_lib.DecodeParams)
    assert L.mykfa_sizeof_kv_append_params() == ctypes.sizeof(_lib.KvAppendParams)
    assert L.mykfa_sizeof_qk_prologue_params() == ctypes.sizeof(_lib.QkPrologueParams)
    assert L.mykfa_sizeof_qk_prologue_bwd_params() == ctypes.sizeof(_lib.QkPrologueBwdParams)
    assert L.mykfa_sizeof_gate_params() == ctypes.sizeof(_lib.GateParams)
    assert L.mykfa_sizeof_ce_params() == ctypes.sizeof(_lib.CeParams)
    assert L.mykfa_sizeof_syrk_params() == ctypes.sizeof(_lib.SyrkParams)


def good_fwd():
    p = _lib.FwdParams()
    p.q = p.k = p.v = p.o = p.lse = 0x10000  # aligned dummies: validation never dereferences
    p.q_batch_stride, p.q_token_stride, p.q_head_stride = 128 * 8 * 64, 8 * 64, 64
    p.k_batch_stride, p.k_token_stride, p.k_head_stride = 128 * 2 * 64, 2 * 64, 64
    p.v_batch_stride, p.v_token_stride, p.v_head_stride = 128 * 2 * 64, 2 * 64, 64
    p.o_batch_stride, p.o_token_stride, p.o_head_stride = 128 * 8 * 64, 8 * 64, 64
    p.lse_head_stride = 2 * 128
    p.batch, p.num_heads, p.num_kv_heads, p.head_dim = 2, 8, 2, 64
    p.max_seqlen_q = p.max_seqlen_k = 128
    p.window_left, p.window_right = _lib.UNBOUNDED, 0
    p.softmax_scale = 0.125
    p.dtype = _lib.DTYPE_BF16
    return p


def test_valid_forward_params_pass(L):
    assert L.mykfa_validate_fwd(ctypes.byref(good_fwd())) == _lib.OK
    assert L.mykfa_last_error() == b""


@pytest.mark.parametrize("field, value, code, text", [
    ("dtype", 7, _lib.ERR_UNSUPPORTED, b"bf16"),
    ("head_dim", 48, _lib.ERR_UNSUPPORTED, b"head_dim"),
    ("num_kv_heads", 3, _lib.ERR_INVALID, b"multiple"),
    ("num_heads", 0, _lib.ERR_INVALID, b"multiple"),
    ("batch", -1, _lib.ERR_INVALID, b"negative"),
    ("window_left", -1, _lib.ERR_INVALID, b"window"),
    ("q", 0, _lib.ERR_INVALID, b"q is NULL"),
    ("q", 0x10008, _lib.ERR_INVALID, b"16-byte aligned"),
    ("k_token_stride", 2 * 64 + 4, _lib.ERR_INVALID, b"multiples of 8"),
    ("lse", 0, _lib.ERR_INVALID, b"lse is NULL"),
    ("lse_head_stride", 10, _lib.ERR_INVALID, b"lse_head_stride"),
    ("softmax_scale", float("nan"), _lib.ERR_INVALID, b"NaN"),
])
def test_forward_validation_errors(L, field, value, code, text):
    p = good_fwd()
    setattr(p, field, value)
    assert L.mykfa_validate_fwd(ctypes.byref(p)) == code
    assert text in L.mykfa_last_error()
    # The launching entry point rejects the same input before any HIP call.
    assert L.mykfa_fwd(ctypes.byref(p), None) == code


def test_varlen_rules(L):
    p = good_fwd()
    p.cu_seqlens_q = 0x20000
    assert L.mykfa_validate_fwd(ctypes.byref(p)) == _lib.ERR_INVALID  # only one cu_seqlens
    p.cu_seqlens_k = 0x20000
    assert L.mykfa_validate_fwd(ctypes.byref(p)) == _lib.ERR_INVALID  # batch strides must be 0
    p.q_batch_stride = p.k_batch_stride = p.v_batch_stride = p.o_batch_stride = 0
    assert L.mykfa_validate_fwd(ctypes.byref(p)) == _lib.OK
    p.seqused_k = 0x30000
    assert L.mykfa_validate_fwd(ctypes.byref(p)) == _lib.ERR_INVALID


def test_empty_problems_succeed_without_a_device(L):
    p = good_fwd()
    p.batch = 0
    assert L.mykfa_fwd(ctypes.byref(p), None) == _lib.OK
    p = good_fwd()
    p.max_seqlen_q = 0
    assert L.mykfa_fwd(ctypes.byref(p), None) == _lib.OK


def test_backward_and_decode_validation(L):
    b = _lib.BwdParams()
    b.fwd = good_fwd()
    assert L.mykfa_validate_bwd(ctypes.byref(b)) == _lib.ERR_INVALID  # dout NULL
    b.dout = b.dq = b.dk = b.dv = b.delta = 0x40000
    for pre in ("do", "dq"):
        setattr(b, f"{pre}_batch_stride", 128 * 8 * 64)
        setattr(b, f"{pre}_token_stride", 8 * 64)
        setattr(b, f"{pre}_head_stride", 64)
    for pre in ("dk", "dv"):
        setattr(b, f"{pre}_batch_stride", 128 * 2 * 64)
        setattr(b, f"{pre}_token_stride", 2 * 64)
        setattr(b, f"{pre}_head_stride", 64)
    assert L.mykfa_validate_bwd(ctypes.byref(b)) == _lib.OK
    b.fwd.seqused_k = 0x50000
    assert L.mykfa_validate_bwd(ctypes.byref(b)) == _lib.ERR_INVALID

    d = _lib.DecodeParams()
    d.fwd = good_fwd()
    d.num_splits = 0
    assert L.mykfa_validate_decode(ctypes.byref(d)) == _lib.OK
    d.num_splits = 5000
    assert L.mykfa_validate_decode(ctypes.byref(d)) == _lib.ERR_INVALID
    d.num_splits = 4
    need = L.mykfa_decode_workspace_size(2, 8, 128, 64, 4)
    # 4 partial segments per sequence on average (O in the 16-bit input type, lse fp32), then
    # (first segment, splits) per sequence
    assert need == 4 * 2 * 8 * 128 * (64 * 2 + 4) + 2 * 2 * 4
    assert L.mykfa_decode_workspace_size(2, 8, 128, 64, 1) == 0  # one split writes o/lse directly
    assert L.mykfa_decode(ctypes.byref(d), None, 0, None) == _lib.ERR_WORKSPACE


def test_buffer_span_limits(L):
    """Rows of one (sequence, head) are addressed through a 32-bit buffer range: token strides
    above 2^24 elements and row spans above 2 GiB are rejected as unsupported."""
    p = good_fwd()
    p.k_token_stride = (1 << 24) + 8
    assert L.mykfa_validate_fwd(ctypes.byref(p)) == _lib.ERR_UNSUPPORTED
    assert b"2^24" in L.mykfa_last_error()
    p = good_fwd()
    p.k_token_stride, p.k_batch_stride = 1 << 20, (1 << 20) * 2048
    p.max_seqlen_k = 2048  # (2047 * 2^20 + 64) * 2 bytes > 2 GiB
    assert L.mykfa_validate_fwd(ctypes.byref(p)) == _lib.ERR_UNSUPPORTED
    assert b"2 GiB" in L.mykfa_last_error()
    p.max_seqlen_k = 1000  # (999 * 2^20 + 64) * 2 bytes < 2 GiB
    assert L.mykfa_validate_fwd(ctypes.byref(p)) == _lib.OK


def test_decode_new_key_rules(L):
    """seqlen_new counts keys after seqused_k[b]; k_new / v_new (both or neither) are written
    into the caches by the decode itself."""
    d = _lib.DecodeParams()
    d.fwd = good_fwd()
    d.seqlen_new = -1
    assert L.mykfa_validate_decode(ctypes.byref(d)) == _lib.ERR_INVALID
    d.seqlen_new = 4
    assert L.mykfa_validate_decode(ctypes.byref(d)) == _lib.ERR_INVALID  # needs seqused_k
    assert b"seqused_k" in L.mykfa_last_error()
    d.fwd.seqused_k = 0x60000
    assert L.mykfa_validate_decode(ctypes.byref(d)) == _lib.OK  # rows already appended
    d.k_new = 0x70000
    assert L.mykfa_validate_decode(ctypes.byref(d)) == _lib.ERR_INVALID  # v_new missing
    d.v_new = 0x80000
    d.kn_batch_stride, d.kn_token_stride, d.kn_head_stride = 4 * 2 * 64, 2 * 64, 64
    d.vn_batch_stride, d.vn_token_stride, d.vn_head_stride = 4 * 2 * 64, 2 * 64, 64
    assert L.mykfa_validate_decode(ctypes.byref(d)) == _lib.OK
    d.k_new = 0x70008
    assert L.mykfa_validate_decode(ctypes.byref(d)) == _lib.ERR_INVALID
    assert b"k_new" in L.mykfa_last_error()


def test_decode_split_heuristic(L):
    # Full 16K caches of a 64-sequence batch: ~1408 keys per split, 12 splits, for one query of
    # a 4-head group and for the 4-query draft alike.
    assert L.mykfa_decode_num_splits(64, 16, 4, 1, 16384) == 12
    assert L.mykfa_decode_num_splits(64, 16, 4, 4, 16384) == 12
    # Never a multiple of the 8 XCDs; short caches are not split; bounds hold.
    # 8 sequences fill the chip only at 64 splits, capped at 4096 / 128 keys = 32, bumped to 33.
    assert L.mykfa_decode_num_splits(8, 32, 4, 1, 4096) == 33
    assert L.mykfa_decode_num_splits(1, 1, 1, 1, 100) == 1
    for args in [(1, 8, 1, 1, 1 << 20), (512, 32, 8, 2, 4096), (64, 4, 4, 1, 256), (3, 64, 8, 16, 9000)]:
        s = L.mykfa_decode_num_splits(*args)
        assert 1 <= s <= 1024 and (s == 1 or s % 8 != 0)


def test_kv_append_validation(L):
    p = _lib.KvAppendParams()
    p.batch, p.seqlen_new, p.capacity, p.num_kv_heads, p.head_dim, p.dtype = 2, 1, 16, 2, 64, _lib.DTYPE_BF16
    assert L.mykfa_validate_kv_append(ctypes.byref(p)) == _lib.ERR_INVALID  # cache_seqlens NULL
    p.cache_seqlens = 0x1000
    assert L.mykfa_validate_kv_append(ctypes.byref(p)) == _lib.ERR_INVALID  # k_cache NULL
    p.k_cache = p.v_cache = p.k_new = p.v_new = 0x2000
    assert L.mykfa_validate_kv_append(ctypes.byref(p)) == _lib.OK
    p.head_dim = 40
    assert L.mykfa_validate_kv_append(ctypes.byref(p)) == _lib.ERR_UNSUPPORTED


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setenv("MYKFA_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(RuntimeError, match="no fallback"):
        _lib.lib()


def _bwd_params(head_dim, window_left=_lib.UNBOUNDED, window_right=0):
    """Valid dense backward params: batch 2, 128 tokens, 8 query / 2 key-value heads."""
    b = _lib.BwdParams()
    f = good_fwd()
    for t, h in (("q", 8), ("k", 2), ("v", 2), ("o", 8)):
        setattr(f, f"{t}_batch_stride", 128 * h * head_dim)
        setattr(f, f"{t}_token_stride", h * head_dim)
        setattr(f, f"{t}_head_stride", head_dim)
    f.head_dim = head_dim
    f.window_left, f.window_right = window_left, window_right
    b.fwd = f
    b.dout = b.dq = b.dk = b.dv = b.delta = 0x40000
    for pre, h in (("do", 8), ("dq", 8), ("dk", 2), ("dv", 2)):
        setattr(b, f"{pre}_batch_stride", 128 * h * head_dim)
        setattr(b, f"{pre}_token_stride", h * head_dim)
        setattr(b, f"{pre}_head_stride", head_dim)
    return b


def test_stored_ds_workspace_size(L):
    """mykfa_bwd_workspace_per_kv_head: one 2 KB dS block per (32-row query tile, key block its
    band touches) for each of a KV head's query heads (compact rows), plus 4 KB for the
    block-queue counters of the queued kernels. head_dim 128 only; 0 for other head dims and for
    invalid params."""
    b = _bwd_params(128)
    assert L.mykfa_validate_bwd(ctypes.byref(b)) == _lib.OK
    seqs, group, sched = 2, 4, 4096
    # Causal, unbounded left, 4 tiles per sequence: rows of 1, 2, 3, 4 blocks.
    assert L.mykfa_bwd_workspace_per_kv_head(ctypes.byref(b)) == group * seqs * 10 * 2048 + sched
    # A 31-key left window: rows of 1, 2, 2, 2 blocks (a tile's band reaches one block back).
    b = _bwd_params(128, 31, 0)
    assert L.mykfa_bwd_workspace_per_kv_head(ctypes.byref(b)) == group * seqs * 7 * 2048 + sched
    assert L.mykfa_bwd_workspace_per_kv_head(ctypes.byref(_bwd_params(64))) == 0
    b = _bwd_params(128)
    b.dout = 0
    assert L.mykfa_bwd_workspace_per_kv_head(ctypes.byref(b)) == 0


def test_stored_ds_halves_check_their_workspace(L):
    """mykfa_bwd_dkdv_ws / mykfa_bwd_dq_ws need every KV head's dS at once; both refuse a
    smaller workspace, and head_dim 64 (no stored-dS path), before anything is launched."""
    b = _bwd_params(128)
    need = 2 * L.mykfa_bwd_workspace_per_kv_head(ctypes.byref(b))
    for fn in (L.mykfa_bwd_dkdv_ws, L.mykfa_bwd_dq_ws):
        assert fn(ctypes.byref(b), 0x50000, need - 1, None) == _lib.ERR_WORKSPACE
        assert b"needed" in L.mykfa_last_error()
        assert fn(ctypes.byref(_bwd_params(64)), 0x50000, 1 << 30, None) == _lib.ERR_UNSUPPORTED


def test_stored_ds_entry_points_need_an_aligned_workspace(L):
    """dS blocks move as 16-byte chunks and the block-queue counters take device-scope atomics:
    mykfa_bwd_ws and both halves refuse a workspace that is not 16-byte aligned, on the host,
    before any launch."""
    b = _bwd_params(128)
    need = 2 * L.mykfa_bwd_workspace_per_kv_head(ctypes.byref(b))
    for fn in (L.mykfa_bwd_ws, L.mykfa_bwd_dkdv_ws, L.mykfa_bwd_dq_ws):
        assert fn(ctypes.byref(b), 0x50008, need, None) == _lib.ERR_INVALID
        assert b"aligned" in L.mykfa_last_error()

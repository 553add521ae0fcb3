"""ctypes binding of libmykfa.so (include/mykfa.h).

The structs below mirror the C parameter structs field for field; their sizes are checked
against the library's own sizeof() at load time. Loading fails loudly when the library
has not been built: there is no fallback implementation.
"""

from __future__ import annotations

import ctypes
import struct
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmykfa.so"
ABI_VERSION = 7  # MYKFA_ABI_VERSION

OK = 0
ERR_INVALID = 1
ERR_UNSUPPORTED = 2
ERR_LAUNCH = 3
ERR_WORKSPACE = 4
DECODE_SCRATCH_BYTES = 16 << 20  # MYKFA_DECODE_SCRATCH_BYTES

DTYPE_BF16 = 0
DTYPE_FP16 = 1
UNBOUNDED = 1 << 30

_i64, _i32, _f32, _ptr = ctypes.c_int64, ctypes.c_int32, ctypes.c_float, ctypes.c_void_p


class FwdParams(ctypes.Structure):
    _fields_ = [
        ("q", _ptr), ("k", _ptr), ("v", _ptr), ("o", _ptr), ("lse", _ptr),
        ("q_batch_stride", _i64), ("q_token_stride", _i64), ("q_head_stride", _i64),
        ("k_batch_stride", _i64), ("k_token_stride", _i64), ("k_head_stride", _i64),
        ("v_batch_stride", _i64), ("v_token_stride", _i64), ("v_head_stride", _i64),
        ("o_batch_stride", _i64), ("o_token_stride", _i64), ("o_head_stride", _i64),
        ("lse_head_stride", _i64),
        ("cu_seqlens_q", _ptr), ("cu_seqlens_k", _ptr), ("seqused_k", _ptr),
        ("batch", _i32), ("num_heads", _i32), ("num_kv_heads", _i32), ("head_dim", _i32),
        ("max_seqlen_q", _i32), ("max_seqlen_k", _i32),
        ("window_left", _i32), ("window_right", _i32),
        ("softmax_scale", _f32), ("dtype", _i32),
    ]


class BwdParams(ctypes.Structure):
    _fields_ = [
        ("fwd", FwdParams),
        ("dout", _ptr), ("dq", _ptr), ("dk", _ptr), ("dv", _ptr), ("delta", _ptr),
        ("do_batch_stride", _i64), ("do_token_stride", _i64), ("do_head_stride", _i64),
        ("dq_batch_stride", _i64), ("dq_token_stride", _i64), ("dq_head_stride", _i64),
        ("dk_batch_stride", _i64), ("dk_token_stride", _i64), ("dk_head_stride", _i64),
        ("dv_batch_stride", _i64), ("dv_token_stride", _i64), ("dv_head_stride", _i64),
    ]


class DecodeParams(ctypes.Structure):
    _fields_ = [
        ("fwd", FwdParams), ("num_splits", _i32), ("seqlen_new", _i32), ("k_new", _ptr), ("v_new", _ptr),
        ("kn_batch_stride", _i64), ("kn_token_stride", _i64), ("kn_head_stride", _i64),
        ("vn_batch_stride", _i64), ("vn_token_stride", _i64), ("vn_head_stride", _i64),
    ]


class KvAppendParams(ctypes.Structure):
    _fields_ = [
        ("k_cache", _ptr), ("v_cache", _ptr), ("k_new", _ptr), ("v_new", _ptr), ("cache_seqlens", _ptr),
        ("kc_batch_stride", _i64), ("kc_token_stride", _i64), ("kc_head_stride", _i64),
        ("vc_batch_stride", _i64), ("vc_token_stride", _i64), ("vc_head_stride", _i64),
        ("kn_batch_stride", _i64), ("kn_token_stride", _i64), ("kn_head_stride", _i64),
        ("vn_batch_stride", _i64), ("vn_token_stride", _i64), ("vn_head_stride", _i64),
        ("batch", _i32), ("seqlen_new", _i32), ("capacity", _i32), ("num_kv_heads", _i32),
        ("head_dim", _i32), ("dtype", _i32),
    ]


class QkPrologueParams(ctypes.Structure):
    _fields_ = [
        ("q_in", _ptr), ("k_in", _ptr), ("q_out", _ptr), ("k_out", _ptr),
        ("qi_batch_stride", _i64), ("qi_token_stride", _i64), ("qi_head_stride", _i64),
        ("ki_batch_stride", _i64), ("ki_token_stride", _i64), ("ki_head_stride", _i64),
        ("qo_batch_stride", _i64), ("qo_token_stride", _i64), ("qo_head_stride", _i64),
        ("ko_batch_stride", _i64), ("ko_token_stride", _i64), ("ko_head_stride", _i64),
        ("position_ids", _ptr), ("pos_batch_stride", _i64), ("pos_token_stride", _i64),
        ("cos", _ptr), ("sin", _ptr), ("table_stride", _i64), ("table_rows", _i32),
        ("q_weight", _ptr), ("k_weight", _ptr), ("eps", _f32),
        ("batch", _i32), ("seqlen", _i32), ("num_heads", _i32), ("num_kv_heads", _i32),
        ("head_dim", _i32), ("dtype", _i32),
    ]


class QkPrologueBwdParams(ctypes.Structure):
    _fields_ = [
        ("fwd", QkPrologueParams),
        ("dq_out", _ptr), ("dk_out", _ptr), ("dq_in", _ptr), ("dk_in", _ptr),
        ("dqo_batch_stride", _i64), ("dqo_token_stride", _i64), ("dqo_head_stride", _i64),
        ("dko_batch_stride", _i64), ("dko_token_stride", _i64), ("dko_head_stride", _i64),
        ("dqi_batch_stride", _i64), ("dqi_token_stride", _i64), ("dqi_head_stride", _i64),
        ("dki_batch_stride", _i64), ("dki_token_stride", _i64), ("dki_head_stride", _i64),
        ("dv_src", _ptr), ("dv_dst", _ptr),
        ("dvs_batch_stride", _i64), ("dvs_token_stride", _i64), ("dvs_head_stride", _i64),
        ("dvd_batch_stride", _i64), ("dvd_token_stride", _i64), ("dvd_head_stride", _i64),
        ("dq_weight", _ptr), ("dk_weight", _ptr),
    ]


class GateParams(ctypes.Structure):
    _fields_ = [
        ("x", _ptr), ("gate", _ptr), ("y", _ptr), ("dy", _ptr), ("dx", _ptr), ("dgate", _ptr),
        ("x_row_stride", _i64), ("gate_row_stride", _i64), ("y_row_stride", _i64),
        ("dy_row_stride", _i64), ("dx_row_stride", _i64), ("dgate_row_stride", _i64),
        ("rows", _i64), ("width", _i32), ("dtype", _i32),
    ]


class CeParams(ctypes.Structure):
    _fields_ = [
        ("logits", _ptr), ("targets", _ptr), ("ce", _ptr), ("lse", _ptr),
        ("row_stride", _i64), ("rows", _i64), ("vocab", _i32), ("ignore_index", _i32),
        ("scale", _f32), ("z_coef", _f32), ("dtype", _i32),
    ]


class SyrkParams(ctypes.Structure):
    _fields_ = [
        ("x", _ptr), ("bias", _ptr), ("out", _ptr),
        ("x_batch_stride", _i64), ("x_row_stride", _i64),
        ("bias_batch_stride", _i64), ("bias_row_stride", _i64),
        ("out_batch_stride", _i64), ("out_row_stride", _i64),
        ("batch", _i32), ("m", _i32), ("k", _i32), ("alpha", _f32), ("beta", _f32), ("dtype", _i32),
    ]


# Every symbol include/mykfa.h declares, with (restype, argtypes).
SIGNATURES = {
    "mykfa_abi_version": (ctypes.c_int, []),
    "mykfa_version": (ctypes.c_char_p, []),
    "mykfa_last_error": (ctypes.c_char_p, []),
    "mykfa_sizeof_fwd_params": (ctypes.c_size_t, []),
    "mykfa_sizeof_bwd_params": (ctypes.c_size_t, []),
    "mykfa_sizeof_decode_params": (ctypes.c_size_t, []),
    "mykfa_sizeof_kv_append_params": (ctypes.c_size_t, []),
    "mykfa_validate_fwd": (ctypes.c_int, [ctypes.POINTER(FwdParams)]),
    "mykfa_validate_bwd": (ctypes.c_int, [ctypes.POINTER(BwdParams)]),
    "mykfa_validate_decode": (ctypes.c_int, [ctypes.POINTER(DecodeParams)]),
    "mykfa_validate_kv_append": (ctypes.c_int, [ctypes.POINTER(KvAppendParams)]),
    "mykfa_fwd": (ctypes.c_int, [ctypes.POINTER(FwdParams), _ptr]),
    "mykfa_bwd_preprocess": (ctypes.c_int, [ctypes.POINTER(BwdParams), _ptr]),
    "mykfa_bwd_dkdv": (ctypes.c_int, [ctypes.POINTER(BwdParams), _ptr]),
    "mykfa_bwd_dq": (ctypes.c_int, [ctypes.POINTER(BwdParams), _ptr]),
    "mykfa_bwd": (ctypes.c_int, [ctypes.POINTER(BwdParams), _ptr]),
    "mykfa_bwd_workspace_per_kv_head": (ctypes.c_size_t, [ctypes.POINTER(BwdParams)]),
    "mykfa_bwd_ws": (ctypes.c_int, [ctypes.POINTER(BwdParams), _ptr, ctypes.c_size_t, _ptr]),
    "mykfa_bwd_dkdv_ws": (ctypes.c_int, [ctypes.POINTER(BwdParams), _ptr, ctypes.c_size_t, _ptr]),
    "mykfa_bwd_dq_ws": (ctypes.c_int, [ctypes.POINTER(BwdParams), _ptr, ctypes.c_size_t, _ptr]),
    "mykfa_decode_num_splits": (ctypes.c_int, [_i32, _i32, _i32, _i32, _i32]),
    "mykfa_decode_workspace_size": (ctypes.c_size_t, [_i32, _i32, _i32, _i32, _i32]),
    "mykfa_decode_splitk": (ctypes.c_int, [ctypes.POINTER(DecodeParams), _ptr, ctypes.c_size_t, _ptr]),
    "mykfa_decode_merge": (ctypes.c_int, [ctypes.POINTER(DecodeParams), _ptr, ctypes.c_size_t, _ptr]),
    "mykfa_decode": (ctypes.c_int, [ctypes.POINTER(DecodeParams), _ptr, ctypes.c_size_t, _ptr]),
    "mykfa_decode_noalloc": (ctypes.c_int, [ctypes.POINTER(DecodeParams), _ptr]),
    "mykfa_kv_append": (ctypes.c_int, [ctypes.POINTER(KvAppendParams), _ptr]),
    "mykfa_sizeof_qk_prologue_params": (ctypes.c_size_t, []),
    "mykfa_sizeof_qk_prologue_bwd_params": (ctypes.c_size_t, []),
    "mykfa_sizeof_gate_params": (ctypes.c_size_t, []),
    "mykfa_validate_qk_prologue": (ctypes.c_int, [ctypes.POINTER(QkPrologueParams)]),
    "mykfa_validate_qk_prologue_bwd": (ctypes.c_int, [ctypes.POINTER(QkPrologueBwdParams)]),
    "mykfa_validate_gate": (ctypes.c_int, [ctypes.POINTER(GateParams), ctypes.c_int]),
    "mykfa_qk_prologue_fwd": (ctypes.c_int, [ctypes.POINTER(QkPrologueParams), _ptr]),
    "mykfa_qk_prologue_bwd_workspace_size": (ctypes.c_size_t, [_i32, _i32, _i32, _i32, _i32]),
    "mykfa_qk_prologue_bwd": (ctypes.c_int, [ctypes.POINTER(QkPrologueBwdParams), _ptr, ctypes.c_size_t, _ptr]),
    "mykfa_gate_fwd": (ctypes.c_int, [ctypes.POINTER(GateParams), _ptr]),
    "mykfa_gate_bwd": (ctypes.c_int, [ctypes.POINTER(GateParams), _ptr]),
    "mykfa_sizeof_ce_params": (ctypes.c_size_t, []),
    "mykfa_validate_ce": (ctypes.c_int, [ctypes.POINTER(CeParams)]),
    "mykfa_ce_rows": (ctypes.c_int, [ctypes.POINTER(CeParams), _ptr]),
    "mykfa_sizeof_syrk_params": (ctypes.c_size_t, []),
    "mykfa_validate_syrk": (ctypes.c_int, [ctypes.POINTER(SyrkParams)]),
    "mykfa_syrk": (ctypes.c_int, [ctypes.POINTER(SyrkParams), _ptr]),
}

_STRUCT_SIZES = {
    "mykfa_sizeof_fwd_params": FwdParams,
    "mykfa_sizeof_bwd_params": BwdParams,
    "mykfa_sizeof_decode_params": DecodeParams,
    "mykfa_sizeof_kv_append_params": KvAppendParams,
    "mykfa_sizeof_qk_prologue_params": QkPrologueParams,
    "mykfa_sizeof_qk_prologue_bwd_params": QkPrologueBwdParams,
    "mykfa_sizeof_gate_params": GateParams,
    "mykfa_sizeof_ce_params": CeParams,
    "mykfa_sizeof_syrk_params": SyrkParams,
}

def _flat_layout(struct_type, base: int = 0, out=None):
    """(offset, struct code) of every scalar field of a (possibly nested) ctypes struct."""
    out = [] if out is None else out
    codes = {_ptr: "Q", _i64: "q", _i32: "i", _f32: "f"}
    for name, ftype in struct_type._fields_:
        off = base + getattr(struct_type, name).offset
        if ftype in codes:
            out.append((off, codes[ftype]))
        else:
            _flat_layout(ftype, off, out)
    return out


def _packer(struct_type) -> struct.Struct:
    """A struct.Struct that writes every field of struct_type, in declaration order, at its
    ctypes offset (pad bytes where the C layout has them): filling a parameter block with one
    pack_into call costs ~1 us where ~30 ctypes attribute stores cost ~8 us, which matters on
    the eager path of small calls. NULL pointers are passed as 0."""
    fmt, pos = "<", 0
    for off, code in _flat_layout(struct_type):
        if off < pos:
            raise RuntimeError(f"{struct_type.__name__}: overlapping fields")
        fmt += "x" * (off - pos) + code
        pos = off + struct.calcsize("<" + code)
    fmt += "x" * (ctypes.sizeof(struct_type) - pos)
    s = struct.Struct(fmt)
    assert s.size == ctypes.sizeof(struct_type)
    return s


FWD_PACK = _packer(FwdParams)
BWD_PACK = _packer(BwdParams)
DECODE_PACK = _packer(DecodeParams)


_lib: ctypes.CDLL | None = None


class MykfaError(RuntimeError):
    """A libmykfa call returned a non-zero status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"mykfa error {code}: {message}")
        self.code = code


def lib() -> ctypes.CDLL:
    """The loaded library; raises if libmykfa.so was not built (no fallback path exists)."""
    global _lib
    if _lib is not None:
        return _lib
    path = os.environ.get("MYKFA_LIB", str(LIB_PATH))
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: the gfx950 FlashAttention library must be built first "
            "(python -m myk_llm_amd.build); there is no fallback implementation")
    handle = ctypes.CDLL(path)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if handle.mykfa_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI version {handle.mykfa_abi_version()} != {ABI_VERSION}")
    for name, struct in _STRUCT_SIZES.items():
        size = getattr(handle, name)()
        if size != ctypes.sizeof(struct):
            raise RuntimeError(f"{path}: {struct.__name__} is {size} bytes in C, {ctypes.sizeof(struct)} here")
    _lib = handle
    return handle


def check(code: int) -> None:
    if code != OK:
        raise MykfaError(code, lib().mykfa_last_error().decode())

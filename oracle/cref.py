"""ctypes wrapper of oracle/attn_ref.c (float64 brute force) — TEST INFRASTRUCTURE ONLY.

Builds libattn_ref.so with the Makefile beside it on first use when it is missing.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libattn_ref.so"
UNBOUNDED = 1 << 30

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def _load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        dp = ctypes.POINTER(ctypes.c_double)
        lib.attn_ref.restype = ctypes.c_int
        lib.attn_ref.argtypes = [ctypes.c_int] * 8 + [ctypes.c_double] + [dp] * 9
        _lib = lib
    return _lib


def _p(a):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def attn_ref(q, k, v, dout=None, *, window_left=UNBOUNDED, window_right=UNBOUNDED, scale=None):
    """q (B, Lq, H, D), k/v (B, Lk, Hkv, D) array-likes; window sides already resolved (ints,
    UNBOUNDED for none). Returns dict with o, lse2 (H, B*Lq) and, with dout, dq/dk/dv, float64."""
    q, k, v = (np.ascontiguousarray(np.asarray(x, dtype=np.float64)) for x in (q, k, v))
    B, Lq, H, D = q.shape
    Lk, Hkv = k.shape[1], k.shape[2]
    scale = 1.0 / np.sqrt(D) if scale is None else float(scale)
    o = np.zeros((B, Lq, H, D))
    lse2 = np.zeros((H, B * Lq))
    res = {"o": o, "lse2": lse2}
    dq = dk = dv = None
    if dout is not None:
        dout = np.ascontiguousarray(np.asarray(dout, dtype=np.float64))
        dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
        res.update(dq=dq, dk=dk, dv=dv)
    rc = _load().attn_ref(B, Lq, Lk, H, Hkv, D, int(window_left), int(window_right), scale, _p(q), _p(k), _p(v),
                          _p(dout), _p(o), _p(lse2), _p(dq), _p(dk), _p(dv))
    if rc != 0:
        raise RuntimeError(f"attn_ref failed with {rc}")
    return res

"""Regenerate tests/golden/*.npz: small seeded attention cases with forward and backward
results computed by the float64 brute force in oracle/attn_ref.c (not by the reference,
which ships no fixtures for this path).

    python tests/golden/make_fixtures.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle.cref import UNBOUNDED, attn_ref  # noqa: E402

# name: (B, Lq, Lk, H, Hkv, D, window_left, window_right) with resolved windows.
CASES = {
    "causal_gqa": (2, 24, 24, 4, 2, 16, UNBOUNDED, 0),
    "window_tail": (1, 9, 33, 4, 1, 32, 7, 0),
    "bidir_asym": (1, 17, 21, 2, 2, 16, 5, 3),
    "more_queries": (1, 30, 12, 2, 1, 16, UNBOUNDED, 0),
}


def main():
    for name, (b, lq, lk, h, hk, d, wl, wr) in CASES.items():
        rng = np.random.default_rng(sum(map(ord, name)))
        q = rng.standard_normal((b, lq, h, d)).astype(np.float32)
        k = rng.standard_normal((b, lk, hk, d)).astype(np.float32)
        v = rng.standard_normal((b, lk, hk, d)).astype(np.float32)
        do = rng.standard_normal((b, lq, h, d)).astype(np.float32)
        r = attn_ref(q, k, v, do, window_left=wl, window_right=wr)
        np.savez_compressed(Path(__file__).parent / f"{name}.npz", q=q, k=k, v=v, dout=do,
                            window=np.array([wl, wr], dtype=np.int64), o=r["o"], lse2=r["lse2"], dq=r["dq"],
                            dk=r["dk"], dv=r["dv"])
        print(f"{name}: written")


if __name__ == "__main__":
    main()

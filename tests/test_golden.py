"""The torch oracle reproduces the committed float64 fixtures (tests/golden/*.npz, written
by tests/golden/make_fixtures.py from the C brute force): forward O, base-2 LSE and the
three gradients."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as A

GOLDEN = sorted((Path(__file__).parent / "golden").glob("*.npz"))


@pytest.mark.parametrize("path", GOLDEN, ids=[p.stem for p in GOLDEN])
def test_oracle_reproduces_golden(path):
    f = np.load(path)
    q, k, v, do = (torch.from_numpy(f[n]) for n in ("q", "k", "v", "dout"))
    wl, wr = (int(x) for x in f["window"])
    window = (wl if wl < A.UNBOUNDED else -1, wr if wr < A.UNBOUNDED else -1)
    o, lse = A.reference_with_lse(q, k, v, False, window)
    np.testing.assert_allclose(o.numpy(), f["o"], rtol=0, atol=3e-5)
    inf = np.isinf(f["lse2"])
    assert np.array_equal(np.isinf(lse.numpy()), inf)
    np.testing.assert_allclose(lse.numpy()[~inf], f["lse2"][~inf], rtol=0, atol=3e-5)
    grads = A.backward_reference(q, k, v, do, False, window)
    for g, n in zip(grads, ("dq", "dk", "dv")):
        np.testing.assert_allclose(g.numpy(), f[n], rtol=0, atol=1e-4)


def test_fixtures_exist():
    assert len(GOLDEN) >= 4

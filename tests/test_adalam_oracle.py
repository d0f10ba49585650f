# SPDX-License-Identifier: Unlicense
"""CPU: the oracle's restatement of AdaLAM's nearest-neighbour search
(adalam.c:38-116) pinned against float64 numpy: the first argmin of the
squared distance (np.argmin's rule), the ratio of the two smallest
(np.partition's second element, so a tie gives ratio 1), the second
clamped to 1e-3, and the column argmin. Ties and the empty and
one-column cases are built so that each rule decides the answer."""

import ctypes as C

import numpy as np
import pytest

from oracle_lib import fp, ip


def nearest(orc, d1, d2, with21=True):
    n1, dim = d1.shape
    n2 = d2.shape[0]
    nn12, sc = np.full(max(n1, 1), -1, np.int32), np.zeros(max(n1, 1), np.float32)
    nn21 = np.full(max(n2, 1), -1, np.int32) if with21 else None
    orc.orc_adalam_nearest(fp(np.ascontiguousarray(d1)), n1, fp(np.ascontiguousarray(d2)), n2,
                           dim, ip(nn12), fp(sc), ip(nn21) if with21 else None)
    return nn12[:n1], sc[:n1], (nn21[:n2] if with21 else None)


def unit_rows(rng, n, dim):
    x = rng.standard_normal((n, dim))
    return (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)


def dist64(d1, d2):
    a, b = d1.astype(np.float64), d2.astype(np.float64)
    return (a * a).sum(1)[:, None] + (b * b).sum(1)[None] - 2 * a @ b.T


@pytest.mark.parametrize("n1,n2,dim", [(300, 257, 128), (64, 1000, 37), (5, 3, 3)])
def test_nearest_vs_float64(orc, n1, n2, dim):
    rng = np.random.default_rng(n1 + n2 + dim)
    d1, d2 = unit_rows(rng, n1, dim), unit_rows(rng, n2, dim)
    nn12, sc, nn21 = nearest(orc, d1, d2)
    D = dist64(d1, d2)
    part = np.partition(D, 1, axis=1)
    sure = part[:, 1] - part[:, 0] > 1e-5
    assert sure.mean() > 0.9
    assert np.array_equal(nn12[sure], D.argmin(1)[sure])
    ref = part[:, 0] / np.maximum(part[:, 1], 1e-3)
    assert np.abs(sc - ref).max() < 1e-5 * np.maximum(1, 1 / np.maximum(part[:, 1], 1e-3)).max()
    cp = np.partition(D, 1, axis=0)
    csure = cp[1] - cp[0] > 1e-5
    assert np.array_equal(nn21[csure], D.argmin(0)[csure])
    a12, s12, none = nearest(orc, d1, d2, with21=False)
    assert none is None and np.array_equal(a12, nn12) and np.array_equal(s12, sc)


def test_nearest_ties_take_the_first_index(orc):
    """Bit-identical rows give bit-identical distances: the first index
    wins both searches and the ratio of a tied pair is exactly 1."""
    rng = np.random.default_rng(3)
    d2 = unit_rows(rng, 40, 128)
    d2[29] = d2[7]
    d1 = unit_rows(rng, 30, 128)
    d1[4] = (d2[7] + 0.3 * unit_rows(rng, 1, 128)[0]).astype(np.float32)
    d1[21] = d1[4]
    nn12, sc, nn21 = nearest(orc, d1, d2)
    assert nn12[4] == 7 and nn12[21] == 7
    assert sc[4] == 1.0 and sc[21] == 1.0
    assert nn21[7] == 4 and nn21[29] == 4


def test_nearest_clamp_and_degenerate_sizes(orc):
    rng = np.random.default_rng(5)
    d2 = unit_rows(rng, 10, 16)
    d1 = np.ascontiguousarray(d2[[3, 8]])
    # An exact copy: best is rounding noise, the ratio uses the 1e-3 clamp
    # only when the second distance is below it (it is not here).
    nn12, sc, _ = nearest(orc, d1, d2)
    assert list(nn12) == [3, 8] and np.all(np.abs(sc) < 1e-5)
    # Two near-copies closer than 1e-3: the ratio divides by 1e-3.
    e = np.zeros(16, np.float32)
    e[0] = 1
    near = np.stack([e, e + np.float32(1e-2) * np.eye(16, dtype=np.float32)[1]])
    nn12, sc, _ = nearest(orc, e[None], near.astype(np.float32))
    D = dist64(e[None], near)[0]
    assert nn12[0] == 0 and D[1] < 1e-3
    assert abs(sc[0] - max(D[0], 0) / 1e-3) < 1e-4
    # One column: the second distance stays FLT_MAX.
    nn12, sc, nn21 = nearest(orc, d1, d2[:1])
    assert list(nn12) == [0, 0] and np.all(sc < 1e-37) and nn21[0] in (0, 1)
    # No columns: index 0 and FLT_MAX / FLT_MAX = 1.
    nn12, sc, nn21 = nearest(orc, d1, np.zeros((0, 16), np.float32))
    assert list(nn12) == [0, 0] and list(sc) == [1.0, 1.0] and len(nn21) == 0
    # No rows: every column points at row 0.
    _, _, nn21 = nearest(orc, np.zeros((0, 16), np.float32), d2)
    assert list(nn21) == [0] * 10

# SPDX-License-Identifier: Unlicense
"""GPU: AdaLAM's nearest-neighbour search (adalam_nearest, the device form
of adalam.c:38-116) against the oracle's restatement of the host loop.

The device sums the dot products in another order than the host loop,
so distances differ by float32 rounding (about 1e-7 for unit
descriptors). Indices are compared bit for bit wherever the two smallest
float64 distances differ by more than 1e-4 (2.5e-5 of the largest
possible distance, 4; the north star's bar is 1e-3), and at least 98 %
of the rows and columns must be such. Lowe's ratio: within
2e-5 / max(second, 1e-3) + 1e-6 absolute. Exact duplicates must tie
exactly: first index, ratio 1."""

import ctypes as C

import numpy as np
import pytest

from oracle_lib import fp, ip

pytestmark = pytest.mark.gpu

MARGIN = 1e-4


def unit_rows(rng, n, dim):
    x = rng.standard_normal((n, dim))
    return (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)


def oracle(orc, d1, d2):
    n1, dim = d1.shape
    n2 = d2.shape[0]
    nn12, sc = np.zeros(max(n1, 1), np.int32), np.zeros(max(n1, 1), np.float32)
    nn21 = np.zeros(max(n2, 1), np.int32)
    orc.orc_adalam_nearest(fp(d1), n1, fp(d2), n2, dim, ip(nn12), fp(sc), ip(nn21))
    return nn12[:n1], sc[:n1], nn21[:n2]


def device(dev, d1, d2, with21=True):
    n1, dim = d1.shape
    n2 = d2.shape[0]
    b1 = dev.upload(d1) if d1.size else dev.zeros(1)
    b2 = dev.upload(d2) if d2.size else dev.zeros(1)
    bi = dev.upload(np.full(max(n1, 1), -5, np.int32))
    bs = dev.upload(np.full(max(n1, 1), -1, np.float32))
    bj = dev.upload(np.full(max(n2, 1), -5, np.int32)) if with21 else None
    work = dev.alloc(int(dev.api.adalam_nearest_work_bytes(n1, n2)) + 256)
    dev.api.adalam_nearest(dev.po, b1.mem, n1, b2.mem, n2, dim, bi.mem, bs.mem,
                           bj.mem if bj else None, work.mem)
    nn12 = dev.read(bi, max(n1, 1), np.int32)[:n1]
    sc = dev.read(bs, max(n1, 1))[:n1]
    nn21 = dev.read(bj, max(n2, 1), np.int32)[:n2] if bj else None
    return nn12, sc, nn21


def margins(d1, d2):
    a, b = d1.astype(np.float64), d2.astype(np.float64)
    D = (a * a).sum(1)[:, None] + (b * b).sum(1)[None] - 2 * a @ b.T
    rp = np.partition(D, 1, axis=1) if D.shape[1] > 1 else np.concatenate(
        [D, np.full_like(D, np.inf)], 1)
    cp = np.partition(D, 1, axis=0) if D.shape[0] > 1 else np.concatenate(
        [D, np.full_like(D, np.inf)], 0)
    return rp[:, 1] - rp[:, 0], rp[:, 1], cp[1] - cp[0]


@pytest.mark.parametrize("n1,n2,dim,near", [(2048, 2048, 128, 0.0), (2048, 2048, 128, 0.05),
                                            (300, 257, 128, 0.0), (64, 1000, 37, 0.0),
                                            (1000, 65, 200, 0.0), (65, 1000, 200, 0.1),
                                            (5, 3, 3, 0.0),
                                            (1, 1, 128, 0.0), (129, 1, 16, 0.0)])
def test_nearest_vs_oracle(dev, ic, orc, n1, n2, dim, near):
    """near > 0: d1 holds noisy copies of distinct rows of d2 (the
    matched-keypoint case: small best distances and ratios), else
    independent rows."""
    print(f"[adalam] nearest {n1}x{n2} dim={dim} near={near}", flush=True)
    rng = np.random.default_rng(n1 * 7 + n2 + dim)
    d2 = unit_rows(rng, n2, dim)
    if near:
        src = d2[rng.permutation(n2)[:n1]]
        d1 = src + near * unit_rows(rng, n1, dim)
        d1 = (d1 / np.linalg.norm(d1, axis=1, keepdims=True)).astype(np.float32)
    else:
        d1 = unit_rows(rng, n1, dim)
    o12, osc, o21 = oracle(orc, d1, d2)
    g12, gsc, g21 = device(dev, d1, d2)
    rm, second, cm = margins(d1, d2)
    sure, csure = rm > MARGIN, cm > MARGIN
    assert sure.mean() >= 0.98 and csure.mean() >= 0.98
    assert np.array_equal(g12[sure], o12[sure])
    assert np.array_equal(g21[csure], o21[csure])
    tol = 2e-5 / np.maximum(second, 1e-3) + 1e-6
    assert np.all(np.abs(gsc.astype(np.float64) - osc) <= tol)
    assert ((g12 >= 0) & (g12 < n2)).all() and ((g21 >= 0) & (g21 < n1)).all()
    # Without nn21 the row results are the same launch's.
    h12, hsc, none = device(dev, d1, d2, with21=False)
    assert none is None and np.array_equal(h12, g12) and np.array_equal(hsc, gsc)


def test_nearest_ties_and_empty_sets(dev, ic, orc):
    rng = np.random.default_rng(3)
    d2 = unit_rows(rng, 140, 128)
    d2[129] = d2[7]
    d1 = unit_rows(rng, 70, 128)
    d1[4] = (d2[7] + 0.3 * unit_rows(rng, 1, 128)[0]).astype(np.float32)
    d1[66] = d1[4]
    g12, gsc, g21 = device(dev, d1, d2)
    assert g12[4] == 7 and g12[66] == 7
    assert gsc[4] == 1.0 and gsc[66] == 1.0
    assert g21[7] == 4 and g21[129] == 4
    # No columns: index 0 and ratio FLT_MAX / FLT_MAX = 1; no rows: 0.
    g12, gsc, g21 = device(dev, d1, np.zeros((0, 128), np.float32))
    assert (g12 == 0).all() and (gsc == 1.0).all() and len(g21) == 0
    g12, gsc, g21 = device(dev, np.zeros((0, 128), np.float32), d2)
    assert len(g12) == 0 and (g21 == 0).all()


def test_nearest_host_entry(dev, ic, orc):
    """adalam_nearest_host, the drop-in for nearest(), gives the device
    form's results from host arrays."""
    rng = np.random.default_rng(11)
    d1, d2 = unit_rows(rng, 333, 128), unit_rows(rng, 517, 128)
    g12, gsc, g21 = device(dev, d1, d2)
    h12, hsc = np.zeros(333, np.int32), np.zeros(333, np.float32)
    h21 = np.zeros(517, np.int32)
    dev.api.adalam_nearest_host(dev.po, d1.ctypes.data, 333, d2.ctypes.data, 517, 128,
                                h12.ctypes.data, hsc.ctypes.data, h21.ctypes.data)
    assert np.array_equal(h12, g12) and np.array_equal(hsc, gsc) and np.array_equal(h21, g21)
    h12b = np.zeros(333, np.int32)
    dev.api.adalam_nearest_host(dev.po, d1.ctypes.data, 333, d2.ctypes.data, 517, 128,
                                h12b.ctypes.data, hsc.ctypes.data, None)
    assert np.array_equal(h12b, g12)


def test_nearest_rejects_short_buffers(dev, ic):
    b = dev.zeros(16)
    with pytest.raises(ic.IcoregError, match="d2"):
        dev.api.adalam_nearest(dev.po, b.mem, 1, b.mem, 2, 16, b.mem, b.mem, None,
                               dev.alloc(4096).mem)

# SPDX-License-Identifier: Unlicense
"""CPU: the oracle's DISK (disk_kernels.cl and the disk.c schedule)
pinned against float64 torch statements (disk_ref.py): the U-Net through
F.conv2d / F.instance_norm / F.prelu / F.avg_pool2d / F.interpolate, the
strict 5 x 5 NMS through F.unfold, the top-n through torch.topk and the
descriptors through F.normalize."""

import ctypes as C
import sys
from pathlib import Path

import numpy as np
import pytest

import disk_ref as R
from oracle_lib import disk_detect, fp, ip, oracle

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "i.coregistration.opencl_amd"))
import synth  # noqa: E402


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


@pytest.mark.parametrize("h,w,thresh", [(40, 52, -np.inf), (33, 20, 0.3)])
def test_nms(orc, h, w, thresh):
    import ctypes as C
    rng = np.random.default_rng(h * w)
    W = w + 7
    heat = rng.standard_normal((h, W)).astype(np.float32)
    heat[10, 10:13] = 5.0          # a plateau: no strict maximum
    mask = np.zeros(h * w, np.uint8)
    orc.orc_disk_nms5x5(fp(heat), W, h, w, np.float32(thresh),
                        mask.ctypes.data_as(C.POINTER(C.c_ubyte)))
    ref = R.nms_mask(heat[:, :w], thresh)
    assert np.array_equal(mask.reshape(h, w).astype(bool), ref)
    assert not ref[10, 10:13].any()


def test_gather(orc):
    rng = np.random.default_rng(9)
    H, W, n = 12, 17, 30
    feat = rng.standard_normal((129, H, W)).astype(np.float32)
    feat[:128, 3, 4] = 0.0         # zero descriptor: eps path
    xy = np.stack([rng.integers(0, W, n), rng.integers(0, H, n)], 1).astype(np.int32)
    xy[0] = (4, 3)
    out = np.zeros((n, 128), np.float32)
    orc.orc_disk_gather_desc(fp(feat), H, W, 128, ip(np.ascontiguousarray(xy)), n, fp(out))
    assert rel(out, R.gather(feat, xy)) < 1e-6
    assert not out[0].any()


@pytest.fixture(scope="module")
def weights():
    return synth.disk_weights()


@pytest.mark.parametrize("H,W,h,w,n,valid", [(64, 64, 64, 64, 50, False),
                                             (96, 128, 90, 100, 2048, True)])
def test_detect(weights, H, W, h, w, n, valid):
    img = synth.disk_image(H, W)
    img[:, h:, :] = 0
    img[:, :, w:] = 0
    v = None
    if valid:
        v = np.ones((h, w), np.uint8)
        v[:20, :30] = 0
    o = disk_detect(weights, img, h, w, n, 0.0, v, full=True)
    out = R.unet(weights, img)
    assert rel(o["out"], out) < 1e-4
    heat = o["out"][128, :h, :w]
    mask = R.nms_mask(heat, 0.0)
    xy = R.select(heat, mask, n, v)
    assert o["n"] == len(xy) and o["n"] > 0
    assert np.array_equal(o["xy"], xy)
    assert np.array_equal(o["score"], heat[xy[:, 1], xy[:, 0]])
    assert rel(o["desc"], R.gather(o["out"], xy)) < 1e-5


def _bruteforce_topn(heat, mask, valid, n):
    """The kept cells by counting, not sorting: with more than n
    candidates a candidate v is kept iff at most n candidates are >= v
    (it is then above the (n+1)-th highest); with n or fewer, iff it is
    above the lowest candidate. Raster order, at most n."""
    m = mask.astype(bool) & (valid.astype(bool) if valid is not None else True)
    ys, xs = np.nonzero(m)
    v = heat[ys, xs].astype(np.float64)
    if len(v) == 0 or n == 0:
        return np.zeros((0, 2), np.int32)
    if len(v) > n:
        keep = np.array([(v >= x).sum() <= n for x in v])
    else:
        keep = v > v.min()
    return np.stack([xs[keep], ys[keep]], 1).astype(np.int32)[:n]


@pytest.mark.parametrize("seed,n,levels,use_valid", [(1, 50, 0, False), (2, 50, 7, False),
                                                     (3, 3, 4, True), (4, 1000, 5, False),
                                                     (5, 0, 0, False), (6, 1, 2, True)])
def test_topn_matches_counting_rule(orc, seed, n, levels, use_valid):
    """orc_disk_topn (disk.c:228-253, qsort and cut) against the counting
    statement of the same rule, with ties at the cut (heat values
    quantised to a few levels), fewer candidates than n, n = 0, a valid
    mask."""
    rng = np.random.default_rng(seed)
    h, w, W = 37, 45, 48
    heat = rng.standard_normal((h, W)).astype(np.float32)
    if levels:
        heat = np.round(heat * levels / 3).astype(np.float32)
    mask = (rng.uniform(size=(h, w)) < 0.15).astype(np.uint8)
    valid = (rng.uniform(size=(h, w)) < 0.7).astype(np.uint8) if use_valid else None
    xy = np.zeros((max(n, 1), 2), np.int32)
    sc = np.zeros(max(n, 1), np.float32)
    up = lambda a: a.ctypes.data_as(C.POINTER(C.c_ubyte)) if a is not None else None
    nk = orc.orc_disk_topn(fp(heat), W, h, w, up(mask), up(valid), n, ip(xy), fp(sc))
    want = _bruteforce_topn(heat[:, :w], mask, valid, n)
    assert nk == len(want)
    assert np.array_equal(xy[:nk], want)
    assert np.array_equal(sc[:nk], heat[want[:, 1], want[:, 0]])

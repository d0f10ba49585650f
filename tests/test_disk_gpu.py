# SPDX-License-Identifier: Unlicense
"""GPU: DISK's kernels and detector on the HIP library against the oracle.

Tolerances: the U-Net output <= 1e-3 of its largest
magnitude; descriptors <= 1e-3; the NMS mask and the kept keypoint set
bit-exact on identical inputs, and on the network's own heatmaps wherever
the oracle's decision margin (a cell against its largest neighbour, a
candidate against the top-n cut) exceeds 1e-3 of the heatmap's scale.
At the config's 512 x 512 size: size-independent properties (strict
local maxima on the device heatmap, raster order, unit descriptors)."""

import ctypes as C
import sys
from pathlib import Path

import numpy as np
import pytest

import disk_ref as R
from oracle_lib import disk_detect, fp, ip

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "i.coregistration.opencl_amd"))
import synth  # noqa: E402

TOL = 1e-3


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


@pytest.mark.parametrize("h,w,W,thresh", [(40, 52, 64, -np.inf), (333, 517, 520, 0.2),
                                          (3, 4, 4, 0.0)])
def test_nms_kernel(dev, ic, orc, h, w, W, thresh):
    print(f"[disk] nms {h}x{w} W={W}", flush=True)
    rng = np.random.default_rng(h + w)
    off = 100
    heat = rng.standard_normal(off + h * W).astype(np.float32)
    plane = heat[off:].reshape(h, W)
    if h > 12 and w > 14:
        plane[10, 10:13] = 9.0
    ref = np.zeros(h * w, np.uint8)
    orc.orc_disk_nms5x5(fp(np.ascontiguousarray(plane)), W, h, w, np.float32(thresh),
                        ref.ctypes.data_as(C.POINTER(C.c_ubyte)))
    bh, bm = dev.upload(heat), dev.zeros((h * w + 3) // 4)
    dev.api.disk_nms5x5(dev.po, bh.mem, off, W, h, w, float(thresh), bm.mem)
    got = dev.read(bm, h * w, np.uint8)
    assert np.array_equal(got, ref)


def test_gather_kernel(dev, ic, orc):
    rng = np.random.default_rng(4)
    H, W, n = 50, 70, 777
    feat = rng.standard_normal((129, H, W)).astype(np.float32)
    xy = np.ascontiguousarray(np.stack([rng.integers(0, W, n), rng.integers(0, H, n)], 1)
                              .astype(np.int32))
    ref = np.zeros((n, 128), np.float32)
    orc.orc_disk_gather_desc(fp(feat), H, W, 128, ip(xy), n, fp(ref))
    bf, bx, bd = dev.upload(feat), dev.upload(xy), dev.zeros(n * 128)
    dev.api.disk_gather_desc(dev.po, bf.mem, H, W, 128, bx.mem, n, bd.mem)
    assert rel(dev.read(bd).reshape(n, 128), ref) < 1e-6


def test_gather_rejects_outside_keypoint(dev, ic):
    feat, xy, d = dev.zeros(129 * 4 * 4), dev.upload(np.array([1, 1, 4, 0], np.int32)), \
        dev.zeros(2 * 128)
    with pytest.raises(ic.IcoregError, match="outside"):
        dev.api.disk_gather_desc(dev.po, feat.mem, 4, 4, 128, xy.mem, 2, d.mem)


@pytest.fixture(scope="module")
def weights(tmp_path_factory):
    p = tmp_path_factory.mktemp("disk") / "disk_random.safetensors"
    return synth.disk_weights_file(p), synth.disk_weights()


def _unsure(heat, thresh, n, valid):
    """Cells whose NMS or top-n decision the oracle takes by less than TOL
    of the heatmap's scale."""
    h, w = heat.shape
    sc = np.abs(heat).max()
    x = np.pad(heat.astype(np.float64), 2, constant_values=-np.inf)
    nb = np.full((h, w), -np.inf)
    for dy in range(5):
        for dx in range(5):
            if dy != 2 or dx != 2:
                nb = np.maximum(nb, x[dy:dy + h, dx:dx + w])
    unsure = (np.abs(heat - nb) < TOL * sc) | (np.abs(heat - thresh) < TOL * sc)
    mask = R.nms_mask(heat, thresh)
    if valid is not None:
        mask &= valid.astype(bool)
    cand = np.sort(heat[mask])[::-1]
    if len(cand):
        cut = cand[min(n, len(cand) - 1)]
        unsure |= mask & (np.abs(heat - cut) < TOL * sc)
    return unsure


@pytest.mark.parametrize("H,W,h,w,n,valid", [(128, 128, 128, 128, 300, False),
                                             (96, 160, 90, 150, 2048, True)])
def test_detect_vs_oracle(dev, ic, weights, H, W, h, w, n, valid):
    print(f"[disk] detect {H}x{W} crop {h}x{w} n={n}", flush=True)
    fpath, wd = weights
    img = synth.disk_image(H, W)
    img[:, h:, :] = 0
    img[:, :, w:] = 0
    v = None
    if valid:
        v = np.ones((h, w), np.uint8)
        v[:20, :30] = 0
    o = disk_detect(wd, img, h, w, n, 0.0, v, full=True)
    net = ic.Disk(dev, fpath, H, W, nmax=2048)
    try:
        g = net.detect(img, h, w, n, 0.0, v)
        out = net.buffer("out", 129 * H * W).reshape(129, H, W)
    finally:
        net.close()
    assert rel(out, o["out"]) < TOL
    heat = o["out"][128, :h, :w]
    unsure = _unsure(heat, 0.0, n, v)
    sg = {tuple(p) for p in g["xy"]}
    so = {tuple(p) for p in o["xy"]}
    for x, y in sg ^ so:
        assert unsure[y, x], (x, y)
    assert len(sg ^ so) <= 0.01 * max(len(so), 1)
    common = sorted(sg & so, key=lambda p: (p[1], p[0]))
    gi = {tuple(p): i for i, p in enumerate(g["xy"])}
    oi = {tuple(p): i for i, p in enumerate(o["xy"])}
    gd = np.array([g["desc"][gi[p]] for p in common])
    od = np.array([o["desc"][oi[p]] for p in common])
    assert rel(gd, od) < TOL
    assert list(map(tuple, g["xy"])) == sorted(map(tuple, g["xy"]), key=lambda p: (p[1], p[0]))


def test_detect_512_properties(dev, ic, weights):
    """The DISK config (512 x 512, n = 2048): every kept keypoint is a
    strict 5 x 5 maximum of the device's own heatmap above thresh and off
    the 2-cell border, the n highest such cells are kept in raster order,
    descriptors have unit norm and equal the normalised channels 0..127."""
    print("[disk] detect 512 properties", flush=True)
    fpath, _ = weights
    img = synth.disk_image(512, 512)
    net = ic.Disk(dev, fpath, 512, 512, nmax=2048)
    try:
        g = net.detect(img, n=2048, thresh=0.0)
        out = net.buffer("out", 129 * 512 * 512).reshape(129, 512, 512)
    finally:
        net.close()
    heat = out[128]
    mask = R.nms_mask(heat, 0.0)
    xy = R.select(heat, mask, 2048)
    assert g["n"] == len(xy) == 2048
    assert np.array_equal(g["xy"], xy)
    assert np.array_equal(g["score"], heat[xy[:, 1], xy[:, 0]])
    assert np.abs(np.linalg.norm(g["desc"], axis=1) - 1).max() < 1e-5
    assert rel(g["desc"], R.gather(out, xy)) < 1e-5


def test_detect_from_torch_checkpoint(dev, ic, weights, tmp_path):
    """The same weights in a torch.save zip archive, held under
    "extractor" as DISK's published checkpoint holds them, give the same
    keypoints, scores and descriptors bit for bit as the safetensors load."""
    print("[disk] detect from a torch.save checkpoint", flush=True)
    fpath, wd = weights
    pth = synth.save_torch(wd, tmp_path / "disk-save.pth", wrap="extractor")
    img = synth.disk_image(128, 128)
    out = []
    for p in (fpath, pth):
        net = ic.Disk(dev, p, 128, 128, nmax=512)
        try:
            out.append(net.detect(img, n=512, thresh=0.0))
        finally:
            net.close()
    a, b = out
    assert a["n"] == b["n"] > 0
    for k in ("xy", "score", "desc"):
        assert np.array_equal(a[k], b[k]), k


@pytest.mark.parametrize("h,w,W,n,levels,use_valid", [
    (37, 45, 48, 50, 0, False), (37, 45, 48, 50, 7, False), (37, 45, 48, 3, 4, True),
    (37, 45, 48, 1000, 5, False), (37, 45, 48, 0, 0, False), (64, 64, 64, 1, 2, True),
    (512, 512, 512, 2048, 0, False), (1024, 1000, 1024, 2048, 9, True),
    (1024, 1000, 1024, 2048, 0, True)])
def test_topn_kernel(dev, ic, orc, h, w, W, n, levels, use_valid):
    """disk_topn (the device's top-n: radix select of the cut, raster
    compaction) bit-exact against the host rule of disk.c:228-253 (the
    oracle), with ties at the cut, a valid mask, more or fewer candidates
    than n, and n = 0."""
    print(f"[disk] topn {h}x{w} W={W} n={n} levels={levels} valid={use_valid}", flush=True)
    rng = np.random.default_rng(h + n + levels)
    off = 64
    heat = rng.standard_normal(off + h * W).astype(np.float32)
    if levels:
        heat = np.round(heat * levels / 3).astype(np.float32)
    plane = np.ascontiguousarray(heat[off:].reshape(h, W))
    mask = (rng.uniform(size=(h, w)) < 0.05).astype(np.uint8)
    valid = (rng.uniform(size=(h, w)) < 0.7).astype(np.uint8) if use_valid else None
    cap = max(n, 1)
    xy_o, sc_o = np.zeros(2 * cap, np.int32), np.zeros(cap, np.float32)
    up = lambda a: a.ctypes.data_as(C.POINTER(C.c_ubyte)) if a is not None else None
    nk_o = orc.orc_disk_topn(fp(plane), W, h, w, up(mask), up(valid), n, ip(xy_o), fp(sc_o))
    bh, bm = dev.upload(heat), dev.upload(mask)
    bv = dev.upload(valid) if valid is not None else None
    bxy, bsc = dev.upload(np.full(2 * cap, -7, np.int32)), dev.zeros(cap)
    bcnt = dev.upload(np.full(1, -1, np.int32))
    work = dev.alloc(int(dev.api.disk_topn_work_bytes(h, w)))
    dev.api.disk_topn(dev.po, bh.mem, off, W, h, w, bm.mem, bv.mem if bv else None, n,
                      bxy.mem, bsc.mem, bcnt.mem, work.mem)
    nk = int(dev.read(bcnt, 1, np.int32)[0])
    assert nk == nk_o
    assert np.array_equal(dev.read(bxy, 2 * cap, np.int32)[:2 * nk], xy_o[:2 * nk])
    assert np.array_equal(dev.read(bsc, cap)[:nk], sc_o[:nk])
    # Continuous scores have no ties at the cut, so exactly n survive;
    # quantised ones lose the tied cut level (v > cut, disk.c:246).
    if n >= 2000 and levels == 0:
        assert nk == n
    assert nk <= n

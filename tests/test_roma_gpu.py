# SPDX-License-Identifier: Unlicense
"""GPU: RoMa's kernels (roma_kernels.cl contracts) on the HIP library
against the oracle on the same float32 inputs. Tolerance 1e-5 of the
largest reference magnitude (2e-5 where the sum runs over 1024 channels),
cls_to_flow's certainty copied bit-exact; edge cases: warps on the
border, far outside, a million cells off and non-finite, modes on the
anchor grid's corners and ties, ragged tiles, the largest channel count
and radius."""

import numpy as np
import pytest

from oracle_lib import fp

pytestmark = pytest.mark.gpu

TOL = 1e-5


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


def warps(rng, H, W):
    gy = -1 + (2 * np.arange(H) + 1) / H
    gx = -1 + (2 * np.arange(W) + 1) / W
    gy, gx = np.meshgrid(gy, gx, indexing="ij")
    f = np.stack([gx, gy]) + 0.3 * rng.standard_normal((2, H, W))
    flat = f.reshape(2, -1)
    k = rng.choice(H * W, 40, replace=False)
    flat[:, k[:10]] *= 3.0
    flat[0, k[10:15]] = 1.0
    flat[1, k[15:20]] = -1.0
    flat[0, k[20]] = 1e6
    flat[1, k[21]] = -3e9
    flat[0, k[22]] = np.nan
    flat[1, k[23]] = np.inf
    flat[0, k[24]] = -np.inf
    return np.ascontiguousarray(f.astype(np.float32))


def smooth_warps(rng, H, W, outliers=True):
    """A smooth warp (the identity plus a displacement of a few cells
    varying slowly over the grid), as the refiners see, with a sprinkle
    of broken cells (far off, non-finite) so that some 4 x 4 patches
    scatter."""
    gy = -1 + (2 * np.arange(H) + 1) / H
    gx = -1 + (2 * np.arange(W) + 1) / W
    gy, gx = np.meshgrid(gy, gx, indexing="ij")
    ph = rng.uniform(0, 2 * np.pi, 4)
    dx = 3.0 / W * (np.sin(2.1 * gy + ph[0]) + np.cos(1.7 * gx + ph[1]))
    dy = 3.0 / H * (np.sin(1.3 * gx + ph[2]) + np.cos(2.5 * gy + ph[3]))
    f = np.stack([gx + dx, gy + dy]) + 0.1 / max(H, W) * rng.standard_normal((2, H, W))
    if outliers:
        flat = f.reshape(2, -1)
        k = rng.choice(H * W, 12, replace=False)
        flat[:, k[:4]] *= 3.0
        flat[0, k[4]] = 1e6
        flat[1, k[5]] = np.nan
        flat[0, k[6]] = -np.inf
        flat[:, k[7:12]] = rng.uniform(-1, 1, (2, 5))
    return np.ascontiguousarray(f.astype(np.float32))


def test_row_norm_cos_exp(dev, ic, orc):
    print("[roma] row_norm / cos_exp", flush=True)
    rng = np.random.default_rng(31)
    N, M, C = 1000, 777, 512
    X = rng.standard_normal((N, C)).astype(np.float32)
    Y = rng.standard_normal((M, C)).astype(np.float32)
    nx, ny = np.zeros(N, np.float32), np.zeros(M, np.float32)
    orc.orc_roma_row_norm(fp(X), N, C, fp(nx))
    orc.orc_roma_row_norm(fp(Y), M, C, fp(ny))
    S = np.ascontiguousarray(X @ Y.T / 8)
    Sref = S.copy()
    orc.orc_roma_cos_exp(fp(Sref), fp(nx), fp(ny), N, M, 0.2, 1e-6)
    bx, by, bnx, bny, bS = (dev.upload(X), dev.upload(Y), dev.zeros(N), dev.zeros(M),
                            dev.upload(S))
    a, m = dev.api, ic.mem
    a.roma_row_norm(dev.po, m(bx), N, C, m(bnx))
    a.roma_row_norm(dev.po, m(by), M, C, m(bny))
    a.roma_cos_exp(dev.po, m(bS), m(bnx), m(bny), N, M, 0.2, 1e-6)
    assert rel(dev.read(bnx), nx) < TOL
    assert rel(dev.read(bny), ny) < TOL
    assert rel(dev.read(bS), Sref) < 1e-4


@pytest.mark.parametrize("res,n", [(64, 700), (8, 33)])
def test_cls_to_flow(dev, ic, orc, res, n):
    print(f"[roma] cls_to_flow res={res} n={n}", flush=True)
    rng = np.random.default_rng(res)
    C = res * res
    ld = C + 1
    L = (2 * rng.standard_normal((n, ld))).astype(np.float32)
    for t, idx in enumerate([[0], [C - 1], [res - 1], [C - res], [5, 9], [C - 2, 1]]):
        L[t, :C] = -5
        L[t, idx] = 9
    flow, cert = np.zeros(2 * n, np.float32), np.zeros(n, np.float32)
    orc.orc_roma_cls_to_flow(fp(L), ld, C, res, n, fp(flow), fp(cert))
    bL, bf, bc = dev.upload(L), dev.zeros(2 * n), dev.zeros(n)
    dev.api.roma_cls_to_flow(dev.po, bL.mem, ld, C, res, n, bf.mem, bc.mem)
    assert rel(dev.read(bf), flow) < TOL
    assert np.array_equal(dev.read(bc), cert)


@pytest.mark.parametrize("C,H,W,smooth", [(3, 37, 45, False), (64, 70, 70, False),
                                          (13, 31, 17, True), (512, 108, 108, True),
                                          (9, 432, 432, True), (1, 29, 33, True),
                                          (16, 40, 52, False), (17, 23, 31, True)])
def test_warp_sample(dev, ic, orc, C, H, W, smooth):
    print(f"[roma] warp_sample C={C} {H}x{W}", flush=True)
    rng = np.random.default_rng(C)
    x = rng.standard_normal((C, H, W)).astype(np.float32)
    f = smooth_warps(rng, H, W) if smooth else warps(rng, H, W)
    n = H * W
    ref = np.zeros((C + 1, n), np.float32)
    orc.orc_roma_warp_sample(fp(x), C, H, W, fp(f), fp(ref), 1)
    bx, bf = dev.upload(x), dev.upload(f)
    out = dev.upload(np.full((C + 1, n), 7.0, np.float32))
    dev.api.roma_warp_sample(dev.po, bx.mem, C, H, W, bf.mem, out.mem, 1)
    got = dev.read(out).reshape(C + 1, n)
    assert np.all(got[0] == 7.0)
    # The element-wise bar (1e-4): the pixel coordinate ((x + 1) W - 1) / 2
    # is rounded differently where the compiler fuses its multiply-add
    # (the oracle's x86 build does not), about 1 ulp of a coordinate of
    # up to 432, which moves a sample by its gradient times that.
    assert rel(got[1:], ref[1:]) < 1e-4


@pytest.mark.parametrize("C,H,W,r,smooth", [(512, 35, 35, 7, False), (1024, 20, 27, 3, False),
                                            (256, 70, 70, 2, False), (24, 9, 13, 7, False),
                                            (512, 35, 37, 3, True), (100, 23, 30, 2, True),
                                            (7, 13, 9, 1, True), (64, 21, 19, 7, True),
                                            (512, 108, 108, 3, True), (256, 216, 216, 2, True),
                                            (37, 20, 22, 3, False), (192, 64, 64, 3, False),
                                            (40, 36, 44, 4, True), (64, 33, 46, 3, True),
                                            (16, 8, 12, 1, False), (512, 108, 108, 3, False),
                                            (36, 17, 28, 2, True), (128, 216, 216, 2, False),
                                            (64, 38, 44, 3, True), (96, 30, 40, 2, True),
                                            (32, 26, 28, 1, True), (1024, 24, 24, 3, True),
                                            (512, 64, 64, 7, True), (48, 128, 128, 1, True),
                                            (64, 40, 52, 2, False), (61, 31, 45, 2, True)])
def test_local_corr(dev, ic, orc, C, H, W, r, smooth):
    """Random warps (most 4 x 4 patches scatter: the per-cell path) and
    smooth ones (the matrix-core path over the patch's window box, with a
    few broken cells), up to the refiner config's 1/8 and 1/4 shapes at
    864 x 864, radius 1 to 7; channel counts that are multiples of 4 (the
    cell-major form, f2 transposed first) and others (channel-major
    reads). Multiples of 32 channels on maps whose width is a multiple of
    4 take the staged form for boxes of up to 144 cells (the 1/8 and 1/4
    shapes, a map whose last patch row is cut, radius 1, 1024 channels).
    Radius 7 on a smooth warp at 64 x 64 (the first refiner's radius and
    channels, on the coarse grid) gives boxes of 19 x 19 cells: the
    matrix-core path's 25-tile limit. 48
    channels at radius 1 (roma_v2ref's 1/2 refiner), and 64 and 61 channels
    at radius 2 on random and smooth warps."""
    print(f"[roma] local_corr C={C} {H}x{W} r={r} smooth={smooth}", flush=True)
    rng = np.random.default_rng(C + r)
    f0 = rng.standard_normal((C, H, W)).astype(np.float32)
    f1 = rng.standard_normal((C, H, W)).astype(np.float32)
    f = smooth_warps(rng, H, W) if smooth else warps(rng, H, W)
    n, K = H * W, (2 * r + 1) ** 2
    ref = np.zeros((K + 2, n), np.float32)
    orc.orc_roma_local_corr(fp(f0), fp(f1), C, H, W, r, fp(f), fp(ref), 2)
    b0, b1, bf = dev.upload(f0), dev.upload(f1), dev.upload(f)
    out = dev.upload(np.full((K + 2, n), 7.0, np.float32))
    dev.api.roma_local_corr(dev.po, b0.mem, b1.mem, C, H, W, r, bf.mem, out.mem, 2)
    got = dev.read(out).reshape(K + 2, n)
    assert np.all(got[:2] == 7.0)
    assert rel(got[2:], ref[2:]) < 2e-5


def test_disp_updates(dev, ic, orc):
    print("[roma] disp / update / update2", flush=True)
    rng = np.random.default_rng(41)
    H, W = 70, 93
    n = H * W
    flow = rng.uniform(-1, 1, (2, n)).astype(np.float32)
    a, m = dev.api, ic.mem
    ref = np.zeros((2, n), np.float32)
    orc.orc_roma_disp(fp(flow), H, W, 35.0, 17.5, fp(ref))
    bflow, bd = dev.upload(flow), dev.zeros(2 * n)
    a.roma_disp(dev.po, m(bflow), H, W, 35.0, 17.5, m(bd))
    assert rel(dev.read(bd), ref) < TOL

    d = (4 * rng.standard_normal((6, n))).astype(np.float32)
    d[3, :6] = [25.0, -30.0, 0.0, 19.9, 20.1, -90.0]
    cert = rng.standard_normal(n).astype(np.float32)
    rf, rc = flow.copy(), cert.copy()
    orc.orc_roma_update(fp(rf), fp(rc), fp(d), n, 0.5, 280.0, 210.0)
    bf, bc, bdd = dev.upload(flow), dev.upload(cert), dev.upload(d)
    a.roma_update(dev.po, m(bf), m(bc), m(bdd), n, 0.5, 280.0, 210.0)
    assert rel(dev.read(bf), rf) < TOL
    assert rel(dev.read(bc), rc) < TOL

    conf = rng.standard_normal((4, n)).astype(np.float32)
    rf2, rc2 = flow.copy(), conf.copy()
    orc.orc_roma2_update(fp(rf2), fp(rc2), fp(d), n, 93.0, 70.0)
    bf2, bc2 = dev.upload(flow), dev.upload(conf)
    a.roma2_update(dev.po, m(bf2), m(bc2), m(bdd), n, 93.0, 70.0)
    assert rel(dev.read(bf2), rf2) < TOL
    assert rel(dev.read(bc2), rc2) < TOL


@pytest.mark.parametrize("C,H,W", [(5, 37, 70), (64, 140, 140), (2, 3, 4), (9, 108, 108)])
def test_dwconv5(dev, ic, orc, C, H, W):
    print(f"[roma] dwconv5 C={C} {H}x{W}", flush=True)
    rng = np.random.default_rng(C * H)
    x = rng.standard_normal((C, H, W)).astype(np.float32)
    w = rng.standard_normal((C, 25)).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32)
    ref = np.zeros((C, H, W), np.float32)
    orc.orc_roma_dwconv5(fp(x), C, H, W, fp(w), fp(b), fp(ref))
    bx, bw, bb, bo = dev.upload(x), dev.upload(w), dev.upload(b), dev.zeros(C * H * W)
    dev.api.roma_dwconv5(dev.po, bx.mem, C, H, W, bw.mem, bb.mem, bo.mem)
    assert rel(dev.read(bo), ref) < TOL


@pytest.mark.parametrize("C,H,W", [(24, 108, 108), (32, 70, 97), (8, 9, 65), (16, 1, 3)])
def test_dwpw_small(dev, ic, orc, C, H, W):
    """The fused refiner block (roma_dwpw_small) against the oracle's
    depthwise 5 x 5 followed by the 1 x 1 in float64 (numpy), and against
    the library's own two-kernel path (roma_dwconv5, ops_conv1x1)."""
    print(f"[roma] dwpw_small C={C} {H}x{W}", flush=True)
    rng = np.random.default_rng(C * H + W)
    x = rng.standard_normal((C, H, W)).astype(np.float32)
    w = rng.standard_normal((C, 25)).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32)
    pw = (rng.standard_normal((C, C)) / np.sqrt(C)).astype(np.float32)
    pb = rng.standard_normal(C).astype(np.float32)
    z = np.zeros((C, H, W), np.float32)
    orc.orc_roma_dwconv5(fp(x), C, H, W, fp(w), fp(b), fp(z))
    ref = (pw.astype(np.float64) @ z.reshape(C, -1).astype(np.float64)
           + pb.astype(np.float64)[:, None]).reshape(C, H, W)
    bx, bw, bb = dev.upload(x), dev.upload(w), dev.upload(b)
    bpw, bpb, bo = dev.upload(pw), dev.upload(pb), dev.zeros(C * H * W)
    dev.api.roma_dwpw_small(dev.po, bx.mem, C, H, W, bw.mem, bb.mem, bpw.mem, bpb.mem, bo.mem)
    got = dev.read(bo).reshape(C, H, W)
    assert rel(got, ref) < TOL
    bz, b2 = dev.zeros(C * H * W), dev.zeros(C * H * W)
    dev.api.roma_dwconv5(dev.po, bx.mem, C, H, W, bw.mem, bb.mem, bz.mem)
    dev.api.ops_conv1x1(dev.po, bz.mem, 0, C, H * W, bpw.mem, bpb.mem, C, b2.mem, 0, 0, 0.0)
    assert rel(got, dev.read(b2).reshape(C, H, W)) < TOL


@pytest.mark.parametrize("H,W,h,w,nimg,imagenet", [
    (1024, 1024, 560, 560, 2, 1), (864, 864, 560, 560, 2, 1), (640, 480, 560, 560, 1, 0),
    (64, 64, 112, 112, 2, 1), (100, 70, 56, 84, 1, 1), (2048, 1000, 140, 112, 1, 0),
    (64, 96, 64, 96, 2, 1), (37, 45, 37, 45, 1, 0)])
def test_prepare_vs_oracle(dev, ic, orc, H, W, h, w, nimg, imagenet):
    """roma_prepare (the host prepare of roma.c:1106-1186 on the device)
    against orc_roma_prepare image by image: the filter weights and sums
    are the same double arithmetic, so the results agree to float32
    rounding at most (bar 1e-6 of the largest magnitude, the north
    star's 1e-4 for elementwise work); reductions, enlargements, mixed
    axes, 15x, same size (normalisation only), ImageNet on and off."""
    print(f"[roma] prepare {H}x{W} -> {h}x{w} nimg={nimg} imagenet={imagenet}", flush=True)
    rng = np.random.default_rng(H + W + h)
    img = rng.uniform(0, 1, (nimg, 3, H, W)).astype(np.float32)
    img[:, :, H // 3:H // 3 + 5, :] = 1.0  # a sharp edge: negative lobes, overshoot
    ref = np.zeros((nimg, 3, h, w), np.float32)
    for k in range(nimg):
        orc.orc_roma_prepare(fp(np.ascontiguousarray(img[k])), H, W, fp(ref[k]), h, w, imagenet)
    bi, bo = dev.upload(img), dev.zeros(nimg * 3 * h * w)
    dev.api.roma_prepare(dev.po, bi.mem, nimg, H, W, bo.mem, h, w, imagenet)
    got = dev.read(bo).reshape(nimg, 3, h, w)
    assert rel(got, ref) < 1e-6
    assert (got == ref).mean() > 0.999


def test_prepare_rejects_large_reductions(dev, ic):
    bi, bo = dev.zeros(3 * 1600 * 16), dev.zeros(3 * 100)
    with pytest.raises(ic.IcoregError, match="15.5"):
        dev.api.roma_prepare(dev.po, bi.mem, 1, 1600, 16, bo.mem, 100, 1, 0)


def test_epilogue_and_sd(dev, ic):
    """roma_epilogue and roma_sd against float64 statements of the host
    loops (roma.c:1330-1349, 1415-1428): attenuation by the negative
    coarse certainty (v1) or none (v2), sigmoid, zero outside [-1, 1]^2,
    clamped warp with NaN kept, det^-0.25 or NaN."""
    rng = np.random.default_rng(2)
    hw = 70001
    flow = rng.uniform(-1.3, 1.3, (2, hw)).astype(np.float32)
    flow[0, :7] = [np.nan, 1.0, -1.0, 1.0000001, np.inf, -np.inf, 0.5]
    cert = rng.normal(0, 4, hw).astype(np.float32)
    low = rng.normal(0, 2, hw).astype(np.float32)
    for use_low in (True, False):
        bf, bc, bl = dev.upload(flow), dev.upload(cert), dev.upload(low)
        dev.api.roma_epilogue(dev.po, bf.mem, bc.mem, bl.mem if use_low else None, hw)
        gf, gc = dev.read(bf).reshape(2, hw), dev.read(bc)
        c = cert.astype(np.float64) - (np.where(low < 0, 0.5 * low, 0) if use_low else 0)
        c = 1 / (1 + np.exp(-c))
        with np.errstate(invalid="ignore"):
            out = (np.abs(flow[0]) > 1) | (np.abs(flow[1]) > 1)
        c[out] = 0
        assert np.abs(gc - c).max() < 1e-6
        assert np.array_equal(np.isnan(gf), np.isnan(flow))
        ok = ~np.isnan(flow)
        assert np.array_equal(gf[ok], np.clip(flow, -1, 1)[ok])
    prec = rng.normal(0, 1, (3, hw)).astype(np.float32)
    prec[0] = np.abs(prec[0]) + 0.1
    prec[2] = np.abs(prec[2]) + 0.1
    bp, bs = dev.upload(np.concatenate([np.zeros(hw, np.float32), prec.ravel()])), dev.zeros(hw)
    dev.api.roma_sd(dev.po, bp.mem, hw, bs.mem, hw)
    gs = dev.read(bs)
    p = prec.astype(np.float64)
    det = p[0] * p[2] - p[1] * p[1]
    assert (det <= 0).any() and (det > 0).any()
    assert np.array_equal(np.isnan(gs), det <= 0)
    pos = det > 0
    assert np.abs(gs[pos] / det[pos] ** -0.25 - 1).max() < 1e-6

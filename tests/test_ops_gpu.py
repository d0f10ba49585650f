# SPDX-License-Identifier: Unlicense
"""GPU: every generic op of the HIP library on the reference's own 33
kernel-check cases (tests/ops_check.c:448-487 of i.coregistration.opencl,
same xorshift64 inputs), against the torch-float64 golden outputs at the
reference's bar (2e-5 of the largest reference magnitude,
ops_compare.py:26) and against the oracle."""

from pathlib import Path

import numpy as np
import pytest

import opcases

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "ops_check_golden.npz"
CASES = opcases.all_cases()


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN)


@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_op_case(case, dev, ic, orc, golden):
    print(f"[case] {case.name}", flush=True)
    got = opcases.hip_run(dev, case, ic)
    ora = opcases.oracle_run(orc, case)
    for name, v in got.items():
        ref = golden[f"{case.name}/{name}"]
        assert v.size == ref.size, name
        assert np.isfinite(v).all(), name
        err = opcases.rel_err(v, ref)
        assert err <= opcases.TOL, f"{case.name}/{name}: {err:.2e} vs golden"
        err_o = opcases.rel_err(v, ora[name])
        assert err_o <= opcases.TOL, f"{case.name}/{name}: {err_o:.2e} vs oracle"


ATT_SHAPES = [
    # (Nq, Nk, nh, d, masked): ELoFTR 400 x 400, 8 x 32; RoMa ViT 16 x 64 and
    # decoder 8 x 128 (reduced token counts); odd sizes and masks.
    (400, 400, 8, 32, 0),
    (97, 161, 4, 64, 0),
    (64, 100, 2, 128, 0),
    (64, 100, 2, 128, 1),
    (50, 77, 3, 40, 1),
    (33, 65, 1, 96, 0),
    (40, 45, 2, 17, 1),
]


@pytest.mark.parametrize("shape", ATT_SHAPES, ids=[str(s) for s in ATT_SHAPES])
def test_attention_shapes(shape, dev, ic, orc):
    Nq, Nk, nh, d, masked = shape
    print(f"[attention] {shape}", flush=True)
    rng = np.random.default_rng(1234 + d)
    E = nh * d
    q = rng.uniform(-2, 2, Nq * E).astype(np.float32)
    k = rng.uniform(-2, 2, Nk * E).astype(np.float32)
    v = rng.uniform(-2, 2, Nk * E).astype(np.float32)
    mask = (rng.uniform(0, 1, Nk) > 0.3).astype(np.uint8) if masked else None
    scale = float(1.0 / np.sqrt(d))
    ref = np.zeros(Nq * E, np.float32)
    from oracle_lib import fp
    orc.orc_attention(fp(q), 0, E, fp(k), 0, E, fp(v), 0, E, fp(ref), 0, E, Nq, Nk,
                      nh, d, scale, mask.ctypes.data if mask is not None else None)
    Q, K, V = dev.upload(q), dev.upload(k), dev.upload(v)
    O = dev.zeros(Nq * E)
    Mk = dev.upload(mask) if masked else None
    dev.api.ops_attention(dev.po, ic.mat(Q, 0, E), ic.mat(K, 0, E), ic.mat(V, 0, E),
                          ic.mat(O, 0, E), Nq, Nk, nh, d, scale, ic.mem(Mk))
    got = dev.read(O, Nq * E)
    err = opcases.rel_err(got, ref)
    assert err <= 1e-5, f"{shape}: {err:.2e}"


@pytest.mark.parametrize("shape", [(400, 400, 8, 32, 2), (161, 97, 4, 64, 3)],
                         ids=["eloftr", "ragged"])
def test_attention_batch(shape, dev, ic, orc):
    """ops_attention_batch against the oracle problem by problem, the
    problems laid out with a gap between them."""
    from oracle_lib import fp
    Nq, Nk, nh, d, nb = shape
    print(f"[attention_batch] {shape}", flush=True)
    rng = np.random.default_rng(99 + nb)
    E = nh * d
    bq, bk, bo = Nq * E + 12, Nk * 2 * E + 8, Nq * E + 4
    q = rng.uniform(-2, 2, nb * bq).astype(np.float32)
    kv = rng.uniform(-2, 2, nb * bk).astype(np.float32)
    Q, KV, O = dev.upload(q), dev.upload(kv), dev.zeros(nb * bo)
    scale = float(1.0 / np.sqrt(d))
    dev.api.ops_attention_batch(dev.po, nb, ic.mat(Q, 0, E), bq, ic.mat(KV, 0, 2 * E), bk,
                                ic.mat(KV, E, 2 * E), bk, ic.mat(O, 0, E), bo, Nq, Nk, nh,
                                d, scale, None)
    got = dev.read(O, nb * bo)
    for i in range(nb):
        ref = np.zeros(Nq * E, np.float32)
        qi, ki = q[i * bq:], kv[i * bk:]
        orc.orc_attention(fp(qi), 0, E, fp(ki), 0, 2 * E, fp(ki), E, 2 * E, fp(ref), 0, E,
                          Nq, Nk, nh, d, scale, None)
        err = opcases.rel_err(got[i * bo:i * bo + Nq * E], ref)
        assert err <= 1e-5, f"{shape} problem {i}: {err:.2e}"
        assert not got[i * bo + Nq * E:(i + 1) * bo].any(), "gap written"


CONV_SHAPES = [
    # (nb, C, H, W, K, k, s, p, norm, act): ELoFTR backbone / fusion, VGG,
    # DISK (5 x 5 with normalisation), stride 2, ragged sizes.
    (2, 64, 40, 48, 64, 3, 1, 1, 0, 2),
    (2, 128, 20, 24, 256, 3, 2, 1, 0, 2),
    (1, 256, 20, 20, 256, 3, 1, 1, 0, 3),
    (2, 1, 64, 96, 64, 3, 2, 1, 0, 2),
    (1, 3, 37, 45, 129, 5, 1, 2, 1, 0),
    (1, 80, 33, 31, 129, 5, 1, 2, 1, 0),
    (1, 7, 21, 35, 10, 5, 2, 2, 1, 2),
    (2, 130, 19, 70, 200, 3, 1, 1, 0, 1),
    # Widths where 8 x 16 output tiles waste less than 4 x 32 ones.
    (1, 64, 40, 80, 96, 3, 1, 1, 0, 2),
    (2, 20, 60, 90, 40, 3, 2, 1, 0, 3),
    (1, 7, 30, 90, 70, 5, 2, 2, 1, 2),
    (1, 9, 17, 48, 20, 5, 1, 2, 1, 1),
    # Winograd F(2 x 2, 3 x 3): normalised input, ragged channels, odd
    # sizes, a partial block of output channels.
    (2, 50, 31, 35, 44, 3, 1, 1, 1, 2),
    (1, 33, 9, 7, 36, 3, 1, 1, 0, 0),
    # Row-split Winograd: 4-byte patch loads (W % 4 != 0) and 16-byte ones,
    # an odd number of 8-channel slices, a partial block of output channels.
    (2, 40, 23, 37, 40, 3, 1, 1, 0, 2),
    (1, 72, 18, 28, 36, 3, 1, 1, 0, 1),
    # Row-split Winograd with whole and split units on 256 CUs: 300 units
    # (256 whole, 44 in 4 pieces), and 336 units (256 whole, 80 in 3
    # pieces, the partial channel block among the split ones).
    (1, 64, 80, 80, 192, 3, 1, 1, 0, 2),
    (2, 48, 30, 90, 200, 3, 1, 1, 0, 1),
    # Two channel groups (256 output channels) in XCD bands, with and
    # without split units (320 units: 256 whole, 64 in pieces).
    (1, 64, 40, 128, 256, 3, 1, 1, 0, 2),
    (2, 256, 20, 24, 256, 3, 1, 1, 0, 1),
    # A last block of 1-8 output channels on the few-channel side kernel:
    # DISK's last layer (129 = 128 + 1) at a size that takes 128-channel
    # blocks, 64-channel blocks with 2, 3 and 6 left, strides 1 and 2.
    (1, 80, 256, 200, 129, 5, 1, 2, 1, 0),
    (2, 16, 41, 39, 66, 5, 2, 2, 1, 2),
    (1, 24, 30, 34, 70, 3, 1, 1, 1, 1),
    (1, 20, 25, 27, 67, 3, 2, 1, 0, 2),
    # Grids smaller than the CU count, cut over the input channels into
    # pieces (DISK's 64 x 64 and 32 x 32 layers, ragged channel slices,
    # pieces together with the few-channel kernel).
    (1, 64, 64, 64, 64, 5, 1, 2, 1, 0),
    (1, 128, 32, 32, 64, 5, 1, 2, 1, 2),
    (2, 37, 24, 20, 48, 3, 1, 1, 1, 1),
    (1, 80, 40, 40, 129, 5, 1, 2, 1, 0),
    # One input channel (the per-pixel kernel): 5 x 5 and 3 x 3, stride 1.
    (1, 1, 37, 45, 20, 5, 1, 2, 0, 1),
    (2, 1, 30, 31, 16, 3, 1, 1, 0, 0),
]


@pytest.mark.parametrize("shape", CONV_SHAPES, ids=[str(s) for s in CONV_SHAPES])
def test_conv_shapes(shape, dev, ic, orc):
    import ctypes as C
    from oracle_lib import fp
    nb, Cc, H, W, K, k, s, p, norm, act = shape
    print(f"[conv] {shape}", flush=True)
    rng = np.random.default_rng(100 + Cc + K)
    x = rng.uniform(-1, 1, nb * Cc * H * W).astype(np.float32)
    w = (rng.uniform(-1, 1, K * Cc * k * k) / np.sqrt(Cc * k * k)).astype(np.float32)
    b = rng.uniform(-1, 1, K).astype(np.float32)
    mean = rng.uniform(-0.5, 0.5, Cc).astype(np.float32) if norm else None
    rstd = rng.uniform(0.5, 2, Cc).astype(np.float32) if norm else None
    alpha = rng.uniform(0, 0.5, Cc).astype(np.float32) if norm else None
    Ho, Wo = opcases.conv_out(H, k, s, p), opcases.conv_out(W, k, s, p)
    ref = np.zeros(nb * K * Ho * Wo, np.float32)
    for i in range(nb):
        orc.orc_conv2d(fp(x[i * Cc * H * W:]), Cc, H, W, fp(w), fp(b), K, k, k, s, s, p, p, 1, 1,
                       1, fp(mean), fp(rstd), fp(alpha), act, 0.1,
                       fp(ref[i * K * Ho * Wo:]))
    X, Wt, B = dev.upload(x), dev.upload(w), dev.upload(b)
    Y = dev.zeros(nb * K * Ho * Wo)
    mb = [dev.upload(v) if v is not None else None for v in (mean, rstd, alpha)]
    g = ic.geom(k, k, s, s, p, p, 1, 1, 1)
    dev.api.ops_conv2d_batch(dev.po, nb, X.mem, Cc * H * W, Cc, H, W, Wt.mem, B.mem, K,
                             C.byref(g), *[ic.mem(v) for v in mb], act, 0.1, Y.mem,
                             K * Ho * Wo)
    got = dev.read(Y, nb * K * Ho * Wo)
    err = opcases.rel_err(got, ref)
    assert err <= 1e-5, f"{shape}: {err:.2e}"


# Same-size 3 x 3 convolutions at the edges of the Winograd kernel's
# blocking: ELoFTR's 80 x 80 layers, outputs that end inside a block of
# 8 x 16 pixels, a partial last block of output channels, maps smaller
# than one 2 x 2 tile, channel counts below the kernel's minimum (which
# take the direct path).
WINO_SHAPES = [
    # (nb, C, H, W, K, act)
    (2, 256, 20, 20, 256, 2),
    (2, 64, 40, 48, 64, 2),
    (1, 64, 37, 45, 36, 1),
    (2, 8, 17, 70, 32, 0),
    (1, 128, 3, 2, 64, 3),
    (1, 40, 50, 33, 96, 2),
    (1, 32, 1, 1, 32, 0),
]


@pytest.mark.parametrize("shape", WINO_SHAPES, ids=[str(s) for s in WINO_SHAPES])
def test_conv_winograd_edges(shape, dev, ic, orc):
    """ops_conv2d_batch on 3 x 3 same-size convolutions (the Winograd
    F(2 x 2, 3 x 3) kernel wherever it applies) against the oracle's direct
    convolution."""
    import ctypes as C
    from oracle_lib import fp
    nb, Cc, H, W, K, act = shape
    print(f"[conv] winograd edges {shape}", flush=True)
    rng = np.random.default_rng(300 + Cc + K)
    x = rng.uniform(-1, 1, nb * Cc * H * W).astype(np.float32)
    w = (rng.uniform(-1, 1, K * Cc * 9) / np.sqrt(Cc * 9)).astype(np.float32)
    b = rng.uniform(-1, 1, K).astype(np.float32)
    ref = np.zeros(nb * K * H * W, np.float32)
    for i in range(nb):
        orc.orc_conv2d(fp(x[i * Cc * H * W:]), Cc, H, W, fp(w), fp(b), K, 3, 3, 1, 1, 1, 1, 1,
                       1, 1, None, None, None, act, 0.1, fp(ref[i * K * H * W:]))
    X, Wt, B = dev.upload(x), dev.upload(w), dev.upload(b)
    Y = dev.zeros(nb * K * H * W)
    g = ic.geom(3, 3, 1, 1, 1, 1, 1, 1, 1)
    dev.api.ops_conv2d_batch(dev.po, nb, X.mem, Cc * H * W, Cc, H, W, Wt.mem, B.mem, K,
                             C.byref(g), None, None, None, act, 0.1, Y.mem, K * H * W)
    err = opcases.rel_err(dev.read(Y, nb * K * H * W), ref)
    assert err <= 1e-5, f"{shape}: {err:.2e}"


# Shapes for the Winograd F(4 x 4) kernel (forced): 80 x 80-like and
# VGG-like layers, outputs that end inside a block and inside a 4 x 4
# tile, a partial block of 16 output channels, 8 x 8-tile blocks (narrow
# maps) and 4 x 16-tile blocks (maps 192 pixels wide or more), an odd
# number of 4-channel slices.
WINO4_SHAPES = [
    # (nb, C, H, W, K, act)
    (2, 256, 20, 20, 256, 2),
    (2, 64, 40, 48, 64, 2),
    (1, 64, 37, 44, 36, 1),
    (2, 32, 17, 72, 32, 0),
    (1, 128, 3, 4, 64, 3),
    (1, 40, 50, 32, 96, 2),
    (2, 32, 26, 200, 48, 0),
    (1, 36, 9, 196, 32, 2),
    (1, 4, 12, 16, 32, 1),
    (1, 8, 12, 64, 40, 4),
    # Grids of at least as many blocks as CUs (two blocks a CU resident).
    (2, 32, 256, 256, 32, 2),
    (2, 16, 208, 208, 48, 3),
]


@pytest.mark.parametrize("shape", WINO4_SHAPES, ids=[str(s) for s in WINO4_SHAPES])
def test_conv_winograd_f4(shape, dev, ic, orc):
    """ops_conv2d_batch with the Winograd F(4 x 4, 3 x 3) kernel forced
    (icoreg_conv_wino_form(4)), with the filters transformed by the call,
    against the oracle's direct convolution: within 1e-5. One to nine
    input-channel slices cover the DMA ring's start and end; every
    activation; K not a multiple of 32; maps 8 and 16 tiles wide; grids
    below and above one block a CU."""
    import ctypes as C
    from oracle_lib import fp
    nb, Cc, H, W, K, act = shape
    form = 4
    print(f"[conv] winograd F(4x4) {shape}", flush=True)
    rng = np.random.default_rng(500 + Cc + K + W)
    x = rng.uniform(-1, 1, nb * Cc * H * W).astype(np.float32)
    w = (rng.uniform(-1, 1, K * Cc * 9) / np.sqrt(Cc * 9)).astype(np.float32)
    b = rng.uniform(-1, 1, K).astype(np.float32)
    ref = np.zeros(nb * K * H * W, np.float32)
    for i in range(nb):
        orc.orc_conv2d(fp(x[i * Cc * H * W:]), Cc, H, W, fp(w), fp(b), K, 3, 3, 1, 1, 1, 1, 1,
                       1, 1, None, None, None, act, 0.1, fp(ref[i * K * H * W:]))
    X, Wt, B = dev.upload(x), dev.upload(w), dev.upload(b)
    Y = dev.zeros(nb * K * H * W)
    g = ic.geom(3, 3, 1, 1, 1, 1, 1, 1, 1)
    lib = ic.lib()
    lib.icoreg_conv_wino_form(form)
    try:
        dev.api.ops_conv2d_batch(dev.po, nb, X.mem, Cc * H * W, Cc, H, W, Wt.mem, B.mem, K,
                                 C.byref(g), None, None, None, act, 0.1, Y.mem, K * H * W)
        got = dev.read(Y, nb * K * H * W)
    finally:
        lib.icoreg_conv_wino_form(0)
    err = opcases.rel_err(got, ref)
    assert err <= 1e-5, f"{shape}: {err:.2e}"


LN_SHAPES = [
    # (rows, C, affine): the RoMa ViT rows (1024) and the float4 variants'
    # lane tails (C / 4 not a multiple of 64), the scalar form (C % 4 != 0).
    (3202, 1024, 1),
    (7, 2048, 1),
    (33, 260, 0),
    (10, 4, 1),
    (5, 2050, 1),
]


@pytest.mark.parametrize("shape", LN_SHAPES, ids=[str(s) for s in LN_SHAPES])
def test_layernorm_shapes(shape, dev, ic, orc):
    from oracle_lib import fp
    rows, Cc, affine = shape
    print(f"[layernorm] {shape}", flush=True)
    rng = np.random.default_rng(500 + Cc)
    x = rng.uniform(-3, 3, rows * Cc).astype(np.float32)
    g = rng.uniform(0.5, 1.5, Cc).astype(np.float32) if affine else None
    b = rng.uniform(-1, 1, Cc).astype(np.float32) if affine else None
    ref = np.zeros(rows * Cc, np.float32)
    orc.orc_layernorm(rows, Cc, fp(x), fp(ref), fp(g), fp(b), 1e-6, opcases.ACT_GELU, 0.0)
    X, Y = dev.upload(x), dev.zeros(rows * Cc)
    G = dev.upload(g) if affine else None
    B = dev.upload(b) if affine else None
    dev.api.ops_layernorm(dev.po, rows, Cc, X.mem, Y.mem, ic.mem(G), ic.mem(B), 1e-6,
                          opcases.ACT_GELU, 0.0)
    got = dev.read(Y, rows * Cc)
    err = opcases.rel_err(got, ref)
    assert err <= 1e-5, f"{shape}: {err:.2e}"


# (C, H, W, points, align_corners, smooth): random points scatter; smooth
# ones are an image-shaped grid in raster order (neighbouring points share
# taps), with W % 4 == 0 and not.
GS_SHAPES = [
    (13, 20, 25, 777, 0, False),   # channel groups with a tail
    (64, 48, 40, 3000, 1, False),
    (512, 108, 108, 11664, 0, False),  # a refiner-sized map
    (512, 108, 108, 11664, 0, True),
    (21, 37, 45, 37 * 45, 1, True),
    (9, 64, 96, 60 * 90, 0, True),
]


def smooth_grid(n, H, W):
    """n points of an image-shaped grid (rows of W) in raster order,
    slightly bent, as normalised (x, y)."""
    h = (n + W - 1) // W
    gx = (2 * (np.arange(W) + 0.5) / W - 1)[None, :] + 0 * np.arange(h)[:, None]
    gy = (2 * (np.arange(h) + 0.5) / h - 1)[:, None] + 0 * np.arange(W)[None, :]
    g = np.stack([gx + 0.03 * np.sin(3 * gy), gy + 0.03 * np.cos(2 * gx)], -1)
    return np.ascontiguousarray(g.reshape(-1, 2)[:n], np.float32)


@pytest.mark.parametrize("shape", GS_SHAPES, ids=[str(s) for s in GS_SHAPES])
def test_grid_sample_shapes(shape, dev, ic, orc):
    """grid_sample over many channels against the oracle, with points
    outside, on the border and non-finite, both align_corners
    conventions, on scattered and smooth grids."""
    from oracle_lib import fp
    Cc, H, W, n, align, smooth = shape
    print(f"[grid_sample] {shape}", flush=True)
    rng = np.random.default_rng(700 + Cc)
    x = rng.standard_normal((Cc, H, W)).astype(np.float32)
    if smooth:
        g = smooth_grid(n, H, W)
        g[5] = [np.nan, 0]
        g[W + 3] = [1e6, 0]
    else:
        g = rng.uniform(-1.2, 1.2, (n, 2)).astype(np.float32)
        g[:4] = [[-1, -1], [1, 1], [np.nan, 0], [0, np.inf]]
        g[4:8] = [[1e6, 0], [-3e9, 2], [1, -1], [-1, 1]]
    ref = np.zeros(Cc * n, np.float32)
    orc.orc_grid_sample(fp(x), Cc, H, W, fp(g), n, align, fp(ref))
    X, Gd, Y = dev.upload(x), dev.upload(g), dev.zeros(Cc * n)
    dev.api.ops_grid_sample(dev.po, X.mem, Cc, H, W, Gd.mem, n, align, Y.mem)
    got = dev.read(Y, Cc * n)
    assert np.isfinite(got).all()
    err = opcases.rel_err(got, ref)
    assert err <= 1e-5, f"{shape}: {err:.2e}"


@pytest.mark.parametrize("soff,doff,nbytes", [(0, 0, 1 << 20), (16, 48, 4096 + 16 * 7),
                                              (4, 0, 4096), (0, 8, 1000), (3, 5, 77),
                                              (0, 0, 16), (256, 1024, 25165824)])
def test_ocl_copy(soff, doff, nbytes, dev, ic):
    """ocl_copy byte for byte: 16-byte aligned ends and sizes (the copy
    kernel), misaligned ones (the runtime's copy); bytes around the
    destination range stay as they were."""
    print(f"[ocl_copy] soff={soff} doff={doff} n={nbytes}", flush=True)
    rng = np.random.default_rng(nbytes)
    src = rng.integers(0, 256, soff + nbytes, dtype=np.uint8)
    dst0 = rng.integers(0, 256, doff + nbytes + 64, dtype=np.uint8)
    S, D = dev.upload(src), dev.upload(dst0)
    dev.api.ocl_copy(dev.pb, S.mem, soff, D.mem, doff, nbytes)
    got = dev.read(D, dst0.nbytes, np.uint8)
    want = dst0.copy()
    want[doff:doff + nbytes] = src[soff:soff + nbytes]
    assert np.array_equal(got, want)

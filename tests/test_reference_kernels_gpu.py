# SPDX-License-Identifier: Unlicense
"""GPU: this library's kernels against the reference's own OpenCL kernels
on the same inputs, on the same GPU: the north star's literal parity
criterion. The reference's eloftr_kernels.cl, disk_kernels.cl and
roma_kernels.cl are compiled where they lie by `make -C oracle ref` (the
options of ocl_backend.c:166-187) and run by oracle/_ref/ref_ocl through
the ROCm OpenCL runtime with the argument conventions and work sizes of
their dispatch in eloftr.c, disk.c and roma.c, on inputs this test writes
to files; the HIP kernels run here on the same arrays.

  * ELoFTR's coarse dual softmax (eloftr_row_lse, col_lse, conf_row,
    conf_col over row blocks, eloftr.c:485-548), against both the HIP
    launchers of those four kernels and the fused block form that
    eloftr_match runs: row maxima within 1e-3; row and column first
    argmaxes bit-exact wherever the float64 dual softmax's relative top-2
    margin exceeds 1e-3.
  * DISK's nms5x5: the mask bit-exact everywhere (comparisons only,
    plateaus included); gather_desc within 1e-6.
  * RoMa's cls_to_flow: the same anchor (warp within 1e-5) wherever the
    logit margin exceeds 1e-3, the certainty logit copied exactly.
  * ops.cl's gemm / gemm_big, attention, layernorm, softmax_rows,
    grid_sample, conv5x5 (with the fused instance norm and PReLU),
    conv2d, chan_stats, resize_bilinear, pool2d and rope with ops.c's
    dispatch, eloftr_kernels.cl's fine matching (the same positions and
    keypoints within 1e-3 px wherever the first stage's float64 top-2
    margin exceeds 1e-3), roma_kernels.cl's local
    correlation, warp sampling and depthwise 5 x 5 with roma.c's, at the
    pipelines' shapes (the ViT's qkv and attention of a 560² image, the
    refiners' 1/8 and 1/4 maps of 864²) and ragged ones: contractions
    within 1e-3 of the reference kernel's outputs, element-wise kernels
    within 1e-4, the depthwise convolution, rotations and average pools
    within 1e-6, max pools bit-exact.
  * the small element-wise kernels of ops.cl and roma_kernels.cl
    (chan_affine, prelu, act_map, unfold, avgpool2, transpose2d, axpby,
    roma_row_norm, roma_cos_exp, roma_disp, roma_update, roma2_update).

Skipped with the reason when the reference's kernels were not built (the
reference is needed at build time) or no OpenCL GPU device is present."""

import ctypes
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import elo_ref

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
REF_DIR = ROOT / "oracle" / "_ref"
EXE = REF_DIR / "ref_ocl"
TOL = 1e-3
MARGIN = 1e-3


def run_reference(*cases, timeout=300):
    need = [EXE] + [REF_DIR / f"{k}.co" for k in ("ops", "roma_kernels", "eloftr_kernels",
                                                 "disk_kernels")]
    if not all(p.exists() for p in need):
        pytest.skip("the reference's OpenCL kernels were not built (make -C oracle ref needs "
                    "the reference sources)")
    print(f"[ref] ref_ocl {' '.join(c.split(':')[0] for c in cases)}", flush=True)
    p = subprocess.run([str(EXE), str(REF_DIR), *cases], capture_output=True, text=True,
                       timeout=timeout)
    if p.returncode != 0 and ("clGetPlatformIDs" in p.stderr or "clGetDeviceIDs" in p.stderr):
        pytest.skip(f"no OpenCL GPU device: {p.stderr.strip()[-200:]}")
    assert p.returncode == 0, p.stderr[-2000:]
    print(p.stdout.strip(), flush=True)


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


def dual_softmax_margins(S):
    """Relative top-2 margins of each row and column of the float64 dual
    softmax softmax_row(S) softmax_col(S)."""
    x = S.astype(np.float64)
    er = np.exp(x - x.max(1, keepdims=True))
    conf = er / er.sum(1, keepdims=True)
    del er
    ec = np.exp(x - x.max(0, keepdims=True))
    conf *= ec / ec.sum(0, keepdims=True)
    del ec, x

    def margins(c, axis):
        t = -np.partition(-c, 1, axis=axis)
        t0, t1 = np.take(t, 0, axis=axis), np.take(t, 1, axis=axis)
        return (t0 - t1) / np.maximum(t0, 1e-300)

    return margins(conf, 1), margins(conf, 0)


def hip_coarse(dev, S, blk, fused):
    """The coarse pass of eloftr.c:485-548 through this library: the four
    generic launchers, or the fused block launchers eloftr_match runs."""
    n = S.shape[0]
    a = dev.api
    lse = dev.zeros(n)
    cm = dev.upload(np.full(n, -np.inf, np.float32))
    cs, rmax = dev.zeros(n), dev.zeros(n)
    cmax = dev.upload(np.full(n, -1.0, np.float32))
    rarg, carg = dev.zeros(n, np.int32), dev.upload(np.full(n, -1, np.int32))
    blocks = [(r0, min(blk, n - r0)) for r0 in range(0, n, blk)]
    bufs = [dev.upload(np.ascontiguousarray(S[r0:r0 + rows])) for r0, rows in blocks]
    for p in range(2):
        for (r0, rows), sb in zip(blocks, bufs):
            if fused and p == 0:
                a.eloftr_lse_block(dev.po, sb.mem, rows, n, r0, lse.mem, cm.mem, cs.mem)
            elif fused:
                a.eloftr_conf_block(dev.po, sb.mem, rows, n, r0, lse.mem, cm.mem, cs.mem,
                                    rmax.mem, rarg.mem, cmax.mem, carg.mem)
            elif p == 0:
                a.eloftr_row_lse(dev.po, sb.mem, rows, n, r0, lse.mem)
                a.eloftr_col_lse(dev.po, sb.mem, rows, n, cm.mem, cs.mem)
            else:
                a.eloftr_conf_row(dev.po, sb.mem, rows, n, r0, lse.mem, cm.mem, cs.mem,
                                  rmax.mem, rarg.mem)
                a.eloftr_conf_col(dev.po, sb.mem, rows, n, r0, lse.mem, cm.mem, cs.mem,
                                  cmax.mem, carg.mem)
    return (dev.read(rmax, n), dev.read(rarg, n, np.int32), dev.read(carg, n, np.int32))


@pytest.mark.parametrize("n,blk,planted", [(6400, 6400, True), (3000, 1024, True),
                                           (2048, 700, False)])
def test_coarse_vs_reference_kernels(dev, ic, tmp_path, n, blk, planted):
    """The 640 x 640 config's 6400 x 6400 scores in one block (the
    library's schedule at that size), three blocks of a 3000-token case,
    and unstructured scores (many near-ties) in three blocks."""
    rng = np.random.default_rng(n + blk)
    if planted:
        F0, F1 = elo_ref.match_features(rng, n, 256)
        S = (np.float32(1.0 / 25.6) * (F0 @ F1.T)).astype(np.float32)
    else:
        S = (2.0 * rng.standard_normal((n, n))).astype(np.float32)
    sf, of = tmp_path / "S.f32", tmp_path / "out.bin"
    S.tofile(sf)
    run_reference(f"coarse:{n}:{blk}:{sf}:{of}")
    out = np.fromfile(of, np.uint8)
    r_rmax = out[:4 * n].view(np.float32)
    r_rarg = out[4 * n:8 * n].view(np.int32)
    r_carg = out[8 * n:12 * n].view(np.int32)
    rm, cm = dual_softmax_margins(S)
    rs, cs = rm > MARGIN, cm > MARGIN
    print(f"[ref] coarse n={n}: margin-sure rows {rs.mean():.3f}, columns {cs.mean():.3f}",
          flush=True)
    assert rs.mean() > (0.9 if planted else 0.3) and cs.mean() > (0.9 if planted else 0.3)
    for fused in (False, True):
        g_rmax, g_rarg, g_carg = hip_coarse(dev, S, blk, fused)
        assert rel(g_rmax, r_rmax) <= TOL, fused
        assert np.array_equal(g_rarg[rs], r_rarg[rs]), fused
        assert np.array_equal(g_carg[cs], r_carg[cs]), fused
        print(f"[ref] coarse n={n} fused={fused}: row argmaxes differ on "
              f"{int((g_rarg != r_rarg).sum())}, columns on {int((g_carg != r_carg).sum())} "
              f"(all within the margin)", flush=True)


@pytest.mark.parametrize("h,w,W,off,thresh,levels", [(512, 512, 512, 0, 0.0, 0),
                                                     (333, 517, 520, 100, 0.2, 0),
                                                     (256, 200, 200, 7, -np.inf, 3)])
def test_nms_vs_reference_kernel(dev, ic, tmp_path, h, w, W, off, thresh, levels):
    """DISK's 512 x 512 config shape, a crop with a row stride and an
    offset, and a quantised heatmap full of plateaus (which strict
    comparisons must reject on both sides)."""
    rng = np.random.default_rng(h + w + levels)
    heat = rng.standard_normal(off + h * W).astype(np.float32)
    if levels:
        heat = np.round(heat * levels).astype(np.float32)
    hf, of = tmp_path / "heat.f32", tmp_path / "mask.u8"
    heat.tofile(hf)
    t = "-inf" if np.isinf(thresh) else f"{thresh}"
    run_reference(f"nms:{h}:{w}:{W}:{off}:{t}:{hf}:{of}")
    ref = np.fromfile(of, np.uint8)
    bh, bm = dev.upload(heat), dev.zeros((h * w + 3) // 4)
    dev.api.disk_nms5x5(dev.po, bh.mem, off, W, h, w, float(thresh), bm.mem)
    got = dev.read(bm, h * w, np.uint8)
    assert ref.sum() > 0
    assert np.array_equal(got, ref)


def test_gather_vs_reference_kernel(dev, ic, tmp_path):
    """DISK's descriptor gather at the config's n = 2048 keypoints on a
    512 x 512 output."""
    rng = np.random.default_rng(5)
    H = W = 512
    n, D = 2048, 128
    feat = rng.standard_normal((D + 1, H, W)).astype(np.float32)
    xy = np.ascontiguousarray(np.stack([rng.integers(0, W, n), rng.integers(0, H, n)], 1)
                              .astype(np.int32))
    ff, xf, of = tmp_path / "feat.f32", tmp_path / "xy.i32", tmp_path / "desc.f32"
    feat.tofile(ff)
    xy.tofile(xf)
    run_reference(f"gather:{H}:{W}:{D}:{n}:{ff}:{xf}:{of}")
    ref = np.fromfile(of, np.float32).reshape(n, D)
    bf, bx, bd = dev.upload(feat), dev.upload(xy), dev.zeros(n * D)
    dev.api.disk_gather_desc(dev.po, bf.mem, H, W, D, bx.mem, n, bd.mem)
    assert rel(dev.read(bd, n * D).reshape(n, D), ref) < 1e-6


def test_cls_to_flow_vs_reference_kernel(dev, ic, tmp_path):
    """RoMa's anchor decoding at the 560 config's 1600 tokens (4096
    anchors on a 64 x 64 grid, ld 4097), with modes on the grid's corners
    and edges (clamped neighbours) and an exact tie (first index wins)."""
    rng = np.random.default_rng(11)
    n, res = 1600, 64
    C, ld = res * res, res * res + 1
    L = (3.0 * rng.standard_normal((n, ld))).astype(np.float32)
    for t, idx in enumerate([0, C - 1, res - 1, C - res, 5]):
        L[t, :C] = -5.0
        L[t, idx] = 9.0
    L[5, :C] = -5.0
    L[5, 17] = L[5, 900] = 9.0
    lf, of = tmp_path / "L.f32", tmp_path / "out.f32"
    L.tofile(lf)
    run_reference(f"cls:{n}:{ld}:{C}:{res}:{lf}:{of}")
    out = np.fromfile(of, np.float32)
    r_flow, r_cert = out[:2 * n].reshape(2, n), out[2 * n:]
    bl, bfl, bce = dev.upload(L), dev.zeros(2 * n), dev.zeros(n)
    dev.api.roma_cls_to_flow(dev.po, bl.mem, ld, C, res, n, bfl.mem, bce.mem)
    g_flow, g_cert = dev.read(bfl, 2 * n).reshape(2, n), dev.read(bce, n)
    s = np.sort(L[:, :C].astype(np.float64), 1)
    margin = (s[:, -1] - s[:, -2]) / np.abs(s[:, -1])
    sure = margin > MARGIN
    sure[5] = True  # the exact tie: both sides take the first index
    assert sure.mean() > 0.9
    assert np.abs(g_flow[:, sure] - r_flow[:, sure]).max() < 1e-5
    assert np.array_equal(g_cert, r_cert)


def smooth_warp(rng, h, w, amp=3.0):
    """The refiners' kind of warp (normalised coordinates): the identity
    plus a slowly varying displacement of a few cells."""
    gy = -1 + (2 * np.arange(h) + 1) / h
    gx = -1 + (2 * np.arange(w) + 1) / w
    gy, gx = np.meshgrid(gy, gx, indexing="ij")
    ph = rng.uniform(0, 2 * np.pi, 4)
    dx = amp / w * (np.sin(2.1 * gy + ph[0]) + np.cos(1.7 * gx + ph[1]))
    dy = amp / h * (np.sin(1.3 * gx + ph[2]) + np.cos(2.5 * gy + ph[3]))
    return np.ascontiguousarray(np.stack([gx + dx, gy + dy]).astype(np.float32))


def files(tmp_path, **arrays):
    """Write each array to tmp_path/<name>.f32; the paths by name."""
    out = {}
    for k, v in arrays.items():
        p = tmp_path / f"{k}.f32"
        np.ascontiguousarray(v, np.float32).tofile(p)
        out[k] = str(p)
    return out


@pytest.mark.parametrize("M,N,K,transb,act", [(1601, 3072, 1024, 1, 0), (1000, 130, 77, 0, 2),
                                              (64, 4097, 1024, 1, 0), (400, 256, 512, 0, 1)])
def test_gemm_vs_reference_kernel(dev, ic, tmp_path, M, N, K, transb, act):
    """ops_gemm: the ViT's qkv product of one 560² image (B given N x K),
    ragged shapes with ReLU, RoMa's anchor-logit width, ELoFTR's MLP with
    GELU: within the contraction bar (1e-3 relative)."""
    rng = np.random.default_rng(M + N + K)
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = (rng.uniform(-1, 1, (N, K) if transb else (K, N)) / np.sqrt(K)).astype(np.float32)
    bias = rng.uniform(-1, 1, N).astype(np.float32)
    f = files(tmp_path, A=A, B=B, bias=bias)
    of = tmp_path / "out.f32"
    run_reference(f"gemmx:{M}:{N}:{K}:{transb}:{act}:{f['A']}:{f['B']}:{f['bias']}:{of}")
    ref = np.fromfile(of, np.float32)
    bA, bB, bb, bC = dev.upload(A), dev.upload(B), dev.upload(bias), dev.zeros(M * N)
    dev.api.ops_gemm(dev.po, M, N, K, ic.mat(bA, 0, K), ic.mat(bB, 0, K if transb else N),
                     transb, ic.mat(bC, 0, N), 1, 1, bb.mem, 0, None, 0, 1.0, act, 0.0)
    assert rel(dev.read(bC, M * N), ref) <= TOL


@pytest.mark.parametrize("rows,C", [(3202, 1024), (33, 260), (7, 2050)])
def test_layernorm_vs_reference_kernel(dev, ic, tmp_path, rows, C):
    """ops_layernorm on the ViT's rows (both images) and ragged widths:
    within the element-wise bar (1e-4)."""
    rng = np.random.default_rng(rows + C)
    x = (rng.standard_normal((rows, C)) * 2 + 0.5).astype(np.float32)
    g, b = rng.uniform(0.5, 1.5, C).astype(np.float32), rng.uniform(-1, 1, C).astype(np.float32)
    f = files(tmp_path, x=x, g=g, b=b)
    of = tmp_path / "out.f32"
    run_reference(f"lnx:{rows}:{C}:1e-06:{f['x']}:{f['g']}:{f['b']}:{of}")
    ref = np.fromfile(of, np.float32)
    bx, bg, bb, by = dev.upload(x), dev.upload(g), dev.upload(b), dev.zeros(rows * C)
    dev.api.ops_layernorm(dev.po, rows, C, bx.mem, by.mem, bg.mem, bb.mem, 1e-6, 0, 0.0)
    assert rel(dev.read(by, rows * C), ref) <= 1e-4


@pytest.mark.parametrize("rows,L,scale", [(1601, 1601, 0.125), (100, 37, 1.0), (3, 5000, 0.5)])
def test_softmax_vs_reference_kernel(dev, ic, tmp_path, rows, L, scale):
    """ops_softmax_rows: a ViT head's score rows and ragged rows, within
    the element-wise bar (1e-4)."""
    rng = np.random.default_rng(rows + L)
    s = (rng.standard_normal((rows, L)) * 4).astype(np.float32)
    f = files(tmp_path, s=s)
    of = tmp_path / "out.f32"
    run_reference(f"smx:{rows}:{L}:{scale}:{f['s']}:{of}")
    ref = np.fromfile(of, np.float32)
    bs = dev.upload(s)
    dev.api.ops_softmax_rows(dev.po, bs.mem, rows, L, scale)
    assert rel(dev.read(bs, rows * L), ref) <= 1e-4


@pytest.mark.parametrize("Nq,Nk,nh,d", [(1601, 1601, 16, 64), (400, 400, 8, 32), (37, 1000, 2, 128)])
def test_attention_vs_reference_kernel(dev, ic, tmp_path, Nq, Nk, nh, d):
    """ops_attention: a ViT layer of one image (16 heads of 64), an
    ELoFTR aggregated-attention shape, and few queries over many keys
    with d = 128: outputs within the contraction bar (1e-3)."""
    rng = np.random.default_rng(Nq + Nk + d)
    E = nh * d
    Q = rng.standard_normal((Nq, E)).astype(np.float32)
    K = rng.standard_normal((Nk, E)).astype(np.float32)
    V = rng.standard_normal((Nk, E)).astype(np.float32)
    scale = 1.0 / np.sqrt(d)
    f = files(tmp_path, q=Q, k=K, v=V)
    of = tmp_path / "out.f32"
    run_reference(f"attnx:{Nq}:{Nk}:{nh}:{d}:{scale}:{f['q']}:{f['k']}:{f['v']}:{of}")
    ref = np.fromfile(of, np.float32)
    bq, bk, bv, bo = dev.upload(Q), dev.upload(K), dev.upload(V), dev.zeros(Nq * E)
    dev.api.ops_attention(dev.po, ic.mat(bq, 0, E), ic.mat(bk, 0, E), ic.mat(bv, 0, E),
                          ic.mat(bo, 0, E), Nq, Nk, nh, d, scale, None)
    assert rel(dev.read(bo, Nq * E), ref) <= TOL


@pytest.mark.parametrize("C,h,w,r,smooth", [(512, 108, 108, 3, True), (256, 216, 216, 2, True),
                                            (64, 37, 50, 3, False), (40, 20, 24, 1, True)])
def test_local_corr_vs_reference_kernel(dev, ic, tmp_path, C, h, w, r, smooth):
    """roma_local_corr at the refiner config's 1/8 and 1/4 shapes of 864²
    on smooth warps, a random warp (the per-cell path) and a channel count
    that is not a multiple of 16: within the contraction bar (1e-3)."""
    rng = np.random.default_rng(C + h + r)
    n = h * w
    f1 = rng.standard_normal((C, n)).astype(np.float32)
    f2 = rng.standard_normal((C, n)).astype(np.float32)
    fl = smooth_warp(rng, h, w) if smooth else rng.uniform(-1.1, 1.1, (2, h, w)).astype(np.float32)
    f = files(tmp_path, f1=f1, f2=f2, fl=fl)
    of = tmp_path / "out.f32"
    run_reference(f"lcx:{C}:{h}:{w}:{r}:{f['f1']}:{f['f2']}:{f['fl']}:{of}")
    K = (2 * r + 1) ** 2
    ref = np.fromfile(of, np.float32)
    b1, b2, bf, bo = dev.upload(f1), dev.upload(f2), dev.upload(fl), dev.zeros(K * n)
    dev.api.roma_local_corr(dev.po, b1.mem, b2.mem, C, h, w, r, bf.mem, bo.mem, 0)
    assert rel(dev.read(bo, K * n), ref) <= TOL


@pytest.mark.parametrize("C,h,w,smooth", [(512, 108, 108, True), (9, 200, 160, True),
                                          (33, 40, 50, False)])
def test_warp_sample_vs_reference_kernel(dev, ic, tmp_path, C, h, w, smooth):
    """roma_warp_sample on the 1/8 shape of 864², RoMa's 9-channel 1/1
    form and a random warp with samples outside: within the element-wise
    bar (1e-4; the sample coordinate is one multiply-add whose fusing may
    differ between the compilers)."""
    rng = np.random.default_rng(C + h)
    n = h * w
    x = rng.standard_normal((C, n)).astype(np.float32)
    fl = smooth_warp(rng, h, w) if smooth else rng.uniform(-1.2, 1.2, (2, h, w)).astype(np.float32)
    f = files(tmp_path, x=x, fl=fl)
    of = tmp_path / "out.f32"
    run_reference(f"warpx:{C}:{h}:{w}:{f['x']}:{f['fl']}:{of}")
    ref = np.fromfile(of, np.float32)
    bx, bf, bo = dev.upload(x), dev.upload(fl), dev.zeros(C * n)
    dev.api.roma_warp_sample(dev.po, bx.mem, C, h, w, bf.mem, bo.mem, 0)
    assert rel(dev.read(bo, C * n), ref) <= 1e-4


@pytest.mark.parametrize("C,H,W,n,align,smooth", [(512, 108, 108, 11664, 0, True),
                                                  (64, 50, 70, 5000, 1, False),
                                                  (3, 33, 17, 999, 0, False)])
def test_grid_sample_vs_reference_kernel(dev, ic, tmp_path, C, H, W, n, align, smooth):
    """ops_grid_sample on a smooth warp of the 1/8 grid of 864² and on
    uniform points past the borders, both corner conventions: within the
    element-wise bar (1e-4)."""
    rng = np.random.default_rng(C + n)
    x = rng.standard_normal((C, H, W)).astype(np.float32)
    if smooth:
        g = np.ascontiguousarray(smooth_warp(rng, H, W).reshape(2, -1).T)
    else:
        g = rng.uniform(-1.1, 1.1, (n, 2)).astype(np.float32)
    f = files(tmp_path, x=x, g=g)
    of = tmp_path / "out.f32"
    run_reference(f"gridx:{C}:{H}:{W}:{n}:{align}:{f['x']}:{f['g']}:{of}")
    ref = np.fromfile(of, np.float32)
    bx, bg, bo = dev.upload(x), dev.upload(g), dev.zeros(C * n)
    dev.api.ops_grid_sample(dev.po, bx.mem, C, H, W, bg.mem, n, align, bo.mem)
    assert rel(dev.read(bo, C * n), ref) <= 1e-4


@pytest.mark.parametrize("C,H,W", [(64, 108, 108), (24, 216, 216), (5, 17, 40)])
def test_dwconv5_vs_reference_kernel(dev, ic, tmp_path, C, H, W):
    """roma_dwconv5 (depthwise 5 x 5, bias, ReLU): the same taps in the
    same order, so within 1e-6."""
    rng = np.random.default_rng(C + H)
    x = rng.standard_normal((C, H, W)).astype(np.float32)
    wt = (rng.standard_normal((C, 25)) / 5).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, C).astype(np.float32)
    f = files(tmp_path, x=x, w=wt, b=b)
    of = tmp_path / "out.f32"
    run_reference(f"dwx:{C}:{H}:{W}:{f['x']}:{f['w']}:{f['b']}:{of}")
    ref = np.fromfile(of, np.float32)
    bx, bw, bb, bo = dev.upload(x), dev.upload(wt), dev.upload(b), dev.zeros(C * H * W)
    dev.api.roma_dwconv5(dev.po, bx.mem, C, H, W, bw.mem, bb.mem, bo.mem)
    assert rel(dev.read(bo, C * H * W), ref) <= 1e-6


@pytest.mark.parametrize("C,H,W,K,norm", [(64, 128, 128, 64, True), (3, 96, 80, 16, False),
                                          (80, 64, 64, 129, True), (12, 37, 45, 10, True)])
def test_conv5x5_vs_reference_kernel(dev, ic, tmp_path, C, H, W, K, norm):
    """DISK's 5 x 5 convolutions (ops.cl's conv5x5: stride 1, padding 2,
    bias), with the input instance-normalised and PReLU-gated as the
    U-Net feeds it, the first layer on the RGB image, the 129-channel
    head, a ragged map: within the contraction bar (1e-3)."""
    rng = np.random.default_rng(C + K + H)
    x = rng.standard_normal((C, H, W)).astype(np.float32) * 2 + 0.3
    w = (rng.standard_normal((K, C, 25)) / np.sqrt(25 * C)).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, K).astype(np.float32)
    mean = x.reshape(C, -1).mean(1).astype(np.float32)
    rstd = (1 / np.sqrt(x.reshape(C, -1).var(1) + 1e-5)).astype(np.float32)
    alpha = rng.uniform(0.05, 0.3, C).astype(np.float32)
    f = files(tmp_path, x=x, w=w, b=b, m=mean, r=rstd, a=alpha)
    of = tmp_path / "out.f32"
    run_reference(f"c5x:{C}:{H}:{W}:{K}:{int(norm)}:{f['x']}:{f['w']}:{f['b']}:{f['m']}:"
                  f"{f['r']}:{f['a']}:{of}")
    ref = np.fromfile(of, np.float32)
    bx, bw, bb, bo = dev.upload(x), dev.upload(w), dev.upload(b), dev.zeros(K * H * W)
    bm, br, ba = dev.upload(mean), dev.upload(rstd), dev.upload(alpha)
    g = ic.geom(5, 5, 1, 1, 2, 2, 1, 1, 1)
    dev.api.ops_conv2d(dev.po, bx.mem, C, H, W, bw.mem, bb.mem, K, ctypes.byref(g),
                       bm.mem if norm else None, br.mem if norm else None,
                       ba.mem if norm else None, 0, 0.0, bo.mem)
    assert rel(dev.read(bo, K * H * W), ref) <= TOL


CONV_GEOMS = [
    # (C, H, W, K, kh, kw, sy, sx, py, px, groups, act): ELoFTR's stride-2
    # layers, a grouped and a depthwise case, a 1 x 1 with LeakyReLU.
    (1, 160, 160, 32, 3, 3, 2, 2, 1, 1, 1, 2),
    (64, 80, 96, 128, 3, 3, 2, 2, 1, 1, 1, 0),
    (32, 33, 41, 48, 3, 3, 1, 1, 1, 1, 4, 2),
    (16, 40, 40, 16, 4, 4, 4, 4, 0, 0, 16, 0),
    (24, 21, 19, 8, 1, 1, 1, 1, 0, 0, 1, 3),
]


@pytest.mark.parametrize("gm", CONV_GEOMS, ids=[str(g) for g in CONV_GEOMS])
def test_conv2d_vs_reference_kernel(dev, ic, tmp_path, gm):
    """ops_conv2d against ops.cl's general conv2d kernel (whatever kernel
    this library picks for the geometry): within 1e-3."""
    C, H, W, K, kh, kw, sy, sx, py, px, groups, act = gm
    Ho, Wo = (H + 2 * py - kh) // sy + 1, (W + 2 * px - kw) // sx + 1
    rng = np.random.default_rng(sum(gm))
    x = rng.standard_normal((C, H, W)).astype(np.float32)
    w = (rng.standard_normal((K, C // groups, kh, kw)) /
         np.sqrt(C // groups * kh * kw)).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, K).astype(np.float32)
    f = files(tmp_path, x=x, w=w, b=b)
    of = tmp_path / "out.f32"
    spec = ":".join(str(v) for v in gm)
    run_reference(f"convx:{spec}:{f['x']}:{f['w']}:{f['b']}:{of}")
    ref = np.fromfile(of, np.float32)
    bx, bw, bb, bo = dev.upload(x), dev.upload(w), dev.upload(b), dev.zeros(K * Ho * Wo)
    g = ic.geom(kh, kw, sy, sx, py, px, 1, 1, groups)
    dev.api.ops_conv2d(dev.po, bx.mem, C, H, W, bw.mem, bb.mem, K, ctypes.byref(g), None, None,
                       None, act, 0.1, bo.mem)
    assert rel(dev.read(bo, K * Ho * Wo), ref) <= TOL


@pytest.mark.parametrize("C,HW", [(64, 512 * 512), (129, 4096), (7, 33)])
def test_chan_stats_vs_reference_kernel(dev, ic, tmp_path, C, HW):
    """ops_chan_stats (instance-norm mean and 1 / std) on DISK's 512²
    layer, its head and a ragged plane: within 1e-4."""
    rng = np.random.default_rng(C + HW)
    x = (rng.standard_normal((C, HW)) * 3 + rng.uniform(-2, 2, (C, 1))).astype(np.float32)
    f = files(tmp_path, x=x)
    of = tmp_path / "out.f32"
    run_reference(f"statx:{C}:{HW}:1e-05:{f['x']}:{of}")
    ref = np.fromfile(of, np.float32)
    bx, bm, br = dev.upload(x), dev.zeros(C), dev.zeros(C)
    dev.api.ops_chan_stats(dev.po, bx.mem, C, HW, 1e-5, bm.mem, br.mem)
    assert rel(dev.read(bm, C), ref[:C]) <= 1e-4
    assert rel(dev.read(br, C), ref[C:]) <= 1e-4


@pytest.mark.parametrize("C,h,w,H,W,align,scale", [(256, 80, 80, 160, 160, 0, 2.0),
                                                   (64, 160, 160, 320, 320, 1, 0.0),
                                                   (3, 37, 45, 20, 23, 0, 0.0)])
def test_resize_vs_reference_kernel(dev, ic, tmp_path, C, h, w, H, W, align, scale):
    """ops_resize (ELoFTR's FPN upsampling by a scale factor, a size with
    aligned corners, a downsampling): within 1e-4."""
    rng = np.random.default_rng(C + H)
    x = rng.standard_normal((C, h, w)).astype(np.float32)
    f = files(tmp_path, x=x)
    of = tmp_path / "out.f32"
    run_reference(f"resx:{C}:{h}:{w}:{H}:{W}:{align}:{scale}:{f['x']}:{of}")
    ref = np.fromfile(of, np.float32)
    bx, bo = dev.upload(x), dev.zeros(C * H * W)
    dev.api.ops_resize(dev.po, bx.mem, C, h, w, bo.mem, H, W, 0, align, scale)
    assert rel(dev.read(bo, C * H * W), ref) <= 1e-4


@pytest.mark.parametrize("C,H,W,ks,s,p,mx", [(64, 864, 864, 2, 2, 0, 1), (256, 80, 80, 4, 4, 0, 1),
                                             (16, 33, 35, 3, 2, 1, 0), (8, 17, 9, 2, 2, 0, 0)])
def test_pool_vs_reference_kernel(dev, ic, tmp_path, C, H, W, ks, s, p, mx):
    """ops_pool2d: VGG's 2 x 2 max pool at 864², ELoFTR's 4 x 4 key
    pooling, padded and ragged average pools: max pools bit-exact,
    average pools within 1e-6."""
    Ho, Wo = (H + 2 * p - ks) // s + 1, (W + 2 * p - ks) // s + 1
    rng = np.random.default_rng(C + H + ks)
    x = rng.standard_normal((C, H, W)).astype(np.float32)
    f = files(tmp_path, x=x)
    of = tmp_path / "out.f32"
    run_reference(f"poolx:{C}:{H}:{W}:{ks}:{s}:{p}:{mx}:{f['x']}:{of}")
    ref = np.fromfile(of, np.float32)
    bx, bo = dev.upload(x), dev.zeros(C * Ho * Wo)
    dev.api.ops_pool2d(dev.po, bx.mem, C, H, W, ks, s, p, mx, bo.mem)
    got = dev.read(bo, C * Ho * Wo)
    if mx:
        assert np.array_equal(got, ref)
    else:
        assert rel(got, ref) <= 1e-6


@pytest.mark.parametrize("rows,nh,d,npos,inter", [(6400, 8, 32, 6400, 0), (1601, 16, 64, 1601, 1),
                                                  (37, 3, 8, 5, 1)])
def test_rope_vs_reference_kernel(dev, ic, tmp_path, rows, nh, d, npos, inter):
    """ops_rope in place: ELoFTR's 80 x 80 tokens (half form), an
    interleaved form, positions cycling: within 1e-6 (a rotation of each
    pair, the same two products)."""
    rng = np.random.default_rng(rows + d)
    ld = nh * d + 4
    x = rng.uniform(-1, 1, (rows, ld)).astype(np.float32)
    ang = rng.uniform(-3.2, 3.2, (npos, d // 2))
    cs = np.empty((npos, d // 2, 2), np.float32)
    cs[..., 0], cs[..., 1] = np.cos(ang), np.sin(ang)
    f = files(tmp_path, x=x, cs=cs)
    of = tmp_path / "out.f32"
    run_reference(f"ropex:{rows}:{ld}:{nh}:{d}:{npos}:{inter}:{f['x']}:{f['cs']}:{of}")
    ref = np.fromfile(of, np.float32)
    bx, bc = dev.upload(x), dev.upload(cs)
    dev.api.ops_rope(dev.po, bx.mem, 0, ld, rows, nh, d, npos, bc.mem, inter)
    assert rel(dev.read(bx, rows * ld), ref) <= 1e-6


@pytest.mark.parametrize("H,W,Mn", [(48, 64, 500), (160, 160, 1000)])
def test_fine_vs_reference_kernel(dev, ic, tmp_path, H, W, Mn):
    """ELoFTR's fine matching (eloftr_kernels.cl's eloftr_fine, one
    work-group per coarse match) against eloftr_fine on the same windows,
    the border cells included: wherever the float64 first-stage top-2
    margin exceeds 1e-3 the same integer positions and sub-pixel
    keypoints within 1e-3 px."""
    rng = np.random.default_rng(H + Mn)
    h, w = H // 8, W // 8
    f0 = rng.standard_normal((64, H, W)).astype(np.float32)
    f1 = rng.standard_normal((64, H, W)).astype(np.float32)
    cells = np.stack([rng.integers(0, w, Mn), rng.integers(0, h, Mn),
                      rng.integers(0, w, Mn), rng.integers(0, h, Mn)], 1).astype(np.int32)
    cells[:3] = [[0, 0, 0, 0], [w - 1, h - 1, w - 1, h - 1], [0, h - 1, w - 1, 0]]
    cells = np.ascontiguousarray(cells)
    f = files(tmp_path, f0=f0, f1=f1)
    cf, of = tmp_path / "cells.i32", tmp_path / "out.f32"
    cells.tofile(cf)
    run_reference(f"finex:{H}:{W}:{Mn}:10.0:{f['f0']}:{f['f1']}:{cf}:{of}")
    ref = np.fromfile(of, np.float32).reshape(-1, 4)
    b0, b1, bc, bo = dev.upload(f0), dev.upload(f1), dev.upload(cells), dev.zeros(4 * Mn)
    dev.api.eloftr_fine(dev.po, b0.mem, b1.mem, H, W, bc.mem, Mn, 10.0, bo.mem)
    got = dev.read(bo, 4 * Mn).reshape(-1, 4)
    _, margin = elo_ref.fine_bruteforce(f0, f1, cells)
    sure = margin > MARGIN
    assert sure.mean() > 0.9
    assert np.array_equal(np.floor(got[sure, :2]), np.floor(ref[sure, :2]))
    assert np.abs(got[sure] - ref[sure]).max() <= 1e-3


def _small_case(kind, rng):
    """Inputs, the reference spec fields and this library's call for one
    small element-wise kernel: (a, b, c, x, y, inputs, ours, tol)."""
    U = lambda *s: rng.uniform(-2, 2, s).astype(np.float32)  # noqa: E731
    if kind == "affine":
        C, HW, act = 24, 999, 3
        X, mu, rs = U(C, HW), U(C), rng.uniform(0.2, 2, C).astype(np.float32)
        g, b = U(C), U(C)
        return (C, HW, act, 0.1, 0.0, [X, mu, rs, g, b],
                lambda d, m, o: d.api.ops_chan_affine(d.po, m[0], o, C, HW, m[1], m[2], m[3],
                                                      m[4], act, 0.1), C * HW, 1e-6)
    if kind == "prelu":
        C, HW = 16, 1234
        X, al = U(C, HW), rng.uniform(0, 0.5, C).astype(np.float32)
        return (C, HW, 0, 0.0, 0.0, [X, al],
                lambda d, m, o: d.api.ops_prelu(d.po, m[0], o, C, HW, m[1]), C * HW, 1e-6)
    if kind == "act":
        n, act = 100003, 1
        X = U(n)
        return (n, 0, act, 0.0, 0.0, [X],
                lambda d, m, o: d.api.ops_act(d.po, m[0], o, n, act, 0.0), n, 1e-4)
    if kind == "unfold":
        C, s, p = 5, 2, 1
        Ho, Wo = (16 + 2 * p - 3) // s + 1, (20 + 2 * p - 3) // s + 1
        X = U(C, 16, 20)

        def ours(d, m, o):
            g = ic_geom(3, 3, s, s, p, p)
            d.api.ops_unfold(d.po, m[0], C, 16, 20, ctypes.byref(g), o)
        return (C, s, p, 0.0, 0.0, [X], ours, C * 9 * Ho * Wo, 0.0)
    if kind == "avgpool2":
        C, H, W = 7, 30, 42
        X = U(C, H, W)
        return (C, H, W, 0.0, 0.0, [X],
                lambda d, m, o: d.api.ops_avgpool2(d.po, m[0], C, H, W, o),
                C * (H // 2) * (W // 2), 1e-6)
    if kind == "transpose":
        B, R, Cc = 3, 37, 129
        X = U(B, R, Cc)
        return (B, R, Cc, 0.0, 0.0, [X],
                lambda d, m, o: d.api.ops_transpose(d.po, m[0], o, B, R, Cc), B * R * Cc, 0.0)
    if kind == "axpby":
        n, bmod = 10000, 77
        A, Bv = U(n), U(bmod)
        return (n, bmod, 0, 0.7, -1.3, [A, Bv],
                lambda d, m, o: d.api.ops_axpby(d.po, o, m[0], 0.7, m[1], -1.3, n, bmod), n,
                1e-6)
    if kind == "rownorm":
        rows, C = 1600, 512
        X = U(rows, C)
        return (rows, C, 0, 0.0, 0.0, [X],
                lambda d, m, o: d.api.roma_row_norm(d.po, m[0], rows, C, o), rows, 1e-5)
    if kind == "cosexp":
        N, M = 300, 411
        S = U(N, M) * 10
        nx, ny = rng.uniform(3, 6, N).astype(np.float32), rng.uniform(3, 6, M).astype(np.float32)
        return (N, M, 0, 0.2, 1e-6, [S, nx, ny], None, N * M, 1e-4)
    if kind == "disp":
        H, W = 108, 96
        fl = U(2, H * W) / 2
        return (H, W, 0, 3.5, 2.5, [fl],
                lambda d, m, o: d.api.roma_disp(d.po, m[0], H, W, 3.5, 2.5, o), 2 * H * W,
                1e-6)
    if kind == "update":
        n = 11664
        return (n, 0, 108, 8.0, 108.0, [U(2, n), U(n), U(3, n)], None, 3 * n, 1e-6)
    if kind == "update2":
        n = 16384
        return (n, 0, 0, 128.0, 128.0, [U(2, n), U(4, n), U(6, n) * 12], None, 6 * n, 1e-5)
    raise ValueError(kind)


def ic_geom(kh, kw, sy, sx, py, px):
    from conftest import load_package
    return load_package().geom(kh, kw, sy, sx, py, px, 1, 1, 1)


SMALL = ["affine", "prelu", "act", "unfold", "avgpool2", "transpose", "axpby", "rownorm",
         "cosexp", "disp", "update", "update2"]


@pytest.mark.parametrize("kind", SMALL)
def test_small_kernels_vs_reference(dev, ic, tmp_path, kind):
    """The small element-wise kernels of ops.cl (chan_affine, prelu,
    act_map, unfold, avgpool2, transpose2d, axpby) and roma_kernels.cl
    (row_norm, cos_exp, disp, update, roma2_update) against this
    library's on the same inputs: copies bit-exact, arithmetic within
    1e-6, transcendental ones within 1e-5 to 1e-4."""
    rng = np.random.default_rng(len(kind) * 7 + 1)
    a, b, c, x, y, ins, ours, nout, tol = _small_case(kind, rng)
    paths = [str(tmp_path / f"in{i}.f32") for i in range(len(ins))]
    for p, v in zip(paths, ins):
        np.ascontiguousarray(v, np.float32).tofile(p)
    paths += ["-"] * (5 - len(paths))
    of = tmp_path / "out.f32"
    run_reference(f"smallx:{kind}:{a}:{b}:{c}:{x!r}:{y!r}:{':'.join(paths)}:{of}")
    ref = np.fromfile(of, np.float32)
    bufs = [dev.upload(v) for v in ins]
    if kind == "cosexp":
        dev.api.roma_cos_exp(dev.po, bufs[0].mem, bufs[1].mem, bufs[2].mem, a, b, x, y)
        got = dev.read(bufs[0], nout)
    elif kind == "update":
        dev.api.roma_update(dev.po, bufs[0].mem, bufs[1].mem, bufs[2].mem, a, x, y, float(c))
        got = np.concatenate([dev.read(bufs[0], 2 * a), dev.read(bufs[1], a)])
    elif kind == "update2":
        dev.api.roma2_update(dev.po, bufs[0].mem, bufs[1].mem, bufs[2].mem, a, x, y)
        got = np.concatenate([dev.read(bufs[0], 2 * a), dev.read(bufs[1], 4 * a)])
    else:
        out = dev.zeros(nout)
        ours(dev, [m.mem for m in bufs], out.mem)
        got = dev.read(out, nout)
    assert got.shape == ref.shape
    if tol == 0.0:
        assert np.array_equal(got, ref)
    else:
        assert rel(got, ref) <= tol

# SPDX-License-Identifier: Unlicense
"""GPU: ELoFTR kernels and network on the HIP library against the oracle.

Tolerances: contractions and features <= 1e-3 of the
largest reference magnitude; index outputs (row / column argmax, fine
window argmax) bit-exact wherever the oracle's relative top-2 margin
exceeds 1e-3."""

import os
import sys
from pathlib import Path

import numpy as np
import pytest

import elo_ref
from oracle_lib import eloftr_forward, fp, ip

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "i.coregistration.opencl_amd"))
import synth  # noqa: E402

GOLDEN = Path(__file__).resolve().parent / "golden" / "eloftr_golden.npz"
TOL = 1e-3
MARGIN = 1e-3


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


@pytest.fixture(scope="module")
def weights_file(tmp_path_factory):
    p = tmp_path_factory.mktemp("w") / "eloftr_random.safetensors"
    return synth.eloftr_weights_file(p)


@pytest.fixture(scope="module")
def weights():
    return synth.eloftr_weights_calibrated()


def test_coarse_kernels_two_blocks(dev, ic, orc):
    """GEMM + row / column LSE + confidence argmaxes over two row blocks
    (the running column statistics and the first-argmax rule across
    blocks) against the oracle's blocked schedule."""
    print("[eloftr] coarse kernels", flush=True)
    rng = np.random.default_rng(21)
    n, D, blk = 1000, 64, 384
    F0, F1 = elo_ref.match_features(rng, n, D)
    alpha = np.float32(1.0) / np.float32(D * 0.1)
    o_rmax = np.zeros(n, np.float32)
    o_rarg, o_carg = np.zeros(n, np.int32), np.zeros(n, np.int32)
    o_rmar, o_cmar = np.zeros(n, np.float32), np.zeros(n, np.float32)
    orc.orc_eloftr_coarse(fp(F0), fp(F1), n, D, alpha, blk, fp(o_rmax), ip(o_rarg),
                          ip(o_carg), fp(o_rmar), fp(o_cmar), None)
    a, M = dev.api, ic.mem
    f0, f1 = dev.upload(F0), dev.upload(F1)
    S = dev.zeros(blk * n)
    lse, cm, cs = dev.zeros(n), dev.upload(np.full(n, -np.inf, np.float32)), dev.zeros(n)
    rmax, rarg = dev.zeros(n), dev.zeros(n, np.int32)
    cmax = dev.upload(np.full(n, -1.0, np.float32))
    carg = dev.upload(np.full(n, -1, np.int32))
    for p in range(2):
        for r0 in range(0, n, blk):
            rows = min(blk, n - r0)
            a.ops_gemm(dev.po, rows, n, D, ic.mat(f0, r0 * D, D), ic.mat(f1, 0, D), 1,
                       ic.mat(S, 0, n), 1, 1, None, 0, None, 0, float(alpha), 0, 0.0)
            if p == 0:
                a.eloftr_row_lse(dev.po, M(S), rows, n, r0, M(lse))
                a.eloftr_col_lse(dev.po, M(S), rows, n, M(cm), M(cs))
            else:
                a.eloftr_conf_row(dev.po, M(S), rows, n, r0, M(lse), M(cm), M(cs), M(rmax), M(rarg))
                a.eloftr_conf_col(dev.po, M(S), rows, n, r0, M(lse), M(cm), M(cs), M(cmax), M(carg))
    g_rmax, g_rarg = dev.read(rmax, n), dev.read(rarg, n, np.int32)
    g_carg = dev.read(carg, n, np.int32)
    assert rel(g_rmax, o_rmax) <= TOL
    sure = o_rmar / np.maximum(o_rmax, 1e-30) > MARGIN
    assert sure.mean() > 0.9
    assert np.array_equal(g_rarg[sure], o_rarg[sure])
    cmaxo = dev.read(cmax, n)
    sure_c = o_cmar / np.maximum(cmaxo, 1e-30) > MARGIN
    assert sure_c.mean() > 0.9
    assert np.array_equal(g_carg[sure_c], o_carg[sure_c])


def test_fine_kernel(dev, ic, orc):
    print("[eloftr] fine kernel", flush=True)
    rng = np.random.default_rng(22)
    H, W = 48, 64
    h, w = H // 8, W // 8
    f0 = rng.standard_normal((64, H, W)).astype(np.float32)
    f1 = rng.standard_normal((64, H, W)).astype(np.float32)
    Mn = 500
    cells = np.stack([rng.integers(0, w, Mn), rng.integers(0, h, Mn),
                      rng.integers(0, w, Mn), rng.integers(0, h, Mn)], 1).astype(np.int32)
    cells[:3] = [[0, 0, 0, 0], [w - 1, h - 1, w - 1, h - 1], [0, h - 1, w - 1, 0]]
    cells = np.ascontiguousarray(cells)
    ref = np.zeros(4 * Mn, np.float32)
    mar = np.zeros(Mn, np.float32)
    orc.orc_eloftr_fine(fp(f0), fp(f1), H, W, ip(cells), Mn, 10.0, fp(ref), fp(mar))
    b0, b1, bc = dev.upload(f0), dev.upload(f1), dev.upload(cells)
    out = dev.zeros(4 * Mn)
    dev.api.eloftr_fine(dev.po, b0.mem, b1.mem, H, W, bc.mem, Mn, 10.0, out.mem)
    got = dev.read(out, 4 * Mn).reshape(-1, 4)
    ref = ref.reshape(-1, 4)
    _, margin = elo_ref.fine_bruteforce(f0, f1, cells)
    sure = margin > MARGIN
    assert sure.mean() > 0.9
    np.testing.assert_array_equal(np.floor(got[sure, :2]), np.floor(ref[sure, :2]))
    np.testing.assert_allclose(got[sure], ref[sure], atol=1e-3, rtol=0)


def test_fine_half_resolution(dev, ic):
    """eloftr_fine_half on half-resolution maps is bit for bit eloftr_fine on
    their 2x resize (ops_resize), including windows at the image border."""
    print("[eloftr] fine kernel, half-resolution maps", flush=True)
    rng = np.random.default_rng(23)
    H, W = 48, 64
    h, w = H // 8, W // 8
    f0 = rng.standard_normal((64, H // 2, W // 2)).astype(np.float32)
    f1 = rng.standard_normal((64, H // 2, W // 2)).astype(np.float32)
    Mn = 300
    cells = np.stack([rng.integers(0, w, Mn), rng.integers(0, h, Mn),
                      rng.integers(0, w, Mn), rng.integers(0, h, Mn)], 1).astype(np.int32)
    cells[:3] = [[0, 0, 0, 0], [w - 1, h - 1, w - 1, h - 1], [0, h - 1, w - 1, 0]]
    cells = np.ascontiguousarray(cells)
    b0, b1, bc = dev.upload(f0), dev.upload(f1), dev.upload(cells)
    u0, u1 = dev.zeros(64 * H * W), dev.zeros(64 * H * W)
    dev.api.ops_resize(dev.po, b0.mem, 64, H // 2, W // 2, u0.mem, H, W, 0, 0, 2.0)
    dev.api.ops_resize(dev.po, b1.mem, 64, H // 2, W // 2, u1.mem, H, W, 0, 0, 2.0)
    full, half = dev.zeros(4 * Mn), dev.zeros(4 * Mn)
    dev.api.eloftr_fine(dev.po, u0.mem, u1.mem, H, W, bc.mem, Mn, 10.0, full.mem)
    dev.api.eloftr_fine_half(dev.po, b0.mem, b1.mem, H, W, bc.mem, Mn, 10.0, half.mem)
    a, b = dev.read(full, 4 * Mn), dev.read(half, 4 * Mn)
    assert np.isfinite(a).all()
    assert np.array_equal(a, b)


def test_network_small_vs_oracle_and_transformers(dev, ic, weights, weights_file, tmp_path):
    print("[eloftr] network 64x96", flush=True)
    g = np.load(GOLDEN)
    H, W = int(g["H"]), int(g["W"])
    g0, g1, _ = synth.eloftr_pair(H, W)
    o = eloftr_forward(weights, g0, g1, backbone=True, coarse=True, fine=True)
    net = ic.Eloftr(dev, weights_file, H, W)
    try:
        r = net.match(g0, g1, dump=str(tmp_path), tile=3)
        n = (H // 8) * (W // 8)
        for k in range(2):
            bb = np.fromfile(tmp_path / f"tile003_eloftr_backbone_{k}.f32", np.float32)
            assert rel(bb, o["backbone"][k]) <= TOL
            assert rel(bb, g["backbone"][k]) <= TOL
            x = net.buffer(f"x{k}", 256 * n)
            assert rel(x, o["coarse"][k]) <= TOL
            assert rel(x, g["coarse"][k]) <= TOL
            cx = np.fromfile(tmp_path / f"tile003_eloftr_coarse_{k}.f32", np.float32)
            assert np.array_equal(cx, x)
            fine = net.buffer(f"fine{k}", 64 * H * W)
            assert rel(fine, o["fine"][k]) <= TOL
            assert rel(fine[g["fine_idx"]], g["fine"][k]) <= TOL
        check_coarse_indices(r, o)
        assert r["nm"] == o["nm"]
    finally:
        net.close()


def test_network_640_properties(dev, ic, weights_file):
    """The benchmark config (640 x 640 grey pair): every output is finite
    and in range, and the matches are exactly the mutual / threshold /
    border selection of the coarse statistics."""
    print("[eloftr] network 640x640", flush=True)
    H = W = 640
    g0, g1, _ = synth.eloftr_pair(H, W)
    net = ic.Eloftr(dev, weights_file, H, W)
    try:
        r = net.match(g0, g1)
        h, w = H // 8, W // 8
        n = h * w
        rm, ra, ca = r["row_max"], r["row_arg"], r["col_arg"]
        assert np.isfinite(rm).all() and (rm >= 0).all() and (rm <= 1.0 + 1e-6).all()
        assert ((ra >= 0) & (ra < n)).all() and ((ca >= 0) & (ca < n)).all()
        inside = lambda k: (2 <= k % w) & (k % w < w - 2) & (2 <= k // w) & (k // w < h - 2)
        i = np.arange(n)
        keep = (rm > 0.2) & (ca[ra] == i) & inside(i) & inside(ra)
        assert r["nm"] == int(keep.sum())
        assert np.array_equal(r["mi"], i[keep]) and np.array_equal(r["mj"], ra[keep])
        x = net.buffer("x0", 256 * n)
        assert np.isfinite(x).all()
        fine = net.buffer("fine1", 64 * H * W)
        assert np.isfinite(fine).all()
        if r["nm"]:
            assert np.isfinite(r["kp"]).all()
    finally:
        net.close()


def test_network_640_matches_properties(dev, ic, weights_file):
    """The fine stage at full size on a 640 x 640 pair that yields
    thousands of coarse matches (B = A shifted by (8, 16) px): the match
    list is the selection of the coarse statistics, and the fine
    keypoints recover the known shift within the random-init network's
    one-pixel spread."""
    H = W = 640
    print("[eloftr] network 640x640 with matches", flush=True)
    g0, g1 = synth.eloftr_noise_pair(H, W, shift=(8, 16))
    net = ic.Eloftr(dev, weights_file, H, W)
    try:
        r = net.match(g0, g1)
    finally:
        net.close()
    h, w = H // 8, W // 8
    n = h * w
    rm, ra, ca = r["row_max"], r["row_arg"], r["col_arg"]
    inside = lambda k: (2 <= k % w) & (k % w < w - 2) & (2 <= k // w) & (k // w < h - 2)
    i = np.arange(n)
    keep = (rm > 0.2) & (ca[ra] == i) & inside(i) & inside(ra)
    assert r["nm"] == int(keep.sum()) > 1000
    assert np.array_equal(r["mi"], i[keep]) and np.array_equal(r["mj"], ra[keep])
    assert np.array_equal(r["mconf"], rm[keep])
    kp = r["kp"]
    assert np.isfinite(kp).all()
    # Keypoints lie in their cells (centre 8 c, +-3.5 px; image 1 also
    # moves by the +-1 px sub-pixel expectation).
    cx0, cy0, cx1, cy1 = r["mi"] % w, r["mi"] // w, r["mj"] % w, r["mj"] // w
    for c, x, e in ((cx0, kp[:, 0], 3.5), (cy0, kp[:, 1], 3.5), (cx1, kp[:, 2], 4.5),
                    (cy1, kp[:, 3], 4.5)):
        assert (np.abs(x - 8 * c) <= e + 1e-4).all()
    d = kp[:, 2:] - kp[:, :2]
    good = (np.abs(d[:, 0] - 16) <= 1.5) & (np.abs(d[:, 1] - 8) <= 1.5)
    assert good.mean() > 0.95


def test_network_wide_vs_oracle(dev, ic, weights, weights_file):
    """A wide 64 x 512 pair (1/8 maps of 8 x 64, aggregated 2 x 16):
    coarse features and scores against the oracle."""
    print("[eloftr] network 64x512", flush=True)
    H, W = 64, 512
    g0, g1, _ = synth.eloftr_pair(H, W)
    o = eloftr_forward(weights, g0, g1, backbone=True, coarse=True, fine=False)
    net = ic.Eloftr(dev, weights_file, H, W)
    try:
        r = net.match(g0, g1)
        n = (H // 8) * (W // 8)
        for k in range(2):
            x = net.buffer(f"x{k}", 256 * n)
            assert rel(x, o["coarse"][k]) <= TOL
        check_coarse_indices(r, o)
        assert r["nm"] == o["nm"]
    finally:
        net.close()


def test_network_matches_vs_oracle(dev, ic, weights, weights_file):
    """A pair that yields coarse matches (unblurred noise, B translated by
    whole cells): the mutual / threshold / border match list, the match
    confidences and the fine keypoints against the oracle."""
    H, W = 128, 160
    print(f"[eloftr] network {H}x{W} with matches", flush=True)
    g0, g1 = synth.eloftr_noise_pair(H, W, shift=(8, 16))
    o = eloftr_forward(weights, g0, g1, coarse=True, fine=True)
    net = ic.Eloftr(dev, weights_file, H, W)
    try:
        r = net.match(g0, g1)
    finally:
        net.close()
    nm = o["nm"]
    assert nm > 50
    # Over half the rows have no confidence at all (exp underflows to 0:
    # no margin), so fewer rows and columns are margin-sure here.
    check_coarse_indices(r, o, min_sure=0.2)
    w = W // 8
    rs = sure_rows(o, w, H // 8)
    assert rs[o["mi"][:nm]].mean() > 0.95
    om = {int(i): k for k, i in enumerate(o["mi"][:nm])}
    gm = {int(i): k for k, i in enumerate(r["mi"])}
    # Matches may differ only on rows whose selection is within the margin.
    for i in set(om) ^ set(gm):
        assert not rs[i], f"match row {i} differs from the oracle with a sure margin"
    if rs[o["mi"][:nm]].all():
        assert r["nm"] == nm
        assert np.array_equal(r["mi"], o["mi"][:nm])
        assert np.array_equal(r["mj"], o["mj"][:nm])
    common = sorted(set(om) & set(gm))
    assert len(common) >= 0.95 * nm
    ko = np.array([om[i] for i in common])
    kg = np.array([gm[i] for i in common])
    assert np.array_equal(r["mj"][kg], o["mj"][ko])
    assert rel(r["mconf"][kg], o["mconf"][ko]) <= TOL
    kp_o = o["kp"][:4 * nm].reshape(-1, 4)[ko]
    kp_g = r["kp"][kg]
    assert np.isfinite(kp_g).all()
    # A whole-cell shift matches all 64 window positions nearly equally
    # well, so the fine argmax is a near tie on most matches.
    fs = o["fine_margin"][ko] > MARGIN
    assert fs.sum() >= 20
    np.testing.assert_allclose(kp_g[fs], kp_o[fs], atol=1e-3, rtol=0)


def sure_rows(o, w, h):
    """Rows whose match decision has a relative top-2 margin above MARGIN
    in its row, in its argmax column, and against the 0.2 threshold."""
    ra = o["row_arg"]
    rs = o["row_margin"] / np.maximum(o["row_max"], 1e-30) > MARGIN
    cs = o["col_margin"] / np.maximum(o["col_max"], 1e-30) > MARGIN
    return rs & cs[ra] & (np.abs(o["row_max"] - 0.2) > MARGIN * 0.2)


def check_coarse_indices(r, o, min_sure=0.8):
    """Row maxima within TOL; row and column first argmaxes bit-exact on
    rows / columns whose relative top-2 margin exceeds MARGIN (at least
    min_sure of them)."""
    assert rel(r["row_max"], o["row_max"]) <= TOL
    sure = o["row_margin"] / np.maximum(o["row_max"], 1e-30) > MARGIN
    assert sure.mean() > min_sure
    assert np.array_equal(r["row_arg"][sure], o["row_arg"][sure])
    sure_c = o["col_margin"] / np.maximum(o["col_max"], 1e-30) > MARGIN
    assert sure_c.mean() > min_sure
    assert np.array_equal(r["col_arg"][sure_c], o["col_arg"][sure_c])


def test_network_from_torch_checkpoint(dev, ic, weights, weights_file, tmp_path):
    """The ELoFTR weights in a torch.save zip archive (under "state_dict")
    give the same coarse statistics and matches bit for bit."""
    H, W = 128, 160
    print(f"[eloftr] network {H}x{W} from a torch.save checkpoint", flush=True)
    pth = synth.save_torch(weights, tmp_path / "eloftr.pth", wrap="state_dict")
    g0, g1 = synth.eloftr_noise_pair(H, W, shift=(8, 16))
    out = []
    for p in (weights_file, pth):
        net = ic.Eloftr(dev, p, H, W)
        try:
            out.append(net.match(g0, g1))
        finally:
            net.close()
    a, b = out
    assert a["nm"] == b["nm"] > 0
    for k in ("row_max", "row_arg", "col_arg", "mi", "mj", "mconf", "kp"):
        assert np.array_equal(a[k], b[k]), k


@pytest.mark.parametrize("h,w,seed", [(80, 80, 0), (13, 37, 1), (1, 1, 2), (100, 2, 3)])
def test_mutual_kernel(dev, ic, h, w, seed):
    """eloftr_mutual (the mutual selection of eloftr.c:606-636 on the
    device) against the rule stated in numpy: kept in raster order when
    the confidence exceeds 0.2 (NaN does not), the column argmax points
    back, and both cells lie 2 cells inside; cells as (x0, y0, x1, y1)."""
    rng = np.random.default_rng(seed)
    n = h * w
    rarg = rng.integers(0, n, n).astype(np.int32)
    carg = rng.integers(0, n, n).astype(np.int32)
    mutual = rng.uniform(size=n) < 0.5
    carg[rarg[mutual]] = np.nonzero(mutual)[0]
    rmax = rng.uniform(0, 0.5, n).astype(np.float32)
    rmax[rng.uniform(size=n) < 0.05] = np.nan
    rmax[rng.uniform(size=n) < 0.05] = 0.2
    i = np.arange(n)
    xi, yi, xj, yj = i % w, i // w, rarg % w, rarg // w
    keep = ((rmax > 0.2) & (carg[rarg] == i) & (xi >= 2) & (yi >= 2) & (xi < w - 2)
            & (yi < h - 2) & (xj >= 2) & (yj >= 2) & (xj < w - 2) & (yj < h - 2))
    br, ba, bc = dev.upload(rmax), dev.upload(rarg), dev.upload(carg)
    bi, bj, bm = dev.upload(np.full(n, -1, np.int32)), dev.upload(np.full(n, -1, np.int32)), \
        dev.zeros(n)
    cells = dev.upload(np.full(4 * n, -1, np.int32))
    cnt = dev.upload(np.full(2, -1, np.int32))
    dev.api.eloftr_mutual(dev.po, br.mem, ba.mem, bc.mem, h, w, 2, 0.2, bi.mem, bj.mem,
                          bm.mem, cells.mem, cnt.mem)
    c = dev.read(cnt, 2, np.int32)
    k = np.nonzero(keep)[0]
    assert c[1] == 0 and c[0] == len(k)
    assert np.array_equal(dev.read(bi, n, np.int32)[:len(k)], k)
    assert np.array_equal(dev.read(bj, n, np.int32)[:len(k)], rarg[k])
    assert np.array_equal(dev.read(bm, n)[:len(k)], rmax[k])
    got = dev.read(cells, 4 * n, np.int32).reshape(n, 4)[:len(k)]
    assert np.array_equal(got, np.stack([xi[k], yi[k], xj[k], yj[k]], 1))
    # An out-of-range row argmax is flagged for the host's error.
    rarg[n // 2] = n
    ba2 = dev.upload(rarg)
    dev.api.eloftr_mutual(dev.po, br.mem, ba2.mem, bc.mem, h, w, 2, 0.2, bi.mem, bj.mem,
                          bm.mem, cells.mem, cnt.mem)
    assert dev.read(cnt, 2, np.int32)[1] == 1


def test_graph_replays_match_eager(dev, ic, weights_file):
    """The pair's whole device stage recorded once as a HIP graph
    (eloftr_match_enqueue between ocl_graph_begin / ocl_graph_end) and
    replayed three times, with eager matches of another pair and host
    synchronisations between the replays: every replay gives the eager
    matches, confidences and keypoints bit for bit."""
    H, W = 128, 160
    print(f"[eloftr] graph replays {H}x{W}", flush=True)
    g0, g1 = synth.eloftr_noise_pair(H, W, shift=(8, 16))
    h0, h1 = synth.eloftr_noise_pair(H, W, shift=(0, 8), seed=5)
    net = ic.Eloftr(dev, weights_file, H, W)
    api, lib = dev.api, ic.lib()
    graph = None
    try:
        b0, b1, c0, c1 = dev.upload(g0), dev.upload(g1), dev.upload(h0), dev.upload(h1)
        net.match_device(b0, b1)
        ref = {k: np.array(v, copy=True) if hasattr(v, "__len__") else v
               for k, v in net.result().items()}
        assert ref["nm"] > 50
        api.ocl_graph_begin(dev.pb)
        api.eloftr_match_enqueue(net.m, b0.mem, b1.mem)
        graph = api.ocl_graph_end(dev.pb)
        for rep in range(3):
            net.match_device(c0, c1)
            other = net.result()["nm"]
            dev.finish()
            api.ocl_graph_launch(dev.pb, graph)
            api.eloftr_match_collect(net.m)
            got = net.result()
            assert got["nm"] == ref["nm"], (rep, other)
            for k in ("mi", "mj", "mconf", "kp"):
                assert np.array_equal(np.asarray(got[k]), ref[k]), (rep, k)
    finally:
        if graph:
            lib.ocl_graph_free(graph)
        net.close()

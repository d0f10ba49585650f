# SPDX-License-Identifier: Unlicense
"""GPU: the HIP path against the oracle at every BASELINE config's full
size, through the fixtures of tests/golden/fullsize_golden.npz (written
in the build container by tests/golden/make_fullsize_golden.py from the
oracle: the C restatement of the reference's kernels and schedules).

Tolerances, as in the small-size tests:
  * features, scores and contractions within 1e-3 of the reference's
    largest magnitude; warps within 1e-3 (normalised units); ELoFTR's
    dual-softmax confidences (exponentials of the score contraction)
    within 1e-3, or where they are not, within the log difference that
    score errors of 1e-3 of the largest score imply (check_conf);
  * integer outputs (row / column first argmax, mutual matches, fine
    window argmax, RoMa anchor cells, kept DISK keypoints) bit-exact
    wherever the oracle's relative top-2 margin exceeds 1e-3;
  * fine keypoints within 1e-3 px on matches whose fine argmax margin
    exceeds 1e-3, and on at least 90 % of all matches.
Each section first checks the checksum of its inputs, so a change of the
synthetic data fails here instead of comparing different inputs."""

import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
sys.path.insert(0, str(ROOT / "i.coregistration.opencl_amd"))
sys.path.insert(0, str(HERE / "golden"))
import synth  # noqa: E402
from make_fullsize_golden import M_NOISE, digest  # noqa: E402

import disk_ref  # noqa: E402

GOLDEN = HERE / "golden" / "fullsize_golden.npz"
TOL = 1e-3
MARGIN = 1e-3


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN)


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


def score_scale(x0, x1):
    """Largest |S| of the coarse scores S = F0 F1^T / (256 * 0.1) from the
    device's (256, n) features, in double on the host."""
    return float(np.abs((x0.astype(np.float64).T @ x1.astype(np.float64)) / 25.6).max())


def check_conf(got, ref, smax, what):
    """Dual-softmax confidences (row maxima, match confidences): each
    within TOL of the largest, or, where that fails, within the error a
    score tolerance implies. A confidence is the exponential of the
    contraction S: log conf = 2 s - lse_row - lse_col moves by at most
    4 delta for a score error delta, and the contraction tolerance allows
    delta = TOL |S|max, so log conf may move by 4 TOL |S|max."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    plain = d <= TOL * max(np.abs(ref).max(), 1e-30)
    with np.errstate(divide="ignore"):
        dl = np.abs(np.log(np.maximum(got, 1e-300)) - np.log(np.maximum(ref, 1e-300)))
    bound = 4 * TOL * smax
    i = int(np.argmax(d))
    print(f"[full] {what}: largest difference {d[i]:.3e} ({ref[i]:.6f} vs {got[i]:.6f}); "
          f"{int((~plain).sum())} beyond TOL of the largest, their log difference at most "
          f"{dl[~plain].max() if (~plain).any() else 0.0:.3e} (bound {bound:.3e}, "
          f"|S|max {smax:.2f})", flush=True)
    assert (plain | ((ref > 0) & (dl <= bound))).all()


def check_coarse(r, g, pre, min_sure, smax):
    """Row maxima as check_conf; row and column first argmaxes bit-exact on
    the rows / columns whose relative top-2 margin exceeds MARGIN (at
    least min_sure of them)."""
    check_conf(r["row_max"], g[pre + "row_max"], smax, f"{pre}row maxima")
    rs = g[pre + "row_margin"] / np.maximum(g[pre + "row_max"], 1e-30) > MARGIN
    cs = g[pre + "col_margin"] / np.maximum(g[pre + "col_max"], 1e-30) > MARGIN
    print(f"[full] {pre}: margin-sure rows {rs.mean():.3f}, columns {cs.mean():.3f}", flush=True)
    assert rs.mean() >= min_sure and cs.mean() >= min_sure
    assert np.array_equal(r["row_arg"][rs], g[pre + "row_arg"][rs])
    assert np.array_equal(r["col_arg"][cs], g[pre + "col_arg"][cs])


@pytest.fixture(scope="module")
def eloftr_weights_file(tmp_path_factory):
    p = tmp_path_factory.mktemp("w") / "eloftr_random.safetensors"
    return synth.eloftr_weights_file(p)


def test_eloftr_640_config_pair_vs_oracle(dev, ic, gold, eloftr_weights_file):
    """The headline pair (640 x 640, blurred noise under a random affine):
    coarse features on 4096 seeded entries, the 6400 row maxima, row and
    column argmaxes, and the (empty or not) match list."""
    H = W = 640
    print(f"[full] ELoFTR {H}x{W} config pair", flush=True)
    g0, g1, _ = synth.eloftr_pair(H, W)
    assert np.array_equal(digest(g0, g1), gold["e_digest"])
    net = ic.Eloftr(dev, eloftr_weights_file, H, W)
    try:
        r = net.match(g0, g1)
        n = (H // 8) * (W // 8)
        idx = gold["e_coarse_idx"]
        x = [net.buffer(f"x{k}", 256 * n) for k in range(2)]
        for k in range(2):
            assert rel(x[k][idx], gold[f"e_coarse{k}"]) <= TOL
    finally:
        net.close()
    check_coarse(r, gold, "e_", 0.9, score_scale(x[0].reshape(256, n), x[1].reshape(256, n)))
    assert r["nm"] == int(gold["e_nm"])


def test_eloftr_640_matches_and_fine_vs_oracle(dev, ic, gold, eloftr_weights_file):
    """The 640 x 640 pair with matches (B = A shifted by whole cells,
    noise 0.05): coarse statistics, the match list (differences only on
    rows decided within the margin), match confidences, and the fine
    keypoints: within 1e-3 px wherever the fine argmax's relative top-2
    margin exceeds 1e-3, and on at least 90 % of all matches."""
    H = W = 640
    print(f"[full] ELoFTR {H}x{W} pair with matches", flush=True)
    g0, g1 = synth.eloftr_noise_pair(H, W, shift=(8, 16), noise=float(gold["m_noise"]))
    assert float(gold["m_noise"]) == M_NOISE
    assert np.array_equal(digest(g0, g1), gold["m_digest"])
    net = ic.Eloftr(dev, eloftr_weights_file, H, W)
    n = (H // 8) * (W // 8)
    try:
        r = net.match(g0, g1)
        x = [net.buffer(f"x{k}", 256 * n) for k in range(2)]
    finally:
        net.close()
    idx = gold["m_coarse_idx"]
    for k in range(2):
        print(f"[full] m_: coarse features {k} within {rel(x[k][idx], gold[f'm_coarse{k}']):.3e}"
              " of the largest", flush=True)
        assert rel(x[k][idx], gold[f"m_coarse{k}"]) <= TOL
    smax = score_scale(x[0].reshape(256, n), x[1].reshape(256, n))
    # The shifted pair's confidences saturate: about 90 % of the rows
    # and columns have no confidence at all (exp underflows to 0, no
    # margin), so fewer of them are margin-sure here (9 %: the matched
    # ones and their neighbours).
    check_coarse(r, gold, "m_", 0.05, smax)
    nm = int(gold["m_nm"])
    assert nm > 500
    h, w = H // 8, W // 8
    ra = gold["m_row_arg"]
    rs = gold["m_row_margin"] / np.maximum(gold["m_row_max"], 1e-30) > MARGIN
    cs = gold["m_col_margin"] / np.maximum(gold["m_col_max"], 1e-30) > MARGIN
    sure = rs & cs[ra] & (np.abs(gold["m_row_max"] - 0.2) > MARGIN * 0.2)
    om = {int(i): k for k, i in enumerate(gold["m_mi"])}
    gm = {int(i): k for k, i in enumerate(r["mi"])}
    for i in set(om) ^ set(gm):
        assert not sure[i], f"match row {i} differs from the oracle with a sure margin"
    common = sorted(set(om) & set(gm))
    assert len(common) >= 0.95 * nm
    ko = np.array([om[i] for i in common])
    kg = np.array([gm[i] for i in common])
    assert np.array_equal(r["mj"][kg], gold["m_mj"][ko])
    check_conf(r["mconf"][kg], gold["m_mconf"][ko], smax, "match confidences")
    kp_o, kp_g = gold["m_kp"][ko], r["kp"][kg]
    assert np.isfinite(kp_g).all()
    err = np.abs(kp_g - kp_o).max(1)
    fs = gold["m_fine_rel_margin"][ko] > MARGIN
    print(f"[full] fine: {len(common)} common matches, {fs.mean():.3f} margin-sure; within "
          f"1e-3 px: {(err <= 1e-3).mean():.4f} of all, {(err[fs] <= 1e-3).mean():.4f} of sure",
          flush=True)
    assert (err[fs] <= 1e-3).all()
    assert (err <= 1e-3).mean() >= 0.9


def _unsure(heat, thresh, n):
    """Cells whose NMS or top-n decision the oracle takes by less than
    TOL of the heatmap's scale."""
    h, w = heat.shape
    sc = np.abs(heat).max()
    x = np.pad(heat.astype(np.float64), 2, constant_values=-np.inf)
    nb = np.full((h, w), -np.inf)
    for dy in range(5):
        for dx in range(5):
            if dy != 2 or dx != 2:
                nb = np.maximum(nb, x[dy:dy + h, dx:dx + w])
    unsure = (np.abs(heat - nb) < TOL * sc) | (np.abs(heat - thresh) < TOL * sc)
    mask = disk_ref.nms_mask(heat, thresh)
    cand = np.sort(heat[mask])[::-1]
    if len(cand):
        cut = cand[min(n, len(cand) - 1)]
        unsure |= mask & (np.abs(heat - cut) < TOL * sc)
    return unsure


def test_disk_512_vs_oracle(dev, ic, gold, tmp_path):
    """DISK at 512 x 512, n = 2048: the heatmap within 1e-3, the kept set
    equal to the oracle's except cells whose NMS or top-n decision is
    within the margin, scores within 1e-3, descriptors of 512 seeded
    keypoints within 1e-3."""
    H = W = 512
    n = 2048
    print(f"[full] DISK {H}x{W} n={n}", flush=True)
    img = synth.disk_image(H, W)
    assert np.array_equal(digest(img), gold["d_digest"])
    fpath = synth.disk_weights_file(tmp_path / "disk_random.safetensors")
    net = ic.Disk(dev, fpath, H, W, nmax=n)
    try:
        g = net.detect(img, n=n, thresh=0.0)
        heat = net.buffer("out", H * W, off=128 * H * W).reshape(H, W)
    finally:
        net.close()
    oh = gold["d_heat"]
    assert rel(heat, oh) < TOL
    oxy = gold["d_xy"].reshape(-1, 2)
    assert g["n"] == int(gold["d_n"]) == n
    unsure = _unsure(oh, 0.0, n)
    sg, so = {tuple(p) for p in g["xy"]}, {tuple(p) for p in oxy}
    print(f"[full] DISK kept sets differ on {len(sg ^ so)} cells", flush=True)
    for x, y in sg ^ so:
        assert unsure[y, x], (x, y)
    assert len(sg ^ so) <= 0.01 * n
    gi = {tuple(p): i for i, p in enumerate(g["xy"])}
    osc = dict(zip(map(tuple, oxy), gold["d_score"]))
    common = [p for p in map(tuple, oxy) if p in gi]
    assert rel([g["score"][gi[p]] for p in common], [osc[p] for p in common]) < TOL
    sel = [(k, tuple(oxy[i])) for k, i in enumerate(gold["d_desc_idx"]) if tuple(oxy[i]) in gi]
    assert len(sel) >= 0.99 * len(gold["d_desc_idx"])
    gd = np.array([g["desc"][gi[p]] for _, p in sel])
    od = gold["d_desc"][[k for k, _ in sel]]
    assert rel(gd, od) < TOL


def _read_dump(folder, what, tile=1):
    return np.fromfile(Path(folder) / f"tile{tile:03d}_roma_{what}.f32", np.float32)


@pytest.fixture(scope="module")
def roma_files(tmp_path_factory):
    return synth.roma_weights_files(tmp_path_factory.mktemp("roma_w"))


def check_anchors(cls_flow, g, pre):
    """The coarse warp's anchor cells: equal (warp within 1e-4) on tokens
    whose anchor logit margin exceeds MARGIN (at least 90 % of them).
    Returns whether every token agrees."""
    sure = g[pre + "anchor_margin"] > MARGIN
    d = np.abs(cls_flow - g[pre + "cls_flow"]).max(0)
    print(f"[full] {pre}: anchor-sure tokens {sure.mean():.3f}; tokens whose warp differs: "
          f"{int((d > 1e-4).sum())}", flush=True)
    assert sure.mean() > 0.9
    assert d[sure].max() < 1e-4
    return bool((d <= 1e-4).all())


def test_roma_560_vs_oracle(dev, ic, gold, roma_files, tmp_path):
    """RoMa's coarse pass at 560 x 560 (DINOv2 x 2, GP, decoder): DINOv2
    features, GP posterior and anchor logits on seeded entries within
    1e-3, anchor cells bit-exact where the logit margin is sure, the
    coarse certainty within 1e-3; then roma_match's final warp and
    certainty at 560 on seeded cells."""
    S = 560
    print(f"[full] RoMa {S}x{S}", flush=True)
    fm, fd, _ = roma_files
    a, b, _ = synth.roma_pair(S, S)
    assert np.array_equal(digest(a, b), gold["r_digest"])
    net = ic.Roma(dev, fm, fd, S, S)
    try:
        got = net.match(a, b, dump=str(tmp_path), tile=1)
        assert net.gp_info() == 0
    finally:
        net.close()
    n16 = (S // 14) ** 2
    for k in range(2):
        assert rel(_read_dump(tmp_path, f"dino_{k}")[gold["r_dino_idx"]], gold[f"r_dino{k}"]) < TOL
    assert rel(_read_dump(tmp_path, "gp")[gold["r_gp_idx"]], gold["r_gp"]) < TOL
    cls_flow = _read_dump(tmp_path, "cls_flow").reshape(2, n16)
    all_agree = check_anchors(cls_flow, gold, "r_")
    assert rel(_read_dump(tmp_path, "cls_cert"), gold["r_cls_cert"]) < TOL
    ci = gold["r_cell_idx"]
    flow = got["flow"].reshape(2, -1)[:, ci]
    cert = got["cert"].ravel()[ci]
    if all_agree:
        assert np.abs(flow - gold["r_flow"]).max() < TOL
        assert np.abs(cert - gold["r_cert"]).max() < TOL
    else:
        # A near-tied anchor moves the warp near its token only.
        ok = np.abs(flow - gold["r_flow"]).max(0) < TOL
        assert ok.mean() > 0.95


def test_refiners_864_vs_oracle(dev, ic, gold, roma_files):
    """The refiner config (864 x 864: VGG19-BN on both images, refiners
    at 1/8 .. 1/1 from the synthetic initial warp; roma_refine_device):
    the final warp and certainty logit on 4096 seeded cells against the
    oracle's fine pass (orc_roma_refine) within 1e-3."""
    H = W = 864
    print(f"[full] refiners {H}x{W}", flush=True)
    fm, fd, _ = roma_files
    a, b, flow8, cert8 = synth.roma_refine_inputs(H, W)
    pa, pb = synth.imagenet_norm(a), synth.imagenet_norm(b)
    assert np.array_equal(digest(pa, pb, flow8, cert8), gold["f_digest"])
    net = ic.Roma(dev, fm, fd, H, W)
    try:
        fl, ce = net.refine_device(dev.upload(np.stack([pa, pb])), dev.upload(flow8),
                                   dev.upload(cert8))
        flow = net.buffer(fl, 2 * H * W).reshape(2, -1)
        cert = net.buffer(ce, H * W)
    finally:
        net.close()
    ci = gold["f_cell_idx"]
    assert np.abs(flow[:, ci] - gold["f_flow"]).max() < TOL
    assert np.abs(cert[ci] - gold["f_cert"]).max() < TOL * max(1.0, np.abs(gold["f_cert"]).max())


def test_roma_v2ref_1024_vs_oracle(dev, ic, gold, roma_files, tmp_path):
    """roma_v2ref at 1024 x 1024 (coarse 560 with both VGG19-BN stacks, v2
    refiners at 1/4, 1/2, 1/1, epilogue): anchor cells as above, then the
    final warp, certainty and standard deviation on 4096 seeded cells."""
    H = W = 1024
    print(f"[full] roma_v2ref {H}x{W}", flush=True)
    fm, fd, f2 = roma_files
    a, b, _ = synth.roma_pair(H, W, seed=synth.BASE_SEED + synth.CONFIG_V2REF)
    assert np.array_equal(digest(a, b), gold["v_digest"])
    net = ic.Roma(dev, fm, fd, H, W, v2_path=f2)
    try:
        got = net.match(a, b, dump=str(tmp_path), tile=1)
        assert net.gp_info() == 0
    finally:
        net.close()
    n16 = (560 // 14) ** 2
    all_agree = check_anchors(_read_dump(tmp_path, "cls_flow").reshape(2, n16), gold, "v_")
    ci = gold["v_cell_idx"]
    flow = got["flow"].reshape(2, -1)[:, ci]
    cert, sd = got["cert"].ravel()[ci], got["sd"].ravel()[ci]
    ok = (np.abs(flow - gold["v_flow"]).max(0) < TOL) & (np.abs(cert - gold["v_cert"]) < TOL)
    both = np.isfinite(sd) & np.isfinite(gold["v_sd"])
    assert both.mean() > 0.99
    ok_sd = np.abs(sd[both] - gold["v_sd"][both]) <= TOL * np.abs(gold["v_sd"][both]).max()
    print(f"[full] v2ref: cells within 1e-3: {ok.mean():.4f}; sd within 1e-3: "
          f"{ok_sd.mean():.4f}", flush=True)
    if all_agree:
        assert ok.all() and ok_sd.all()
    else:
        assert ok.mean() > 0.95 and ok_sd.mean() > 0.95

# SPDX-License-Identifier: Unlicense
"""Write tests/golden/fullsize_golden.npz: the oracle's outputs (oracle/,
the C restatement of the reference's kernels and schedules) on every
BASELINE config at its full size, compact enough to commit, so that the
GPU tests compare the HIP path with the oracle at the benchmark sizes
without running the oracle (minutes of CPU) on the GPU box.

Sections (inputs and weights are the seeded synthetic ones of synth.py;
each section stores a checksum of its inputs so a test fails loudly if
they drift):

  e_*  ELoFTR 640 x 640, the config pair: coarse row maxima, row and
       column first argmaxes with their top-2 margins, a seeded
       subsample of the coarse features; the mutual selection.
  m_*  ELoFTR 640 x 640 on the pair that yields coarse matches (B = A
       shifted by whole cells, noise 0.05): the same, plus the match
       list, the fine
       keypoints and each match's relative top-2 margin of the fine
       argmax (elo_ref.fine_bruteforce on the oracle's fine maps).
  d_*  DISK 512 x 512, n = 2048: the heatmap, kept keypoints, scores,
       descriptors of a seeded subset.
  r_*  RoMa at 560 x 560 (coarse 560): DINOv2 features and GP posterior
       (subsamples), anchor logits (subsample) with each token's argmax
       and relative top-2 margin, the coarse warp and certainty, the
       final warp and certainty on seeded cells.
  f_*  RoMa refiners at 864 x 864 from the synthetic initial 1/8 warp
       (orc_roma_refine): the final warp and certainty logit on seeded
       cells.
  v_*  roma_v2ref at 1024 x 1024: coarse warp, anchor argmaxes and
       margins, final warp, certainty and standard deviation on seeded
       cells.

    python tests/golden/make_fullsize_golden.py [section ...]

Existing sections in the file are kept when only some are rebuilt.
"""

import hashlib
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(ROOT / "i.coregistration.opencl_amd"))

import elo_ref  # noqa: E402
import synth  # noqa: E402
from oracle_lib import disk_detect, eloftr_forward, roma_forward, roma_refine  # noqa: E402

OUT = HERE / "fullsize_golden.npz"
NSAMPLE = 4096
# B's noise in the ELoFTR pair with matches: decisive fine argmaxes (see
# synth.eloftr_noise_pair).
M_NOISE = 0.05


def digest(*arrays):
    """Checksum of input arrays (their float32 / int bytes)."""
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return np.frombuffer(h.digest()[:16], np.uint8).copy()


def sample(n, k, seed):
    """k sorted distinct indices of range(n), seeded."""
    rng = np.random.default_rng(seed)
    return np.sort(rng.choice(n, size=min(k, n), replace=False)).astype(np.int64)


def coarse_stats(o, pre):
    return {f"{pre}row_max": o["row_max"], f"{pre}row_arg": o["row_arg"],
            f"{pre}col_arg": o["col_arg"], f"{pre}row_margin": o["row_margin"],
            f"{pre}col_margin": o["col_margin"], f"{pre}col_max": o["col_max"]}


def section_e():
    H = W = 640
    w = synth.eloftr_weights_calibrated()
    g0, g1, _ = synth.eloftr_pair(H, W)
    o = eloftr_forward(w, g0, g1, coarse=True)
    n = (H // 8) * (W // 8)
    idx = sample(256 * n, NSAMPLE, 101)
    out = {"e_digest": digest(g0, g1), "e_nm": np.int64(o["nm"]), "e_coarse_idx": idx,
           "e_coarse0": o["coarse"][0][idx], "e_coarse1": o["coarse"][1][idx]}
    out.update(coarse_stats(o, "e_"))
    return out


def section_m():
    H = W = 640
    w = synth.eloftr_weights_calibrated()
    g0, g1 = synth.eloftr_noise_pair(H, W, shift=(8, 16), noise=M_NOISE)
    o = eloftr_forward(w, g0, g1, coarse=True, fine=True)
    nm = o["nm"]
    cells_i, cells_j = o["mi"][:nm], o["mj"][:nm]
    wc = W // 8
    cells = np.stack([cells_i % wc, cells_i // wc, cells_j % wc, cells_j // wc], 1)
    fine0 = o["fine"][0].reshape(64, H, W)
    fine1 = o["fine"][1].reshape(64, H, W)
    kp_bf, rmargin = elo_ref.fine_bruteforce(fine0, fine1, cells)
    kp = o["kp"][:4 * nm].reshape(-1, 4)
    print(f"[m] nm {nm}; oracle kp vs float64 brute force on sure matches: "
          f"{np.abs(kp - kp_bf)[rmargin > 1e-3].max():.2e} px; relative fine margin > 1e-3: "
          f"{(rmargin > 1e-3).mean():.3f}, > 1e-4: {(rmargin > 1e-4).mean():.3f}, > 1e-5: "
          f"{(rmargin > 1e-5).mean():.3f}", flush=True)
    n = (H // 8) * (W // 8)
    idx = sample(256 * n, NSAMPLE, 102)
    out = {"m_digest": digest(g0, g1), "m_noise": np.float64(M_NOISE), "m_nm": np.int64(nm),
           "m_coarse_idx": idx, "m_coarse0": o["coarse"][0][idx],
           "m_coarse1": o["coarse"][1][idx], "m_mi": o["mi"][:nm],
           "m_mj": o["mj"][:nm], "m_mconf": o["mconf"][:nm], "m_kp": kp,
           "m_fine_rel_margin": rmargin.astype(np.float32)}
    out.update(coarse_stats(o, "m_"))
    return out


def section_d():
    H = W = 512
    n = 2048
    w = synth.disk_weights()
    img = synth.disk_image(H, W)
    r = disk_detect(w, img, n=n, thresh=0.0, full=True)
    nk = r["n"]
    heat = r["out"][128]
    sel = sample(nk, 512, 303)
    return {"d_digest": digest(img), "d_n": np.int64(nk), "d_xy": r["xy"][:nk].astype(np.int32),
            "d_score": r["score"][:nk], "d_heat": heat.astype(np.float32), "d_desc_idx": sel,
            "d_desc": r["desc"][:nk][sel]}


def _anchor(logits):
    s = np.sort(logits[:, :4096], 1)
    arg = np.argmax(logits[:, :4096], 1)
    return arg.astype(np.int32), ((s[:, -1] - s[:, -2]) /
                                  np.maximum(np.abs(s[:, -1]), 1e-30)).astype(np.float32)


def section_r():
    S = 560
    wm, wd = synth.roma_weights(), synth.dino_weights()
    a, b, _ = synth.roma_pair(S, S)
    o = roma_forward(wm, wd, None, a, b, S)
    assert o["info"] == 0
    n16 = (S // 14) ** 2
    arg, margin = _anchor(o["logits"])
    di = sample(1024 * n16, NSAMPLE, 401)
    gi = sample(512 * n16, NSAMPLE, 402)
    li = sample(4097 * n16, NSAMPLE, 403)
    ci = sample(S * S, NSAMPLE, 404)
    print(f"[r] anchor margins: min {margin.min():.2e}, < 1e-3: {(margin < 1e-3).sum()}, "
          f"< 1e-4: {(margin < 1e-4).sum()}", flush=True)
    return {"r_digest": digest(a, b), "r_dino_idx": di, "r_dino0": o["dino"][0].ravel()[di],
            "r_dino1": o["dino"][1].ravel()[di], "r_gp_idx": gi, "r_gp": o["gp"].ravel()[gi],
            "r_logit_idx": li, "r_logit": o["logits"].ravel()[li], "r_anchor": arg,
            "r_anchor_margin": margin, "r_cls_flow": o["cls_flow"], "r_cls_cert": o["cls_cert"],
            "r_cell_idx": ci, "r_flow": o["flow"].reshape(2, -1)[:, ci],
            "r_cert": o["cert"].ravel()[ci]}


def section_f():
    H = W = 864
    wm, wd = synth.roma_weights(), synth.dino_weights()
    a, b, flow8, cert8 = synth.roma_refine_inputs(H, W)
    pa, pb = synth.imagenet_norm(a), synth.imagenet_norm(b)
    o = roma_refine(wm, wd, pa, pb, flow8, cert8, 560)
    ci = sample(H * W, NSAMPLE, 510)
    return {"f_digest": digest(pa, pb, flow8, cert8), "f_cell_idx": ci,
            "f_flow": o["flow"].reshape(2, -1)[:, ci], "f_cert": o["cert"].ravel()[ci]}


def section_v():
    H = W = 1024
    wm, wd, w2 = synth.roma_weights(), synth.dino_weights(), synth.roma2_weights()
    a, b, _ = synth.roma_pair(H, W, seed=synth.BASE_SEED + synth.CONFIG_V2REF)
    o = roma_forward(wm, wd, w2, a, b, 560)
    assert o["info"] == 0
    arg, margin = _anchor(o["logits"])
    ci = sample(H * W, NSAMPLE, 601)
    print(f"[v] anchor margins: min {margin.min():.2e}, < 1e-3: {(margin < 1e-3).sum()}, "
          f"< 1e-4: {(margin < 1e-4).sum()}", flush=True)
    return {"v_digest": digest(a, b), "v_anchor": arg, "v_anchor_margin": margin,
            "v_cls_flow": o["cls_flow"], "v_cell_idx": ci,
            "v_flow": o["flow"].reshape(2, -1)[:, ci], "v_cert": o["cert"].ravel()[ci],
            "v_sd": o["sd"].ravel()[ci]}


SECTIONS = {"e": section_e, "m": section_m, "d": section_d, "r": section_r, "f": section_f,
            "v": section_v}


def main(names):
    names = names or list(SECTIONS)
    data = dict(np.load(OUT)) if OUT.exists() else {}
    for s in names:
        t0 = time.time()
        got = SECTIONS[s]()
        data = {k: v for k, v in data.items() if not k.startswith(s + "_")}
        data.update(got)
        np.savez_compressed(OUT, **data)
        print(f"[{s}] {len(got)} arrays in {time.time() - t0:.0f} s", flush=True)
    print(f"{OUT}: {OUT.stat().st_size / 1e6:.2f} MB")


if __name__ == "__main__":
    main(sys.argv[1:])

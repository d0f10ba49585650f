# SPDX-License-Identifier: Unlicense
"""CPU: pins of the oracle's ELoFTR functions.

* coarse dual softmax (eloftr_kernels.cl:10-144) against the brute-force
  float64 formulation over the whole score matrix;
* mutual / threshold / border selection (eloftr.c:552-566) by its defining
  properties;
* two-stage fine matching (eloftr_kernels.cl:146-295) against the authors'
  formulation in float64;
* the whole network schedule (eloftr.c:358-681) against Hugging Face
  transformers' EfficientLoFTR in float64 (committed fixture)."""

import sys
from pathlib import Path

import numpy as np
import pytest

import elo_ref
from oracle_lib import eloftr_forward, fp, ip

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "i.coregistration.opencl_amd"))
import synth  # noqa: E402

GOLDEN = Path(__file__).resolve().parent / "golden" / "eloftr_golden.npz"


def oracle_coarse(orc, F0, F1, alpha, blk):
    n, D = F0.shape
    rmax = np.zeros(n, np.float32)
    rarg, carg = np.zeros(n, np.int32), np.zeros(n, np.int32)
    rmar, cmar = np.zeros(n, np.float32), np.zeros(n, np.float32)
    orc.orc_eloftr_coarse(fp(F0), fp(F1), n, D, alpha, blk, fp(rmax), ip(rarg),
                          ip(carg), fp(rmar), fp(cmar), None)
    return rmax, rarg, carg, rmar, cmar


@pytest.mark.parametrize("blk", [500, 128, 37])
def test_coarse_vs_bruteforce(orc, blk):
    rng = np.random.default_rng(11)
    F0, F1 = elo_ref.match_features(rng, 500, 64)
    alpha = np.float32(1.0) / np.float32(64 * 0.1)
    conf, rmax, rarg, carg = elo_ref.coarse_bruteforce(F0, F1, float(alpha))
    o_rmax, o_rarg, o_carg, o_rmar, o_cmar = oracle_coarse(orc, F0, F1, alpha, blk)
    assert np.abs(o_rmax - rmax).max() <= 1e-5 * rmax.max()
    rel_r = o_rmar / np.maximum(o_rmax, 1e-30)
    sure = rel_r > 1e-4
    assert sure.mean() > 0.9
    assert np.array_equal(o_rarg[sure], rarg[sure])
    cmax = conf.max(0)
    sure_c = o_cmar / np.maximum(cmax, 1e-30) > 1e-4
    assert np.array_equal(o_carg[sure_c], carg[sure_c])


def test_coarse_ties_take_first_index(orc):
    """Exact ties (duplicated tokens) resolve to the lowest index along
    rows and columns, the reference's first-argmax rule."""
    rng = np.random.default_rng(3)
    F0 = rng.standard_normal((64, 16)).astype(np.float32)
    F1 = np.concatenate([F0[:32], F0[:32]])      # columns j and j + 32 tie
    _, rarg, carg, _, _ = oracle_coarse(orc, F0, F1, np.float32(1.0), 64)
    assert (rarg < 32).all()


def test_select_properties(orc):
    rng = np.random.default_rng(5)
    h, w = 20, 24
    n = h * w
    F0, F1 = elo_ref.match_features(rng, n, 64, noise=0.5)
    rmax, rarg, carg, _, _ = oracle_coarse(orc, F0, F1, np.float32(1 / 6.4), n)
    mi, mj = np.zeros(n, np.int32), np.zeros(n, np.int32)
    mc = np.zeros(n, np.float32)
    nm = orc.orc_eloftr_select(fp(rmax), ip(rarg), ip(carg), h, w, 0.2, 2, ip(mi),
                               ip(mj), fp(mc))
    want = []
    for i in range(n):
        j = rarg[i]
        inside = lambda k: 2 <= k % w < w - 2 and 2 <= k // w < h - 2
        if rmax[i] > 0.2 and carg[j] == i and inside(i) and inside(j):
            want.append((i, j))
    assert nm == len(want) and nm > 50
    assert list(zip(mi[:nm], mj[:nm])) == want
    assert np.array_equal(mc[:nm], rmax[mi[:nm]])


def test_fine_vs_bruteforce(orc):
    rng = np.random.default_rng(9)
    H, W = 48, 64
    f0 = rng.standard_normal((64, H, W)).astype(np.float32)
    f1 = rng.standard_normal((64, H, W)).astype(np.float32)
    h, w = H // 8, W // 8
    cells = np.stack([rng.integers(0, w, 300), rng.integers(0, h, 300),
                      rng.integers(0, w, 300), rng.integers(0, h, 300)], 1).astype(np.int32)
    cells[:4] = [[0, 0, 0, 0], [w - 1, h - 1, w - 1, h - 1], [0, h - 1, w - 1, 0], [3, 2, 0, 0]]
    out = np.zeros(4 * len(cells), np.float32)
    mar = np.zeros(len(cells), np.float32)
    orc.orc_eloftr_fine(fp(f0), fp(f1), H, W, ip(np.ascontiguousarray(cells)), len(cells),
                        10.0, fp(out), fp(mar))
    ref, margin = elo_ref.fine_bruteforce(f0, f1, cells)
    out = out.reshape(-1, 4)
    sure = margin > 1e-4
    assert sure.mean() > 0.9
    np.testing.assert_allclose(out[sure], ref[sure], atol=1e-4, rtol=0)


@pytest.fixture(scope="module")
def golden_run():
    g = np.load(GOLDEN)
    H, W = int(g["H"]), int(g["W"])
    w = synth.eloftr_weights_calibrated()
    g0, g1, _ = synth.eloftr_pair(H, W)
    ck = np.array([float(np.sum(np.asarray(v, np.float64) ** 2)) for _, v in sorted(w.items())])
    assert np.allclose(ck, g["weights_checksum"], rtol=1e-12), "weight generator changed"
    o = eloftr_forward(w, g0, g1, backbone=True, coarse=True, fine=True)
    return g, o


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return np.abs(a - b).max() / np.abs(b).max()


def test_network_backbone_vs_transformers(golden_run):
    g, o = golden_run
    for k in range(2):
        assert rel(o["backbone"][k], g["backbone"][k]) < 1e-4


def test_network_transformer_vs_transformers(golden_run):
    g, o = golden_run
    for k in range(2):
        assert rel(o["coarse"][k], g["coarse"][k]) < 1e-4


def test_network_fusion_vs_transformers(golden_run):
    g, o = golden_run
    for k in range(2):
        assert rel(o["fine"][k][g["fine_idx"]], g["fine"][k]) < 1e-4


def test_network_planted_error_is_caught(golden_run):
    """A plausible mistake (the two images exchanged, which the order of
    the cross attentions makes visible) changes the transformer output far
    beyond the tolerance: the fixture discriminates."""
    g, _ = golden_run
    w = synth.eloftr_weights_calibrated()
    g0, g1, _ = synth.eloftr_pair(int(g["H"]), int(g["W"]))
    o = eloftr_forward(w, g1, g0, coarse=True)
    assert rel(o["coarse"][0], g["coarse"][0]) > 1e-2

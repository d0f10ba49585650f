# SPDX-License-Identifier: Unlicense
"""CPU: the oracle's restatement of roma_kernels.cl pinned against float64
torch statements of RoMa's published operations (roma_ref.py): cosine
kernel, cls_to_flow_refine, grid_sample, local_correlation, displacement,
v1 / v2 updates, depthwise 5 x 5. Each check would fail on a swapped axis,
a dropped term or an off-by-one cell offset."""

import numpy as np
import pytest
import torch

import roma_ref as R
from oracle_lib import fp

TOL = 2e-5


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


def test_row_norm_and_cos_exp(orc):
    rng = np.random.default_rng(1)
    N, M, C = 37, 53, 96
    X = rng.standard_normal((N, C)).astype(np.float32)
    Y = rng.standard_normal((M, C)).astype(np.float32)
    nx, ny = np.zeros(N, np.float32), np.zeros(M, np.float32)
    orc.orc_roma_row_norm(fp(X), N, C, fp(nx))
    orc.orc_roma_row_norm(fp(Y), M, C, fp(ny))
    assert rel(nx, torch.linalg.norm(R.t64(X), dim=1).numpy()) < TOL
    S = np.ascontiguousarray(X @ Y.T)
    T, eps = 0.2, 1e-6
    orc.orc_roma_cos_exp(fp(S), fp(nx), fp(ny), N, M, T, eps)
    x, y = R.t64(X), R.t64(Y)
    cos = (x @ y.T) / (x.norm(dim=1)[:, None] * y.norm(dim=1)[None] + eps)
    assert rel(S, torch.exp((cos - 1) / T).numpy()) < 1e-4


@pytest.mark.parametrize("res", [8, 16])
def test_cls_to_flow(orc, res):
    rng = np.random.default_rng(res)
    C, n = res * res, 300
    ld = C + 3
    L = (3 * rng.standard_normal((n, ld))).astype(np.float32)
    # modes on the grid's edges and corners (clamped neighbours) and a tie
    L[0, :C] = -5
    L[0, 0] = 9
    L[1, :C] = -5
    L[1, C - 1] = 9
    L[2, :C] = -5
    L[2, res - 1] = 9
    L[3, :C] = -5
    L[3, 5] = L[3, 9] = 9
    flow, cert = np.zeros(2 * n, np.float32), np.zeros(n, np.float32)
    orc.orc_roma_cls_to_flow(fp(L), ld, C, res, n, fp(flow), fp(cert))
    ref = R.cls_to_flow_refine(R.t64(L[:, :C]).T).numpy()
    assert rel(flow, ref) < TOL
    assert np.array_equal(cert, L[:, C])


def warps(rng, H, W, n_out=40):
    """Warps (2, H, W) around the identity, with some far outside, some
    on the border and one a million cells off (non-finite warps are the
    GPU tests' case: torch leaves them unspecified)."""
    gy, gx = np.meshgrid(R.cell_centres(H).numpy(), R.cell_centres(W).numpy(), indexing="ij")
    f = np.stack([gx, gy]) + 0.3 * rng.standard_normal((2, H, W))
    flat = f.reshape(2, -1)
    k = rng.choice(H * W, n_out, replace=False)
    flat[:, k[:10]] *= 3.0
    flat[0, k[10:15]] = 1.0
    flat[1, k[15:20]] = -1.0
    flat[0, k[20]] = 1e6
    return f.astype(np.float32)


def test_warp_sample(orc):
    rng = np.random.default_rng(3)
    C, H, W = 5, 19, 23
    x = rng.standard_normal((C, H, W)).astype(np.float32)
    f = warps(rng, H, W)
    out = np.zeros((C + 2, H * W), np.float32)
    orc.orc_roma_warp_sample(fp(x), C, H, W, fp(f), fp(out), 2)
    ref = R.grid_sample_flow(R.t64(x), R.t64(f)).reshape(C, -1).numpy()
    assert rel(out[2:], ref) < TOL
    assert not out[:2].any()


@pytest.mark.parametrize("C,H,W,r", [(16, 12, 17, 3), (32, 9, 11, 7), (8, 15, 13, 2)])
def test_local_corr(orc, C, H, W, r):
    rng = np.random.default_rng(C + r)
    f0 = rng.standard_normal((C, H, W)).astype(np.float32)
    f1 = rng.standard_normal((C, H, W)).astype(np.float32)
    f = warps(rng, H, W, n_out=24)
    K = (2 * r + 1) ** 2
    out = np.zeros((K + 1, H * W), np.float32)
    orc.orc_roma_local_corr(fp(f0), fp(f1), C, H, W, r, fp(f), fp(out), 1)
    ref = R.local_correlation(R.t64(f0), R.t64(f1), R.t64(f), r).reshape(K, -1).numpy()
    assert rel(out[1:], ref) < 1e-4
    assert not out[0].any()


def test_disp_and_updates(orc):
    rng = np.random.default_rng(5)
    H, W = 14, 22
    n = H * W
    flow = rng.uniform(-1, 1, (2, n)).astype(np.float32)
    out = np.zeros((2, n), np.float32)
    orc.orc_roma_disp(fp(flow), H, W, 11.0, 7.0, fp(out))
    assert rel(out, R.disp(R.t64(flow), H, W, 11.0, 7.0).numpy()) < TOL

    d = (4 * rng.standard_normal((6, n))).astype(np.float32)
    d[3, :5] = [25.0, -30.0, 0.0, 19.9, 20.1]
    f1, c1 = flow.copy(), rng.standard_normal(n).astype(np.float32)
    c1_0 = c1.copy()
    orc.orc_roma_update(fp(f1), fp(c1), fp(d), n, 0.5, 80.0, 60.0)
    ref_f = R.t64(flow) + 0.5 * R.t64(d[:2]) / torch.tensor([[320.0], [240.0]], dtype=torch.float64)
    assert rel(f1, ref_f.numpy()) < TOL
    assert rel(c1, c1_0 + d[2]) < TOL

    f2, conf = flow.copy(), rng.standard_normal((4, n)).astype(np.float32)
    conf0 = conf.copy()
    orc.orc_roma2_update(fp(f2), fp(conf), fp(d), n, 40.0, 30.0)
    rf, rc = R.update2(R.t64(flow), R.t64(conf0), R.t64(d), 40.0, 30.0)
    assert rel(f2, rf.numpy()) < TOL
    assert rel(conf, rc.numpy()) < 1e-4


def test_dwconv5(orc):
    rng = np.random.default_rng(6)
    C, H, W = 6, 21, 40
    x = rng.standard_normal((C, H, W)).astype(np.float32)
    w = rng.standard_normal((C, 25)).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32)
    out = np.zeros((C, H, W), np.float32)
    orc.orc_roma_dwconv5(fp(x), C, H, W, fp(w), fp(b), fp(out))
    assert rel(out, R.dwconv5_relu(R.t64(x), R.t64(w), R.t64(b)).numpy()) < TOL


# ---- the network ---------------------------------------------------------------------

import sys  # noqa: E402
from pathlib import Path  # noqa: E402

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "i.coregistration.opencl_amd"))
import synth  # noqa: E402
from oracle_lib import roma_forward  # noqa: E402

COARSE, TILE = 112, 64


@pytest.mark.parametrize("H,W,h,w", [(112, 112, 56, 56), (64, 96, 112, 112), (90, 70, 56, 28)])
def test_prepare_matches_antialiased_bicubic(orc, H, W, h, w):
    """Host resampling (Pillow's antialiased bicubic, roma.c:1106-1186)
    against torch's antialias=True bicubic, both directions, then the
    ImageNet normalisation."""
    rng = np.random.default_rng(H + w)
    img = rng.uniform(0, 1, (3, H, W)).astype(np.float32)
    out = np.zeros((3, h, w), np.float32)
    orc.orc_roma_prepare(fp(img), H, W, fp(out), h, w, 1)
    ref = R.prepare(img, h, w).numpy()
    assert np.abs(out - ref).max() < 2e-5


@pytest.fixture(scope="module")
def roma_weights():
    return synth.roma_weights(), synth.dino_weights(), synth.roma2_weights()


def _margins(logits):
    s = np.sort(logits[:, :4096], 1)
    return (s[:, -1] - s[:, -2]) / np.maximum(np.abs(s[:, -1]), 1e-30)


@pytest.mark.parametrize("v2", [False, True])
def test_roma_forward_matches_float64_restatement(roma_weights, v2):
    """The oracle's whole RoMa match (float32, the reference's schedule)
    against a float64 torch statement built from library routines:
    transformers' Dinov2Layer for the 24 DINOv2 blocks and the 5 decoder
    blocks, torch.linalg.cholesky for the GP, F.grid_sample /
    local_correlation / depthwise F.conv2d + F.batch_norm for the
    refiners, antialiased bicubic resizes. Stage by stage; the refiners
    start from the oracle's coarse warp so that an anchor argmax decided
    by a near-tie cannot hide a refiner difference."""
    wm, wd, w2 = roma_weights
    a, b, _ = synth.roma_pair(TILE, TILE)
    o = roma_forward(wm, wd, w2 if v2 else None, a, b, COARSE)
    assert o["info"] == 0
    r = R.roma_match(wm, wd, w2 if v2 else None, a, b, COARSE, cls_flow_in=o["cls_flow"])
    for k in range(2):
        assert rel(o["dino"][k], r["dino"][k]) < 1e-3
    assert rel(o["gp"], r["gp"]) < 1e-3
    assert rel(o["logits"], r["logits"]) < 1e-3
    sure = _margins(o["logits"]) > 1e-3
    assert sure.mean() > 0.9
    assert np.abs(o["cls_flow"][:, sure] - r["cls_flow"][:, sure]).max() < 1e-4
    for key, f in o["scale_flow"].items():
        assert np.abs(f - r["scale_flow"][key]).max() < 1e-3, key
    assert np.abs(o["flow"] - r["flow"]).max() < 1e-3
    assert np.abs(o["cert"] - r["cert"]).max() < 1e-3
    if v2:
        both = np.isfinite(o["sd"]) & np.isfinite(r["sd"])
        assert both.mean() > 0.99
        assert rel(o["sd"][both], r["sd"][both]) < 1e-3


def test_roma_coarse_is_the_coarse_pass(orc, roma_weights):
    """orc_roma_coarse (the coarse unit alone: DINOv2 x 2, GP, decoder,
    cls_to_flow on prepared images) gives the coarse warp and certainty
    of the oracle's whole match bit for bit."""
    from oracle_lib import roma_coarse
    wm, wd, _ = roma_weights
    a, b, _ = synth.roma_pair(COARSE, COARSE)
    o = roma_forward(wm, wd, None, a, b, COARSE)
    pa, pb = (np.zeros((3, COARSE, COARSE), np.float32) for _ in range(2))
    orc.orc_roma_prepare(fp(np.ascontiguousarray(a)), COARSE, COARSE, fp(pa), COARSE, COARSE, 1)
    orc.orc_roma_prepare(fp(np.ascontiguousarray(b)), COARSE, COARSE, fp(pb), COARSE, COARSE, 1)
    flow, cert, info = roma_coarse(wm, wd, pa, pb)
    assert info == 0
    assert np.array_equal(flow, o["cls_flow"])
    assert np.array_equal(cert, o["cls_cert"])


def test_roma_refine_is_the_fine_pass(orc, roma_weights):
    """orc_roma_refine (the refiner config's unit: VGG19-BN and the v1
    refiners of scales 8 .. 1 from a given 1/8 warp) reproduces the fine
    pass of the oracle's whole match bit for bit when started from that
    match's own inputs: the tile's prepared images and the coarse pass's
    last warp resized to 1/8. The certainty logit only accumulates the
    refiners' deltas, so the warps do not depend on the starting one."""
    from oracle_lib import roma_refine
    wm, wd, _ = roma_weights
    a, b, _ = synth.roma_pair(TILE, TILE)
    o = roma_forward(wm, wd, None, a, b, COARSE)
    pa, pb = np.zeros((3, TILE, TILE), np.float32), np.zeros((3, TILE, TILE), np.float32)
    orc.orc_roma_prepare(fp(np.ascontiguousarray(a)), TILE, TILE, fp(pa), TILE, TILE, 1)
    orc.orc_roma_prepare(fp(np.ascontiguousarray(b)), TILE, TILE, fp(pb), TILE, TILE, 1)
    f0 = np.ascontiguousarray(o["scale_flow"][(0, 1)])
    h8 = TILE // 8
    f8 = np.zeros((2, h8, h8), np.float32)
    orc.orc_resize(fp(f0), 2, COARSE, COARSE, fp(f8), h8, h8, 0, 0, 0.0)
    r = roma_refine(wm, wd, pa, pb, f8, np.zeros((h8, h8), np.float32), COARSE)
    for s in (8, 4, 2, 1):
        assert np.array_equal(r["scale_flow"][s], o["scale_flow"][(1, s)]), s
    assert np.array_equal(r["flow"], r["scale_flow"][1])


def test_vit_block_vs_torch(orc):
    """orc_vit_block (the DINOv2 block the oracle runs, roma.c:675-713, and
    the CPU baseline times) against torch float64: pre-norm attention with
    16 heads, exact-erf GELU MLP, both residuals. A swapped q / k slice, a
    missing residual or a tanh GELU fails the bound."""
    from oracle_lib import vit_block
    rng = np.random.default_rng(7)
    N, D = 19, 1024
    s = 1.0 / np.sqrt(D)
    w = [1 + 0.1 * rng.standard_normal(D), 0.1 * rng.standard_normal(D),
         s * rng.standard_normal((3 * D, D)), 0.1 * rng.standard_normal(3 * D),
         s * rng.standard_normal((D, D)), 0.1 * rng.standard_normal(D),
         1 + 0.1 * rng.standard_normal(D), 0.1 * rng.standard_normal(D),
         s * rng.standard_normal((4 * D, D)), 0.1 * rng.standard_normal(4 * D),
         0.5 * s * rng.standard_normal((D, 4 * D)), 0.1 * rng.standard_normal(D)]
    w = [a.astype(np.float32) for a in w]
    X = rng.standard_normal((N, D)).astype(np.float32)
    got = vit_block(w, X)
    t = [R.t64(a) for a in w]
    x = R.t64(X)
    ln = torch.nn.functional.layer_norm
    h = ln(x, (D,), t[0], t[1], 1e-6)
    qkv = (h @ t[2].T + t[3]).reshape(N, 3, 16, 64).permute(1, 2, 0, 3)
    a = torch.softmax(qkv[0] @ qkv[1].transpose(1, 2) / 8.0, -1) @ qkv[2]
    x = x + a.permute(1, 0, 2).reshape(N, D) @ t[4].T + t[5]
    h = ln(x, (D,), t[6], t[7], 1e-6)
    x = x + torch.nn.functional.gelu(h @ t[8].T + t[9]) @ t[10].T + t[11]
    assert rel(got, x.numpy()) < 1e-5


def test_oracle_threads(orc):
    """The thread count the CPU baseline pins is the one the oracle's loops
    use afterwards."""
    n0 = orc.orc_threads()
    orc.orc_set_threads(3)
    try:
        assert orc.orc_threads() == 3
    finally:
        orc.orc_set_threads(n0)

# SPDX-License-Identifier: Unlicense
"""GPU: the RoMa network on the HIP library against the oracle.

Tolerances: features and contractions <= 1e-3 of
the largest reference magnitude; warps <= 1e-3 (normalised units); the
anchor argmax of the coarse warp bit-exact (same cell) wherever the
oracle's relative top-2 logit margin exceeds 1e-3. Where a near-tie
decides the argmax differently, the oracle's refiners are re-run from
the HIP coarse warp, so that the refiners are still compared on the
same input.

The Gaussian-process solve (device, double precision) is checked against
numpy's float64 Cholesky solve, and at the full 560 x 560 size through
its residual."""

import sys
from pathlib import Path

import numpy as np
import pytest

from oracle_lib import roma_forward

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "i.coregistration.opencl_amd"))
import synth  # noqa: E402

COARSE, TILE = 112, 64


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


def cos_kernel(rng, n, d=64):
    x = rng.standard_normal((n, d))
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    return np.exp((x @ x.T - 1) / 0.2).astype(np.float32)


@pytest.mark.parametrize("n,d", [(1600, 512), (100, 512), (65, 7), (1, 3), (31, 5),
                                 (32, 64), (33, 65), (64, 130), (127, 9), (200, 512)])
def test_gp_solve(dev, ic, n, d):
    print(f"[roma] gp_solve n={n} d={d}", flush=True)
    rng = np.random.default_rng(n)
    K = cos_kernel(rng, n)
    F = rng.standard_normal((n, d)).astype(np.float32)
    ref = np.linalg.solve(K.astype(np.float64) + 0.1 * np.eye(n), F.astype(np.float64))
    bK, bF = dev.upload(K), dev.upload(F)
    work = dev.alloc(int(dev.api.roma_gp_work_bytes(n, d)))
    info = dev.upload(np.full(1, 7, np.int32))
    dev.api.roma_gp_solve(dev.po, bK.mem, n, 0.1, bF.mem, d, work.mem, info.mem)
    got = dev.read(bF).reshape(n, d)
    assert dev.read(info, 1, np.int32)[0] == 0
    assert rel(got, ref) < 1e-5


def test_gp_solve_reports_indefinite(dev, ic):
    """A kernel that is not positive definite (here -I, so the first pivot
    is -0.9) sets info to the failing column + 1; the factor is NaN from
    there, no fault."""
    n, d = 70, 3
    K = -np.eye(n, dtype=np.float32)
    bK, bF = dev.upload(K), dev.upload(np.ones((n, d), np.float32))
    work = dev.alloc(int(dev.api.roma_gp_work_bytes(n, d)))
    info = dev.zeros(1, np.int32)
    dev.api.roma_gp_solve(dev.po, bK.mem, n, 0.1, bF.mem, d, work.mem, info.mem)
    assert dev.read(info, 1, np.int32)[0] == 1


def test_gp_solve_wait_gives_up_and_events_form(dev, ic):
    """The solve's bounded in-kernel waits (the diagonal kernels' and the
    panels' first products') forced to give up from the host
    (icoreg_gp_test_wait: the panel flags never set, 64 polls): every
    launch still exits, info is -1; roma_gp_solve_events (stream
    event waits) on the same inputs gives the solution, and with the
    default hooks both forms give the same bits."""
    print("[roma] gp_solve forced give-up, n=300 d=64", flush=True)
    lib = ic.lib()
    n, d = 300, 64  # 5 panels: diagonal blocks 2, 3, 4 wait
    rng = np.random.default_rng(3)
    K = cos_kernel(rng, n)
    F = rng.standard_normal((n, d)).astype(np.float32)
    ref = np.linalg.solve(K.astype(np.float64) + 0.1 * np.eye(n), F.astype(np.float64))
    bK = dev.upload(K)
    work = dev.alloc(int(dev.api.roma_gp_work_bytes(n, d)))
    info = dev.zeros(1, np.int32)
    lib.icoreg_gp_test_wait(64, 0)
    try:
        bF = dev.upload(F)
        dev.api.roma_gp_solve(dev.po, bK.mem, n, 0.1, bF.mem, d, work.mem, info.mem)
        dev.finish()
        assert dev.read(info, 1, np.int32)[0] == -1
        bF = dev.upload(F)
        dev.api.roma_gp_solve_events(dev.po, bK.mem, n, 0.1, bF.mem, d, work.mem, info.mem)
        ev = dev.read(bF).reshape(n, d)
        assert dev.read(info, 1, np.int32)[0] == 0
        assert rel(ev, ref) < 1e-5
    finally:
        lib.icoreg_gp_test_wait(0, 1)
    bF = dev.upload(F)
    dev.api.roma_gp_solve(dev.po, bK.mem, n, 0.1, bF.mem, d, work.mem, info.mem)
    assert dev.read(info, 1, np.int32)[0] == 0
    assert np.array_equal(dev.read(bF).reshape(n, d), ev)


@pytest.fixture(scope="module")
def weights(tmp_path_factory):
    d = tmp_path_factory.mktemp("roma_w")
    files = synth.roma_weights_files(d)
    return files, (synth.roma_weights(), synth.dino_weights(), synth.roma2_weights())


def _margins(logits):
    s = np.sort(logits[:, :4096], 1)
    return (s[:, -1] - s[:, -2]) / np.maximum(np.abs(s[:, -1]), 1e-30)


def _read_dump(folder, what, tile=1):
    return np.fromfile(Path(folder) / f"tile{tile:03d}_roma_{what}.f32", np.float32)


@pytest.mark.parametrize("v2", [False, True])
def test_roma_match_vs_oracle(dev, ic, weights, tmp_path, v2):
    print(f"[roma] match v2={v2} coarse={COARSE} tile={TILE}", flush=True)
    (fm, fd, f2), (wm, wd, w2) = weights
    a, b, _ = synth.roma_pair(TILE, TILE)
    net = ic.Roma(dev, fm, fd, TILE, TILE, v2_path=f2 if v2 else None, coarse=COARSE)
    try:
        got = net.match(a, b, dump=str(tmp_path), tile=1)
    finally:
        net.close()
    o = roma_forward(wm, wd, w2 if v2 else None, a, b, COARSE)
    assert o["info"] == 0
    n16 = (COARSE // 14) ** 2
    for k in range(2):
        assert rel(_read_dump(tmp_path, f"dino_{k}"), o["dino"][k]) < 1e-3
    assert rel(_read_dump(tmp_path, "gp"), o["gp"]) < 1e-3
    cls_flow = _read_dump(tmp_path, "cls_flow").reshape(2, n16)
    sure = _margins(o["logits"]) > 1e-3
    assert sure.mean() > 0.9
    assert np.abs(cls_flow[:, sure] - o["cls_flow"][:, sure]).max() < 1e-4
    assert rel(_read_dump(tmp_path, "cls_cert"), o["cls_cert"]) < 1e-3
    if np.abs(cls_flow - o["cls_flow"]).max() > 1e-4:
        print("[roma] near-tie anchors differ; oracle refiners re-run from the HIP warp",
              flush=True)
        o = roma_forward(wm, wd, w2 if v2 else None, a, b, COARSE, cls_flow_in=cls_flow)
    for (p, s), f in o["scale_flow"].items():
        g = _read_dump(tmp_path, f"p{p}_s{s}_flow").reshape(f.shape)
        assert np.abs(g - f).max() < 1e-3, (p, s)
    assert np.abs(got["flow"] - o["flow"]).max() < 1e-3
    assert np.abs(got["cert"] - o["cert"]).max() < 1e-3
    if v2:
        both = np.isfinite(got["sd"]) & np.isfinite(o["sd"])
        assert both.mean() > 0.99
        assert rel(got["sd"][both], o["sd"][both]) < 1e-3


def test_roma_coarse_560_properties(dev, ic, weights, tmp_path):
    """The benchmark's unit at full size (DINOv2 x 2 on 560 x 560, GP on
    1600 tokens, decoder): the GP solve's residual |(K + 0.1 I) X - B| /
    |B| in float64 from the device's own K, X and basis, a finite warp
    inside -1..1 on the 40 x 40 grid, and the same warp as the coarse
    stage of roma_match on the same inputs."""
    print("[roma] coarse 560 properties", flush=True)
    (fm, fd, _), _ = weights
    a, b, _ = synth.roma_pair(560, 560)
    net = ic.Roma(dev, fm, fd, 560, 560)
    try:
        mean = np.array([0.485, 0.456, 0.406], np.float32)[:, None, None]
        std = np.array([0.229, 0.224, 0.225], np.float32)[:, None, None]
        pair = dev.upload(np.stack([(a - mean) / std, (b - mean) / std]))
        net.coarse_device(pair)
        dev.finish()
        assert net.gp_info() == 0
        n = 1600
        K = net.buffer("g_kyy", n * n).reshape(n, n).astype(np.float64)
        X = net.buffer("g_f", n * 512).reshape(n, 512).astype(np.float64)
        flow = net.buffer("fl0", 2 * n).reshape(2, n)
        cert = net.buffer("ce0", n)
        assert np.isfinite(flow).all() and np.isfinite(cert).all()
        assert np.abs(flow).max() <= 1.0
        # The basis is what the solve started from: recompute it as the
        # library does (roma.c:326-350) from the weights file.
        w = synth.roma_weights()
        c = 40
        i = np.arange(n)
        x = (-1.0 + 1.0 / c + (i % c) * (2.0 - 2.0 / c) / (c - 1)).astype(np.float32)
        y = (-1.0 + 1.0 / c + (i // c) * (2.0 - 2.0 / c) / (c - 1)).astype(np.float32)
        pw = w["decoder.gps.16.pos_conv.weight"][:, :, 0, 0]
        v = (pw[:, 0][None] * x[:, None] + pw[:, 1][None] * y[:, None]
             + w["decoder.gps.16.pos_conv.bias"][None]).astype(np.float32)
        basis = np.cos(np.float32(8.0 * np.pi) * v).astype(np.float64)
        res = (K + 0.1 * np.eye(n)) @ X - basis
        assert np.abs(res).max() / np.abs(basis).max() < 1e-4
        got = net.match(a, b, dump=str(tmp_path), tile=1)
        assert np.isfinite(got["flow"]).all()
        assert ((got["cert"] >= 0) & (got["cert"] <= 1)).all()
        cls_full = _read_dump(tmp_path, "cls_flow").reshape(2, n)
        assert np.abs(cls_full - flow).max() < 1e-5
    finally:
        net.close()


def test_roma_match_from_torch_checkpoints(dev, ic, weights, tmp_path):
    """RoMa from torch.save files the way the published ones are laid out
    (the matcher's tensors under "matcher.model.", DINOv2 in the legacy
    pickle stream here) gives the same warp and certainty bit for bit as
    the safetensors load."""
    print(f"[roma] match from torch.save checkpoints coarse={COARSE} tile={TILE}", flush=True)
    (fm, fd, _), (wm, wd, _) = weights
    pm = synth.save_torch(wm, tmp_path / "roma_outdoor.pth", prefix="matcher.model.")
    pd = synth.save_torch(wd, tmp_path / "dinov2_vitl14_pretrain.pth", legacy=True)
    a, b, _ = synth.roma_pair(TILE, TILE)
    out = []
    for m, d in ((fm, fd), (pm, pd)):
        net = ic.Roma(dev, m, d, TILE, TILE, coarse=COARSE)
        try:
            out.append(net.match(a, b))
        finally:
            net.close()
    for k in ("flow", "cert"):
        assert np.array_equal(out[0][k], out[1][k]), k


def _refine_from_dumps(dev, ic, net, folder, H, W, coarse):
    """roma_refine_device on roma_match's own fine-pass inputs read back
    from its dumps: the normalised pair and the coarse pass's final warp
    and certainty, resized to 1/8 as roma_match resizes them."""
    pair = np.concatenate([_read_dump(folder, "in_f_0"), _read_dump(folder, "in_f_1")])
    f0 = dev.upload(_read_dump(folder, "p0_s1_flow"))
    c0 = dev.upload(_read_dump(folder, "p0_s1_cert"))
    h8, w8 = H // 8, W // 8
    f8, c8 = dev.zeros(2 * h8 * w8), dev.zeros(h8 * w8)
    dev.api.ops_resize(dev.po, f0.mem, 2, coarse, coarse, f8.mem, h8, w8, 0, 0, 0.0)
    dev.api.ops_resize(dev.po, c0.mem, 1, coarse, coarse, c8.mem, h8, w8, 0, 0, 0.0)
    fl, ce = net.refine_device(dev.upload(pair), f8, c8)
    return net.buffer(fl, 2 * H * W), net.buffer(ce, H * W)


def test_refine_device_is_the_fine_pass(dev, ic, weights, tmp_path):
    """roma_refine_device (the refiner benchmark's unit) reproduces the
    fine pass of roma_match bit for bit from the same inputs."""
    print(f"[roma] refine_device vs match coarse={COARSE} tile={TILE}", flush=True)
    (fm, fd, _), _ = weights
    a, b, _ = synth.roma_pair(TILE, TILE)
    net = ic.Roma(dev, fm, fd, TILE, TILE, coarse=COARSE)
    try:
        net.match(a, b, dump=str(tmp_path), tile=1)
        flow, cert = _refine_from_dumps(dev, ic, net, tmp_path, TILE, TILE, COARSE)
    finally:
        net.close()
    assert np.array_equal(flow, _read_dump(tmp_path, "p1_s1_flow"))
    assert np.array_equal(cert, _read_dump(tmp_path, "p1_s1_cert"))


def test_refiners_864_properties(dev, ic, weights, tmp_path):
    """The refiner config at full size (864 x 864: VGG19-BN on both
    images, refiners at 1/8 .. 1/1 with C = 512, 256, 64, 9 and local
    correlation radii 3 and 2): from the synthetic initial warp the
    outputs are finite and stay near it, and roma_match's own fine pass
    at 864 x 864 is reproduced bit for bit by roma_refine_device."""
    H = W = 864
    print(f"[roma] refiners {H}x{W}", flush=True)
    (fm, fd, _), _ = weights
    a, b, flow8, cert8 = synth.roma_refine_inputs(H, W)
    net = ic.Roma(dev, fm, fd, H, W)
    try:
        pair = dev.upload(np.stack([synth.imagenet_norm(a), synth.imagenet_norm(b)]))
        fl, ce = net.refine_device(pair, dev.upload(flow8), dev.upload(cert8))
        flow = net.buffer(fl, 2 * H * W).reshape(2, H, W)
        cert = net.buffer(ce, H * W)
        assert np.isfinite(flow).all() and np.isfinite(cert).all()
        # The refiners move the warp by bounded steps: the result stays
        # within a few cells of the initial warp (resized to full size).
        up = np.repeat(np.repeat(flow8, 8, 1), 8, 2)
        assert np.median(np.abs(flow - up)) < 0.1
        got = net.match(a, b, dump=str(tmp_path), tile=1)
        assert np.isfinite(got["flow"]).all()
        assert ((got["cert"] >= 0) & (got["cert"] <= 1)).all()
        flow2, cert2 = _refine_from_dumps(dev, ic, net, tmp_path, H, W, 560)
    finally:
        net.close()
    assert np.array_equal(flow2, _read_dump(tmp_path, "p1_s1_flow"))
    assert np.array_equal(cert2, _read_dump(tmp_path, "p1_s1_cert"))


def test_roma_v2ref_1024_properties(dev, ic, weights):
    """The full roma_v2ref config at 1024 x 1024 (RoMa coarse at 560 with
    both VGG19-BN stacks, v2 refiners at 1/4, 1/2, 1/1, host epilogue):
    finite warp in -1..1, certainty in 0..1, a finite positive standard
    deviation wherever the precision is positive definite (almost
    everywhere)."""
    H = W = 1024
    print(f"[roma] v2ref {H}x{W}", flush=True)
    (fm, fd, f2), _ = weights
    a, b, _ = synth.roma_pair(H, W, seed=synth.BASE_SEED + synth.CONFIG_V2REF)
    net = ic.Roma(dev, fm, fd, H, W, v2_path=f2)
    try:
        got = net.match(a, b)
        assert net.gp_info() == 0
    finally:
        net.close()
    flow, cert, sd = got["flow"], got["cert"], got["sd"]
    assert np.isfinite(flow).all() and np.abs(flow).max() <= 1.0
    assert np.isfinite(cert).all() and ((cert >= 0) & (cert <= 1)).all()
    ok = np.isfinite(sd)
    assert ok.mean() > 0.99 and (sd[ok] > 0).all()


def test_roma_match_recovers_from_gp_give_up(dev, ic, weights):
    """roma_match with the GP solve's in-kernel wait forced to give up
    (coarse 168: 144 tokens, 3 panels, diagonal block 2 waits): it re-runs
    the solve with stream event waits and returns the same warp and
    certainty bit for bit as an undisturbed run."""
    print("[roma] match with a forced GP give-up, coarse=168 tile=64", flush=True)
    (fm, fd, _), _ = weights
    a, b, _ = synth.roma_pair(TILE, TILE)
    lib = ic.lib()
    out = []
    for forced in (False, True):
        net = ic.Roma(dev, fm, fd, TILE, TILE, coarse=168)
        try:
            if forced:
                lib.icoreg_gp_test_wait(64, 0)
            out.append(net.match(a, b))
            assert net.gp_retries() == int(forced)
            assert net.gp_info() == 0
        finally:
            lib.icoreg_gp_test_wait(0, 1)
            net.close()
    for k in ("flow", "cert"):
        assert np.isfinite(out[0][k]).all()
        assert np.array_equal(out[0][k], out[1][k]), k


def test_coarse_graph_replays_match_eager(dev, ic, weights):
    """RoMa's coarse pass (DINOv2, GP solve, decoder: roma_coarse_device,
    no host transfer inside) recorded once as a HIP graph and replayed
    three times, with eager passes on another pair and synchronisations
    between: every replay gives the eager warp, certainty and GP solution
    bit for bit."""
    print(f"[roma] coarse graph replays coarse={COARSE}", flush=True)
    (fm, fd, _), _ = weights
    a, b, _ = synth.roma_pair(COARSE, COARSE)
    c, d, _ = synth.roma_pair(COARSE, COARSE, seed=11)
    net = ic.Roma(dev, fm, fd, COARSE, COARSE, coarse=COARSE)
    api, lib = dev.api, ic.lib()
    n = (COARSE // 14) ** 2
    graph = None
    try:
        p0, p1 = dev.upload(np.stack([a, b])), dev.upload(np.stack([c, d]))
        read = lambda: [net.buffer("fl0", 2 * n), net.buffer("ce0", n),
                        net.buffer("g_f", n * 512)]
        net.coarse_device(p0)
        ref = read()
        api.ocl_graph_begin(dev.pb)
        net.coarse_device(p0)
        graph = api.ocl_graph_end(dev.pb)
        for rep in range(3):
            net.coarse_device(p1)
            dev.finish()
            api.ocl_graph_launch(dev.pb, graph)
            dev.finish()
            for k, (g, r) in enumerate(zip(read(), ref)):
                assert np.array_equal(g, r), (rep, k)
    finally:
        if graph:
            lib.ocl_graph_free(graph)
        net.close()

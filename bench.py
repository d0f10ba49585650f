# SPDX-License-Identifier: Unlicense
"""Benchmark of the MI355X matcher tensor path (BASELINE.json metric).

The metric names two workloads. `value` is the first: one step = one
Efficient LoFTR 640 x 640 grey tile pair through the whole device stage of
the reference's eloftr_match (eloftr.c:654-681):
backbone x 2, 4 x (self, self, cross, cross) aggregated attention, coarse
dual-softmax matching with the host mutual selection, FPN fusion x 2 and
two-stage fine matching; seeded synthetic pair and seeded random-init
weights (synth.py), both images resident in HBM before timing.

The second, RoMa's coarse forward on a 560 x 560 RGB pair (DINOv2 ViT-L/14
x 2, Gaussian process, coordinate decoder; roma.c:715-919), is reported
under "roma560" with its own throughput and GEMM roofline.

Prints one JSON line (the driver's contract) with the per-kernel roofline
of the dominant kernel (the same-size 3 x 3 convolutions as Winograd
F(2 x 2, 3 x 3) on the fp32 matrix cores: HIP events around each of its
launches over the profiled steps; its FLOPs are the 16 transform-domain
products it performs, and the direct-convolution rate of the same layers is
reported beside it) and the CPU baseline (the oracle, a C port of the
reference kernels, on a bounded sample timed on this host).

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu-baseline]
                    [--no-roma] [--roma-steps 10] [--copy-calib MiB]
"""

import argparse
import importlib.util
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
PKG_DIR = ROOT / "i.coregistration.opencl_amd"
PEAK_FP32_MFMA = 157.3  # TFLOP/s, MI355X dense fp32 matrix
PEAK_HBM = 8000.0        # GB/s


def load_package():
    if "icoreg_amd" in sys.modules:
        return sys.modules["icoreg_amd"]
    spec = importlib.util.spec_from_file_location(
        "icoreg_amd", PKG_DIR / "__init__.py", submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["icoreg_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def eloftr_flops(H, W, nm=0):
    """Algorithmic FLOPs of one ELoFTR pair by kernel family: 2 M N K per
    contraction, 2 K Ho Wo C kh kw per convolution, 4 heads Nq Nk d per
    attention, one score GEMM (the second pass is a recompute)."""
    h, w = H // 8, W // 8
    n, na = h * w, (h // 4) * (w // 4)
    conv = gemm = attn = other = 0.0
    # Backbone (eloftr.c:367-394), both images.
    layers = [(1, 64, 2)] + [(64, 64, 1)] * 2 + [(64, 128, 2)] + [(128, 128, 1)] * 3 + \
             [(128, 256, 2)] + [(256, 256, 1)] * 13
    Hc, Wc = H, W
    for ci, co, s in layers:
        Hc, Wc = Hc // s, Wc // s
        conv += 2 * 2.0 * co * Hc * Wc * ci * 9
    # Transformer: 16 aggregated attention blocks (eloftr.c:405-463).
    D = 256
    per = (4 * 2.0 * na * D * D            # q, k, v, o projections
           + 2.0 * n * 512 * 512 + 2.0 * n * 256 * 512)  # fc1, fc2
    gemm += 16 * per
    attn += 16 * 4.0 * 8 * na * na * 32
    other += 16 * 2.0 * D * na * 16         # depthwise 4 x 4 aggregation
    # Coarse scores (one pass).
    gemm += 2.0 * n * n * D
    # Fusion (eloftr.c:573-604), both images.
    H4, W4, H2, W2 = 2 * h, 2 * w, 4 * h, 4 * w
    gemm += 2 * (2.0 * 256 * n * 256 + 2.0 * 256 * H4 * W4 * 128 + 2.0 * 128 * H2 * W2 * 64)
    conv += 2 * (2.0 * 256 * H4 * W4 * 256 * 9 + 2.0 * 128 * H4 * W4 * 256 * 9
                 + 2.0 * 128 * H2 * W2 * 128 * 9 + 2.0 * 64 * H2 * W2 * 128 * 9)
    other += nm * (2.0 * 64 * 100 * 56 + 2.0 * 9 * 8)
    return {"conv": conv, "gemm": gemm, "attention": attn, "other": other,
            "total": conv + gemm + attn + other}


def eloftr_conv_layers(H, W):
    """(ci, co, hin, win, stride) of the 25 direct 3 x 3 convolution
    launches of one pair (each launch covers both images): 21 backbone
    layers (eloftr.c:367-394), 4 fusion layers (eloftr.c:573-604)."""
    out, Hc, Wc = [], H, W
    for ci, co, st in [(1, 64, 2)] + [(64, 64, 1)] * 2 + [(64, 128, 2)] + [(128, 128, 1)] * 3 + \
            [(128, 256, 2)] + [(256, 256, 1)] * 13:
        out.append((ci, co, Hc, Wc, st))
        Hc, Wc = Hc // st, Wc // st
    H4, W4, H2, W2 = H // 4, W // 4, H // 2, W // 2
    out += [(256, 256, H4, W4, 1), (256, 128, H4, W4, 1), (128, 128, H2, W2, 1),
            (128, 64, H2, W2, 1)]
    return out


def eloftr_wino_layers(H, W):
    """The stride-1 layers, which run as Winograd convolutions (22 launches
    per pair); the 3 stride-2 layers run direct."""
    return [l for l in eloftr_conv_layers(H, W) if l[4] == 1]


def eloftr_wino_forms(dev, H, W):
    """The Winograd form the library gives each stride-1 layer of a pair on
    this device (icoreg_conv_wino_choice): 4 for F(4 x 4, 3 x 3), 2 for
    F(2 x 2, 3 x 3)."""
    lib = load_package().lib()
    return [lib.icoreg_conv_wino_choice(dev.po, 2, ci, h, w, co)
            for ci, co, h, w, _ in eloftr_wino_layers(H, W)]


def eloftr_wino_flops(H, W, forms):
    """Algorithmic matrix FLOPs of the Winograd launches of one pair: per
    image, 2 x 16 x K x C per 2 x 2 output tile for F(2 x 2) (the 16
    transform-domain products; ceil(Ho / 2) ceil(Wo / 2) tiles), 2 x 36 x
    K x C per 4 x 4 tile for F(4 x 4). The input and output transforms
    (vector-ALU work) are not counted."""
    f = 0.0
    for (ci, co, h, w, _), form in zip(eloftr_wino_layers(H, W), forms):
        if form == 4:
            f += 2 * 2.0 * 36 * co * ci * ((h + 3) // 4) * ((w + 3) // 4)
        else:
            f += 2 * 2.0 * 16 * co * ci * ((h + 1) // 2) * ((w + 1) // 2)
    return f


def eloftr_wino_direct_flops(H, W):
    """The same layers' direct-convolution FLOPs (2 K Ho Wo C 9 per image):
    the work a direct kernel would do for the same outputs."""
    return sum(2 * 2.0 * co * h * w * ci * 9 for ci, co, h, w, _ in eloftr_wino_layers(H, W))


def eloftr_wino_bytes(H, W, forms):
    """Algorithmic HBM bytes of the Winograd launches of one pair: both
    images' input and output read / written once, the transformed filters
    (16 K C for F(2 x 2), 36 K C for F(4 x 4)) and bias once per launch."""
    b = 0
    for (ci, co, h, w, _), form in zip(eloftr_wino_layers(H, W), forms):
        b += 4 * (2 * (ci * h * w + co * h * w) + (36 if form == 4 else 16) * co * ci + co)
    return b


def conv_traffic(profile=ROOT / "profiles" / "eloftr_640_wino_traffic.md"):
    """Measured HBM bytes per Winograd convolution launch, from the
    committed rocprofv3 counter summary (the line
    'traffic_bytes_per_launch: N'), or None."""
    import re
    try:
        m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", profile.read_text())
    except OSError:
        return None
    return int(m.group(1)) if m else None


def conv_counters(profile=ROOT / "profiles" / "eloftr_640_wino_sq_counters.md"):
    """The Winograd kernel's matrix-pipe share of its CUs' busy cycles and
    its CU-busy share of the dispatch, from the committed rocprofv3 SQ
    counter summary, or None."""
    import re
    try:
        t = profile.read_text()
    except OSError:
        return None
    m1 = re.search(r"mfma_issue_share_of_busy_cycles:\s*([0-9.]+)", t)
    m2 = re.search(r"cu_busy_share:\s*([0-9.]+)", t)
    if not (m1 and m2):
        return None
    return {"mfma_issue_share_of_busy_cycles": float(m1.group(1)),
            "cu_busy_share": float(m2.group(1)),
            "source": "profiles/eloftr_640_wino_sq_counters.md"}


def roma_coarse_flops(coarse=560):
    """Algorithmic FLOPs of RoMa's coarse forward on one pair (DINOv2 x 2,
    GP, decoder), by kernel family; the GP's double-precision Cholesky
    (n^3 / 3) and solves (2 n^2 d) are reported apart as fp64."""
    c16 = coarse // 14
    n, nt, D = c16 * c16, c16 * c16 + 1, 1024
    gemm = attn = 0.0
    gemm += 2 * 2.0 * D * n * 3 * 14 * 14                        # patch embedding
    blk = 2.0 * nt * D * (3 * D + D + 4 * D + 4 * D)
    gemm += 2 * 24 * blk
    attn += 2 * 24 * 4.0 * 16 * nt * nt * 64
    gemm += 2 * 2.0 * n * 512 * D                                 # proj to 512
    gemm += 3 * 2.0 * n * n * 512                                 # K_yy, K_xy, K_xy X
    gemm += 5 * 2.0 * n * D * (3 * D + D + 4 * D + 4 * D)
    attn += 5 * 4.0 * 8 * n * n * 128
    gemm += 2.0 * n * 4097 * D                                    # to_out
    fp64 = n ** 3 / 3.0 + 2.0 * n * n * 512
    return {"gemm": gemm, "attention": attn, "fp64": fp64, "total": gemm + attn}


def bench_roma(ic, dev, synth, wdir, steps, warmup, profile_steps):
    """RoMa coarse forward (DINOv2 ViT-L/14 x 2 at 560 x 560, GP on 1600
    tokens, coordinate decoder, cls_to_flow) of one pair already in HBM."""
    fm, fd, _ = synth.roma_weights_files(wdir)
    a, b, _ = synth.roma_pair(560, 560)
    net = ic.Roma(dev, fm, fd, 560, 560)
    mean = np.array([0.485, 0.456, 0.406], np.float32)[:, None, None]
    std = np.array([0.229, 0.224, 0.225], np.float32)[:, None, None]
    pair = dev.upload(np.stack([(a - mean) / std, (b - mean) / std]))
    for _ in range(warmup):
        net.coarse_device(pair)
    dev.finish()
    dev.reset_events()
    t0 = time.perf_counter()
    e0 = dev.event()
    for _ in range(steps):
        net.coarse_device(pair)
    e1 = dev.event()
    dev.finish()
    wall = time.perf_counter() - t0
    ms = max(dev.elapsed_ms(e0, e1), wall * 1e3) / steps
    info = net.gp_info()
    if info > 0:
        raise RuntimeError("RoMa GP kernel not positive definite")
    if info < 0:
        # The solve's in-kernel wait for its second stream gave up: only
        # where kernels are serialized (a counter-collecting profiler);
        # roma_match would rerun the solve with event waits.
        print("[bench] RoMa GP: in-kernel wait gave up (serialized kernels); "
              "the timed passes include it", file=sys.stderr, flush=True)
    # The same pass replayed from one HIP graph.
    graph = None
    try:
        dev.api.ocl_graph_begin(dev.pb)
        net.coarse_device(pair)
        graph = dev.api.ocl_graph_end(dev.pb)
        for _ in range(warmup):
            dev.api.ocl_graph_launch(dev.pb, graph)
        dev.finish()
        dev.reset_events()
        t0 = time.perf_counter()
        e0 = dev.event()
        for _ in range(steps):
            dev.api.ocl_graph_launch(dev.pb, graph)
        e1 = dev.event()
        dev.finish()
        ms_g = max(dev.elapsed_ms(e0, e1), (time.perf_counter() - t0) * 1e3) / steps
        # The replays' GP solve (stream-event form) succeeded and their
        # warp, certainty and GP solution are the eager pass's.
        if net.gp_info() != 0:
            raise RuntimeError("RoMa graph replay: GP solve failed")
        n16 = (560 // 14) ** 2
        outs = lambda: [net.buffer("fl0", 2 * n16), net.buffer("ce0", n16),
                        net.buffer("g_f", n16 * 512)]
        replayed = outs()
        net.coarse_device(pair)
        dev.finish()
        # (An eager pass whose GP wait gave up has no result to compare.)
        if info == 0 and not all(np.array_equal(a, b) for a, b in zip(replayed, outs())):
            raise RuntimeError("RoMa graph replay differs from the eager pass")
    finally:
        if graph:
            ic.lib().ocl_graph_free(graph)
    dev.profile_reset()
    dev.set_profile(2)
    for _ in range(profile_steps):
        net.coarse_device(pair)
    dev.finish()
    table = dev.profile_table()
    dev.set_profile(0)
    net.close()
    fl = roma_coarse_flops()
    ps = profile_steps
    gemm_ms = table.get("gemm", (0.0, 0))[0] / ps
    attn_ms = table.get("attention", (0.0, 0))[0] / ps
    kernels = {k: {"ms_per_step": round(v[0] / ps, 4), "launches_per_step": v[1] / ps}
               for k, v in sorted(table.items(), key=lambda kv: -kv[1][0])}
    print("[bench] RoMa per-kernel ms per pair: " + json.dumps(kernels), file=sys.stderr,
          flush=True)
    gp_ms = table.get("roma_gp_solve", (0.0, 0))[0] / ps
    g_tf = fl["gemm"] / (gemm_ms * 1e-3) / 1e12 if gemm_ms > 0 else 0.0
    a_tf = fl["attention"] / (attn_ms * 1e-3) / 1e12 if attn_ms > 0 else 0.0
    return {
        "workload": "RoMa coarse forward, 560x560 RGB pair: DINOv2 ViT-L/14 x 2 (1601 tokens), "
                    "GP on 1600 tokens (device fp64 solve), coordinate decoder, cls_to_flow",
        "pairs_per_s": round(1000.0 / ms, 3), "ms_per_pair": round(ms, 4),
        "graph": {"pairs_per_s": round(1000.0 / ms_g, 3), "ms_per_pair": round(ms_g, 4),
                  "workload": f"the same pass replayed from one HIP graph ({steps} replays)"},
        "gflop_per_pair": round(fl["total"] / 1e9, 1),
        "pipeline_tflops": round(fl["total"] / (ms * 1e-3) / 1e12, 2),
        "gp_solve_ms": round(gp_ms, 4),
        "kernels": kernels,
        "roofline": {"kernel": "gemm_mfma (fp32 MFMA GEMM: qkv, proj, MLP, GP, to_out)",
                     "bound": "mfma", "achieved": round(g_tf, 2), "peak": PEAK_FP32_MFMA,
                     "unit": "TFLOP/s", "frac": round(g_tf / PEAK_FP32_MFMA, 4),
                     "gflop_per_step": round(fl["gemm"] / 1e9, 1)},
        "attention": {"achieved": round(a_tf, 2), "unit": "TFLOP/s",
                      "frac": round(a_tf / PEAK_FP32_MFMA, 4),
                      "gflop_per_step": round(fl["attention"] / 1e9, 1)},
    }


VGG_BLOCKS = ((2, 64), (2, 128), (4, 256), (4, 512))
# RoMa's v1 refiners at scales 8, 4, 2, 1: features, embedding, radius
# (roma.c:60-64); input channels 2 f + e + (2 r + 1)^2.
REFINE_V1 = ((8, 512, 64, 3), (4, 256, 32, 2), (2, 64, 16, 0), (1, 9, 6, 0))
PROJ_V1 = {8: (512, 512), 4: (256, 256), 2: (128, 64), 1: (64, 9)}


def vgg_flops(H, W, nblk=4, proj=PROJ_V1):
    """One image through VGG19-BN's first nblk blocks plus the 1 x 1
    projections to the refiner features (roma.c:740-768)."""
    f, cin, h, w = 0.0, 3, H, W
    for b, (n, c) in enumerate(VGG_BLOCKS[:nblk]):
        for _ in range(n):
            f += 2.0 * c * cin * 9 * h * w
            cin = c
        pi, po = proj[1 << b]
        f += 2.0 * po * pi * h * w
        h, w = h // 2, w // 2
    return f


def refiner_flops(H, W, table=REFINE_V1):
    """The v1 refiners on an H x W pass: per scale the displacement
    embedding, local correlation ((2 r + 2)^2 whole-cell dot products per
    cell), 9 depthwise 5 x 5 + 1 x 1 blocks and the output convolution."""
    f = 0.0
    for s, feat, emb, r in table:
        n = (H // s) * (W // s)
        cin = 2 * feat + emb + ((2 * r + 1) ** 2 if r else 0)
        f += 2.0 * emb * 2 * n
        if r:
            f += 2.0 * feat * (2 * r + 2) ** 2 * n
        f += 9 * (2.0 * cin * 25 * n + 2.0 * cin * cin * n)
        f += 2.0 * 3 * cin * n
    return f


def disk_flops(H=512, W=512):
    """DISK's nine 5 x 5 convolutions on one H x W image (disk.c:28-30)."""
    cin = (3, 16, 32, 64, 64, 128, 128, 96, 80)
    cout = (16, 32, 64, 64, 64, 64, 64, 64, 129)
    lvl = (0, 1, 2, 3, 4, 3, 2, 1, 0)
    return sum(2.0 * co * ci * 25 * (H >> l) * (W >> l) for ci, co, l in zip(cin, cout, lvl))


def hbm_kernel_bytes(kind, C, n, r=0):
    """Compulsory HBM bytes of a refiner sampling kernel on n cells:
    warp sample reads the C x n map and the warp, writes C x n; local
    correlation reads both C x n maps and the warp, writes (2 r + 1)^2 x n."""
    if kind == "warp_sample":
        return 4 * C * n + 8 * n + 4 * C * n
    return 2 * 4 * C * n + 8 * n + 4 * (2 * r + 1) ** 2 * n


def time_launches(dev, fn, reps=20):
    """Mean ms of fn() over reps launches after one warm-up, HIP events on
    the library's stream around one replay of a HIP graph that holds the
    reps calls: the launches run back to back on the device, without the
    host's per-call time (a few microseconds of Python and ctypes, as long
    as the smaller kernels themselves) between them."""
    fn()
    dev.finish()
    api = dev.api
    api.ocl_graph_begin(dev.pb)
    try:
        for _ in range(reps):
            fn()
    finally:
        graph = api.ocl_graph_end(dev.pb)
    try:
        api.ocl_graph_launch(dev.pb, graph)
        dev.finish()
        dev.reset_events()
        e0 = dev.event()
        api.ocl_graph_launch(dev.pb, graph)
        e1 = dev.event()
        dev.finish()
    finally:
        api.ocl_graph_free(graph)
    return dev.elapsed_ms(e0, e1) / reps


def bench_local_corr_shapes(dev):
    """roma_local_corr (cell-major copy of f2 plus correlation) alone at the
    refiners' shapes, on seeded features and a smooth warp, each timed over
    20 launches: the v1 refiners at 1/8 and 1/4 of 864 x 864, the first
    refiner's radius 7 and 512 channels on 64 x 64 and 40 x 40 cells (the
    coarse grid), roma_v2ref's refiners at 1/4 and 1/2 of 1024 x 1024.
    frac_hbm: compulsory bytes / time / 8 TB/s."""
    out = []
    rng = np.random.default_rng(7)
    api, po = dev.api, dev.po
    for C, h, r in ((512, 108, 3), (256, 216, 2), (512, 64, 7), (512, 40, 7), (192, 256, 3),
                    (48, 512, 1)):
        n = h * h
        f1 = dev.upload(rng.standard_normal((C, n), np.float32))
        f2 = dev.upload(rng.standard_normal((C, n), np.float32))
        gx = (2 * (np.arange(h) + 0.5) / h - 1)[None, :] + 0 * np.arange(h)[:, None]
        gy = (2 * (np.arange(h) + 0.5) / h - 1)[:, None] + 0 * np.arange(h)[None, :]
        fl = np.stack([gx + 0.03 * np.sin(gy * 3), gy + 0.03 * np.cos(gx * 2)]).astype(np.float32)
        flow = dev.upload(fl)
        d = dev.zeros((2 * r + 1) ** 2 * n)
        ms = time_launches(dev, lambda: api.roma_local_corr(po, f1.mem, f2.mem, C, h, h, r,
                                                            flow.mem, d.mem, 0))
        b = hbm_kernel_bytes("local_corr", C, n, r)
        out.append({"C": C, "cells": f"{h}x{h}", "r": r, "us": round(ms * 1e3, 2),
                    "GBps": round(b / ms / 1e6, 1), "frac_hbm": round(b / ms / 1e6 / PEAK_HBM, 4)})
        for t in (f1, f2, flow, d):
            t.release()
    return out


def bench_hbm_kernels(ic, dev, H=864, W=864):
    """The memory-bound kernels alone at their config shapes: the refiner
    stack's (864 x 864: s8, s4, s2, s1) warp sample, local correlation
    and depthwise 5 x 5, grid_sample at s8, on seeded features and a
    smooth warp; DISK's NMS at 512 x 512. Each timed over 20 launches;
    achieved GB/s = compulsory bytes / mean launch time, reported with
    the rate of a device-to-device copy moving the same bytes (copy_GBps,
    the practical ceiling at that size) and the fraction of it."""
    out = []
    rng = np.random.default_rng(7)
    for s, feat, emb, r in REFINE_V1:
        h, w = H // s, W // s
        n = h * w
        f1 = dev.upload(rng.standard_normal((feat, n), np.float32))
        f2 = dev.upload(rng.standard_normal((feat, n), np.float32))
        gx = (2 * (np.arange(w) + 0.5) / w - 1)[None, :] + 0 * np.arange(h)[:, None]
        gy = (2 * (np.arange(h) + 0.5) / h - 1)[:, None] + 0 * np.arange(w)[None, :]
        fl = np.stack([gx + 0.03 * np.sin(gy * 3), gy + 0.03 * np.cos(gx * 2)]).astype(np.float32)
        flow = dev.upload(fl)
        side = 2 * r + 1
        d = dev.zeros((feat + side * side) * n)
        api, po = dev.api, dev.po
        ms = time_launches(dev, lambda: api.roma_warp_sample(po, f2.mem, feat, h, w, flow.mem,
                                                             d.mem, 0))
        b = hbm_kernel_bytes("warp_sample", feat, n)
        out.append({"kernel": "warp_sample", "scale": s, "C": feat, "cells": n,
                    "ms": round(ms, 5), "bytes": b, "GBps": round(b / ms / 1e6, 1),
                    "frac_hbm": round(b / ms / 1e6 / PEAK_HBM, 4)})
        if r:
            ms = time_launches(dev, lambda: api.roma_local_corr(po, f1.mem, f2.mem, feat, h, w, r,
                                                                flow.mem, d.mem, 0))
            b = hbm_kernel_bytes("local_corr", feat, n, r)
            out.append({"kernel": "local_corr", "scale": s, "C": feat, "r": r, "cells": n,
                        "ms": round(ms, 5), "bytes": b, "GBps": round(b / ms / 1e6, 1),
                        "frac_hbm": round(b / ms / 1e6 / PEAK_HBM, 4)})
        # The refiner's depthwise 5 x 5 on its input width at this scale
        # (2 feat + emb + (2 r + 1)^2 channels): reads and writes it once.
        cin = 2 * feat + emb + (2 * r + 1) ** 2 * (r > 0)
        x = dev.upload(rng.standard_normal((cin, n), np.float32))
        y = dev.zeros(cin * n)
        wdw, bdw = dev.upload(rng.standard_normal((cin, 25), np.float32)), dev.zeros(cin)
        ms = time_launches(dev, lambda: api.roma_dwconv5(po, x.mem, cin, h, w, wdw.mem, bdw.mem,
                                                         y.mem))
        b = 2 * 4 * cin * n + 26 * 4 * cin
        out.append({"kernel": "dwconv5", "scale": s, "C": cin, "cells": n,
                    "ms": round(ms, 5), "bytes": b, "GBps": round(b / ms / 1e6, 1),
                    "frac_hbm": round(b / ms / 1e6 / PEAK_HBM, 4)})
        for t in (f1, f2, flow, d, x, y, wdw, bdw):
            t.release()
    # grid_sample (ops.cl's contract) at the s8 shape on a smooth warp.
    C8, h8 = 512, H // 8
    n8 = h8 * h8
    gx = (2 * (np.arange(h8) + 0.5) / h8 - 1)[None, :] + 0 * np.arange(h8)[:, None]
    gy = (2 * (np.arange(h8) + 0.5) / h8 - 1)[:, None] + 0 * np.arange(h8)[None, :]
    g = np.stack([gx + 0.03 * np.sin(gy * 3), gy + 0.03 * np.cos(gx * 2)], -1)
    src, grid = dev.upload(rng.standard_normal((C8, n8), np.float32)), \
        dev.upload(np.ascontiguousarray(g.reshape(n8, 2), np.float32))
    dst = dev.zeros(C8 * n8)
    ms = time_launches(dev, lambda: api.ops_grid_sample(po, src.mem, C8, h8, h8, grid.mem, n8, 0,
                                                        dst.mem))
    b = 8 * C8 * n8 + 8 * n8
    out.append({"kernel": "grid_sample", "scale": 8, "C": C8, "cells": n8, "ms": round(ms, 5),
                "bytes": b, "GBps": round(b / ms / 1e6, 1),
                "frac_hbm": round(b / ms / 1e6 / PEAK_HBM, 4)})
    # DISK's NMS on the 512 x 512 heatmap: reads it, writes the byte mask.
    heat = dev.upload(rng.standard_normal(512 * 512).astype(np.float32))
    mask = dev.zeros(512 * 512 // 4)
    ms = time_launches(dev, lambda: api.disk_nms5x5(po, heat.mem, 0, 512, 512, 512, 0.0,
                                                    mask.mem))
    b = 5 * 512 * 512
    out.append({"kernel": "nms5x5", "C": 1, "cells": 512 * 512, "ms": round(ms, 5),
                "bytes": b, "GBps": round(b / ms / 1e6, 1),
                "frac_hbm": round(b / ms / 1e6 / PEAK_HBM, 4)})
    for t in (src, grid, dst, heat, mask):
        t.release()
    # The practical ceiling at each size: a device-to-device copy that
    # reads half the kernel's compulsory bytes and writes the other half,
    # timed the same way.
    rates = {}
    for e in out:
        half = (e["bytes"] // 2 + 255) // 256 * 256
        if half not in rates:
            a, b = dev.alloc(half, "copy ceiling"), dev.alloc(half, "copy ceiling")
            ms = time_launches(dev, lambda: api.ocl_copy(dev.pb, a.mem, 0, b.mem, 0, half))
            rates[half] = 2 * half / ms / 1e6
            a.release()
            b.release()
        e["copy_GBps"] = round(rates[half], 1)
        e["frac_copy"] = round(e["GBps"] / rates[half], 4)
    return out


def bench_adalam(ic, dev, n=2048, dim=128):
    """AdaLAM's nearest-neighbour search (adalam_nearest) on two sets of n
    unit descriptors, the DISK config's keypoint count: distance tiles on
    the matrix cores, top-2 per row and argmin per column fused, timed
    over 20 launches. Algorithmic work 2 n^2 dim flop."""
    rng = np.random.default_rng(9)
    d = rng.standard_normal((2, n, dim))
    d = (d / np.linalg.norm(d, axis=2, keepdims=True)).astype(np.float32)
    b1, b2 = dev.upload(d[0]), dev.upload(d[1])
    nn12, sc, nn21 = dev.zeros(n), dev.zeros(n), dev.zeros(n)
    work = dev.alloc(int(dev.api.adalam_nearest_work_bytes(n, n)))
    api, po = dev.api, dev.po
    ms = time_launches(dev, lambda: api.adalam_nearest(po, b1.mem, n, b2.mem, n, dim, nn12.mem,
                                                       sc.mem, nn21.mem, work.mem))
    fl = 2.0 * n * n * dim
    for x in (b1, b2, nn12, sc, nn21, work):
        x.release()
    return {"workload": f"AdaLAM nearest neighbours, {n} x {n} unit descriptors of {dim} "
                        "(nn12, Lowe ratio, nn21)",
            "ms": round(ms, 5), "gflop": round(fl / 1e9, 3),
            "tflops": round(fl / (ms * 1e-3) / 1e12, 2)}


def cpu_adalam(n=2048, dim=128):
    """The oracle's restatement of the host loop (adalam.c:38-116, OpenMP
    over rows as there) on the same sizes, timed once."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_lib import fp, ip, oracle
    orc = oracle()
    nproc, thr = _cpu_threads()
    orc.orc_set_threads(thr)
    rng = np.random.default_rng(9)
    d = rng.standard_normal((2, n, dim))
    d = np.ascontiguousarray((d / np.linalg.norm(d, axis=2, keepdims=True)).astype(np.float32))
    nn12, sc, nn21 = np.zeros(n, np.int32), np.zeros(n, np.float32), np.zeros(n, np.int32)
    d1, d2 = np.ascontiguousarray(d[0]), np.ascontiguousarray(d[1])
    t0 = time.perf_counter()
    orc.orc_adalam_nearest(fp(d1), n, fp(d2), n, dim, ip(nn12), fp(sc), ip(nn21))
    dt = time.perf_counter() - t0
    return {"value": round(dt * 1e3, 3), "unit": "ms", "cores": int(orc.orc_threads()),
            "kind": "port", "sample": f"oracle/ orc_adalam_nearest on the same {n} x {n} x {dim} "
                                      f"sets, one run, {thr} OpenMP threads"}


REF_DIR = ROOT / "oracle" / "_ref"
REF_CASES = ["vitblock:1601", "gemm:1601:3072:1024:1", "gemm:1601:4096:1024:1",
             "gemm:1601:1024:4096:1", "attention:400:400:8:32",
             "localcorr:512:108:108:3", "localcorr:256:216:216:2",
             "warpsample:512:108:108", "warpsample:256:216:216", "warpsample:64:432:432",
             "warpsample:9:864:864", "gridsample:512:108:108:11664"]


def _ours_case(ic, dev, case):
    """This library's kernels on a reference case's shapes: the mean ms of
    one launch (one block schedule for vitblock), HIP events."""
    kind, *a = case.split(":")
    a = [int(x) for x in a]
    rng = np.random.default_rng(1)
    api, po = dev.api, dev.po
    keep = []

    def up(*shape, s=1.0):
        b = dev.upload((s * rng.uniform(-1, 1, shape)).astype(np.float32))
        keep.append(b)
        return b

    def zeros(n):
        b = dev.zeros(n)
        keep.append(b)
        return b

    if kind == "gemm":
        M, N, K, tb = a
        A, B, Cb = up(M, K), up(N, K) if tb else up(K, N), zeros(M * N)
        fn = lambda: api.ops_gemm(po, M, N, K, ic.mat(A, 0, K), ic.mat(B, 0, K if tb else N), tb,
                                  ic.mat(Cb, 0, N), 1, 1, None, 0, None, 0, 1.0, 0, 0.0)
    elif kind == "vitblock":
        N, D = a[0], 1024
        x, t, qkv = up(N, D), zeros(N * D), zeros(N * 3 * D)
        o, h = zeros(N * D), zeros(N * 4 * D)
        wq, wp, w1, w2 = up(3 * D, D, s=0.03), up(D, D, s=0.03), up(4 * D, D, s=0.03), \
            up(D, 4 * D, s=0.03)
        bb, gg = up(4 * D, s=0.1), up(D)

        def fn():
            api.ops_layernorm(po, N, D, x.mem, t.mem, gg.mem, bb.mem, 1e-6, 0, 0.0)
            api.ops_linear(po, N, D, 3 * D, t.mem, 0, wq.mem, bb.mem, qkv.mem, 0, 0, 0.0, 0)
            api.ops_attention(po, ic.mat(qkv, 0, 3 * D), ic.mat(qkv, D, 3 * D),
                              ic.mat(qkv, 2 * D, 3 * D), ic.mat(o, 0, D), N, N, 16, 64,
                              0.125, None)
            api.ops_linear(po, N, D, D, o.mem, 0, wp.mem, bb.mem, x.mem, 0, 0, 0.0, 1)
            api.ops_layernorm(po, N, D, x.mem, t.mem, gg.mem, bb.mem, 1e-6, 0, 0.0)
            api.ops_linear(po, N, D, 4 * D, t.mem, 0, w1.mem, bb.mem, h.mem, 0, 1, 0.0, 0)
            api.ops_linear(po, N, 4 * D, D, h.mem, 0, w2.mem, bb.mem, x.mem, 0, 0, 0.0, 1)
    elif kind == "attention":
        Nq, Nk, nh, d = a
        Q, K, V, O = up(Nq, nh * d), up(Nk, nh * d), up(Nk, nh * d), zeros(Nq * nh * d)
        fn = lambda: api.ops_attention(po, ic.mat(Q, 0, nh * d), ic.mat(K, 0, nh * d),
                                       ic.mat(V, 0, nh * d), ic.mat(O, 0, nh * d), Nq, Nk, nh,
                                       d, 1.0 / np.sqrt(d), None)
    elif kind in ("localcorr", "warpsample"):
        Cc, hh, ww = a[:3]
        n = hh * ww
        gx = (2 * (np.arange(ww) + 0.5) / ww - 1)[None, :] + 0 * np.arange(hh)[:, None]
        gy = (2 * (np.arange(hh) + 0.5) / hh - 1)[:, None] + 0 * np.arange(ww)[None, :]
        fl = dev.upload(np.stack([gx + 0.03 * np.sin(gy * 3),
                                  gy + 0.03 * np.cos(gx * 2)]).astype(np.float32))
        keep.append(fl)
        f1, f2 = up(Cc, n), up(Cc, n)
        if kind == "localcorr":
            r = a[3]
            out = zeros((2 * r + 1) ** 2 * n)
            fn = lambda: api.roma_local_corr(po, f1.mem, f2.mem, Cc, hh, ww, r, fl.mem,
                                             out.mem, 0)
        else:
            out = zeros(Cc * n)
            fn = lambda: api.roma_warp_sample(po, f2.mem, Cc, hh, ww, fl.mem, out.mem, 0)
    elif kind == "gridsample":
        Cc, H, W, n = a
        src, out = up(Cc, H * W), zeros(Cc * n)
        if n == H * W:  # a smooth warp of the same grid, as the reference case
            gx = (2 * (np.arange(W) + 0.5) / W - 1)[None, :] + 0 * np.arange(H)[:, None]
            gy = (2 * (np.arange(H) + 0.5) / H - 1)[:, None] + 0 * np.arange(W)[None, :]
            g = np.stack([gx + 0.03 * np.sin(gy * 3), gy + 0.03 * np.cos(gx * 2)], -1)
            grid = dev.upload(np.ascontiguousarray(g.reshape(n, 2), np.float32))
            keep.append(grid)
        else:
            grid = up(n, 2, s=1.05)
        fn = lambda: api.ops_grid_sample(po, src.mem, Cc, H, W, grid.mem, n, 0, out.mem)
    else:
        raise ValueError(case)
    ms = time_launches(dev, fn, reps=10)
    for b in keep:
        b.release()
    return ms


def reference_same_gpu(ic, dev):
    """The reference's own OpenCL kernels (ops.cl, roma_kernels.cl, built
    by oracle/Makefile's `ref` target from the reference sources) on this
    GPU through the ROCm OpenCL runtime, at the headline shapes, beside
    this library's kernels on the same shapes. None when the reference
    build is absent."""
    exe = REF_DIR / "ref_ocl"
    if not exe.exists():
        return None
    import subprocess
    p = subprocess.run([str(exe), str(REF_DIR)] + REF_CASES, capture_output=True, text=True,
                       timeout=300)
    if p.returncode != 0:
        return {"error": p.stderr.strip()[-500:]}
    rows = []
    for line in p.stdout.splitlines():
        r = json.loads(line)
        ours = _ours_case(ic, dev, r["case"])
        row = {"case": r["case"], "reference_kernel": r["kernel"],
               "reference_ms": round(r["ms"], 5), "ours_ms": round(ours, 5),
               "speedup": round(r["ms"] / ours, 2), "reference_check_rel": r["check_rel"]}
        if "gflop" in r:
            row["reference_tflops"] = round(r["gflop"] / r["ms"], 2)
            row["ours_tflops"] = round(r["gflop"] / ours, 2)
        if "bytes" in r:
            row["reference_GBps"] = round(r["bytes"] / r["ms"] / 1e6, 1)
            row["ours_GBps"] = round(r["bytes"] / ours / 1e6, 1)
        if "parts_ms" in r:
            row["reference_parts_ms"] = r["parts_ms"]
        rows.append(row)
    return {"what": "the reference's ops.cl / roma_kernels.cl compiled for gfx950 and run "
                    "through the ROCm OpenCL runtime on the same MI355X, argument conventions "
                    "of its ops.c / roma.c dispatch, outputs checked in double; ours on the "
                    "same shapes (vitblock: the reference's DINOv2 block schedule on one "
                    "1601-token image against this library's)",
            "cases": rows}


def _kernel_table(table, steps):
    return {k: {"ms_per_step": round(v[0] / steps, 4), "launches_per_step": v[1] / steps}
            for k, v in sorted(table.items(), key=lambda kv: -kv[1][0])}


def bench_refiners(ic, dev, synth, wdir, steps, warmup, profile_steps, H=864):
    """The refiner config (roma_refine_device): VGG19-BN on both 864 x 864
    images, then RoMa's refiners at 1/8 .. 1/1 from the synthetic initial
    warp, on a pair already in HBM."""
    fm, fd, _ = synth.roma_weights_files(wdir)
    a, b, flow8, cert8 = synth.roma_refine_inputs(H, H)
    net = ic.Roma(dev, fm, fd, H, H)
    pair = dev.upload(np.stack([synth.imagenet_norm(a), synth.imagenet_norm(b)]))
    f8, c8 = dev.upload(flow8), dev.upload(cert8)
    run = lambda: net.refine_device(pair, f8, c8)
    for _ in range(warmup):
        run()
    dev.finish()
    dev.reset_events()
    t0 = time.perf_counter()
    e0 = dev.event()
    for _ in range(steps):
        run()
    e1 = dev.event()
    dev.finish()
    ms = max(dev.elapsed_ms(e0, e1), (time.perf_counter() - t0) * 1e3) / steps
    dev.profile_reset()
    dev.set_profile(2)
    for _ in range(profile_steps):
        run()
    dev.finish()
    table = dev.profile_table()
    dev.set_profile(0)
    net.close()
    fl = 2 * vgg_flops(H, H) + refiner_flops(H, H)
    kern = _kernel_table(table, profile_steps)
    print("[bench] refiners per-kernel ms per pair: " + json.dumps(kern), file=sys.stderr,
          flush=True)
    return {"workload": f"RoMa refiner stack, {H}x{H} RGB pair in HBM: VGG19-BN x 2, v1 "
                        "refiners at 1/8, 1/4, 1/2, 1/1 (local correlation r = 3, 2) from the "
                        "synthetic initial warp (roma_refine_device)",
            "pairs_per_s": round(1000.0 / ms, 3), "ms_per_pair": round(ms, 4),
            "gflop_per_pair": round(fl / 1e9, 1),
            "pipeline_tflops": round(fl / (ms * 1e-3) / 1e12, 2), "kernels": kern}


def bench_v2ref(ic, dev, synth, wdir, steps, warmup, H=1024):
    """roma_v2ref end to end on a 1024 x 1024 pair: host images in (PIL
    bicubic resampling, upload), RoMa coarse at 560 with both VGG19-BN
    stacks, v2 refiners at 1/4, 1/2, 1/1 of the coarse and of the tile
    pass, host epilogue out (roma_match)."""
    fm, fd, f2 = synth.roma_weights_files(wdir)
    a, b, _ = synth.roma_pair(H, H, seed=synth.BASE_SEED + synth.CONFIG_V2REF)
    net = ic.Roma(dev, fm, fd, H, H, v2_path=f2)
    for _ in range(warmup):
        net.match(a, b)
    dev.finish()
    t0 = time.perf_counter()
    for _ in range(steps):
        net.match(a, b)
    dev.finish()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    dev.profile_reset()
    dev.set_profile(2)
    net.match(a, b)
    dev.finish()
    table = dev.profile_table()
    dev.set_profile(0)
    net.close()
    kern = _kernel_table(table, 1)
    dev_ms = sum(v["ms_per_step"] for v in kern.values())
    print("[bench] v2ref per-kernel ms per pair: " + json.dumps(kern), file=sys.stderr,
          flush=True)
    return {"workload": f"roma_v2ref end to end on a {H}x{H} RGB pair (host images in, "
                        "roma_match: coarse 560 + v2 refiners, host epilogue out)",
            "pairs_per_s": round(1000.0 / ms, 3), "ms_per_pair": round(ms, 3),
            "device_kernel_ms_per_pair": round(dev_ms, 3), "kernels": kern}


def bench_disk(ic, dev, synth, wdir, steps, warmup, H=512, n=2048):
    """DISK on one 512 x 512 RGB image, host image in and keypoints out
    (disk_detect: U-Net, NMS, top-n, descriptors)."""
    fpath = synth.disk_weights_file(wdir / "disk_random.safetensors")
    img = synth.disk_image(H, H)
    net = ic.Disk(dev, fpath, H, H, nmax=n)
    for _ in range(warmup):
        r = net.detect(img, n=n, thresh=0.0)
    t0 = time.perf_counter()
    for _ in range(steps):
        r = net.detect(img, n=n, thresh=0.0)
    ms = (time.perf_counter() - t0) * 1e3 / steps
    dev.profile_reset()
    dev.set_profile(2)
    net.detect(img, n=n, thresh=0.0)
    dev.finish()
    table = dev.profile_table()
    dev.set_profile(0)
    net.close()
    kern = _kernel_table(table, 1)
    fl = disk_flops(H, H)
    conv_ms = sum(v["ms_per_step"] for k, v in kern.items() if k.startswith("conv"))
    print("[bench] DISK per-kernel ms per image: " + json.dumps(kern), file=sys.stderr,
          flush=True)
    return {"workload": f"DISK {H}x{H} RGB image, n = {n} (host image in, keypoints and "
                        "descriptors out)",
            "images_per_s": round(1000.0 / ms, 3), "ms_per_image": round(ms, 4),
            "keypoints": int(r["n"]), "gflop_per_image": round(fl / 1e9, 1),
            "conv_tflops": round(fl / (conv_ms * 1e-3) / 1e12, 2) if conv_ms else None,
            "kernels": kern}


def _cpu_threads():
    """(CPUs this process may run on, OpenMP threads the baseline pins):
    the box's CPU share per GPU is 16 threads."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return n, min(n, 16)


def cpu_baseline(weights, H=640, W=640):
    """The oracle (C port of the reference kernels and eloftr.c schedule,
    OpenMP) timed on one whole H x W pair of the config: no scaling."""
    sys.path.insert(0, str(ROOT / "tests"))
    sys.path.insert(0, str(PKG_DIR))
    import synth
    from oracle_lib import eloftr_forward, oracle
    orc = oracle()
    nproc, thr = _cpu_threads()
    orc.orc_set_threads(thr)
    g0, g1, _ = synth.eloftr_pair(H, W)
    t0 = time.perf_counter()
    eloftr_forward(weights, g0, g1)
    dt = time.perf_counter() - t0
    return {"value": 1.0 / dt, "unit": "tile-pairs/s", "cores": int(orc.orc_threads()),
            "kind": "port",
            "sample": f"oracle/ (C port of the reference kernels + eloftr.c schedule, OpenMP) "
                      f"full ELoFTR pass on one {H}x{W} pair (the config itself, no scaling) "
                      f"in {dt:.1f} s; {thr} OpenMP threads set by omp_set_num_threads, "
                      f"{nproc} CPUs visible to the process"}


def cpu_baseline_roma(coarse=560, blocks=2):
    """The oracle's DINOv2 ViT-L block (roma.c:675-713, the block() the
    oracle's RoMa forward runs) timed on `blocks` whole blocks at the
    config's token count; the pair's 48 blocks plus the rest of the
    coarse pass are priced at the blocks' rate by algorithmic FLOPs."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_lib import oracle, vit_block
    orc = oracle()
    nproc, thr = _cpu_threads()
    orc.orc_set_threads(thr)
    D = 1024
    nt = (coarse // 14) ** 2 + 1
    rng = np.random.default_rng(0)
    s = 1.0 / np.sqrt(D)
    shapes = [(D,), (D,), (3 * D, D), (3 * D,), (D, D), (D,), (D,), (D,), (4 * D, D),
              (4 * D,), (D, 4 * D), (D,)]
    w = [(s * rng.standard_normal(sh)).astype(np.float32) for sh in shapes]
    X = rng.standard_normal((nt, D)).astype(np.float32)
    vit_block(w, X[:64])  # first touch of the weights and the thread pool
    t0 = time.perf_counter()
    for _ in range(blocks):
        X = vit_block(w, X)
    dt = (time.perf_counter() - t0) / blocks
    blk = 2.0 * nt * D * 12 * D + 4.0 * 16 * nt * nt * 64
    fl = roma_coarse_flops(coarse)
    pair_s = dt * fl["total"] / blk
    return {"value": 1.0 / pair_s, "unit": "tile-pairs/s", "cores": int(orc.orc_threads()),
            "kind": "port",
            "sample": f"oracle/ DINOv2 ViT-L/14 block (C port, OpenMP) timed on {blocks} whole "
                      f"blocks at {nt} tokens ({dt:.2f} s per block, {blk / 1e9:.1f} GFLOP); "
                      f"the coarse pair ({fl['total'] / 1e9:.0f} GFLOP: 48 such blocks, "
                      f"patch embedding, GP, decoder) priced at that rate "
                      f"(x{fl['total'] / blk:.1f}); {thr} OpenMP threads, {nproc} CPUs visible"}


def cpu_baseline_roma_full(coarse=560):
    """The oracle's whole coarse forward (orc_roma_coarse: DINOv2 on both
    images, GP, decoder) on the config's pair, timed once (about two
    minutes on 16 threads: only with --cpu-full)."""
    sys.path.insert(0, str(ROOT / "tests"))
    sys.path.insert(0, str(PKG_DIR))
    import synth
    from oracle_lib import oracle, roma_coarse
    orc = oracle()
    nproc, thr = _cpu_threads()
    orc.orc_set_threads(thr)
    a, b, _ = synth.roma_pair(coarse, coarse)
    wm, wd = synth.roma_weights(), synth.dino_weights()
    t0 = time.perf_counter()
    _, _, info = roma_coarse(wm, wd, synth.imagenet_norm(a), synth.imagenet_norm(b))
    dt = time.perf_counter() - t0
    return {"value": 1.0 / dt, "unit": "tile-pairs/s", "cores": int(orc.orc_threads()),
            "kind": "port", "gp_info": int(info),
            "sample": f"oracle/ orc_roma_coarse (C port, OpenMP): the whole coarse forward of "
                      f"the {coarse}x{coarse} config pair once, {dt:.1f} s; {thr} OpenMP "
                      f"threads, {nproc} CPUs visible"}


def cpu_baseline_disk(side=256, H=512):
    """The oracle's DISK detection (disk.c:164-273: U-Net, NMS, top-n,
    descriptors) on a side x side crop of the config image, scaled to the
    H x H image by pixels (every layer's work is per pixel)."""
    sys.path.insert(0, str(ROOT / "tests"))
    sys.path.insert(0, str(PKG_DIR))
    import synth
    from oracle_lib import disk_detect, oracle
    orc = oracle()
    nproc, thr = _cpu_threads()
    orc.orc_set_threads(thr)
    img = np.ascontiguousarray(synth.disk_image(H, H)[:, :side, :side])
    w = synth.disk_weights()
    t0 = time.perf_counter()
    disk_detect(w, img, n=2048 * side * side // (H * H), thresh=0.0)
    dt = time.perf_counter() - t0
    scale = (H * H) / (side * side)
    return {"value": 1.0 / (dt * scale), "unit": "images/s", "cores": int(orc.orc_threads()),
            "kind": "port",
            "sample": f"oracle/ DISK detect (C port, OpenMP) on the {side}x{side} crop of the "
                      f"config image in {dt:.1f} s, scaled x{scale:.0f} by pixels to {H}x{H}; "
                      f"{thr} OpenMP threads, {nproc} CPUs visible"}


def cpu_baseline_refiners(side=288, H=864):
    """The oracle's refiner config unit (orc_roma_refine: VGG19-BN on both
    images, v1 refiners at 1/8 .. 1/1 from the synthetic initial warp) on
    a side x side pair of the same recipe, scaled to H x H by pixels."""
    sys.path.insert(0, str(ROOT / "tests"))
    sys.path.insert(0, str(PKG_DIR))
    import synth
    from oracle_lib import oracle, roma_refine
    orc = oracle()
    nproc, thr = _cpu_threads()
    orc.orc_set_threads(thr)
    a, b, f8, c8 = synth.roma_refine_inputs(side, side)
    wm, wd = synth.roma_weights(), synth.dino_weights()
    t0 = time.perf_counter()
    roma_refine(wm, wd, synth.imagenet_norm(a), synth.imagenet_norm(b), f8, c8, 560)
    dt = time.perf_counter() - t0
    scale = (H * H) / (side * side)
    return {"value": 1.0 / (dt * scale), "unit": "tile-pairs/s", "cores": int(orc.orc_threads()),
            "kind": "port",
            "sample": f"oracle/ orc_roma_refine (C port, OpenMP, its weight load included) on "
                      f"a {side}x{side} pair of the refiner recipe in {dt:.1f} s, scaled "
                      f"x{scale:.0f} by pixels to "
                      f"{H}x{H}; {thr} OpenMP threads, {nproc} CPUs visible"}


def bench_host_loop(ic, dev, net, pairs, steps):
    """ELoFTR over host-resident pairs, PCIe included: eloftr_match (a
    blocking upload from pageable memory, the device stage, the match
    read) against the overlapped loop that ocl_write_async allows (pair
    t + 1 copied into page-locked memory and uploaded into the other
    device slot while pair t computes, eloftr_match_enqueue / collect)."""
    import ctypes as C
    a = dev.api
    H, W = pairs[0][0].shape
    n = H * W
    # At least two pairs: the warm-up loops below run two.
    seq = [pairs[t % len(pairs)] for t in range(max(steps, 2))]
    for g0, g1 in seq[:2]:
        a.eloftr_match(net.m, g0.ctypes.data, g1.ctypes.data, None, 1)
    dev.finish()
    t0 = time.perf_counter()
    for g0, g1 in seq[:steps]:
        a.eloftr_match(net.m, g0.ctypes.data, g1.ctypes.data, None, 1)
    blocking = (time.perf_counter() - t0) * 1e3 / steps

    ptr = [a.ocl_host_alloc(dev.pb, 8 * n) for _ in range(2)]
    view = [np.ctypeslib.as_array((C.c_float * (2 * n)).from_address(p)) for p in ptr]
    slots = [(dev.alloc(4 * n), dev.alloc(4 * n)) for _ in range(2)]
    tickets = [None, None]

    def upload(t):
        s = t % 2
        if tickets[s] is not None:
            a.ocl_write_wait(dev.pb, tickets[s][1])
        view[s][:n] = seq[t][0].ravel()
        view[s][n:] = seq[t][1].ravel()
        tickets[s] = (a.ocl_write_async(dev.pb, slots[s][0].mem, 0, ptr[s], 4 * n),
                      a.ocl_write_async(dev.pb, slots[s][1].mem, 0, ptr[s] + 4 * n, 4 * n))

    def loop(k):
        upload(0)
        for t in range(k):
            s = t % 2
            a.ocl_write_join(dev.pb, tickets[s][0])
            a.ocl_write_join(dev.pb, tickets[s][1])
            a.eloftr_match_enqueue(net.m, slots[s][0].mem, slots[s][1].mem)
            if t + 1 < k:
                upload(t + 1)
            a.eloftr_match_collect(net.m)

    try:
        loop(2)
        dev.finish()
        t0 = time.perf_counter()
        loop(steps)
        overlapped = (time.perf_counter() - t0) * 1e3 / steps
    finally:
        for p in ptr:
            a.ocl_host_free(p)
    return {"workload": f"ELoFTR {H}x{W} grey pairs in host memory, {steps} in a row, "
                        "upload + device stage + match read (host wall clock)",
            "blocking_pairs_per_s": round(1000.0 / blocking, 3),
            "overlapped_pairs_per_s": round(1000.0 / overlapped, 3),
            "ms_per_pair": {"blocking": round(blocking, 4), "overlapped": round(overlapped, 4)}}


def copy_calibration(dev, mib):
    """One device-to-device copy of mib MiB: the known-size reference that
    scales the HBM byte counters of a rocprofv3 --pmc run."""
    nb = mib << 20
    src, dst = dev.alloc(nb, "calibration"), dev.alloc(nb, "calibration")
    dev.api.ocl_fill(dev.pb, src.mem, 0, nb // 4, 1.0)
    dev.finish()
    dev.api.ocl_copy(dev.pb, src.mem, 0, dst.mem, 0, nb)
    dev.finish()
    print(f"[bench] calibration copy of {mib} MiB done", file=sys.stderr, flush=True)
    src.release()
    dst.release()


DETAIL = ROOT / "gpurun_out" / "bench_detail.json"


def write_detail(obj):
    """The full records of a run (per-kernel tables, every memory-bound
    kernel and reference case) as JSON under gpurun_out/, and on stderr."""
    text = json.dumps(obj)
    print("[bench] detail: " + text, file=sys.stderr, flush=True)
    try:
        DETAIL.parent.mkdir(exist_ok=True)
        DETAIL.write_text(text + "\n")
    except OSError as e:
        print(f"[bench] could not write {DETAIL}: {e}", file=sys.stderr, flush=True)


def _short_cpu(c):
    if not c:
        return c
    return {"value": round(c["value"], 5), "unit": c["unit"], "cores": c["cores"],
            "kind": c["kind"], "sample": c["sample"]}


def _short_roma(r):
    """RoMa 560 coarse: throughput, the GEMM roofline and the attention
    share, the HIP-graph rate and the CPU baseline."""
    if not r:
        return r
    out = {"pairs_per_s": r["pairs_per_s"], "ms_per_pair": r["ms_per_pair"],
           "graph_pairs_per_s": r["graph"]["pairs_per_s"],
           "gflop_per_pair": r["gflop_per_pair"], "pipeline_tflops": r["pipeline_tflops"],
           "roofline": {k: r["roofline"][k] for k in ("bound", "achieved", "peak", "unit", "frac")},
           "attention_frac": r["attention"]["frac"], "gp_solve_ms": r.get("gp_solve_ms")}
    out["roofline"]["kernel"] = "gemm_mfma (fp32 MFMA GEMMs of the ViT, GP and decoder)"
    if r.get("cpu_baseline"):
        out["cpu_baseline"] = _short_cpu(r["cpu_baseline"])
    if r.get("cpu_baseline_full"):
        out["cpu_baseline_full"] = _short_cpu(r["cpu_baseline_full"])
    return out


def _short_extra(extra):
    """One figure or two per extra leg; memory-bound kernels as
    [kernel, scale, GB/s, fraction of HBM peak]; reference cases as
    their speed-ups."""
    out = {}
    if "refiners864" in extra:
        e = extra["refiners864"]
        out["refiners864"] = {"pairs_per_s": e["pairs_per_s"],
                              "pipeline_tflops": e["pipeline_tflops"]}
        if e.get("cpu_baseline"):
            out["refiners864"]["cpu_baseline"] = _short_cpu(e["cpu_baseline"])
    if "roma_v2ref1024" in extra:
        e = extra["roma_v2ref1024"]
        out["roma_v2ref1024"] = {"pairs_per_s": e["pairs_per_s"],
                                 "device_kernel_ms_per_pair": e["device_kernel_ms_per_pair"]}
    if "disk512" in extra:
        e = extra["disk512"]
        out["disk512"] = {"images_per_s": e["images_per_s"], "conv_tflops": e["conv_tflops"],
                          "keypoints": e["keypoints"]}
        if e.get("cpu_baseline"):
            out["disk512"]["cpu_baseline"] = _short_cpu(e["cpu_baseline"])
    if "adalam_nn2048" in extra:
        e = extra["adalam_nn2048"]
        out["adalam_nn2048"] = {"ms": e["ms"], "tflops": e["tflops"]}
        if e.get("cpu_baseline"):
            out["adalam_nn2048"]["cpu_ms"] = e["cpu_baseline"]["value"]
    if "hbm_kernels" in extra:
        out["hbm_kernels"] = [[e["kernel"], e.get("scale"), e["GBps"], e["frac_hbm"]]
                              for e in extra["hbm_kernels"]]
    ref = extra.get("reference_opencl_same_gpu")
    if ref and "cases" in ref:
        out["reference_opencl_speedup"] = {c["case"]: c["speedup"] for c in ref["cases"]}
    elif ref:
        out["reference_opencl_speedup"] = ref
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--size", type=int, default=640)
    ap.add_argument("--profile-steps", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-full", action="store_true",
                    help="also time the oracle's whole RoMa coarse pass (about two minutes)")
    ap.add_argument("--no-roma", action="store_true")
    ap.add_argument("--roma-only", action="store_true",
                    help="run only the RoMa leg and print its JSON object (for profiling)")
    ap.add_argument("--roma-steps", type=int, default=10)
    ap.add_argument("--leg", choices=["refiners864", "v2ref1024", "disk512", "adalam_nn2048",
                                      "localcorr"],
                    help="run only this extra leg and print its JSON (for profiling)")
    ap.add_argument("--hbm-only", action="store_true",
                    help="run only the memory-bound kernels' leg (and --copy-calib) and "
                         "print its JSON (for counter profiles)")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the refiner, roma_v2ref, DISK and HBM-kernel legs")
    ap.add_argument("--copy-calib", type=int, default=0,
                    help="MiB: one device-to-device copy of this size, the known-size "
                         "reference for HBM byte counters under rocprofv3 --pmc")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus}: this build runs on one GPU only (tiles are "
              "independent; the multi-GPU design is in DESIGN.md). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(1)

    ic = load_package()
    sys.path.insert(0, str(PKG_DIR))
    import synth

    H = W = args.size
    dev = ic.Device("auto")
    print(f"[bench] {dev.name} ({dev.arch}), {dev.ocl.cu_count} CUs", file=sys.stderr, flush=True)
    wdir = Path(tempfile.gettempdir()) / "icoreg_bench"
    if args.leg:
        wd = Path(tempfile.gettempdir()) / "icoreg_bench"
        fn = {"refiners864": lambda: bench_refiners(ic, dev, synth, wd, 10, 2, 2),
              "v2ref1024": lambda: bench_v2ref(ic, dev, synth, wd, 3, 1),
              "disk512": lambda: bench_disk(ic, dev, synth, wd, 20, 3),
              "adalam_nn2048": lambda: bench_adalam(ic, dev),
              "localcorr": lambda: bench_local_corr_shapes(dev)}[args.leg]
        print(json.dumps({args.leg: fn()}), flush=True)
        dev.close()
        return
    if args.hbm_only:
        if args.copy_calib:
            copy_calibration(dev, args.copy_calib)
        print(json.dumps({"hbm_kernels": bench_hbm_kernels(ic, dev)}), flush=True)
        dev.close()
        return
    if args.roma_only:
        print(json.dumps(bench_roma(ic, dev, synth, wdir, args.roma_steps, 2,
                                    args.profile_steps)), flush=True)
        dev.close()
        return
    wfile = synth.eloftr_weights_file(wdir / "eloftr_random_calibrated.safetensors")
    g0, g1, _ = synth.eloftr_pair(H, W)
    net = ic.Eloftr(dev, wfile, H, W)
    b0, b1 = dev.upload(g0), dev.upload(g1)

    for _ in range(args.warmup):
        net.match_device(b0, b1)
    dev.finish()
    dev.reset_events()
    t0 = time.perf_counter()
    e0 = dev.event()
    for _ in range(args.steps):
        net.match_device(b0, b1)
    e1 = dev.event()
    dev.finish()
    wall = time.perf_counter() - t0
    gpu_ms = dev.elapsed_ms(e0, e1)
    ms = max(gpu_ms, wall * 1e3) / args.steps
    res = net.result()
    nm = int(res["nm"])

    # The same pair from a HIP graph: the whole device stage recorded once
    # (eloftr_match_enqueue) and replayed, the matches read after the
    # last replay.
    graph = None
    try:
        dev.api.ocl_graph_begin(dev.pb)
        dev.api.eloftr_match_enqueue(net.m, b0.mem, b1.mem)
        graph = dev.api.ocl_graph_end(dev.pb)
        for _ in range(args.warmup):
            dev.api.ocl_graph_launch(dev.pb, graph)
        dev.finish()
        dev.reset_events()
        t0 = time.perf_counter()
        e0 = dev.event()
        for _ in range(args.steps):
            dev.api.ocl_graph_launch(dev.pb, graph)
        e1 = dev.event()
        dev.finish()
        wall = time.perf_counter() - t0
        ms_g = max(dev.elapsed_ms(e0, e1), wall * 1e3) / args.steps
        dev.api.eloftr_match_collect(net.m)
        graph_leg = {"workload": f"the headline pair, its device stage replayed from one HIP "
                                 f"graph ({args.steps} replays)",
                     "pairs_per_s": round(1000.0 / ms_g, 3), "ms_per_pair": round(ms_g, 4),
                     "coarse_matches": int(net.result()["nm"])}
    finally:
        if graph:
            ic.lib().ocl_graph_free(graph)

    if args.copy_calib:
        copy_calibration(dev, args.copy_calib)

    # Per-kernel times over a few more steps (event pairs, no sync).
    dev.profile_reset()
    dev.set_profile(2)
    for _ in range(args.profile_steps):
        net.match_device(b0, b1)
    dev.finish()
    table = dev.profile_table()
    dev.set_profile(0)
    ps = args.profile_steps
    fl = eloftr_flops(H, W, nm)
    # The Winograd convolutions, both forms: F(4 x 4) (conv_wino4) where the
    # launch fills the GPU, F(2 x 2) (conv_wino) on the others.
    forms = eloftr_wino_forms(dev, H, W)
    wino_ms = (table.get("conv_wino", (0.0, 0))[0] + table.get("conv_wino4", (0.0, 0))[0]) / ps
    wino_calls = (table.get("conv_wino", (0.0, 0))[1] + table.get("conv_wino4", (0.0, 0))[1]) / ps
    wino_fl = eloftr_wino_flops(H, W, forms)
    achieved = wino_fl / (wino_ms * 1e-3) / 1e12 if wino_ms > 0 else 0.0
    direct_eq = eloftr_wino_direct_flops(H, W) / (wino_ms * 1e-3) / 1e12 if wino_ms > 0 else 0.0
    kernels = {k: {"ms_per_step": round(v[0] / ps, 4), "launches_per_step": v[1] / ps}
               for k, v in sorted(table.items(), key=lambda kv: -kv[1][0])}
    print("[bench] per-kernel ms per pair: " + json.dumps(kernels), file=sys.stderr, flush=True)

    # Fine stage at its largest size (every coarse cell matched once), so
    # that its cost shows whatever the number of coarse matches.
    h, w = H // 8, W // 8
    n = h * w
    cells = np.stack(np.meshgrid(np.arange(w), np.arange(h)), -1).reshape(-1, 2)
    cells = np.ascontiguousarray(np.concatenate([cells, cells], 1).astype(np.int32))
    bc, bo = dev.upload(cells), dev.zeros(4 * n)
    # The matcher's own form: windows sampled from the half-resolution maps.
    f0m, f1m = ic.lib().icoreg_eloftr_buffer(net.m, b"fineh0"), ic.lib().icoreg_eloftr_buffer(net.m, b"fineh1")
    dev.api.eloftr_fine_half(dev.po, f0m, f1m, H, W, bc.mem, n, 10.0, bo.mem)
    dev.finish()
    dev.reset_events()
    ea = dev.event()
    for _ in range(5):
        dev.api.eloftr_fine_half(dev.po, f0m, f1m, H, W, bc.mem, n, 10.0, bo.mem)
    eb = dev.event()
    fine_nmax_ms = dev.elapsed_ms(ea, eb) / 5

    # The same network on a pair that yields coarse matches (unblurred
    # noise, B = A shifted by whole cells): with random-init weights the
    # config pair keeps almost no match, so its fine stage has nothing to
    # do; this line times the whole device stage with thousands of them.
    m0, m1 = synth.eloftr_noise_pair(H, W, shift=(8, 16))
    c0, c1 = dev.upload(m0), dev.upload(m1)
    for _ in range(args.warmup):
        net.match_device(c0, c1)
    dev.finish()
    dev.reset_events()
    t0 = time.perf_counter()
    e0 = dev.event()
    for _ in range(args.steps):
        net.match_device(c0, c1)
    e1 = dev.event()
    dev.finish()
    wall = time.perf_counter() - t0
    ms_m = max(dev.elapsed_ms(e0, e1), wall * 1e3) / args.steps
    nm_m = int(net.result()["nm"])
    with_matches = {
        "workload": f"ELoFTR {H}x{W} grey pair, full device stage, unblurred-noise pair "
                    "with B = A shifted by (8, 16) px",
        "coarse_matches": nm_m, "pairs_per_s": round(1000.0 / ms_m, 3),
        "ms_per_pair": round(ms_m, 4)}
    host_loop = bench_host_loop(ic, dev, net, [(g0, g1), (m0, m1)], args.steps)

    net.close()
    roma = None
    if not args.no_roma:
        roma = bench_roma(ic, dev, synth, wdir, args.roma_steps, 2, args.profile_steps)

    extra = {}
    if not args.no_extra:
        extra["refiners864"] = bench_refiners(ic, dev, synth, wdir, 10, 2, 2)
        extra["hbm_kernels"] = bench_hbm_kernels(ic, dev)
        extra["roma_v2ref1024"] = bench_v2ref(ic, dev, synth, wdir, 3, 1)
        extra["disk512"] = bench_disk(ic, dev, synth, wdir, 20, 3)
        extra["adalam_nn2048"] = bench_adalam(ic, dev)

    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline: oracle ELoFTR pass at the config size", file=sys.stderr,
              flush=True)
        cpu = cpu_baseline(synth.eloftr_weights_calibrated(), H, W)
        if roma is not None:
            print("[bench] CPU baseline: oracle ViT-L blocks at 1601 tokens", file=sys.stderr,
                  flush=True)
            roma["cpu_baseline"] = cpu_baseline_roma()
        if "adalam_nn2048" in extra:
            extra["adalam_nn2048"]["cpu_baseline"] = cpu_adalam()
        if "disk512" in extra:
            print("[bench] CPU baseline: oracle DISK on a 256x256 crop", file=sys.stderr,
                  flush=True)
            extra["disk512"]["cpu_baseline"] = cpu_baseline_disk()
        if "refiners864" in extra:
            print("[bench] CPU baseline: oracle refiners on a 288x288 pair", file=sys.stderr,
                  flush=True)
            extra["refiners864"]["cpu_baseline"] = cpu_baseline_refiners()
        if args.cpu_full and roma is not None:
            print("[bench] CPU baseline: oracle's whole RoMa coarse pass", file=sys.stderr,
                  flush=True)
            roma["cpu_baseline_full"] = cpu_baseline_roma_full()
        print("[bench] baseline: the reference's OpenCL kernels on this GPU", file=sys.stderr,
              flush=True)
        extra["reference_opencl_same_gpu"] = reference_same_gpu(ic, dev)

    # The full records (per-kernel tables, every memory-bound kernel and
    # reference case) go to a file and to stderr; the JSON line on stdout
    # keeps the figures, so that the whole line fits a log's tail.
    detail = {"eloftr640": {"kernels": kernels, "with_matches": with_matches,
                            "graph": graph_leg, "host_loop": host_loop,
                            "fine_ms_at_max_matches": round(fine_nmax_ms, 4)},
              "roma560": roma, "cpu_baseline": cpu, **extra}
    write_detail(detail)
    n4 = sum(1 for f in forms if f == 4)
    rf = {"kernel": f"3x3 stride-1 conv on fp32 MFMA: Winograd F(4x4,3x3) (conv_wino4, {n4} "
                    f"launches) where the launch fills the GPU, F(2x2,3x3) (conv_wino, "
                    f"{len(forms) - n4}) on the others",
          "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP32_MFMA,
          "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA, 4),
          "traffic": conv_traffic() if H == W == 640 else None,
          "algorithmic_bytes_per_launch": round(eloftr_wino_bytes(H, W, forms) / len(forms)),
          "launches_per_step": wino_calls, "gflop_per_step": round(wino_fl / 1e9, 2),
          "direct_equivalent_tflops": round(direct_eq, 2)}
    cc = conv_counters() if H == W == 640 else None
    if cc:
        rf["sq_counters"] = {k: v for k, v in cc.items() if k != "source"}
    line = {
        "metric": "tile-pairs/sec (1 GPU) ELoFTR 640² & RoMa 560², fp32; % MFMA/HBM peak",
        "value": round(1000.0 / ms, 3),
        "unit": "tile-pairs/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded blurred-noise grey pair, B = random affine of A + noise; "
                "seeded He-normal weights, data-calibrated BatchNorm statistics)",
        "config": {"workload": f"ELoFTR {H}x{W} grey pair, full device stage (coarse + fine)",
                   "coarse_matches": nm, "gflop_per_pair": round(fl["total"] / 1e9, 1),
                   "roma560_pairs_per_s": roma["pairs_per_s"] if roma else None},
        "roofline": rf,
        "cpu_baseline": _short_cpu(cpu),
        "eloftr_with_matches": {"coarse_matches": nm_m, "pairs_per_s": with_matches["pairs_per_s"],
                                "ms_per_pair": with_matches["ms_per_pair"]},
        "eloftr_graph_pairs_per_s": graph_leg["pairs_per_s"],
        "eloftr_host_pairs_per_s": {"blocking": host_loop["blocking_pairs_per_s"],
                                    "overlapped": host_loop["overlapped_pairs_per_s"]},
        "pipeline_tflops": round(fl["total"] / (ms * 1e-3) / 1e12, 2),
        "roma560": _short_roma(roma),
        **_short_extra(extra),
        "detail": str(DETAIL.relative_to(ROOT)),
    }
    print(json.dumps(line), flush=True)
    dev.close()


if __name__ == "__main__":
    main()

# SPDX-License-Identifier: Unlicense
"""Synthetic inputs and seeded random-init weights of the benchmark configs.

No checkpoint or dataset is available offline, so every network runs on
weights drawn here and written as safetensors with the reference's tensor
names and shapes (the names its loaders require: eloftr.c:110-230 of
i.coregistration.opencl), read back through the C loader like real
weights. Recipe (seeds: base 20261201 + config index, numpy PCG64):

* image A: uniform white noise, Gaussian blur sigma 2 px, min-max to 0..1;
* ELoFTR image B: A under a random affine (rotation +-5 deg, scale
  0.95..1.05, shift +-20 px), bilinear, plus N(0, 0.01) noise;
* weights: He-normal (std sqrt(2 / fan_in)), no biases where the model has
  none; BatchNorm and LayerNorm parameters randomised around identity
  (scales drawn so that the 21 RepVGG blocks keep activations of order 1,
  as trained weights do).
"""

from pathlib import Path

import numpy as np

BASE_SEED = 20261201
CONFIG_ELOFTR = 1


def smooth_noise(rng, shape, sigma=2.0):
    from scipy.ndimage import gaussian_filter
    x = rng.uniform(0.0, 1.0, shape)
    if len(shape) == 3:
        x = np.stack([gaussian_filter(c, sigma, mode="reflect") for c in x])
    else:
        x = gaussian_filter(x, sigma, mode="reflect")
    x = (x - x.min()) / max(x.max() - x.min(), 1e-12)
    return x.astype(np.float32)


def random_affine(rng, img, rot_deg=5.0, scale=(0.95, 1.05), shift=20.0):
    """img (H, W) warped by a random affine about the centre, bilinear."""
    from scipy.ndimage import map_coordinates
    H, W = img.shape
    th = np.deg2rad(rng.uniform(-rot_deg, rot_deg))
    s = rng.uniform(*scale)
    tx, ty = rng.uniform(-shift, shift, 2)
    c, sn = np.cos(th) * s, np.sin(th) * s
    yy, xx = np.mgrid[0:H, 0:W].astype(np.float64)
    cx, cy = (W - 1) / 2.0, (H - 1) / 2.0
    # Output pixel p samples A at M^-1 (p - c - t) + c.
    det = c * c + sn * sn
    dx, dy = xx - cx - tx, yy - cy - ty
    sx = (c * dx + sn * dy) / det + cx
    sy = (-sn * dx + c * dy) / det + cy
    out = map_coordinates(img.astype(np.float64), [sy, sx], order=1, mode="constant",
                          cval=0.0)
    return out.astype(np.float32), np.array([[c, -sn, tx], [sn, c, ty]])


def eloftr_pair(H=640, W=640, seed=BASE_SEED + CONFIG_ELOFTR):
    """Grey pair (H x W each) for the ELoFTR config and the true affine."""
    rng = np.random.default_rng(seed)
    a = smooth_noise(rng, (H, W))
    b, M = random_affine(rng, a)
    b = b + rng.normal(0.0, 0.01, b.shape).astype(np.float32)
    return a, b.astype(np.float32), M


def eloftr_noise_pair(H, W, shift=(8, 16), seed=BASE_SEED + CONFIG_ELOFTR + 100, noise=0.01):
    """Grey pair that yields coarse matches with random-init weights:
    A is unblurred uniform noise, B is A translated by shift = (dy, dx) px
    (whole 8-px cells), zeros where B leaves A, plus N(0, noise). With the
    config pair (blurred noise) random-init features barely separate the
    cells and the mutual selection keeps almost nothing; sub-cell shifts
    keep almost no coarse match either. A larger noise (0.05) leaves fewer
    coarse matches but makes the fine stage's argmax decisive: with 0.01
    the 64 window positions of a whole-cell shift match almost equally
    well."""
    rng = np.random.default_rng(seed)
    a = rng.uniform(0.0, 1.0, (H, W)).astype(np.float32)
    dy, dx = shift
    b = np.zeros_like(a)
    b[max(dy, 0):H + min(dy, 0), max(dx, 0):W + min(dx, 0)] = \
        a[max(-dy, 0):H - max(dy, 0), max(-dx, 0):W - max(dx, 0)]
    b = b + rng.normal(0.0, noise, b.shape).astype(np.float32)
    return a, b.astype(np.float32)


def _he(rng, shape):
    fan_in = int(np.prod(shape[1:])) if len(shape) > 1 else shape[0]
    return (rng.standard_normal(shape) * np.sqrt(2.0 / fan_in)).astype(np.float32)


def _bn(rng, d, prefix, c, gamma=(0.8, 1.2)):
    d[f"{prefix}.weight"] = rng.uniform(*gamma, c).astype(np.float32)
    d[f"{prefix}.bias"] = rng.uniform(-0.1, 0.1, c).astype(np.float32)
    d[f"{prefix}.running_mean"] = rng.uniform(-0.1, 0.1, c).astype(np.float32)
    d[f"{prefix}.running_var"] = rng.uniform(0.5, 1.5, c).astype(np.float32)


def eloftr_weights(seed=BASE_SEED + CONFIG_ELOFTR):
    """State dict of EfficientLoFTRForKeypointMatching, names and shapes of
    eloftr.c:110-230, seeded random values."""
    rng = np.random.default_rng(seed + 1000)
    d = {}
    blocks, outs, strides = (1, 2, 4, 14), (64, 64, 128, 256), (2, 1, 2, 2)
    cin = 1
    for s in range(4):
        for b in range(blocks[s]):
            co, st = outs[s], strides[s] if b == 0 else 1
            pre = f"efficientloftr.backbone.stages.{s}.blocks.{b}"
            d[f"{pre}.conv1.conv.weight"] = _he(rng, (co, cin, 3, 3))
            _bn(rng, d, f"{pre}.conv1.norm", co, (0.35, 0.55))
            d[f"{pre}.conv2.conv.weight"] = _he(rng, (co, cin, 1, 1))
            _bn(rng, d, f"{pre}.conv2.norm", co, (0.35, 0.55))
            if cin == co and st == 1:
                _bn(rng, d, f"{pre}.identity", co, (0.35, 0.55))
            cin = co
    D, MLP = 256, 512
    for i in range(4):
        for kind in ("self_attention", "cross_attention"):
            pre = f"efficientloftr.local_feature_transformer.layers.{i}.{kind}"
            d[f"{pre}.aggregation.q_aggregation.weight"] = _he(rng, (D, 1, 4, 4))
            d[f"{pre}.aggregation.norm.weight"] = rng.uniform(0.8, 1.2, D).astype(np.float32)
            d[f"{pre}.aggregation.norm.bias"] = rng.uniform(-0.1, 0.1, D).astype(np.float32)
            for p in ("q", "k", "v", "o"):
                d[f"{pre}.attention.{p}_proj.weight"] = _he(rng, (D, D))
            d[f"{pre}.mlp.fc1.weight"] = _he(rng, (MLP, 2 * D))
            d[f"{pre}.mlp.fc2.weight"] = _he(rng, (D, MLP))
            d[f"{pre}.mlp.layer_norm.weight"] = rng.uniform(0.8, 1.2, D).astype(np.float32)
            d[f"{pre}.mlp.layer_norm.bias"] = rng.uniform(-0.1, 0.1, D).astype(np.float32)
    d["refinement_layer.out_conv.weight"] = _he(rng, (256, 256, 1, 1))
    dims = (256, 128, 64)
    for i in range(2):
        hid, inter = dims[i + 1], dims[i]
        pre = f"refinement_layer.out_conv_layers.{i}"
        d[f"{pre}.out_conv1.weight"] = _he(rng, (inter, hid, 1, 1))
        d[f"{pre}.out_conv2.weight"] = _he(rng, (inter, inter, 3, 3))
        _bn(rng, d, f"{pre}.batch_norm", inter)
        d[f"{pre}.out_conv3.weight"] = _he(rng, (hid, inter, 3, 3))
    return d


def calibrate_backbone_bn(w, images, eps=1e-5):
    """Set every RepVGG BatchNorm's running mean / variance to the batch
    statistics of its input on images (N, H, W), block by block, as a
    trained network's running statistics are: without this, random
    running statistics leave the ReLU features with a large common mode
    and no contrast between cells. In place on the float32 dict w."""
    import torch
    import torch.nn.functional as F

    x = torch.from_numpy(np.asarray(images, np.float32))[:, None].double()
    blocks, strides = (1, 2, 4, 14), (2, 1, 2, 2)
    for s in range(4):
        for b in range(blocks[s]):
            pre = f"efficientloftr.backbone.stages.{s}.blocks.{b}"
            st = strides[s] if b == 0 else 1
            out = 0
            for conv, norm, pad in (("conv1", "conv1.norm", 1), ("conv2", "conv2.norm", 0)):
                y = F.conv2d(x, torch.from_numpy(w[f"{pre}.{conv}.conv.weight"]).double(),
                             stride=st, padding=pad)
                out = out + _bn_calibrated(w, f"{pre}.{norm}", y, eps)
            if f"{pre}.identity.weight" in w:
                out = out + _bn_calibrated(w, f"{pre}.identity", x, eps)
            x = torch.relu(out)
    return w


def _bn_calibrated(w, prefix, y, eps):
    mean = y.mean(dim=(0, 2, 3))
    var = y.var(dim=(0, 2, 3), unbiased=False)
    w[f"{prefix}.running_mean"] = mean.numpy().astype(np.float32)
    w[f"{prefix}.running_var"] = var.numpy().astype(np.float32)
    g = np.float64(1.0) * w[f"{prefix}.weight"]
    bt = w[f"{prefix}.bias"]
    import torch
    return ((y - mean[None, :, None, None]) / torch.sqrt(var + eps)[None, :, None, None]
            * torch.from_numpy(g)[None, :, None, None]
            + torch.from_numpy(bt.astype(np.float64))[None, :, None, None])


def eloftr_weights_calibrated(seed=BASE_SEED + CONFIG_ELOFTR, size=256):
    """eloftr_weights with the backbone BatchNorm statistics calibrated on
    a size x size crop of the config's synthetic pair."""
    w = eloftr_weights(seed)
    a, b, _ = eloftr_pair(size, size, seed)
    return calibrate_backbone_bn(w, np.stack([a, b]))


def save_safetensors(tensors, path):
    from safetensors.numpy import save_file
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    save_file({k: np.ascontiguousarray(v) for k, v in tensors.items()}, str(path))
    return path


def save_torch(tensors, path, legacy=False, wrap=None, prefix=""):
    """Write tensors with torch.save, as the published checkpoints are:
    the zip archive (or the legacy pickle stream with legacy=True), names
    prefixed by prefix, the dict optionally wrapped as {wrap: dict, ...}
    the way training checkpoints hold it."""
    import torch
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    sd = {prefix + k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in tensors.items()}
    obj = {wrap: sd, "epoch": 7} if wrap else sd
    torch.save(obj, str(path), _use_new_zipfile_serialization=not legacy)
    return path


def eloftr_weights_file(path, seed=BASE_SEED + CONFIG_ELOFTR):
    """Write (once) and return the ELoFTR weights file."""
    path = Path(path)
    if not path.exists():
        save_safetensors(eloftr_weights_calibrated(seed), path)
    return path


# ---- RoMa ---------------------------------------------------------------------

CONFIG_ROMA = 2


def tps_warp(rng, img, n_ctrl=4, disp=15.0):
    """img (C, H, W) warped by a thin-plate spline through n_ctrl x n_ctrl
    control points with displacements U(-disp, disp) px: output pixel p
    samples img at p + d(p), bilinear, zeros outside. Returns the warped
    image and d (2, H, W) (x, y)."""
    from scipy.interpolate import RBFInterpolator
    from scipy.ndimage import map_coordinates
    C, H, W = img.shape
    cy, cx = np.meshgrid(np.linspace(0, H - 1, n_ctrl), np.linspace(0, W - 1, n_ctrl),
                         indexing="ij")
    ctrl = np.stack([cx.ravel(), cy.ravel()], 1)
    dd = rng.uniform(-disp, disp, ctrl.shape)
    yy, xx = np.mgrid[0:H, 0:W].astype(np.float64)
    pts = np.stack([xx.ravel(), yy.ravel()], 1)
    d = RBFInterpolator(ctrl, dd, kernel="thin_plate_spline")(pts).T.reshape(2, H, W)
    out = np.stack([map_coordinates(c.astype(np.float64), [yy + d[1], xx + d[0]], order=1,
                                    mode="constant", cval=0.0) for c in img])
    return out.astype(np.float32), d


def roma_pair(H=560, W=560, seed=BASE_SEED + CONFIG_ROMA):
    """RGB pair (3, H, W) in 0..1 for the RoMa configs: blurred noise A and
    B = a TPS warp of A (16 control points, +-15 px)."""
    rng = np.random.default_rng(seed)
    a = smooth_noise(rng, (3, H, W))
    b, d = tps_warp(rng, a)
    return a, np.clip(b, 0.0, 1.0).astype(np.float32), d


CONFIG_REFINE = 3
CONFIG_V2REF = 4


def imagenet_norm(img):
    """(3, H, W) in 0..1 normalised with the ImageNet mean and deviation,
    as RoMa's inputs are (roma.c:1170-1186)."""
    mean = np.array([0.485, 0.456, 0.406], np.float32)[:, None, None]
    std = np.array([0.229, 0.224, 0.225], np.float32)[:, None, None]
    return ((img - mean) / std).astype(np.float32)


def roma_refine_inputs(H=864, W=864, seed=BASE_SEED + CONFIG_REFINE, noise_px=2.0):
    """The refiner config's inputs: the RoMa pair at H x W (A blurred
    noise, B = A under a TPS warp) and the initial 1/8-scale warp of A
    onto B, the TPS ground truth at the cell centres perturbed by
    N(0, noise_px) px, normalised to -1..1 with align_corners = 0
    (roma_kernels.cl:1-7), with a zero certainty logit. B(p) = A(p + d(p)),
    so a point q of A lies near q - d(q) in B (first order)."""
    a, b, d = roma_pair(H, W, seed)
    rng = np.random.default_rng(seed + 500)
    h, w = H // 8, W // 8
    ys = (np.arange(h) * 8 + 3.5)[:, None]
    xs = (np.arange(w) * 8 + 3.5)[None, :]
    yi = np.clip(np.rint(ys).astype(int), 0, H - 1)
    xi = np.clip(np.rint(xs).astype(int), 0, W - 1)
    qx = xs - d[0][yi, xi] + rng.normal(0.0, noise_px, (h, w))
    qy = ys - d[1][yi, xi] + rng.normal(0.0, noise_px, (h, w))
    flow = np.stack([(2 * qx + 1) / W - 1, (2 * qy + 1) / H - 1]).astype(np.float32)
    return a, b, flow, np.zeros((h, w), np.float32)


def _rn(rng, shape, std):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std))


def _he32(rng, shape, gain=1.0):
    fan_in = int(np.prod(shape[1:])) if len(shape) > 1 else shape[0]
    return _rn(rng, shape, gain * np.sqrt(2.0 / fan_in))


def _bias(rng, n, a=0.05):
    return rng.uniform(-a, a, n).astype(np.float32)


def _ln(rng, d, prefix, n):
    d[f"{prefix}.weight"] = rng.uniform(0.8, 1.2, n).astype(np.float32)
    d[f"{prefix}.bias"] = _bias(rng, n, 0.1)


def _vit_block(rng, d, pre, D, qkv_bias, ls):
    _ln(rng, d, f"{pre}.norm1", D)
    d[f"{pre}.attn.qkv.weight"] = _he32(rng, (3 * D, D))
    if qkv_bias:
        d[f"{pre}.attn.qkv.bias"] = _bias(rng, 3 * D)
    d[f"{pre}.attn.proj.weight"] = _he32(rng, (D, D))
    d[f"{pre}.attn.proj.bias"] = _bias(rng, D)
    _ln(rng, d, f"{pre}.norm2", D)
    d[f"{pre}.mlp.fc1.weight"] = _he32(rng, (4 * D, D))
    d[f"{pre}.mlp.fc1.bias"] = _bias(rng, 4 * D)
    d[f"{pre}.mlp.fc2.weight"] = _he32(rng, (D, 4 * D))
    d[f"{pre}.mlp.fc2.bias"] = _bias(rng, D)
    if ls:
        d[f"{pre}.ls1.gamma"] = rng.uniform(0.1, 0.5, D).astype(np.float32)
        d[f"{pre}.ls2.gamma"] = rng.uniform(0.1, 0.5, D).astype(np.float32)


def _vgg(rng, d, pre, nblk):
    idx, cin = 0, 3
    for blk, (nconv, co) in enumerate(zip((2, 2, 4, 4), (64, 128, 256, 512))):
        if blk >= nblk:
            break
        for _ in range(nconv):
            d[f"{pre}.{idx}.weight"] = _he32(rng, (co, cin, 3, 3))
            d[f"{pre}.{idx}.bias"] = _bias(rng, co)
            _bn(rng, d, f"{pre}.{idx + 1}", co)
            cin = co
            idx += 3
        idx += 1


def _refiner_blocks(rng, d, pre, cin, dw, bn, pw):
    for b in range(9):
        blk = f"{pre}.block1" if b == 0 else f"{pre}.hidden_blocks.{b - 1}"
        d[f"{blk}.{dw}.weight"] = _he32(rng, (cin, 1, 5, 5))
        d[f"{blk}.{dw}.bias"] = _bias(rng, cin)
        _bn(rng, d, f"{blk}.{bn}", cin)
        d[f"{blk}.{pw}.weight"] = _he32(rng, (cin, cin, 1, 1))
        d[f"{blk}.{pw}.bias"] = _bias(rng, cin)


ROMA_REFINERS = {16: (512, 128, 7), 8: (512, 64, 3), 4: (256, 32, 2), 2: (64, 16, 0), 1: (9, 6, 0)}
ROMA_PROJ_IN = {16: 1024, 8: 512, 4: 256, 2: 128, 1: 64}
ROMA2_REFINERS = {4: (256, 192, 79, 3), 2: (128, 48, 23, 1), 1: (64, 12, 8, 0)}


def roma_weights(seed=BASE_SEED + CONFIG_ROMA):
    """RoMa RegressionMatcher state dict (roma_outdoor names and shapes,
    roma.c:213-436), seeded: He-normal weights, small random biases,
    BatchNorm and LayerNorm parameters randomised around identity."""
    rng = np.random.default_rng(seed + 1000)
    d = {}
    _vgg(rng, d, "encoder.cnn.layers", 4)
    for s, (feat, _, _) in ROMA_REFINERS.items():
        d[f"decoder.proj.{s}.0.weight"] = _he32(rng, (feat, ROMA_PROJ_IN[s], 1, 1))
        d[f"decoder.proj.{s}.0.bias"] = _bias(rng, feat)
        _bn(rng, d, f"decoder.proj.{s}.1", feat)
    d["decoder.gps.16.pos_conv.weight"] = _rn(rng, (512, 2, 1, 1), 0.1)
    d["decoder.gps.16.pos_conv.bias"] = _bias(rng, 512, 0.1)
    for i in range(5):
        _vit_block(rng, d, f"decoder.embedding_decoder.blocks.{i}", 1024, False, False)
    d["decoder.embedding_decoder.to_out.weight"] = _he32(rng, (4097, 1024))
    d["decoder.embedding_decoder.to_out.bias"] = _bias(rng, 4097)
    for s, (feat, emb, rad) in ROMA_REFINERS.items():
        cin = 2 * feat + emb + ((2 * rad + 1) ** 2 if rad else 0)
        pre = f"decoder.conv_refiner.{s}"
        _refiner_blocks(rng, d, pre, cin, "0", "1", "3")
        d[f"{pre}.out_conv.weight"] = _he32(rng, (3, cin, 1, 1), 0.01)
        d[f"{pre}.out_conv.bias"] = _bias(rng, 3)
        d[f"{pre}.disp_emb.weight"] = _he32(rng, (emb, 2, 1, 1))
        d[f"{pre}.disp_emb.bias"] = _bias(rng, emb)
    return d


def dino_weights(seed=BASE_SEED + CONFIG_ROMA):
    """DINOv2 ViT-L/14 state dict (dinov2_vitl14_pretrain names and shapes,
    roma.c:300-324), seeded."""
    rng = np.random.default_rng(seed + 2000)
    D = 1024
    d = {"patch_embed.proj.weight": _he32(rng, (D, 3, 14, 14)),
         "patch_embed.proj.bias": _bias(rng, D),
         "cls_token": _rn(rng, (1, 1, D), 0.5),
         "pos_embed": _rn(rng, (1, 37 * 37 + 1, D), 0.5)}
    for i in range(24):
        _vit_block(rng, d, f"blocks.{i}", D, True, True)
    _ln(rng, d, "norm", D)
    return d


def roma2_weights(seed=BASE_SEED + CONFIG_ROMA):
    """RoMa v2 refiners and their VGG19-BN (refiners.*, refiner_features.*
    names and shapes, roma.c:452-544), seeded."""
    rng = np.random.default_rng(seed + 3000)
    d = {}
    _vgg(rng, d, "refiner_features.layers", 3)
    for s, (fin, feat, emb, rad) in ROMA2_REFINERS.items():
        cin = 2 * feat + emb + ((2 * rad + 1) ** 2 if rad else 0)
        pre = f"refiners.{s}"
        d[f"{pre}.proj.weight"] = _he32(rng, (feat, fin))
        d[f"{pre}.proj.bias"] = _bias(rng, feat)
        _refiner_blocks(rng, d, pre, cin, "conv_depthwise", "norm", "conv_pointwise")
        d[f"{pre}.disp_emb.weight"] = _he32(rng, (emb, 2, 1, 1))
        d[f"{pre}.disp_emb.bias"] = _bias(rng, emb)
        d[f"{pre}.warp_head.weight"] = _he32(rng, (2, cin, 1, 1), 0.01)
        d[f"{pre}.warp_head.bias"] = _bias(rng, 2)
        d[f"{pre}.confidence_head.weight"] = _he32(rng, (4, cin, 1, 1), 0.1)
        d[f"{pre}.confidence_head.bias"] = _bias(rng, 4)
    return d


def roma_weights_files(folder, seed=BASE_SEED + CONFIG_ROMA):
    """Write (once) and return the paths of the RoMa, DINOv2 and RoMa v2
    weight files."""
    folder = Path(folder)
    out = []
    for name, fn in (("roma_random", roma_weights), ("dinov2_random", dino_weights),
                     ("romav2_random", roma2_weights)):
        p = folder / f"{name}_{seed}.safetensors"
        if not p.exists():
            save_safetensors(fn(seed), p)
        out.append(p)
    return out


# ---- DISK ---------------------------------------------------------------------

CONFIG_DISK = 0
DISK_CIN = (3, 16, 32, 64, 64, 128, 128, 96, 80)
DISK_COUT = (16, 32, 64, 64, 64, 64, 64, 64, 129)


def disk_image(H=512, W=512, seed=BASE_SEED + CONFIG_DISK):
    """(3, H, W) blurred noise in 0..1, the DISK config's input."""
    return smooth_noise(np.random.default_rng(seed), (3, H, W))


def disk_weights(seed=BASE_SEED + CONFIG_DISK):
    """DISK U-Net state dict (kornia DISK names and shapes, disk.c:43-82),
    seeded: He-normal 5 x 5 convolutions, small biases, PReLU slopes
    U(0.1, 0.3)."""
    rng = np.random.default_rng(seed + 1000)
    d = {}
    for l in range(9):
        pre = f"unet.path_down.{l}.1" if l < 5 else f"unet.path_up.{l - 5}.conv"
        d[f"{pre}.3.weight"] = _he32(rng, (DISK_COUT[l], DISK_CIN[l], 5, 5))
        d[f"{pre}.3.bias"] = _bias(rng, DISK_COUT[l])
        if l > 0:
            d[f"{pre}.1.weight"] = rng.uniform(0.1, 0.3, DISK_CIN[l]).astype(np.float32)
    return d


def disk_weights_file(path, seed=BASE_SEED + CONFIG_DISK):
    path = Path(path)
    if not path.exists():
        save_safetensors(disk_weights(seed), path)
    return path

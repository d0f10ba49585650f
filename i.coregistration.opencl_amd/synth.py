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


def eloftr_weights_file(path, seed=BASE_SEED + CONFIG_ELOFTR):
    """Write (once) and return the ELoFTR weights file."""
    path = Path(path)
    if not path.exists():
        save_safetensors(eloftr_weights_calibrated(seed), path)
    return path

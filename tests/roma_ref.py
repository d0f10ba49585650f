# SPDX-License-Identifier: Unlicense
"""Independent float64 torch statements of RoMa's published building
blocks (Edstedt et al., RoMa, CVPR 2024; romatch/utils/local_correlation
and cls_to_flow_refine), used to pin the oracle's restatement of
roma_kernels.cl (i.coregistration.opencl). Written from the published
definitions in tensor form (grid_sample over shifted grids, gather of
neighbour classes), not from the oracle's loops."""

import math

import numpy as np
import torch
import torch.nn.functional as F


def t64(a):
    return torch.from_numpy(np.asarray(a, np.float64))


def cell_centres(n):
    """Normalised centres of n cells, align_corners = False."""
    return torch.linspace(-1 + 1 / n, 1 - 1 / n, n, dtype=torch.float64)


def grid_sample_flow(feat, flow):
    """feat (C, H, W) sampled at flow (2, H, W) (x, y): F.grid_sample,
    bilinear, zero padding, align_corners = False."""
    C, H, W = feat.shape
    grid = flow.permute(1, 2, 0)[None]
    return F.grid_sample(feat[None], grid, mode="bilinear", padding_mode="zeros",
                         align_corners=False)[0]


def local_correlation(f0, f1, flow, r):
    """RoMa's local_correlation with corr_in_other: f0, f1 (C, h, w),
    flow (2, h, w); (2 r + 1)^2 channels, offset k = a (2 r + 1) + b
    shifting the warp by (b - r, a - r) cells."""
    C, h, w = f0.shape
    side = 2 * r + 1
    wy = torch.linspace(-2 * r / h, 2 * r / h, side, dtype=torch.float64)
    wx = torch.linspace(-2 * r / w, 2 * r / w, side, dtype=torch.float64)
    gy, gx = torch.meshgrid(wy, wx, indexing="ij")
    win = torch.stack([gx, gy], -1).reshape(-1, 2)               # (K, 2)
    coords = flow.permute(1, 2, 0)[:, :, None, :] + win[None, None]  # (h, w, K, 2)
    wf = F.grid_sample(f1[None], coords.reshape(1, h, w * side * side, 2),
                       mode="bilinear", padding_mode="zeros", align_corners=False)
    wf = wf.reshape(C, h, w, side * side)
    return (f0[..., None] / math.sqrt(C) * wf).sum(0).permute(2, 0, 1)


def cls_to_flow_refine(logits):
    """logits (C, n) anchor classes of a res x res grid: softmax, mode and
    its four neighbours (clamped indices), probability-weighted mean
    anchor position (2, n)."""
    C, n = logits.shape
    res = round(math.sqrt(C))
    gy, gx = torch.meshgrid(cell_centres(res), cell_centres(res), indexing="ij")
    G = torch.stack([gx, gy], -1).reshape(C, 2)
    p = logits.softmax(0)
    mode = p.max(0).indices
    idx = torch.stack([mode - 1, mode, mode + 1, mode - res, mode + res], 0).clamp(0, C - 1)
    nb = torch.gather(p, 0, idx)                                  # (5, n)
    flow = (nb[..., None] * G[idx]).sum(0) / nb.sum(0)[:, None]   # (n, 2)
    return flow.T


def disp(flow, H, W, fx, fy):
    gy, gx = torch.meshgrid(cell_centres(H), cell_centres(W), indexing="ij")
    g = torch.stack([gx, gy]).reshape(2, -1)
    return torch.tensor([fx, fy], dtype=torch.float64)[:, None] * (flow - g)


def update2(flow, conf, d, W, H):
    """RoMa v2 refiner update: warp step and precision of the Cholesky
    factor L = [[softplus(d3) + 1e-6, 0], [d4, softplus(d5) + 1e-6]]
    (L L^T entries 00, 10, 11)."""
    flow = flow + d[:2] / torch.tensor([4.0 * W, 4.0 * H], dtype=torch.float64)[:, None]
    l00 = F.softplus(d[3], threshold=20) + 1e-6
    l10 = d[4]
    l11 = F.softplus(d[5], threshold=20) + 1e-6
    L = torch.zeros(d.shape[1], 2, 2, dtype=torch.float64)
    L[:, 0, 0], L[:, 1, 0], L[:, 1, 1] = l00, l10, l11
    P = L @ L.transpose(1, 2)
    conf = conf + torch.stack([d[2], P[:, 0, 0], P[:, 1, 0], P[:, 1, 1]])
    return flow, conf


def dwconv5_relu(x, w, b):
    C = x.shape[0]
    return F.relu(F.conv2d(x[None], w.reshape(C, 1, 5, 5), b, padding=2, groups=C)[0])

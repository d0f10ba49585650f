# SPDX-License-Identifier: Unlicense
"""Float64 torch statement of DISK's U-Net and keypoint selection (kornia
DISK: Unet(3, size=5, down=[16, 32, 64, 64, 64], up=[64, 64, 64, 129]),
nms2d with strict maxima, heatmap_to_keypoints), from library routines
(F.conv2d, F.instance_norm, F.prelu, F.avg_pool2d, F.interpolate, F.unfold,
torch.topk, F.normalize), to pin the oracle's restatement of disk.c and
disk_kernels.cl (i.coregistration.opencl)."""

import numpy as np
import torch
import torch.nn.functional as F

CIN = (3, 16, 32, 64, 64, 128, 128, 96, 80)


def _t(w, k):
    return torch.from_numpy(np.asarray(w[k], np.float64))


def _block(w, l, x):
    pre = f"unet.path_down.{l}.1" if l < 5 else f"unet.path_up.{l - 5}.conv"
    if l > 0:
        x = F.prelu(F.instance_norm(x, eps=1e-5), _t(w, f"{pre}.1.weight"))
    return F.conv2d(x, _t(w, f"{pre}.3.weight"), _t(w, f"{pre}.3.bias"), padding=2)


@torch.no_grad()
def unet(w, img):
    """(129, H, W) output of a (3, H, W) image."""
    x = torch.from_numpy(np.asarray(img, np.float64))[None]
    skips = [_block(w, 0, x)]
    for l in range(1, 5):
        skips.append(_block(w, l, F.avg_pool2d(skips[-1], 2)))
    y = skips[-1]
    for j in range(4):
        up = F.interpolate(y, scale_factor=2, mode="bilinear", align_corners=False)
        y = _block(w, 5 + j, torch.cat([up, skips[3 - j]], 1))
    return y[0].numpy()


def nms_mask(heat, thresh):
    """Cells strictly above their 24 neighbours (5 x 5) and thresh, the
    2-cell border excluded: the centre compared with the maximum of the
    unfolded window without it."""
    h, w = heat.shape
    x = torch.from_numpy(np.asarray(heat, np.float64))[None, None]
    pat = F.unfold(x, 5, padding=2)[0]                    # (25, h w)
    pat = torch.cat([pat[:12], pat[13:]])                 # drop the centre
    mx = pat.max(0).values.reshape(h, w)
    m = (x[0, 0] > mx) & (x[0, 0] > thresh)
    m[:2] = False
    m[-2:] = False
    m[:, :2] = False
    m[:, -2:] = False
    return m.numpy()


def select(heat, mask, n, valid=None):
    """heatmap_to_keypoints: the n highest candidates by torch.topk, in
    raster order (with n or fewer candidates the reference drops the
    lowest, disk.c:228-253)."""
    m = mask if valid is None else mask & valid.astype(bool)
    ys, xs = np.nonzero(m)
    v = heat[ys, xs]
    if len(v) == 0:
        return np.zeros((0, 2), np.int32)
    if len(v) > n:
        keep = torch.topk(torch.from_numpy(v.astype(np.float64)), n).indices.numpy()
    else:
        keep = np.argsort(-v, kind="stable")[:len(v) - 1]
    keep = np.sort(keep)
    return np.stack([xs[keep], ys[keep]], 1).astype(np.int32)


def gather(out, xy):
    f = torch.from_numpy(np.asarray(out[:128], np.float64))
    d = f[:, xy[:, 1], xy[:, 0]].T
    return F.normalize(d, dim=1, eps=1e-12).numpy()

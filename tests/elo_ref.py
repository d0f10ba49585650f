# SPDX-License-Identifier: Unlicense
"""Independent float64 formulations of ELoFTR's matching stages (torch),
used to pin the oracle: the dual softmax over the full score matrix as
the reference's comparison script writes it (tests/reference_compare_eloftr.py
:80-104 of i.coregistration.opencl), and the authors' two-stage fine
matching (same file :107-142), written here as whole-tensor operations
rather than the kernels' loops."""

import numpy as np


def coarse_bruteforce(F0, F1, alpha):
    """conf = softmax_row(S) softmax_col(S), S = alpha F0 F1^T; returns
    (conf, row max, first row argmax, first column argmax)."""
    import torch
    S = alpha * torch.from_numpy(F0.astype(np.float64)) @ torch.from_numpy(F1.astype(np.float64)).T
    conf = torch.softmax(S, 1) * torch.softmax(S, 0)
    rmax, rarg = conf.max(1)
    carg = conf.argmax(0)
    return conf.numpy(), rmax.numpy(), rarg.numpy(), carg.numpy()


def windows(f, H, W, cx, cy, size, off):
    """(M, size*size, 64) windows of f (64, H, W) at cell * 8 + off, zero
    outside the image."""
    M = len(cx)
    ar = np.arange(size)
    xs = cx[:, None] * 8 + off + ar[None, :]          # (M, size)
    ys = cy[:, None] * 8 + off + ar[None, :]
    X = np.broadcast_to(xs[:, None, :], (M, size, size))
    Y = np.broadcast_to(ys[:, :, None], (M, size, size))
    ok = (X >= 0) & (X < W) & (Y >= 0) & (Y < H)
    Xc, Yc = np.clip(X, 0, W - 1), np.clip(Y, 0, H - 1)
    v = f[:, Yc, Xc]                                   # (64, M, size, size)
    v = np.where(ok[None], v, 0.0)
    return np.transpose(v, (1, 2, 3, 0)).reshape(M, size * size, 64)


def fine_bruteforce(f0, f1, cells, T=10.0):
    """The authors' two-stage fine matching on (64, H, W) features;
    returns (M, 4) positions (x0, y0, x1, y1; pixel index - 3.5) and the
    first-stage relative top-2 margin."""
    import torch
    _, H, W = f0.shape
    cells = np.asarray(cells).reshape(-1, 4)
    w0 = torch.from_numpy(windows(f0.astype(np.float64), H, W, cells[:, 0], cells[:, 1], 8, 0))
    w1 = torch.from_numpy(windows(f1.astype(np.float64), H, W, cells[:, 2], cells[:, 3], 10, -1))
    M = w0.shape[0]
    conf = (w0[..., :56] / 8.0) @ (w1[..., :56] / 8.0).transpose(1, 2)      # (M, 64, 100)
    ff = w0[..., 56:] @ (w1[..., 56:] / np.sqrt(8.0)).transpose(1, 2)
    sm = torch.softmax(conf, 1) * torch.softmax(conf, 2)
    sm = sm.reshape(M, 64, 10, 10)[..., 1:-1, 1:-1].reshape(M, -1)
    top2 = sm.topk(2, -1).values
    margin = ((top2[:, 0] - top2[:, 1]) / top2[:, 0]).numpy()
    idx = sm.argmax(-1)
    il, ir = idx // 64, idx % 64
    ii, jj = ir // 8, ir % 8
    d = torch.arange(-1, 2)
    ar = torch.arange(M)[:, None, None]
    sel = ff.reshape(M, 64, 10, 10)[ar, il[:, None, None], ii[:, None, None] + d[None, :, None],
                                    jj[:, None, None] + d[None, None, :]].reshape(M, 9)
    heat = torch.softmax(sel / T, -1).reshape(M, 3, 3)
    ex = (heat.sum(1) * d).sum(-1)
    ey = (heat.sum(2) * d).sum(-1)
    c = torch.from_numpy(cells.astype(np.float64))
    x0 = c[:, 0] * 8 + (il % 8) - 3.5
    y0 = c[:, 1] * 8 + (il // 8) - 3.5
    x1 = c[:, 2] * 8 + jj - 3.5 + ex
    y1 = c[:, 3] * 8 + ii - 3.5 + ey
    return torch.stack([x0, y0, x1, y1], -1).numpy(), margin


def match_features(rng, n, D, noise=0.3, scale=3.0):
    """Token features with a planted permutation (peaky dual softmax)."""
    F0 = rng.standard_normal((n, D)).astype(np.float32) * scale
    perm = rng.permutation(n)
    F1 = (F0[perm] + noise * rng.standard_normal((n, D))).astype(np.float32)
    return F0, F1

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


# ---- the whole match, float64 ------------------------------------------------------

def _t(w, k):
    return torch.from_numpy(np.asarray(w[k], np.float64))


def _dinov2_layer(w, pre, D, heads, eps, qkv_bias, ls):
    """transformers' Dinov2Layer loaded from a timm/DINOv2-named block."""
    from transformers import Dinov2Config
    from transformers.models.dinov2.modeling_dinov2 import Dinov2Layer
    cfg = Dinov2Config(hidden_size=D, num_attention_heads=heads, mlp_ratio=4,
                       layer_norm_eps=eps, qkv_bias=True, layerscale_value=1.0,
                       hidden_act="gelu", attn_implementation="eager")
    layer = Dinov2Layer(cfg).double().eval()
    qkv = _t(w, f"{pre}.attn.qkv.weight")
    qb = _t(w, f"{pre}.attn.qkv.bias") if qkv_bias else torch.zeros(3 * D, dtype=torch.float64)
    sd = {"norm1.weight": _t(w, f"{pre}.norm1.weight"), "norm1.bias": _t(w, f"{pre}.norm1.bias"),
          "attention.attention.query.weight": qkv[:D], "attention.attention.query.bias": qb[:D],
          "attention.attention.key.weight": qkv[D:2 * D], "attention.attention.key.bias": qb[D:2 * D],
          "attention.attention.value.weight": qkv[2 * D:], "attention.attention.value.bias": qb[2 * D:],
          "attention.output.dense.weight": _t(w, f"{pre}.attn.proj.weight"),
          "attention.output.dense.bias": _t(w, f"{pre}.attn.proj.bias"),
          "norm2.weight": _t(w, f"{pre}.norm2.weight"), "norm2.bias": _t(w, f"{pre}.norm2.bias"),
          "mlp.fc1.weight": _t(w, f"{pre}.mlp.fc1.weight"), "mlp.fc1.bias": _t(w, f"{pre}.mlp.fc1.bias"),
          "mlp.fc2.weight": _t(w, f"{pre}.mlp.fc2.weight"), "mlp.fc2.bias": _t(w, f"{pre}.mlp.fc2.bias"),
          "layer_scale1.lambda1": _t(w, f"{pre}.ls1.gamma") if ls else torch.ones(D, dtype=torch.float64),
          "layer_scale2.lambda1": _t(w, f"{pre}.ls2.gamma") if ls else torch.ones(D, dtype=torch.float64)}
    layer.load_state_dict(sd)
    return layer


def _conv_bn(w, x, conv, bn, groups=1, padding=0, relu=False):
    bias = _t(w, f"{conv}.bias") if f"{conv}.bias" in w else None
    y = F.conv2d(x, _t(w, f"{conv}.weight"), bias, padding=padding, groups=groups)
    y = F.batch_norm(y, _t(w, f"{bn}.running_mean"), _t(w, f"{bn}.running_var"),
                     _t(w, f"{bn}.weight"), _t(w, f"{bn}.bias"), False, 0.0, 1e-5)
    return F.relu(y) if relu else y


def prepare(img, h, w, imagenet=True):
    """RoMa's transforms: antialiased bicubic resize (PIL's filter, which
    torch's antialias=True bicubic follows) and ImageNet normalisation."""
    x = t64(img)[None]
    if x.shape[-2:] != (h, w):
        x = F.interpolate(x, size=(h, w), mode="bicubic", antialias=True, align_corners=False)
    x = x[0]
    if imagenet:
        m = torch.tensor([0.485, 0.456, 0.406], dtype=torch.float64)[:, None, None]
        s = torch.tensor([0.229, 0.224, 0.225], dtype=torch.float64)[:, None, None]
        x = (x - m) / s
    return x


def _vgg(w, pre, x, nblk):
    """VGG19-BN features before each pooling (block outputs)."""
    feats, idx = [], 0
    for blk, nconv in enumerate((2, 2, 4, 4)[:nblk]):
        for _ in range(nconv):
            x = _conv_bn(w, x, f"{pre}.{idx}", f"{pre}.{idx + 1}", padding=1, relu=True)
            idx += 3
        feats.append(x)
        if blk < nblk - 1:
            x = F.max_pool2d(x, 2, 2)
        idx += 1
    return feats


def _dino(wd, img, c16):
    D = 1024
    x = F.conv2d(img[None], _t(wd, "patch_embed.proj.weight"), _t(wd, "patch_embed.proj.bias"),
                 stride=14)[0]
    tok = x.reshape(D, -1).T
    pos = _t(wd, "pos_embed")[0]
    pp = pos[1:].reshape(1, 37, 37, D).permute(0, 3, 1, 2)
    pp = F.interpolate(pp, scale_factor=((c16 + 0.1) / 37, (c16 + 0.1) / 37), mode="bicubic",
                       align_corners=False)
    pp = pp[0].reshape(D, -1).T
    x = torch.cat([_t(wd, "cls_token")[0], tok], 0) + torch.cat([pos[:1], pp], 0)
    x = x[None]
    for i in range(24):
        x = _dinov2_layer(wd, f"blocks.{i}", D, 16, 1e-6, True, True)(x)
        x = x[0] if isinstance(x, tuple) else x
    x = F.layer_norm(x, (D,), _t(wd, "norm.weight"), _t(wd, "norm.bias"), 1e-6)
    return x[0, 1:]                                   # (n16, 1024)


def _refine(w, pre, fa, fb, flow, radius, fx, fy, nout):
    """One ConvRefiner on (C, h, w) features of both images and a (2, h, w)
    warp: (nout, h, w) output."""
    C, h, wd = fa.shape
    x_hat = grid_sample_flow(fb, flow)
    gy, gx = torch.meshgrid(cell_centres(h), cell_centres(wd), indexing="ij")
    disp = torch.stack([gx, gy])
    fac = torch.tensor([fx, fy], dtype=torch.float64)[:, None, None]
    emb = F.conv2d((fac * (flow - disp))[None], _t(w, f"{pre}.disp_emb.weight"),
                   _t(w, f"{pre}.disp_emb.bias"))[0]
    parts = [fa, x_hat, emb]
    if radius:
        parts.append(local_correlation(fa, fb, flow, radius))
    d = torch.cat(parts, 0)[None]
    cin = d.shape[1]
    v2 = f"{pre}.block1.conv_depthwise.weight" in w
    dw, bn, pw = ("conv_depthwise", "norm", "conv_pointwise") if v2 else ("0", "1", "3")
    for b in range(9):
        blk = f"{pre}.block1" if b == 0 else f"{pre}.hidden_blocks.{b - 1}"
        d = _conv_bn(w, d, f"{blk}.{dw}", f"{blk}.{bn}", groups=cin, padding=2, relu=True)
        d = F.conv2d(d, _t(w, f"{blk}.{pw}.weight"), _t(w, f"{blk}.{pw}.bias"))
    if v2:
        ow = torch.cat([_t(w, f"{pre}.warp_head.weight"), _t(w, f"{pre}.confidence_head.weight")])
        ob = torch.cat([_t(w, f"{pre}.warp_head.bias"), _t(w, f"{pre}.confidence_head.bias")])
    else:
        ow, ob = _t(w, f"{pre}.out_conv.weight"), _t(w, f"{pre}.out_conv.bias")
    return F.conv2d(d, ow, ob)[0]


def _resize(x, h, w):
    return F.interpolate(x[None], size=(h, w), mode="bilinear", align_corners=False)[0]


@torch.no_grad()
def roma_match(wm, wd, w2, imgA, imgB, coarse, imagenet=True, cls_flow_in=None):
    """RoMa's match (v1, or with RoMa v2's refiners when w2 is given) in
    float64: warp (2, H, W), certainty (H, W), sd (v2) and the stage
    outputs the oracle reports."""
    _, H, W = imgA.shape
    c16 = coarse // 14
    n16 = c16 * c16
    out = {"scale_flow": {}}
    scales = (16, 8, 4, 2, 1)
    proj = {}

    def vgg_proj(imgs, h, w_):
        P = {s: [] for s in (8, 4, 2, 1)}
        P2 = {s: [] for s in (4, 2, 1)}
        for x in imgs:
            f = _vgg(wm, "encoder.cnn.layers", x[None], 4)
            for s, fs in zip((1, 2, 4, 8), f):
                P[s].append(_conv_bn(wm, fs, f"decoder.proj.{s}.0", f"decoder.proj.{s}.1")[0])
            if w2:
                f2 = _vgg(w2, "refiner_features.layers", x[None], 3)
                for s, fs in zip((1, 2, 4), f2):
                    y = fs[0].reshape(fs.shape[1], -1).T @ _t(w2, f"refiners.{s}.proj.weight").T \
                        + _t(w2, f"refiners.{s}.proj.bias")
                    P2[s].append(y.T.reshape(-1, fs.shape[2], fs.shape[3]))
        return P, P2

    imgs_c = [prepare(x, coarse, coarse, imagenet) for x in (imgA, imgB)]
    P, P2 = vgg_proj(imgs_c, coarse, coarse)
    toks = [_dino(wd, x, c16) for x in imgs_c]
    out["dino"] = [t.T.numpy() for t in toks]
    g = [F.linear(t, _t(wm, "decoder.proj.16.0.weight")[:, :, 0, 0], _t(wm, "decoder.proj.16.0.bias"))
         for t in toks]
    g = [F.batch_norm(y[:, :, None], _t(wm, "decoder.proj.16.1.running_mean"),
                      _t(wm, "decoder.proj.16.1.running_var"), _t(wm, "decoder.proj.16.1.weight"),
                      _t(wm, "decoder.proj.16.1.bias"), False, 0.0, 1e-5)[:, :, 0] for y in g]
    P[16] = [y.T.reshape(512, c16, c16) for y in g]

    def cosk(a, b):
        c = (a @ b.T) / (a.norm(dim=1)[:, None] * b.norm(dim=1)[None] + 1e-6)
        return torch.exp((c - 1) / 0.2)

    kyy, kxy = cosk(g[1], g[1]), cosk(g[0], g[1])
    gy, gx = torch.meshgrid(cell_centres(c16), cell_centres(c16), indexing="ij")
    grid = torch.stack([gx, gy]).reshape(2, -1).T                     # (n16, 2)
    pv = grid @ _t(wm, "decoder.gps.16.pos_conv.weight")[:, :, 0, 0].T \
        + _t(wm, "decoder.gps.16.pos_conv.bias")
    basis = torch.cos(8 * math.pi * pv)
    L = torch.linalg.cholesky(kyy + 0.1 * torch.eye(n16, dtype=torch.float64))
    mu = kxy @ torch.cholesky_solve(basis, L)
    out["gp"] = mu.numpy()
    x = torch.cat([mu, g[0]], 1)[None]
    for i in range(5):
        x = _dinov2_layer(wm, f"decoder.embedding_decoder.blocks.{i}", 1024, 8, 1e-5, False, False)(x)
        x = x[0] if isinstance(x, tuple) else x
    logits = F.linear(x[0], _t(wm, "decoder.embedding_decoder.to_out.weight"),
                      _t(wm, "decoder.embedding_decoder.to_out.bias"))
    out["logits"] = logits.numpy()
    flow = cls_to_flow_refine(logits[:, :4096].T).reshape(2, c16, c16)
    cert = logits[:, 4096].reshape(1, c16, c16)
    out["cls_flow"] = flow.reshape(2, -1).numpy()
    if cls_flow_in is not None:
        flow = t64(cls_flow_in).reshape(2, c16, c16)

    def run_v1(flow, cert, Hp, Wp, sf, slist, p):
        for i, s in enumerate(slist):
            feat = P[s]
            hs, ws = flow.shape[1:]
            rad = {16: 7, 8: 3, 4: 2, 2: 0, 1: 0}[s]
            d = _refine(wm, f"decoder.conv_refiner.{s}", feat[0], feat[1], flow, rad,
                        40 / 32 * sf, 40 / 32 * sf, 3)
            flow = flow + s * torch.stack([d[0] / (4 * Wp), d[1] / (4 * Hp)])
            cert = cert + d[2:3]
            if p == 0 and s == 16:
                out["cert16"] = cert.clone()
            out["scale_flow"][(p, s)] = flow.numpy().copy()
            if i < len(slist) - 1:
                n = slist[i + 1]
                hn, wn = (Hp // n, Wp // n)
                flow, cert = _resize(flow, hn, wn), _resize(cert, hn, wn)
        return flow, cert

    def run_v2(flow, conf, Hp, Wp, zero_prec):
        for j, s in enumerate((4, 2, 1)):
            if zero_prec and j == 0:
                conf = torch.cat([conf[:1], torch.zeros_like(conf[1:])])
            hs, ws = Hp // s, Wp // s
            flow, conf = _resize(flow, hs, ws), _resize(conf, hs, ws)
            rad = {4: 3, 2: 1, 1: 0}[s]
            d = _refine(w2, f"refiners.{s}", P2[s][0], P2[s][1], flow, rad, Wp / 512, Hp / 512, 6)
            flow = flow + torch.stack([d[0] / (4 * ws), d[1] / (4 * hs)])
            l00 = F.softplus(d[3], threshold=20) + 1e-6
            l10 = d[4]
            l11 = F.softplus(d[5], threshold=20) + 1e-6
            conf = conf + torch.stack([d[2], l00 * l00, l00 * l10, l10 * l10 + l11 * l11])
        return flow, conf

    if w2:
        flow, cert = run_v1(flow, cert, coarse, coarse, 1.0, (16, 8), 0)
        conf = torch.cat([cert, torch.zeros(3, *cert.shape[1:], dtype=torch.float64)])
        flow, conf = run_v2(flow, conf, coarse, coarse, False)
        imgs_f = [prepare(x, H, W, imagenet) for x in (imgA, imgB)]
        P, P2 = vgg_proj(imgs_f, H, W)
        flow, conf = run_v2(flow, conf, H, W, True)
        det = conf[1] * conf[3] - conf[2] * conf[2]
        out["sd"] = torch.where(det > 0, det.clamp(min=1e-300) ** -0.25,
                                torch.tensor(float("nan"), dtype=torch.float64)).numpy()
        c = torch.sigmoid(conf[0])
    else:
        flow, cert = run_v1(flow, cert, coarse, coarse, 1.0, scales, 0)
        imgs_f = [prepare(x, H, W, imagenet) for x in (imgA, imgB)]
        P, P2 = vgg_proj(imgs_f, H, W)
        sf = math.sqrt(H * W) / coarse
        flow, cert = _resize(flow, H // 8, W // 8), _resize(cert, H // 8, W // 8)
        flow, cert = run_v1(flow, cert, H, W, sf, (8, 4, 2, 1), 1)
        low = _resize(out["cert16"], H, W)
        c = torch.sigmoid(cert[0] - torch.where(low[0] < 0, 0.5 * low[0], torch.zeros_like(low[0])))
    off = (flow.abs() > 1).any(0)
    out["cert"] = torch.where(off, torch.zeros_like(c), c).numpy()
    out["flow"] = flow.clamp(-1, 1).numpy()
    return out

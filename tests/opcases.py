# SPDX-License-Identifier: Unlicense
"""The generic-op cases of the reference's kernel check, for three runners.

The reference checks its generic kernels with ``tests/ops_check.c``
(i.coregistration.opencl): 33 cases on inputs drawn from one xorshift64
stream (seed 88172645463325252, ``ops_check.c:33-42``) in a fixed order
(``ops_check.c:448-487``), recomputed in torch float64 by
``tests/ops_compare.py:73-235``. This module restates that case list and
draw order, and runs each case through:

* ``golden64`` — torch float64 closed forms (F.conv2d, F.layer_norm, ...),
  used by ``tests/golden/make_golden.py`` to write the committed fixture;
* ``oracle`` — the C restatement in ``oracle/`` (CPU);
* ``hip`` — the HIP library through its C-ABI (GPU).
"""

import ctypes as C
import math

import numpy as np

ACT_NONE, ACT_GELU, ACT_RELU, ACT_LEAKY, ACT_GELU_TANH = range(5)
SEED = 88172645463325252
MASK64 = (1 << 64) - 1
# ops_compare.py:26 — the reference's own bar for these cases.
TOL = 2e-5


class XorShift:
    """xorshift64 of ops_check.c:33-42, float32 arithmetic as in C."""

    def __init__(self, seed=SEED):
        self.s = seed

    def raw(self, n):
        out = np.empty(n, np.uint64)
        s = self.s
        for i in range(n):
            s ^= (s << 13) & MASK64
            s ^= s >> 7
            s ^= (s << 17) & MASK64
            out[i] = s
        self.s = s
        return out

    def uniform(self, n, lo, hi):
        lo, hi = np.float32(lo), np.float32(hi)
        u = ((self.raw(n) >> np.uint64(11)).astype(np.float64)
             * (1.0 / 9007199254740992.0)).astype(np.float32)
        return (lo + (hi - lo) * u).astype(np.float32)


def f32(x):
    return np.float32(x)


class Case:
    """One case: name, op, parameters, inputs drawn in the reference order."""

    def __init__(self, name, op, **p):
        self.name, self.op, self.p = name, op, p
        self.inp = {}

    def __getitem__(self, k):
        return self.p[k]

    def __repr__(self):
        return f"Case({self.name})"


def _gemm(rng, name, M, N, K, transb, nb, act, residual):
    c = Case(name, "gemm", M=M, N=N, K=K, transb=transb, nb=nb, act=act,
             residual=residual, alpha=0.5, slope=0.1)
    c.inp["a"] = rng.uniform(nb * M * K, -1, 1)
    c.inp["b"] = rng.uniform(nb * N * K, -1, 1)
    c.inp["bias"] = rng.uniform(N, -1, 1)
    if residual:
        c.inp["r"] = rng.uniform(nb * M * N, -1, 1)
    return c


def _conv1x1(rng, name, Cc, HW, K):
    c = Case(name, "conv1x1", C=Cc, HW=HW, K=K, act=ACT_RELU)
    c.inp["x"] = rng.uniform(Cc * HW, -1, 1)
    c.inp["w"] = rng.uniform(K * Cc, -1, 1)
    c.inp["bias"] = rng.uniform(K, -1, 1)
    return c


def _conv(rng, name, Cc, H, W, K, k, s, p, d, groups, act, norm):
    c = Case(name, "conv2d", C=Cc, H=H, W=W, K=K, k=k, s=s, p=p, d=d,
             groups=groups, act=act, slope=0.2, norm=norm)
    c.inp["x"] = rng.uniform(Cc * H * W, -1, 1)
    c.inp["w"] = rng.uniform(K * (Cc // groups) * k * k, -0.3, 0.3)
    c.inp["bias"] = rng.uniform(K, -1, 1)
    if norm:
        c.inp["mean"] = rng.uniform(Cc, -0.5, 0.5)
        c.inp["rstd"] = rng.uniform(Cc, 0.5, 2.0)
        c.inp["alpha"] = rng.uniform(Cc, 0.0, 0.5)
    return c


def _instnorm(rng, name, Cc, HW):
    c = Case(name, "instnorm", C=Cc, HW=HW, eps=1e-5, act=ACT_LEAKY, slope=0.01)
    c.inp["x"] = rng.uniform(Cc * HW, -2, 3)
    c.inp["g"] = rng.uniform(Cc, 0.5, 1.5)
    c.inp["bias"] = rng.uniform(Cc, -1, 1)
    return c


def _layernorm(rng, name, rows, Cc):
    c = Case(name, "layernorm", rows=rows, C=Cc, eps=1e-6, act=ACT_GELU)
    c.inp["x"] = rng.uniform(rows * Cc, -2, 3)
    c.inp["g"] = rng.uniform(Cc, 0.5, 1.5)
    c.inp["bias"] = rng.uniform(Cc, -1, 1)
    return c


def _softmax(rng, name, rows, L, scale):
    c = Case(name, "softmax", rows=rows, L=L, scale=float(f32(scale)))
    c.inp["x"] = rng.uniform(rows * L, -20, 20)
    return c


def _attention(rng, name, Nq, Nk, nh, d, masked):
    E = nh * d
    scale = float(f32(1.0) / np.sqrt(f32(d), dtype=np.float32))
    c = Case(name, "attention", Nq=Nq, Nk=Nk, nh=nh, d=d, scale=scale,
             masked=masked)
    c.inp["qkv"] = rng.uniform(Nk * 3 * E, -2, 2)
    if masked:
        c.inp["mask"] = (rng.uniform(Nk, 0, 1) > f32(0.3)).astype(np.float32)
    return c


def _rope(rng, name, rows, nh, d, npos, interleaved):
    ld = nh * d + 6
    c = Case(name, "rope", rows=rows, nh=nh, d=d, npos=npos, ld=ld, off=3,
             interleaved=interleaved)
    c.inp["x"] = rng.uniform(rows * ld + 3, -1, 1)
    c.inp["angles"] = rng.uniform(npos * d // 2, -3.2, 3.2)
    ang = c.inp["angles"].astype(np.float64)
    cs = np.empty(npos * d, np.float32)
    cs[0::2] = np.cos(ang).astype(np.float32)
    cs[1::2] = np.sin(ang).astype(np.float32)
    c.table = cs
    return c


def _resize(rng, name, Cc, h, w, H, W, align, scale):
    c = Case(name, "resize", C=Cc, h=h, w=w, H=H, W=W, coff=2, align=align,
             scale=float(scale))
    c.inp["x"] = rng.uniform(Cc * h * w, -1, 1)
    return c


def _grid_sample(rng, name, Cc, H, W, n, align):
    c = Case(name, "grid_sample", C=Cc, H=H, W=W, n=n, align=align)
    c.inp["x"] = rng.uniform(Cc * H * W, -1, 1)
    c.inp["grid"] = rng.uniform(2 * n, -1.2, 1.2)
    return c


def _unfold(rng, name, Cc, H, W, k, s, p):
    c = Case(name, "unfold", C=Cc, H=H, W=W, k=k, s=s, p=p)
    c.inp["x"] = rng.uniform(Cc * H * W, -1, 1)
    return c


def _pool(rng, name, Cc, H, W, k, s, p, mx):
    c = Case(name, "pool", C=Cc, H=H, W=W, k=k, s=s, p=p, max=mx)
    c.inp["x"] = rng.uniform(Cc * H * W, -1, 1)
    return c


def _transpose(rng, name, B, R, Cc):
    c = Case(name, "transpose", B=B, R=R, C=Cc)
    c.inp["x"] = rng.uniform(B * R * Cc, -1, 1)
    return c


def _elementwise(rng, name, Cc, HW):
    n = Cc * HW
    c = Case(name, "elementwise", C=Cc, HW=HW, slope=0.05, a=0.5, b=-2.0)
    c.inp["x"] = rng.uniform(n, -3, 3)
    c.inp["alpha"] = rng.uniform(Cc, 0, 0.5)
    c.inp["b"] = rng.uniform(HW, -1, 1)
    return c


def _fold_bn(rng, name, Cc, H, W, K):
    per = Cc * 9
    c = Case(name, "fold_bn", C=Cc, H=H, W=W, K=K, eps=1e-5)
    c.inp["w"] = rng.uniform(K * per, -0.3, 0.3)
    c.inp["bias"] = rng.uniform(K, -1, 1)
    c.inp["gamma"] = rng.uniform(K, 0.5, 1.5)
    c.inp["beta"] = rng.uniform(K, -1, 1)
    c.inp["mean"] = rng.uniform(K, -1, 1)
    c.inp["var"] = rng.uniform(K, 0.2, 2.0)
    c.inp["x"] = rng.uniform(Cc * H * W, -1, 1)
    return c


def all_cases():
    """The 33 cases of ops_check.c:448-487, inputs drawn in order."""
    r = XorShift()
    return [
        _gemm(r, "gemm_small_nt", 37, 29, 21, 0, 1, ACT_GELU, 0),
        _gemm(r, "gemm_small_t", 70, 65, 33, 1, 3, ACT_LEAKY, 1),
        _gemm(r, "gemm_big_t", 300, 200, 96, 1, 2, ACT_RELU, 1),
        _gemm(r, "gemm_big_nt", 256, 130, 64, 0, 1, ACT_NONE, 0),
        _conv1x1(r, "conv1x1", 48, 300, 40),
        _conv(r, "conv5x5_norm", 12, 37, 45, 10, 5, 1, 2, 1, 1, ACT_NONE, 1),
        _conv(r, "conv5x5_first", 3, 33, 20, 16, 5, 1, 2, 1, 1, ACT_NONE, 0),
        _conv(r, "conv3x3_s2_g2", 6, 37, 29, 8, 3, 2, 1, 1, 2, ACT_RELU, 0),
        _conv(r, "conv3x3_dil2", 5, 21, 26, 7, 3, 1, 2, 2, 1, ACT_LEAKY, 0),
        _conv(r, "conv_dw4_s4", 8, 32, 40, 8, 4, 4, 0, 1, 8, ACT_NONE, 0),
        _conv(r, "conv5x5_norm_relu", 6, 19, 23, 5, 5, 1, 2, 1, 1, ACT_RELU, 1),
        _conv(r, "conv3x3_im2col", 24, 37, 29, 20, 3, 1, 1, 1, 1, ACT_RELU, 0),
        _conv(r, "conv3x3_s2_im2col_blocks", 16, 33, 41, 12, 3, 2, 1, 1, 1,
              ACT_LEAKY, 0),
        _instnorm(r, "instnorm", 7, 1000),
        _layernorm(r, "layernorm_96", 50, 96),
        _layernorm(r, "layernorm_1030", 9, 1030),
        _softmax(r, "softmax", 7, 300, 0.1),
        _softmax(r, "softmax_short", 5, 20, 10.0),
        _attention(r, "attention_d40", 50, 77, 3, 40, 0),
        _attention(r, "attention_d128_mask", 33, 300, 2, 128, 1),
        _attention(r, "attention_d32", 260, 260, 8, 32, 0),
        _rope(r, "rope_interleaved", 20, 2, 16, 10, 1),
        _rope(r, "rope_half", 20, 2, 16, 10, 0),
        _resize(r, "resize_x2", 3, 16, 24, 32, 48, 0, 2.0),
        _resize(r, "resize_size", 2, 13, 17, 29, 31, 0, 0),
        _resize(r, "resize_align", 2, 13, 17, 29, 31, 1, 0),
        _grid_sample(r, "grid_sample", 3, 20, 25, 500, 0),
        _grid_sample(r, "grid_sample_align", 3, 20, 25, 500, 1),
        _unfold(r, "unfold", 4, 12, 10, 3, 2, 1),
        _unfold(r, "unfold_8", 2, 16, 16, 8, 8, 0),
        _pool(r, "avgpool2", 3, 16, 22, 2, 2, 0, 0),
        _pool(r, "maxpool4", 3, 16, 24, 4, 4, 0, 1),
        _pool(r, "avgpool3_pad", 2, 15, 17, 3, 2, 1, 0),
        _transpose(r, "transpose", 2, 37, 50),
        _elementwise(r, "elementwise", 5, 77),
        _fold_bn(r, "fold_bn", 4, 11, 13, 6),
    ]


def conv_out(n, k, s, p, d=1):
    return (n + 2 * p - d * (k - 1) - 1) // s + 1


def fold_bn_host(c):
    """ops_fold_bn (ops.c:612-626) on the host, as the reference's check
    does before uploading (ops_check.c:415): double-precision scale."""
    K, per = c["K"], c["C"] * 9
    w = c.inp["w"].astype(np.float32).copy().reshape(K, per)
    b = c.inp["bias"].astype(np.float32).copy()
    s = (c.inp["gamma"].astype(np.float64)
         / np.sqrt(c.inp["var"].astype(np.float64) + np.float64(np.float32(c["eps"]))))
    w = (w.astype(np.float64) * s[:, None]).astype(np.float32)
    b = ((b - c.inp["mean"]).astype(np.float64) * s
         + c.inp["beta"].astype(np.float64)).astype(np.float32)
    return w.reshape(-1), b


# ---- golden: torch float64 (ops_compare.py:73-235 restated) -----------------

def golden64(c):
    import torch
    import torch.nn.functional as F

    def t(name, *shape):
        v = torch.from_numpy(c.inp[name].astype(np.float64))
        return v.reshape(*shape) if shape else v

    def act(x, a, slope):
        if a == ACT_GELU:
            return F.gelu(x)
        if a == ACT_RELU:
            return F.relu(x)
        if a == ACT_LEAKY:
            return F.leaky_relu(x, slope)
        if a == ACT_GELU_TANH:
            return F.gelu(x, approximate="tanh")
        return x

    op = c.op
    if op == "gemm":
        M, N, K, nb = c["M"], c["N"], c["K"], c["nb"]
        a = t("a", nb, M, K)
        b = t("b", nb, N, K) if c["transb"] else t("b", nb, K, N).transpose(1, 2)
        v = c["alpha"] * a @ b.transpose(1, 2) + t("bias")
        v = act(v, c["act"], c["slope"])
        if c["residual"]:
            v = v + t("r", nb, M, N)
        return {"out": v}
    if op == "conv1x1":
        Cc, HW, K = c["C"], c["HW"], c["K"]
        v = t("w", K, Cc) @ t("x", Cc, HW) + t("bias")[:, None]
        return {"out": act(v, c["act"], 0)}
    if op == "conv2d":
        Cc, H, W, K, k, g = c["C"], c["H"], c["W"], c["K"], c["k"], c["groups"]
        x = t("x", 1, Cc, H, W)
        if c["norm"]:
            x = (x - t("mean")[None, :, None, None]) * t("rstd")[None, :, None, None]
            x = F.prelu(x, t("alpha"))
        y = F.conv2d(x, t("w", K, Cc // g, k, k), t("bias"), stride=c["s"],
                     padding=c["p"], dilation=c["d"], groups=g)
        return {"out": act(y, c["act"], c["slope"])}
    if op == "instnorm":
        Cc, HW = c["C"], c["HW"]
        y = F.instance_norm(t("x", 1, Cc, HW), weight=t("g"), bias=t("bias"),
                            eps=c["eps"])
        return {"out": act(y, c["act"], c["slope"])}
    if op == "layernorm":
        rows, Cc = c["rows"], c["C"]
        y = F.layer_norm(t("x", rows, Cc), (Cc,), t("g"), t("bias"), c["eps"])
        return {"out": act(y, c["act"], 0)}
    if op == "softmax":
        return {"out": torch.softmax(c["scale"] * t("x", c["rows"], c["L"]), -1)}
    if op == "attention":
        Nq, Nk, nh, d = c["Nq"], c["Nk"], c["nh"], c["d"]
        qkv = t("qkv", Nk, 3, nh, d)
        q, k, v = (qkv[:, i].transpose(0, 1) for i in range(3))
        mask = None
        if c["masked"]:
            mask = t("mask").bool()[None, None, :]
        o = F.scaled_dot_product_attention(q[:, :Nq][None], k[None], v[None],
                                           attn_mask=mask, scale=c["scale"])
        return {"out": o[0].transpose(0, 1).reshape(Nq, nh * d)}
    if op == "rope":
        rows, nh, d, npos, ld, off = (c["rows"], c["nh"], c["d"], c["npos"],
                                      c["ld"], c["off"])
        flat = t("x")
        x = flat[off:off + rows * ld].reshape(rows, ld)[:, :nh * d].reshape(rows, nh, d)
        ang = t("angles", npos, d // 2)[torch.arange(rows) % npos][:, None, :]
        cos, sin = torch.cos(ang), torch.sin(ang)
        if c["interleaved"]:
            a, b = x[..., 0::2], x[..., 1::2]
            y = torch.stack((a * cos - b * sin, a * sin + b * cos), -1).reshape(rows, nh, d)
        else:
            a, b = x[..., :d // 2], x[..., d // 2:]
            y = torch.cat((a * cos - b * sin, a * sin + b * cos), -1)
        out = flat.clone()
        view = out[off:off + rows * ld].reshape(rows, ld)
        view[:, :nh * d] = y.reshape(rows, nh * d)
        return {"out": out}
    if op == "resize":
        Cc, h, w, H, W, coff = c["C"], c["h"], c["w"], c["H"], c["W"], c["coff"]
        x = t("x", 1, Cc, h, w)
        if c["scale"] > 0:
            y = F.interpolate(x, scale_factor=c["scale"], mode="bilinear",
                              align_corners=False)
        else:
            y = F.interpolate(x, size=(H, W), mode="bilinear",
                              align_corners=bool(c["align"]))
        out = torch.zeros(Cc + coff, H, W, dtype=torch.float64)
        out[coff:] = y[0]
        return {"out": out}
    if op == "grid_sample":
        Cc, H, W, n = c["C"], c["H"], c["W"], c["n"]
        y = F.grid_sample(t("x", 1, Cc, H, W), t("grid", 1, 1, n, 2),
                          mode="bilinear", padding_mode="zeros",
                          align_corners=bool(c["align"]))
        return {"out": y.reshape(Cc, n)}
    if op == "unfold":
        Cc, H, W, k, s, p = c["C"], c["H"], c["W"], c["k"], c["s"], c["p"]
        return {"out": F.unfold(t("x", 1, Cc, H, W), k, stride=s, padding=p)[0]}
    if op == "pool":
        Cc, H, W, k, s, p = c["C"], c["H"], c["W"], c["k"], c["s"], c["p"]
        x = t("x", 1, Cc, H, W)
        y = (F.max_pool2d(x, k, s, p) if c["max"]
             else F.avg_pool2d(x, k, s, p, count_include_pad=True))
        return {"out": y}
    if op == "transpose":
        return {"out": t("x", c["B"], c["R"], c["C"]).transpose(1, 2)}
    if op == "elementwise":
        Cc, HW = c["C"], c["HW"]
        x = t("x", Cc, HW)
        r = {"prelu": F.prelu(x[None], t("alpha"))[0]}
        for a in (ACT_GELU, ACT_RELU, ACT_LEAKY, ACT_GELU_TANH):
            r[f"act{a}"] = act(x, a, c["slope"])
        r["axpby"] = c["a"] * x + c["b"] * t("b")[None, :]
        return r
    if op == "fold_bn":
        Cc, H, W, K = c["C"], c["H"], c["W"], c["K"]
        y = F.conv2d(t("x", 1, Cc, H, W), t("w", K, Cc, 3, 3), t("bias"), padding=1)
        y = F.batch_norm(y, t("mean"), t("var"), t("gamma"), t("beta"),
                         training=False, eps=c["eps"])
        return {"out": y}
    raise ValueError(op)


# ---- oracle runner (liboracle.so, CPU) ----------------------------------------

def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float)) if a is not None else None


def oracle_run(orc, c):
    """Run case c through the C oracle; outputs as float32 arrays."""
    p, inp = c.p, c.inp
    op = c.op
    if op == "gemm":
        M, N, K, nb = p["M"], p["N"], p["K"], p["nb"]
        out = inp["r"].copy() if p["residual"] else np.zeros(nb * M * N, np.float32)
        orc.orc_gemm(M, N, K, _fp(inp["a"]), 0, K, M * K, 0, _fp(inp["b"]), 0,
                     K if p["transb"] else N, N * K, 0, p["transb"], _fp(out), 0,
                     N, M * N, 0, nb, 1, _fp(inp["bias"]), 0,
                     _fp(out) if p["residual"] else None, 0, C.c_float(0.5),
                     p["act"], C.c_float(0.1))
        return {"out": out}
    if op == "conv1x1":
        Cc, HW, K = p["C"], p["HW"], p["K"]
        out = np.zeros(K * HW, np.float32)
        orc.orc_gemm(K, HW, Cc, _fp(inp["w"]), 0, Cc, 0, 0, _fp(inp["x"]), 0, HW,
                     0, 0, 0, _fp(out), 0, HW, 0, 0, 1, 1, _fp(inp["bias"]), 1,
                     None, 0, C.c_float(1.0), p["act"], C.c_float(0.0))
        return {"out": out}
    if op == "conv2d":
        Cc, H, W, K, k = p["C"], p["H"], p["W"], p["K"], p["k"]
        Ho, Wo = conv_out(H, k, p["s"], p["p"], p["d"]), conv_out(W, k, p["s"], p["p"], p["d"])
        out = np.zeros(K * Ho * Wo, np.float32)
        norm = p["norm"]
        orc.orc_conv2d(_fp(inp["x"]), Cc, H, W, _fp(inp["w"]), _fp(inp["bias"]), K,
                       k, k, p["s"], p["s"], p["p"], p["p"], p["d"], p["d"],
                       p["groups"], _fp(inp["mean"]) if norm else None,
                       _fp(inp["rstd"]) if norm else None,
                       _fp(inp["alpha"]) if norm else None, p["act"],
                       C.c_float(p["slope"]), _fp(out))
        return {"out": out}
    if op == "instnorm":
        Cc, HW = p["C"], p["HW"]
        mean, rstd = np.zeros(Cc, np.float32), np.zeros(Cc, np.float32)
        out = np.zeros(Cc * HW, np.float32)
        orc.orc_chan_stats(_fp(inp["x"]), Cc, HW, C.c_float(p["eps"]), _fp(mean), _fp(rstd))
        orc.orc_chan_affine(_fp(inp["x"]), _fp(out), Cc, HW, _fp(mean), _fp(rstd),
                            _fp(inp["g"]), _fp(inp["bias"]), p["act"], C.c_float(p["slope"]))
        return {"out": out}
    if op == "layernorm":
        out = np.zeros(p["rows"] * p["C"], np.float32)
        orc.orc_layernorm(p["rows"], p["C"], _fp(inp["x"]), _fp(out), _fp(inp["g"]),
                          _fp(inp["bias"]), C.c_float(p["eps"]), p["act"], C.c_float(0))
        return {"out": out}
    if op == "softmax":
        out = inp["x"].copy()
        orc.orc_softmax_rows(_fp(out), p["rows"], p["L"], C.c_float(p["scale"]))
        return {"out": out}
    if op == "attention":
        Nq, Nk, nh, d = p["Nq"], p["Nk"], p["nh"], p["d"]
        E = nh * d
        out = np.zeros(Nq * E, np.float32)
        mask = None
        if p["masked"]:
            mask = inp["mask"].astype(np.uint8)
        qkv = inp["qkv"]
        orc.orc_attention(_fp(qkv), 0, 3 * E, _fp(qkv), E, 3 * E, _fp(qkv), 2 * E,
                          3 * E, _fp(out), 0, E, Nq, Nk, nh, d, C.c_float(p["scale"]),
                          mask.ctypes.data_as(C.c_void_p) if mask is not None else None)
        return {"out": out}
    if op == "rope":
        out = inp["x"].copy()
        orc.orc_rope(_fp(out), p["off"], p["ld"], p["rows"], p["nh"], p["d"], p["npos"],
                     _fp(c.table), p["interleaved"])
        return {"out": out}
    if op == "resize":
        Cc, H, W = p["C"], p["H"], p["W"]
        out = np.zeros((Cc + 2) * H * W, np.float32)
        orc.orc_resize(_fp(inp["x"]), Cc, p["h"], p["w"], _fp(out), H, W, 2,
                       p["align"], C.c_float(p["scale"]))
        return {"out": out}
    if op == "grid_sample":
        out = np.zeros(p["C"] * p["n"], np.float32)
        orc.orc_grid_sample(_fp(inp["x"]), p["C"], p["H"], p["W"], _fp(inp["grid"]),
                            p["n"], p["align"], _fp(out))
        return {"out": out}
    if op == "unfold":
        Cc, H, W, k, s, pp = p["C"], p["H"], p["W"], p["k"], p["s"], p["p"]
        n = Cc * k * k * conv_out(H, k, s, pp) * conv_out(W, k, s, pp)
        out = np.zeros(n, np.float32)
        orc.orc_unfold(_fp(inp["x"]), Cc, H, W, k, k, s, s, pp, pp, _fp(out))
        return {"out": out}
    if op == "pool":
        Cc, H, W, k, s, pp = p["C"], p["H"], p["W"], p["k"], p["s"], p["p"]
        out = np.zeros(Cc * conv_out(H, k, s, pp) * conv_out(W, k, s, pp), np.float32)
        if k == 2 and s == 2 and pp == 0 and not p["max"]:
            orc.orc_avgpool2(_fp(inp["x"]), Cc, H, W, _fp(out))
        else:
            orc.orc_pool2d(_fp(inp["x"]), Cc, H, W, k, s, pp, p["max"], _fp(out))
        return {"out": out}
    if op == "transpose":
        out = np.zeros_like(inp["x"])
        orc.orc_transpose(_fp(inp["x"]), _fp(out), p["B"], p["R"], p["C"])
        return {"out": out}
    if op == "elementwise":
        Cc, HW = p["C"], p["HW"]
        n = Cc * HW
        r = {}
        out = np.zeros(n, np.float32)
        orc.orc_prelu(_fp(inp["x"]), _fp(out), Cc, HW, _fp(inp["alpha"]))
        r["prelu"] = out.copy()
        for a in (ACT_GELU, ACT_RELU, ACT_LEAKY, ACT_GELU_TANH):
            orc.orc_act_map(_fp(inp["x"]), _fp(out), n, a, C.c_float(p["slope"]))
            r[f"act{a}"] = out.copy()
        orc.orc_axpby(_fp(out), _fp(inp["x"]), C.c_float(0.5), _fp(inp["b"]),
                      C.c_float(-2.0), n, HW)
        r["axpby"] = out.copy()
        return r
    if op == "fold_bn":
        Cc, H, W, K = p["C"], p["H"], p["W"], p["K"]
        w = inp["w"].copy()
        b = inp["bias"].copy()
        orc.orc_fold_bn(_fp(w), _fp(b), K, Cc * 9, _fp(inp["gamma"]), _fp(inp["beta"]),
                        _fp(inp["mean"]), _fp(inp["var"]), C.c_float(p["eps"]))
        out = np.zeros(K * H * W, np.float32)
        orc.orc_conv2d(_fp(inp["x"]), Cc, H, W, _fp(w), _fp(b), K, 3, 3, 1, 1, 1, 1,
                       1, 1, 1, None, None, None, ACT_NONE, C.c_float(0), _fp(out))
        return {"out": out}
    raise ValueError(op)


# ---- HIP runner (libicoreg.so through its C-ABI, GPU) ---------------------------

def hip_run(dev, c, ic):
    """Run case c on the device dev (ic: the binding module)."""
    p, inp, a = c.p, c.inp, dev.api
    pb, po = dev.pb, dev.po
    up = {k: dev.upload(v) for k, v in inp.items() if k not in ("mask",)}
    M = ic.mem
    op = c.op
    if op == "gemm":
        Mm, N, K, nb = p["M"], p["N"], p["K"], p["nb"]
        out = dev.upload(inp["r"]) if p["residual"] else dev.zeros(nb * Mm * N)
        a.ops_gemm(po, Mm, N, K, ic.bmat(up["a"], 0, K, Mm * K, 0),
                   ic.bmat(up["b"], 0, K if p["transb"] else N, N * K, 0), p["transb"],
                   ic.bmat(out, 0, N, Mm * N, 0), nb, 1, M(up["bias"]), 0,
                   M(out) if p["residual"] else None, 0, 0.5, p["act"], 0.1)
        return {"out": dev.read(out, nb * Mm * N)}
    if op == "conv1x1":
        Cc, HW, K = p["C"], p["HW"], p["K"]
        out = dev.zeros(K * HW)
        a.ops_conv1x1(po, M(up["x"]), 0, Cc, HW, M(up["w"]), M(up["bias"]), K, M(out),
                      0, p["act"], 0.0)
        return {"out": dev.read(out, K * HW)}
    if op == "conv2d":
        Cc, H, W, K, k = p["C"], p["H"], p["W"], p["K"], p["k"]
        Ho, Wo = conv_out(H, k, p["s"], p["p"], p["d"]), conv_out(W, k, p["s"], p["p"], p["d"])
        out = dev.zeros(K * Ho * Wo)
        g = ic.geom(k, k, p["s"], p["s"], p["p"], p["p"], p["d"], p["d"], p["groups"])
        norm = p["norm"]
        a.ops_conv2d(po, M(up["x"]), Cc, H, W, M(up["w"]), M(up["bias"]), K, C.byref(g),
                     M(up["mean"]) if norm else None, M(up["rstd"]) if norm else None,
                     M(up["alpha"]) if norm else None, p["act"], p["slope"], M(out))
        return {"out": dev.read(out, K * Ho * Wo)}
    if op == "instnorm":
        Cc, HW = p["C"], p["HW"]
        mean, rstd, out = dev.zeros(Cc), dev.zeros(Cc), dev.zeros(Cc * HW)
        a.ops_chan_stats(po, M(up["x"]), Cc, HW, p["eps"], M(mean), M(rstd))
        a.ops_chan_affine(po, M(up["x"]), M(out), Cc, HW, M(mean), M(rstd), M(up["g"]),
                          M(up["bias"]), p["act"], p["slope"])
        return {"out": dev.read(out, Cc * HW)}
    if op == "layernorm":
        n = p["rows"] * p["C"]
        out = dev.zeros(n)
        a.ops_layernorm(po, p["rows"], p["C"], M(up["x"]), M(out), M(up["g"]),
                        M(up["bias"]), p["eps"], p["act"], 0.0)
        return {"out": dev.read(out, n)}
    if op == "softmax":
        a.ops_softmax_rows(po, M(up["x"]), p["rows"], p["L"], p["scale"])
        return {"out": dev.read(up["x"], p["rows"] * p["L"])}
    if op == "attention":
        Nq, Nk, nh, d = p["Nq"], p["Nk"], p["nh"], p["d"]
        E = nh * d
        out = dev.zeros(Nq * E)
        mask = dev.upload(inp["mask"].astype(np.uint8)) if p["masked"] else None
        a.ops_attention(po, ic.mat(up["qkv"], 0, 3 * E), ic.mat(up["qkv"], E, 3 * E),
                        ic.mat(up["qkv"], 2 * E, 3 * E), ic.mat(out, 0, E), Nq, Nk, nh, d,
                        p["scale"], M(mask))
        return {"out": dev.read(out, Nq * E)}
    if op == "rope":
        tab = dev.upload(c.table)
        a.ops_rope(po, M(up["x"]), p["off"], p["ld"], p["rows"], p["nh"], p["d"],
                   p["npos"], M(tab), p["interleaved"])
        return {"out": dev.read(up["x"], inp["x"].size)}
    if op == "resize":
        Cc, H, W = p["C"], p["H"], p["W"]
        out = dev.zeros((Cc + 2) * H * W)
        a.ops_resize(po, M(up["x"]), Cc, p["h"], p["w"], M(out), H, W, 2, p["align"],
                     p["scale"])
        return {"out": dev.read(out, (Cc + 2) * H * W)}
    if op == "grid_sample":
        out = dev.zeros(p["C"] * p["n"])
        a.ops_grid_sample(po, M(up["x"]), p["C"], p["H"], p["W"], M(up["grid"]), p["n"],
                          p["align"], M(out))
        return {"out": dev.read(out, p["C"] * p["n"])}
    if op == "unfold":
        Cc, H, W, k, s, pp = p["C"], p["H"], p["W"], p["k"], p["s"], p["p"]
        n = Cc * k * k * conv_out(H, k, s, pp) * conv_out(W, k, s, pp)
        out = dev.zeros(n)
        g = ic.geom(k, k, s, s, pp, pp, 1, 1, 1)
        a.ops_unfold(po, M(up["x"]), Cc, H, W, C.byref(g), M(out))
        return {"out": dev.read(out, n)}
    if op == "pool":
        Cc, H, W, k, s, pp = p["C"], p["H"], p["W"], p["k"], p["s"], p["p"]
        n = Cc * conv_out(H, k, s, pp) * conv_out(W, k, s, pp)
        out = dev.zeros(n)
        if k == 2 and s == 2 and pp == 0 and not p["max"]:
            a.ops_avgpool2(po, M(up["x"]), Cc, H, W, M(out))
        else:
            a.ops_pool2d(po, M(up["x"]), Cc, H, W, k, s, pp, p["max"], M(out))
        return {"out": dev.read(out, n)}
    if op == "transpose":
        n = inp["x"].size
        out = dev.zeros(n)
        a.ops_transpose(po, M(up["x"]), M(out), p["B"], p["R"], p["C"])
        return {"out": dev.read(out, n)}
    if op == "elementwise":
        Cc, HW = p["C"], p["HW"]
        n = Cc * HW
        out = dev.zeros(n)
        r = {}
        a.ops_prelu(po, M(up["x"]), M(out), Cc, HW, M(up["alpha"]))
        r["prelu"] = dev.read(out, n)
        for act in (ACT_GELU, ACT_RELU, ACT_LEAKY, ACT_GELU_TANH):
            a.ops_act(po, M(up["x"]), M(out), n, act, p["slope"])
            r[f"act{act}"] = dev.read(out, n)
        a.ops_axpby(po, M(out), M(up["x"]), 0.5, M(up["b"]), -2.0, n, HW)
        r["axpby"] = dev.read(out, n)
        return r
    if op == "fold_bn":
        Cc, H, W, K = p["C"], p["H"], p["W"], p["K"]
        w = inp["w"].copy()
        b = inp["bias"].copy()
        ff = [inp[k].copy() for k in ("gamma", "beta", "mean", "var")]
        a.ops_fold_bn(w.ctypes.data, b.ctypes.data, K, Cc * 9, *[f.ctypes.data for f in ff],
                      float(np.float32(p["eps"])))
        wd, bd = dev.upload(w), dev.upload(b)
        out = dev.zeros(K * H * W)
        g = ic.geom(3, 3, 1, 1, 1, 1, 1, 1, 1)
        a.ops_conv2d(po, M(up["x"]), Cc, H, W, M(wd), M(bd), K, C.byref(g), None, None,
                     None, ACT_NONE, 0.0, M(out))
        return {"out": dev.read(out, K * H * W)}
    raise ValueError(op)


def rel_err(got, ref):
    """max |got - ref| / max |ref| (ops_compare.py:269-270)."""
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    scale = max(np.abs(ref).max(), 1e-30)
    return float(np.abs(got - ref).max() / scale)

# SPDX-License-Identifier: Unlicense
"""Loader of the oracle (oracle/liboracle.so, test infrastructure only)."""

import ctypes as C
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
ORACLE_SO = ROOT / "oracle" / "liboracle.so"

_F, _I, _L, _P = C.c_float, C.c_int, C.c_long, C.c_void_p
_FP = C.POINTER(C.c_float)
_IP = C.POINTER(C.c_int)

SIGS = {
    "orc_rng_seed": (None, [C.c_uint64]),
    "orc_rng_state": (C.c_uint64, []),
    "orc_urand": (_F, [_F, _F]),
    "orc_rand_fill": (None, [_FP, _L, _F, _F]),
    "orc_act": (_F, [_F, _I, _F]),
    "orc_gemm": (None, [_I, _I, _I, _FP, _L, _I, _L, _L, _FP, _L, _I, _L, _L, _I,
                        _FP, _L, _I, _L, _L, _I, _I, _FP, _I, _FP, _L, _F, _I, _F]),
    "orc_conv2d": (None, [_FP, _I, _I, _I, _FP, _FP, _I, _I, _I, _I, _I, _I, _I,
                          _I, _I, _I, _FP, _FP, _FP, _I, _F, _FP]),
    "orc_chan_stats": (None, [_FP, _I, _I, _F, _FP, _FP]),
    "orc_chan_affine": (None, [_FP, _FP, _I, _I, _FP, _FP, _FP, _FP, _I, _F]),
    "orc_prelu": (None, [_FP, _FP, _I, _I, _FP]),
    "orc_act_map": (None, [_FP, _FP, _L, _I, _F]),
    "orc_layernorm": (None, [_L, _I, _FP, _FP, _FP, _FP, _F, _I, _F]),
    "orc_softmax_rows": (None, [_FP, _L, _I, _F]),
    "orc_attention": (None, [_FP, _L, _I, _FP, _L, _I, _FP, _L, _I, _FP, _L, _I,
                             _I, _I, _I, _I, _F, _P]),
    "orc_rope": (None, [_FP, _L, _I, _L, _I, _I, _I, _FP, _I]),
    "orc_resize": (None, [_FP, _I, _I, _I, _FP, _I, _I, _I, _I, _F]),
    "orc_grid_sample": (None, [_FP, _I, _I, _I, _FP, _I, _I, _FP]),
    "orc_unfold": (None, [_FP, _I, _I, _I, _I, _I, _I, _I, _I, _I, _FP]),
    "orc_avgpool2": (None, [_FP, _I, _I, _I, _FP]),
    "orc_pool2d": (None, [_FP, _I, _I, _I, _I, _I, _I, _I, _FP]),
    "orc_transpose": (None, [_FP, _FP, _I, _I, _I]),
    "orc_axpby": (None, [_FP, _FP, _F, _FP, _F, _L, _L]),
    "orc_fold_bn": (None, [_FP, _FP, _I, _L, _FP, _FP, _FP, _FP, _F]),
    "orc_eloftr_coarse": (None, [_FP, _FP, _I, _I, _F, _I, _FP, _IP, _IP, _FP, _FP, _FP]),
    "orc_eloftr_select": (_I, [_FP, _IP, _IP, _I, _I, _F, _I, _IP, _IP, _FP]),
    "orc_eloftr_fine": (None, [_FP, _FP, _I, _I, _IP, _I, _F, _FP, _FP]),
    "orc_roma_row_norm": (None, [_FP, _I, _I, _FP]),
    "orc_roma_cos_exp": (None, [_FP, _FP, _FP, _I, _I, _F, _F]),
    "orc_roma_cls_to_flow": (None, [_FP, _I, _I, _I, _I, _FP, _FP]),
    "orc_roma_warp_sample": (None, [_FP, _I, _I, _I, _FP, _FP, _I]),
    "orc_roma_local_corr": (None, [_FP, _FP, _I, _I, _I, _I, _FP, _FP, _I]),
    "orc_roma_disp": (None, [_FP, _I, _I, _F, _F, _FP]),
    "orc_roma_update": (None, [_FP, _FP, _FP, _I, _F, _F, _F]),
    "orc_roma2_update": (None, [_FP, _FP, _FP, _I, _F, _F]),
    "orc_roma_dwconv5": (None, [_FP, _I, _I, _I, _FP, _FP, _FP]),
}

class Named(C.Structure):
    _fields_ = [("name", C.c_char_p), ("data", _FP), ("numel", C.c_long)]


class EloftrOut(C.Structure):
    _fields_ = [
        ("backbone", _FP * 2), ("coarse", _FP * 2),
        ("row_max", _FP), ("row_margin", _FP), ("col_margin", _FP),
        ("row_arg", _IP), ("col_arg", _IP),
        ("nm", C.c_int), ("mi", _IP), ("mj", _IP),
        ("mconf", _FP), ("kp", _FP), ("fine_margin", _FP),
        ("fine", _FP * 2), ("col_max", _FP),
    ]


SIGS["orc_eloftr_forward"] = (_I, [C.POINTER(Named), _I, _FP, _FP, _I, _I, _F,
                                   C.POINTER(EloftrOut)])

class RomaOut(C.Structure):
    _fields_ = [
        ("dino", _FP * 2), ("gp", _FP), ("logits", _FP),
        ("cls_flow", _FP), ("cls_cert", _FP),
        ("scale_flow", (_FP * 5) * 2),
        ("flow", _FP), ("cert", _FP), ("sd", _FP),
    ]


SIGS["orc_roma_forward"] = (_I, [C.POINTER(Named), _I, C.POINTER(Named), _I,
                                 C.POINTER(Named), _I, _FP, _FP, _I, _I, _I, _I, _FP,
                                 C.POINTER(RomaOut)])
SIGS["orc_roma_coarse"] = (_I, [C.POINTER(Named), _I, C.POINTER(Named), _I, _FP, _FP, _I, _FP,
                                _FP])
SIGS["orc_roma_refine"] = (_I, [C.POINTER(Named), _I, C.POINTER(Named), _I, _FP, _FP, _I, _I,
                                _I, _FP, _FP, C.POINTER(RomaOut)])
_UP = C.POINTER(C.c_ubyte)
SIGS["orc_disk_nms5x5"] = (None, [_FP, _I, _I, _I, _F, _UP])
SIGS["orc_disk_topn"] = (_I, [_FP, _I, _I, _I, _UP, _UP, _I, _IP, _FP])
SIGS["orc_disk_gather_desc"] = (None, [_FP, _I, _I, _I, _IP, _I, _FP])
SIGS["orc_disk_detect"] = (_I, [C.POINTER(Named), _I, _FP, _I, _I, _I, _I, _I, _F, _UP,
                                _IP, _FP, _FP, _FP])
SIGS["orc_roma_prepare"] = (None, [_FP, _I, _I, _FP, _I, _I, _I])
SIGS["orc_adalam_nearest"] = (None, [_FP, _I, _FP, _I, _I, _IP, _FP, _IP])
SIGS["orc_vit_block"] = (None, [_FP * 12, _FP, _I, _I, _F])
SIGS["orc_threads"] = (_I, [])
SIGS["orc_set_threads"] = (None, [_I])

_lib = None


def vit_block(w, X, heads=16, eps=1e-6):
    """orc_vit_block on a copy of X (N x 1024); w: the 12 float32 arrays in
    the order norm1 g, b; qkv W, b; proj W, b; norm2 g, b; fc1 W, b; fc2 W, b."""
    import numpy as np
    X = np.ascontiguousarray(X, np.float32).copy()
    ws = [np.ascontiguousarray(a, np.float32) for a in w]
    arr = (_FP * 12)(*[fp(a) for a in ws])
    oracle().orc_vit_block(arr, fp(X), X.shape[0], heads, eps)
    return X


def named_array(weights):
    """(ctypes array of Named, keep-alive list) for a dict of float32 arrays."""
    import numpy as np
    keep = []
    arr = (Named * len(weights))()
    for i, (k, v) in enumerate(sorted(weights.items())):
        a = np.ascontiguousarray(v, dtype=np.float32)
        kb = k.encode()
        keep += [a, kb]
        arr[i] = Named(kb, a.ctypes.data_as(_FP), a.size)
    return arr, keep


def eloftr_forward(weights, g0, g1, pos_scale=1.0, backbone=False, coarse=False,
                   fine=False):
    """Run the oracle's Efficient LoFTR on grey images; dict of outputs."""
    import numpy as np
    l = oracle()
    H, W = g0.shape
    n = (H // 8) * (W // 8)
    arr, keep = named_array(weights)
    out = {k: np.zeros(n, np.float32)
           for k in ("row_max", "row_margin", "col_margin", "col_max", "mconf")}
    for k in ("row_arg", "col_arg", "mi", "mj"):
        out[k] = np.zeros(n, np.int32)
    out["kp"] = np.zeros(4 * n, np.float32)
    out["fine_margin"] = np.zeros(n, np.float32)
    st = EloftrOut()
    for k in ("row_max", "row_margin", "col_margin", "col_max", "mconf", "kp", "fine_margin"):
        setattr(st, k, fp(out[k]))
    for k in ("row_arg", "col_arg", "mi", "mj"):
        setattr(st, k, ip(out[k]))
    for name, flag, size in (("backbone", backbone, 256 * n), ("coarse", coarse, 256 * n),
                             ("fine", fine, 64 * H * W)):
        if flag:
            bufs = [np.zeros(size, np.float32) for _ in range(2)]
            out[name] = bufs
            getattr(st, name)[0] = fp(bufs[0])
            getattr(st, name)[1] = fp(bufs[1])
    g0 = np.ascontiguousarray(g0, np.float32)
    g1 = np.ascontiguousarray(g1, np.float32)
    nm = l.orc_eloftr_forward(arr, len(weights), fp(g0), fp(g1), H, W, pos_scale,
                              C.byref(st))
    out["nm"] = nm
    return out


ROMA_SCALES = (16, 8, 4, 2, 1)


def roma_forward(wmain, wdino, wv2, imgA, imgB, coarse, imagenet=1, cls_flow_in=None):
    """Run the oracle's RoMa match on (3, H, W) images; dict of outputs:
    flow, cert, (sd), dino (2 x (1024, n16)), gp, logits, cls_flow,
    cls_cert, scale_flow[(p, s)] and the GP status info."""
    import numpy as np
    l = oracle()
    _, H, W = imgA.shape
    c16 = coarse // 14
    n16 = c16 * c16
    a1, k1 = named_array(wmain)
    a2, k2 = named_array(wdino)
    a3, k3 = named_array(wv2) if wv2 else (None, [])
    out = {"flow": np.zeros((2, H, W), np.float32), "cert": np.zeros((H, W), np.float32),
           "dino": [np.zeros((1024, n16), np.float32) for _ in range(2)],
           "gp": np.zeros((n16, 512), np.float32),
           "logits": np.zeros((n16, 4097), np.float32),
           "cls_flow": np.zeros((2, n16), np.float32), "cls_cert": np.zeros(n16, np.float32),
           "scale_flow": {}}
    st = RomaOut()
    for k in ("flow", "cert", "gp", "logits", "cls_flow", "cls_cert"):
        setattr(st, k, fp(out[k]))
    st.dino[0], st.dino[1] = fp(out["dino"][0]), fp(out["dino"][1])
    if wv2:
        out["sd"] = np.zeros((H, W), np.float32)
        st.sd = fp(out["sd"])
    nsc = 2 if wv2 else 5
    for p in range(2):
        for si, s in enumerate(ROMA_SCALES):
            if (p == 0 and si >= nsc) or (p == 1 and (wv2 or si == 0)):
                continue
            hs = (c16 if si == 0 else coarse // s) if p == 0 else H // s
            ws = (c16 if si == 0 else coarse // s) if p == 0 else W // s
            buf = np.zeros((2, hs, ws), np.float32)
            out["scale_flow"][(p, s)] = buf
            st.scale_flow[p][si] = fp(buf)
    A = np.ascontiguousarray(imgA, np.float32)
    B = np.ascontiguousarray(imgB, np.float32)
    cf = None if cls_flow_in is None else np.ascontiguousarray(cls_flow_in, np.float32)
    out["info"] = l.orc_roma_forward(a1, len(wmain), a2, len(wdino), a3,
                                     len(wv2) if wv2 else 0, fp(A), fp(B), H, W, coarse,
                                     imagenet, fp(cf), C.byref(st))
    return out


def roma_coarse(wmain, wdino, pairA, pairB):
    """Run the oracle's coarse forward alone (DINOv2 x 2, GP, decoder) on
    ImageNet-normalised (3, c, c) images; (cls_flow (2, n16), cls_cert
    (n16), GP status)."""
    import numpy as np
    l = oracle()
    c = pairA.shape[1]
    n16 = (c // 14) ** 2
    a1, k1 = named_array(wmain)
    a2, k2 = named_array(wdino)
    flow, cert = np.zeros((2, n16), np.float32), np.zeros(n16, np.float32)
    A = np.ascontiguousarray(pairA, np.float32)
    B = np.ascontiguousarray(pairB, np.float32)
    info = l.orc_roma_coarse(a1, len(wmain), a2, len(wdino), fp(A), fp(B), c, fp(flow),
                             fp(cert))
    return flow, cert, info


def roma_refine(wmain, wdino, pairA, pairB, flow8, cert8, coarse=560):
    """Run the oracle's fine pass alone (the refiner config's unit) on
    ImageNet-normalised (3, H, W) images from the 1/8 warp and certainty
    logit; dict: flow (2, H, W), cert (H, W) (the last refiner's, no
    epilogue) and scale_flow[s] for s = 8, 4, 2, 1."""
    import numpy as np
    l = oracle()
    _, H, W = pairA.shape
    a1, k1 = named_array(wmain)
    a2, k2 = named_array(wdino)
    out = {"flow": np.zeros((2, H, W), np.float32), "cert": np.zeros((H, W), np.float32),
           "scale_flow": {}}
    st = RomaOut()
    st.flow, st.cert = fp(out["flow"]), fp(out["cert"])
    for si, s in enumerate(ROMA_SCALES):
        if si == 0:
            continue
        buf = np.zeros((2, H // s, W // s), np.float32)
        out["scale_flow"][s] = buf
        st.scale_flow[1][si] = fp(buf)
    A = np.ascontiguousarray(pairA, np.float32)
    B = np.ascontiguousarray(pairB, np.float32)
    f8 = np.ascontiguousarray(flow8, np.float32)
    c8 = np.ascontiguousarray(cert8, np.float32)
    l.orc_roma_refine(a1, len(wmain), a2, len(wdino), fp(A), fp(B), H, W, coarse, fp(f8),
                      fp(c8), C.byref(st))
    return out


def disk_detect(weights, img, h=None, w=None, n=2048, thresh=0.0, valid=None,
                full=False):
    """Run the oracle's DISK detection on a (3, H, W) image."""
    import numpy as np
    l = oracle()
    _, H, W = img.shape
    h = H if h is None else h
    w = W if w is None else w
    arr, keep = named_array(weights)
    xy = np.zeros(2 * n, np.int32)
    score = np.zeros(n, np.float32)
    desc = np.zeros((n, 128), np.float32)
    out = np.zeros((129, H, W), np.float32) if full else None
    img = np.ascontiguousarray(img, np.float32)
    v = None if valid is None else np.ascontiguousarray(valid, np.uint8)
    nk = l.orc_disk_detect(arr, len(weights), fp(img), H, W, h, w, n, thresh,
                           v.ctypes.data_as(_UP) if v is not None else None, ip(xy),
                           fp(score), fp(desc), fp(out))
    r = {"n": nk, "xy": xy[:2 * nk].reshape(-1, 2), "score": score[:nk], "desc": desc[:nk]}
    if full:
        r["out"] = out
    return r


def oracle():
    global _lib
    if _lib is None:
        if not ORACLE_SO.exists():
            raise RuntimeError(f"{ORACLE_SO} not built (make -C oracle)")
        l = C.CDLL(str(ORACLE_SO))
        for name, (res, args) in SIGS.items():
            if not hasattr(l, name):
                continue
            f = getattr(l, name)
            f.restype, f.argtypes = res, args
        _lib = l
    return _lib


def fp(a):
    return a.ctypes.data_as(_FP) if a is not None else None


def ip(a):
    return a.ctypes.data_as(_IP) if a is not None else None

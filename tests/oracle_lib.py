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
    "orc_eloftr_coarse": (None, [_FP, _FP, _I, _I, _F, _I, _FP, _IP, _IP, _FP, _FP]),
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
        ("fine", _FP * 2),
    ]


SIGS["orc_eloftr_forward"] = (_I, [C.POINTER(Named), _I, _FP, _FP, _I, _I, _F,
                                   C.POINTER(EloftrOut)])

_lib = None


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
    out = {k: np.zeros(n, np.float32) for k in ("row_max", "row_margin", "col_margin", "mconf")}
    for k in ("row_arg", "col_arg", "mi", "mj"):
        out[k] = np.zeros(n, np.int32)
    out["kp"] = np.zeros(4 * n, np.float32)
    out["fine_margin"] = np.zeros(n, np.float32)
    st = EloftrOut()
    for k in ("row_max", "row_margin", "col_margin", "mconf", "kp", "fine_margin"):
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

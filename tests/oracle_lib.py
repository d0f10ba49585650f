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
}

_lib = None


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

# SPDX-License-Identifier: Unlicense
"""ctypes binding of libicoreg.so, the MI355X (gfx950) matcher tensor path.

The product is the C-ABI library built from ``csrc/`` (``make`` in this
folder); this module only loads it and exposes its entry points to Python
(tests, bench, smoke). There is no Python or CPU fallback: if the library
is missing, or no gfx950 device is present, every call raises.

The directory name is not a valid Python identifier, so load it with
``importlib`` (see ``load()`` in bench.py / tests/conftest.py).
"""

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBPATH = HERE / "libicoreg.so"

ACT_NONE, ACT_GELU, ACT_RELU, ACT_LEAKY, ACT_GELU_TANH = range(5)
FATAL_EXIT, FATAL_RECORD = 0, 1


class IcoregError(RuntimeError):
    """A fatal error of the library (the reference's G_fatal_error)."""


class OclBuf(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("bytes", C.c_size_t), ("owned", C.c_int)]


Mem = C.POINTER(OclBuf)


class OclBackend(C.Structure):
    _fields_ = [
        ("device", C.c_int),
        ("stream", C.c_void_p),
        ("device_name", C.c_char * 256),
        ("platform_name", C.c_char * 256),
        ("max_alloc", C.c_uint64),
        ("global_mem", C.c_uint64),
        ("is_gpu", C.c_int),
        ("profile", C.c_int),
        ("cu_count", C.c_int),
        ("arch", C.c_char * 64),
        ("aux_stream", C.c_void_p),
        ("aux_events", C.c_void_p),
        ("aux_nevents", C.c_int),
        ("copy_stream", C.c_void_p),
        ("copy_events", C.c_void_p),
        ("copy_tickets", C.c_longlong),
    ]


class Ops(C.Structure):
    _fields_ = [
        ("ocl", C.POINTER(OclBackend)),
        ("scratch", Mem),
        ("scratch_bytes", C.c_size_t),
        ("im2col_bytes", C.c_size_t),
    ]


class Opnd(C.Structure):
    _fields_ = [
        ("buf", Mem),
        ("off", C.c_int64),
        ("ld", C.c_int32),
        ("s0", C.c_int64),
        ("s1", C.c_int64),
    ]


class ConvGeom(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("kh", "kw", "sy", "sx", "py", "px", "dy", "dx", "groups")]


_I, _L, _F, _P, _S = C.c_int, C.c_long, C.c_float, C.c_void_p, C.c_char_p
_B = C.POINTER(OclBackend)
_O = C.POINTER(Ops)

# name -> (restype, argtypes)
SIGNATURES = {
    # backend (include/hip_backend.h)
    "ocl_init": (None, [_B, _S, _S]),
    "ocl_free": (None, [_B]),
    "ocl_errstr": (_S, [C.c_int32]),
    "ocl_check": (None, [C.c_int32, _S]),
    "ocl_alloc": (Mem, [_B, C.c_size_t, _S]),
    "ocl_upload": (Mem, [_B, _P, C.c_size_t, _S]),
    "ocl_write": (None, [_B, Mem, C.c_size_t, _P, C.c_size_t]),
    "ocl_read": (None, [_B, Mem, C.c_size_t, _P, C.c_size_t]),
    "ocl_host_alloc": (C.c_void_p, [_B, C.c_size_t]),
    "ocl_host_free": (None, [C.c_void_p]),
    "ocl_write_async": (C.c_longlong, [_B, Mem, C.c_size_t, _P, C.c_size_t]),
    "ocl_write_join": (None, [_B, C.c_longlong]),
    "ocl_write_wait": (None, [_B, C.c_longlong]),
    "ocl_release": (None, [C.POINTER(Mem)]),
    "ocl_copy": (None, [_B, Mem, C.c_size_t, Mem, C.c_size_t, C.c_size_t]),
    "ocl_copy_rect": (None, [_B, Mem, C.c_size_t, C.c_size_t, Mem, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t]),
    "ocl_fill": (None, [_B, Mem, C.c_size_t, C.c_size_t, _F]),
    "ocl_graph_begin": (None, [_B]),
    "ocl_graph_end": (_P, [_B]),
    "ocl_graph_launch": (None, [_B, _P]),
    "ocl_graph_free": (None, [_P]),
    "ocl_finish": (None, [_B]),
    "ocl_wrap": (Mem, [_P, C.c_size_t]),
    "ocl_event_record": (_I, [_B]),
    "ocl_event_ms": (_F, [_B, _I, _I]),
    "ocl_event_reset": (None, [_B]),
    "icoreg_set_fatal_mode": (None, [_I]),
    "icoreg_last_error": (_S, []),
    "icoreg_clear_error": (None, []),
    "icoreg_prof_entry": (_I, [_I, C.POINTER(_S), C.POINTER(C.c_double), C.POINTER(C.c_long)]),
    "icoreg_prof_reset": (None, []),
    "icoreg_prof_flush": (_I, []),
    # generic ops (include/ops.h)
    "ops_init": (None, [_O, _B]),
    "ops_free": (None, [_O]),
    "ops_report": (None, []),
    "ops_mat": (Opnd, [Mem, _L, _I]),
    "ops_bmat": (Opnd, [Mem, _L, _I, _L, _L]),
    "ops_gemm": (None, [_O, _I, _I, _I, Opnd, Opnd, _I, Opnd, _I, _I, Mem, _I, Mem, _L, _F, _I, _F]),
    "ops_linear": (None, [_O, _I, _I, _I, Mem, _L, Mem, Mem, Mem, _L, _I, _F, _I]),
    "ops_conv1x1": (None, [_O, Mem, _L, _I, _I, Mem, Mem, _I, Mem, _L, _I, _F]),
    "ops_geom": (ConvGeom, [_I, _I, _I]),
    "ops_conv_out": (_I, [_I, _I, _I, _I, _I]),
    "ops_conv2d": (None, [_O, Mem, _I, _I, _I, Mem, Mem, _I, C.POINTER(ConvGeom), Mem, Mem, Mem, _I, _F, Mem]),
    "ops_conv2d_batch": (None, [_O, _I, Mem, _L, _I, _I, _I, Mem, Mem, _I, C.POINTER(ConvGeom),
                                Mem, Mem, Mem, _I, _F, Mem, _L]),
    "ops_chan_stats": (None, [_O, Mem, _I, _I, _F, Mem, Mem]),
    "ops_chan_affine": (None, [_O, Mem, Mem, _I, _I, Mem, Mem, Mem, Mem, _I, _F]),
    "ops_prelu": (None, [_O, Mem, Mem, _I, _I, Mem]),
    "ops_act": (None, [_O, Mem, Mem, _L, _I, _F]),
    "ops_layernorm": (None, [_O, _L, _I, Mem, Mem, Mem, Mem, _F, _I, _F]),
    "ops_softmax_rows": (None, [_O, Mem, _L, _I, _F]),
    "ops_attention": (None, [_O, Opnd, Opnd, Opnd, Opnd, _I, _I, _I, _I, _F, Mem]),
    "ops_attention_noalloc": (None, [_O, Opnd, Opnd, Opnd, Opnd, _I, _I, _I, _I, _F, Mem]),
    "ops_attention_batch": (None, [_O, _I, Opnd, _L, Opnd, _L, Opnd, _L, Opnd, _L, _I,
                                   _I, _I, _I, _F, Mem]),
    "ops_rope": (None, [_O, Mem, _L, _I, _L, _I, _I, _I, Mem, _I]),
    "ops_resize": (None, [_O, Mem, _I, _I, _I, Mem, _I, _I, _I, _I, _F]),
    "ops_grid_sample": (None, [_O, Mem, _I, _I, _I, Mem, _I, _I, Mem]),
    "ops_unfold": (None, [_O, Mem, _I, _I, _I, C.POINTER(ConvGeom), Mem]),
    "ops_avgpool2": (None, [_O, Mem, _I, _I, _I, Mem]),
    "ops_pool2d": (None, [_O, Mem, _I, _I, _I, _I, _I, _I, _I, Mem]),
    "ops_transpose": (None, [_O, Mem, Mem, _I, _I, _I]),
    "ops_axpby": (None, [_O, Mem, Mem, _F, Mem, _F, _L, _L]),
    "ops_fold_bn": (None, [_P, _P, _I, _L, _P, _P, _P, _P, _F]),
    "ocl_fill_u32": (None, [_B, Mem, C.c_size_t, C.c_size_t, C.c_uint32]),
    # checkpoints (include/pth_loader.h)
    "pth_open": (None, [_P, _S]),
    "pth_close": (None, [_P]),
    "pth_find": (_P, [_P, _S]),
    "pth_require": (_P, [_P, _S, _I, C.POINTER(C.c_long)]),
    "pth_strip_prefix": (_I, [_P, _S]),
    "pth_numel": (C.c_long, [_P]),
    "pth_bytes": (C.c_double, [_P, _S]),
    "pth_read_f32": (C.POINTER(C.c_float), [_P, _P]),
    # ELoFTR (include/eloftr.h, include/icoreg_kernels.h)
    "eloftr_load": (None, [_P, _O, _P]),
    "eloftr_alloc": (None, [_P, _I, _I]),
    "eloftr_match": (None, [_P, _P, _P, _S, _I]),
    "eloftr_match_device": (None, [_P, Mem, Mem]),
    "eloftr_match_enqueue": (None, [_P, Mem, Mem]),
    "eloftr_match_collect": (None, [_P]),
    "eloftr_free": (None, [_P]),
    "eloftr_row_lse": (None, [_O, Mem, _I, _I, _I, Mem]),
    "eloftr_col_lse": (None, [_O, Mem, _I, _I, Mem, Mem]),
    "eloftr_conf_row": (None, [_O, Mem, _I, _I, _I, Mem, Mem, Mem, Mem, Mem]),
    "eloftr_conf_col": (None, [_O, Mem, _I, _I, _I, Mem, Mem, Mem, Mem, Mem]),
    "eloftr_lse_block": (None, [_O, Mem, _I, _I, _I, Mem, Mem, Mem]),
    "eloftr_conf_block": (None, [_O, Mem, _I, _I, _I, Mem, Mem, Mem, Mem, Mem, Mem, Mem]),
    "eloftr_fine": (None, [_O, Mem, Mem, _I, _I, Mem, _I, _F, Mem]),
    "eloftr_fine_half": (None, [_O, Mem, Mem, _I, _I, Mem, _I, _F, Mem]),
    "eloftr_fine_half_count": (None, [_O, Mem, Mem, _I, _I, Mem, Mem, _I, _F, Mem]),
    "eloftr_mutual": (None, [_O, Mem, Mem, Mem, _I, _I, _I, _F, Mem, Mem, Mem, Mem, Mem]),
    "roma_row_norm": (None, [_O, Mem, _I, _I, Mem]),
    "roma_cos_exp": (None, [_O, Mem, Mem, Mem, _I, _I, _F, _F]),
    "roma_cls_to_flow": (None, [_O, Mem, _I, _I, _I, _I, Mem, Mem]),
    "roma_warp_sample": (None, [_O, Mem, _I, _I, _I, Mem, Mem, _I]),
    "roma_local_corr": (None, [_O, Mem, Mem, _I, _I, _I, _I, Mem, Mem, _I]),
    "roma_disp": (None, [_O, Mem, _I, _I, _F, _F, Mem]),
    "roma_update": (None, [_O, Mem, Mem, Mem, _I, _F, _F, _F]),
    "roma2_update": (None, [_O, Mem, Mem, Mem, _I, _F, _F]),
    "roma_dwconv5": (None, [_O, Mem, _I, _I, _I, Mem, Mem, Mem]),
    "roma_dwpw_small": (None, [_O, Mem, _I, _I, _I, Mem, Mem, Mem, Mem, Mem]),
    "roma_gp_work_bytes": (C.c_size_t, [_I, _I]),
    "roma_gp_solve": (None, [_O, Mem, _I, _F, Mem, _I, Mem, Mem]),
    "roma_gp_solve_events": (None, [_O, Mem, _I, _F, Mem, _I, Mem, Mem]),
    "roma_prepare": (None, [_O, Mem, _I, _I, _I, Mem, _I, _I, _I]),
    "roma_epilogue": (None, [_O, Mem, Mem, Mem, _L]),
    "roma_sd": (None, [_O, Mem, _L, Mem, _L]),
    "disk_nms5x5": (None, [_O, Mem, _L, _I, _I, _I, _F, Mem]),
    "disk_gather_desc": (None, [_O, Mem, _I, _I, _I, Mem, _I, Mem]),
    "disk_topn_work_bytes": (C.c_size_t, [_I, _I]),
    "disk_topn": (None, [_O, Mem, _L, _I, _I, _I, Mem, Mem, _I, Mem, Mem, Mem, Mem]),
    "disk_gather_desc_count": (None, [_O, Mem, _I, _I, _I, Mem, Mem, _I, Mem]),
    # AdaLAM's nearest-neighbour search (include/adalam_nn.h)
    "adalam_nearest_work_bytes": (C.c_size_t, [_I, _I]),
    "adalam_nearest": (None, [_O, Mem, _I, Mem, _I, _I, Mem, Mem, Mem, Mem]),
    "adalam_nearest_host": (None, [_O, _P, _I, _P, _I, _I, _P, _P, _P]),
    # DISK model (include/disk.h)
    "disk_load": (None, [_P, _O, _P]),
    "disk_alloc": (None, [_P, _I, _I, _I]),
    "disk_detect": (_I, [_P, _P, _I, _I, _I, _I, _I, _F, _P, _P, _P, _P]),
    "disk_free": (None, [_P]),
    # RoMa model (include/roma.h)
    "roma_load": (None, [_P, _O, _P, _P]),
    "roma_load_v2": (None, [_P, _P]),
    "roma_set_coarse": (None, [_P, _I]),
    "roma_alloc": (None, [_P, _I, _I]),
    "roma_match": (None, [_P, _P, _P, _S, _I]),
    "roma_coarse_device": (None, [_P, Mem]),
    "roma_refine_device": (None, [_P, Mem, Mem, Mem]),
    "roma_free": (None, [_P]),
    # binding glue (include/icoreg_glue.h)
    "icoreg_sizeof_backend": (C.c_size_t, []),
    "icoreg_sizeof_ops": (C.c_size_t, []),
    "icoreg_pth_new": (_P, []),
    "icoreg_eloftr_new": (_P, []),
    "icoreg_struct_delete": (None, [_P]),
    "icoreg_eloftr_result": (_I, [_P, C.POINTER(C.POINTER(C.c_int)), C.POINTER(C.POINTER(C.c_int)),
                                  C.POINTER(C.POINTER(C.c_float)), C.POINTER(C.POINTER(C.c_float))]),
    "icoreg_eloftr_coarse_stats": (_I, [_P, C.POINTER(C.POINTER(C.c_float)),
                                        C.POINTER(C.POINTER(C.c_int)), C.POINTER(C.POINTER(C.c_int))]),
    "icoreg_eloftr_set_pos_scale": (None, [_P, _F]),
    "icoreg_eloftr_buffer": (Mem, [_P, _S]),
    "icoreg_roma_new": (_P, []),
    "icoreg_disk_new": (_P, []),
    "icoreg_disk_buffer": (Mem, [_P, _S]),
    "icoreg_roma_result": (_I, [_P, C.POINTER(C.POINTER(C.c_float)), C.POINTER(C.POINTER(C.c_float)),
                                C.POINTER(C.POINTER(C.c_float))]),
    "icoreg_roma_buffer": (Mem, [_P, _S]),
    "icoreg_roma_gp_info": (_I, [_P]),
    "icoreg_roma_last": (_I, [_P]),
    "icoreg_roma_set_imagenet": (None, [_P, _I]),
    "icoreg_gp_test_wait": (None, [_I, _I]),
    "icoreg_conv_wino_form": (None, [_I]),
    "icoreg_conv_wino_choice": (_I, [_P, _I, _I, _I, _I, _I]),
    "icoreg_roma_gp_retries": (_I, [_P]),
}

# Entry points that never raise through the fatal path (no error check).
_NO_CHECK = {"ocl_graph_free", "icoreg_set_fatal_mode", "icoreg_last_error", "icoreg_clear_error",
             "ocl_errstr", "ops_mat", "ops_bmat", "ops_geom", "ops_conv_out",
             "ocl_wrap", "icoreg_prof_entry", "icoreg_prof_reset", "icoreg_prof_flush", "ops_report",
             "pth_find", "pth_numel", "pth_bytes", "pth_strip_prefix",
             "icoreg_pth_new", "icoreg_eloftr_new", "icoreg_struct_delete",
             "icoreg_sizeof_backend", "icoreg_sizeof_ops",
             "icoreg_eloftr_result", "icoreg_eloftr_coarse_stats",
             "icoreg_eloftr_set_pos_scale", "icoreg_eloftr_buffer", "roma_gp_work_bytes",
             "icoreg_roma_new", "icoreg_roma_result", "icoreg_roma_buffer",
             "icoreg_roma_set_imagenet", "icoreg_disk_new", "icoreg_disk_buffer",
             "icoreg_roma_last", "disk_topn_work_bytes", "adalam_nearest_work_bytes",
             "icoreg_gp_test_wait", "icoreg_roma_gp_retries", "icoreg_conv_wino_form",
             "icoreg_conv_wino_choice"}

_lib = None


def library_path():
    return LIBPATH


def lib():
    """The loaded library with argument types set; raises if not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIBPATH.exists():
        raise IcoregError(f"{LIBPATH} is not built (run make in {HERE}); "
                          "this path has no fallback")
    l = C.CDLL(str(LIBPATH))
    for name, (res, args) in SIGNATURES.items():
        f = getattr(l, name)
        f.restype = res
        f.argtypes = args
    l.icoreg_set_fatal_mode(FATAL_RECORD)
    _lib = l
    return l


def exported_symbols():
    return sorted(SIGNATURES)


class _Checked:
    """Calls into the library; a recorded fatal error becomes IcoregError."""

    def __init__(self, l):
        self._l = l

    def __getattr__(self, name):
        f = getattr(self._l, name)
        if name in _NO_CHECK:
            return f

        def call(*args):
            self._l.icoreg_clear_error()
            r = f(*args)
            msg = self._l.icoreg_last_error()
            if msg:
                raise IcoregError(msg.decode())
            return r
        return call


def api():
    return _Checked(lib())


class Buffer:
    """A device buffer of the library (cl_mem), freed with the object."""

    def __init__(self, dev, mem, nbytes):
        self.dev, self.mem, self.nbytes = dev, mem, nbytes

    def release(self):
        if self.mem:
            lib().ocl_release(C.byref(self.mem))
            self.mem = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class Device:
    """One gfx950 device: the backend struct and the ops struct."""

    def __init__(self, device="auto"):
        self.api = api()
        self.ocl = OclBackend()
        self.api.ocl_init(C.byref(self.ocl), device.encode(), None)
        self.ops = Ops()
        self.api.ops_init(C.byref(self.ops), C.byref(self.ocl))
        self.pb = C.byref(self.ocl)
        self.po = C.byref(self.ops)

    @property
    def name(self):
        return self.ocl.device_name.decode()

    @property
    def arch(self):
        return self.ocl.arch.decode()

    def alloc(self, nbytes, what="buffer"):
        m = self.api.ocl_alloc(self.pb, int(nbytes), what.encode())
        return Buffer(self, m, int(nbytes))

    def zeros(self, n, dtype=np.float32):
        b = self.alloc(max(int(n), 1) * np.dtype(dtype).itemsize)
        self.api.ocl_fill(self.pb, b.mem, 0, b.nbytes // 4, 0.0)
        return b

    def upload(self, a, what="upload"):
        a = np.ascontiguousarray(a)
        b = self.alloc(max(a.nbytes, 4), what)
        if a.nbytes:
            self.api.ocl_write(self.pb, b.mem, 0, a.ctypes.data, a.nbytes)
        return b

    def write(self, buf, a, off_bytes=0):
        a = np.ascontiguousarray(a)
        self.api.ocl_write(self.pb, buf.mem, off_bytes, a.ctypes.data, a.nbytes)

    def read(self, buf, count=None, dtype=np.float32, off_bytes=0):
        dtype = np.dtype(dtype)
        if count is None:
            count = (buf.nbytes - off_bytes) // dtype.itemsize
        out = np.empty(int(count), dtype)
        if out.nbytes:
            self.api.ocl_read(self.pb, buf.mem, off_bytes, out.ctypes.data, out.nbytes)
        return out

    def finish(self):
        self.api.ocl_finish(self.pb)

    def event(self):
        return self.api.ocl_event_record(self.pb)

    def elapsed_ms(self, e0, e1):
        return self.api.ocl_event_ms(self.pb, e0, e1)

    def reset_events(self):
        self.api.ocl_event_reset(self.pb)

    def set_profile(self, mode):
        """0 off, 1 synchronous per launch, 2 asynchronous event pairs."""
        self.ocl.profile = mode

    def profile_table(self):
        """{name: (total ms, launches)} of the launch timing table."""
        l = lib()
        l.icoreg_prof_flush()
        out, i = {}, 0
        what, ms, calls = C.c_char_p(), C.c_double(), C.c_long()
        while l.icoreg_prof_entry(i, C.byref(what), C.byref(ms), C.byref(calls)):
            out[what.value.decode()] = (ms.value, calls.value)
            i += 1
        return out

    def profile_reset(self):
        lib().icoreg_prof_reset()

    def close(self):
        if self.ocl.stream:
            self.api.ops_free(self.po)
            self.api.ocl_free(self.pb)


def mat(buf, off, ld):
    return Opnd(buf.mem if buf is not None else None, off, ld, 0, 0)


def bmat(buf, off, ld, s0, s1):
    return Opnd(buf.mem if buf is not None else None, off, ld, s0, s1)


def mem(buf):
    """cl_mem of a Buffer, or NULL."""
    return buf.mem if buf is not None else None


def geom(kh, kw, sy, sx, py, px, dy, dx, groups):
    return ConvGeom(kh, kw, sy, sx, py, px, dy, dx, groups)


class Eloftr:
    """Efficient LoFTR on the device: eloftr_load / eloftr_alloc /
    eloftr_match of the C-ABI, weights from a safetensors file."""

    def __init__(self, dev, weights_path, H, W, pos_scale=1.0):
        self.dev = dev
        a = dev.api
        self.pf = lib().icoreg_pth_new()
        a.pth_open(self.pf, str(weights_path).encode())
        self.m = lib().icoreg_eloftr_new()
        a.eloftr_load(self.m, dev.po, self.pf)
        lib().icoreg_eloftr_set_pos_scale(self.m, pos_scale)
        a.eloftr_alloc(self.m, H, W)
        self.H, self.W = H, W
        self.h, self.w = H // 8, W // 8

    def match(self, g0, g1, dump=None, tile=1):
        g0 = np.ascontiguousarray(g0, np.float32)
        g1 = np.ascontiguousarray(g1, np.float32)
        self.dev.api.eloftr_match(self.m, g0.ctypes.data, g1.ctypes.data,
                                  dump.encode() if dump else None, tile)
        return self.result()

    def match_device(self, b0, b1):
        self.dev.api.eloftr_match_device(self.m, b0.mem, b1.mem)

    def result(self):
        mi, mj = C.POINTER(C.c_int)(), C.POINTER(C.c_int)()
        mc, kp = C.POINTER(C.c_float)(), C.POINTER(C.c_float)()
        nm = lib().icoreg_eloftr_result(self.m, C.byref(mi), C.byref(mj), C.byref(mc), C.byref(kp))
        rm, ra, ca = C.POINTER(C.c_float)(), C.POINTER(C.c_int)(), C.POINTER(C.c_int)()
        n = lib().icoreg_eloftr_coarse_stats(self.m, C.byref(rm), C.byref(ra), C.byref(ca))
        arr = lambda p, k: np.ctypeslib.as_array(p, (k,)).copy() if k else np.zeros(0)
        return {"nm": nm, "mi": arr(mi, nm), "mj": arr(mj, nm), "mconf": arr(mc, nm),
                "kp": arr(kp, 4 * nm).reshape(-1, 4), "row_max": arr(rm, n),
                "row_arg": arr(ra, n), "col_arg": arr(ca, n)}

    def buffer(self, name, count):
        mem = lib().icoreg_eloftr_buffer(self.m, name.encode())
        out = np.empty(count, np.float32)
        self.dev.api.ocl_read(self.dev.pb, mem, 0, out.ctypes.data, out.nbytes)
        return out

    def close(self):
        if self.m:
            self.dev.api.eloftr_free(self.m)
            lib().icoreg_struct_delete(self.m)
            self.m = None
        if self.pf:
            self.dev.api.pth_close(self.pf)
            lib().icoreg_struct_delete(self.pf)
            self.pf = None


class Roma:
    """RoMa on the device: roma_load (+ roma_load_v2) / roma_alloc /
    roma_match of the C-ABI, weights from safetensors files."""

    def __init__(self, dev, weights_path, dino_path, H, W, v2_path=None, coarse=560):
        self.dev = dev
        a = dev.api
        self.pfs = []
        for p in (weights_path, dino_path) + ((v2_path,) if v2_path else ()):
            pf = lib().icoreg_pth_new()
            a.pth_open(pf, str(p).encode())
            self.pfs.append(pf)
        self.m = lib().icoreg_roma_new()
        a.roma_load(self.m, dev.po, self.pfs[0], self.pfs[1])
        if v2_path:
            a.roma_load_v2(self.m, self.pfs[2])
        a.roma_set_coarse(self.m, coarse)
        a.roma_alloc(self.m, H, W)
        self.H, self.W, self.coarse, self.v2 = H, W, coarse, bool(v2_path)
        self.c16 = coarse // 14

    def match(self, imgA, imgB, dump=None, tile=1):
        A = np.ascontiguousarray(imgA, np.float32)
        B = np.ascontiguousarray(imgB, np.float32)
        self.dev.api.roma_match(self.m, A.ctypes.data, B.ctypes.data,
                                dump.encode() if dump else None, tile)
        return self.result()

    def coarse_device(self, pair):
        self.dev.api.roma_coarse_device(self.m, pair.mem)

    def refine_device(self, pair, flow8, cert8):
        """roma_refine_device; returns the names of the buffers holding
        the full-size warp and certainty logit."""
        self.dev.api.roma_refine_device(self.m, pair.mem, flow8.mem, cert8.mem)
        k = lib().icoreg_roma_last(self.m)
        return f"fl{k}", f"ce{k}"

    def result(self):
        f, c, s = (C.POINTER(C.c_float)(), C.POINTER(C.c_float)(), C.POINTER(C.c_float)())
        n = lib().icoreg_roma_result(self.m, C.byref(f), C.byref(c), C.byref(s))
        out = {"flow": np.ctypeslib.as_array(f, (2 * n,)).copy().reshape(2, self.H, self.W),
               "cert": np.ctypeslib.as_array(c, (n,)).copy().reshape(self.H, self.W)}
        if self.v2:
            out["sd"] = np.ctypeslib.as_array(s, (n,)).copy().reshape(self.H, self.W)
        return out

    def buffer(self, name, count, off=0):
        mem = lib().icoreg_roma_buffer(self.m, name.encode())
        out = np.empty(count, np.float32)
        self.dev.api.ocl_read(self.dev.pb, mem, off * 4, out.ctypes.data, out.nbytes)
        return out

    def gp_info(self):
        return lib().icoreg_roma_gp_info(self.m)

    def gp_retries(self):
        """GP solves roma_match re-ran with event waits after the solve's
        in-kernel wait gave up."""
        return lib().icoreg_roma_gp_retries(self.m)

    def close(self):
        if self.m:
            self.dev.api.roma_free(self.m)
            lib().icoreg_struct_delete(self.m)
            self.m = None
        for pf in self.pfs:
            self.dev.api.pth_close(pf)
            lib().icoreg_struct_delete(pf)
        self.pfs = []


class Disk:
    """DISK on the device: disk_load / disk_alloc / disk_detect of the
    C-ABI, weights from a safetensors file."""

    def __init__(self, dev, weights_path, H, W, nmax=2048):
        self.dev = dev
        a = dev.api
        self.pf = lib().icoreg_pth_new()
        a.pth_open(self.pf, str(weights_path).encode())
        self.m = lib().icoreg_disk_new()
        a.disk_load(self.m, dev.po, self.pf)
        a.disk_alloc(self.m, H, W, nmax)
        self.H, self.W, self.nmax = H, W, nmax

    def detect(self, img, h=None, w=None, n=2048, thresh=0.0, valid=None):
        _, H, W = img.shape
        h = H if h is None else h
        w = W if w is None else w
        img = np.ascontiguousarray(img, np.float32)
        n = min(n, self.nmax)
        xy = np.zeros(2 * n, np.int32)
        score = np.zeros(n, np.float32)
        desc = np.zeros((n, 128), np.float32)
        v = None if valid is None else np.ascontiguousarray(valid, np.uint8)
        nk = self.dev.api.disk_detect(self.m, img.ctypes.data, H, W, h, w, n, thresh,
                                      v.ctypes.data if v is not None else None,
                                      xy.ctypes.data, score.ctypes.data, desc.ctypes.data)
        return {"n": nk, "xy": xy[:2 * nk].reshape(-1, 2), "score": score[:nk],
                "desc": desc[:nk]}

    def buffer(self, name, count, dtype=np.float32, off=0):
        mem = lib().icoreg_disk_buffer(self.m, name.encode())
        out = np.empty(count, dtype)
        self.dev.api.ocl_read(self.dev.pb, mem, off * out.itemsize, out.ctypes.data,
                              out.nbytes)
        return out

    def close(self):
        if self.m:
            self.dev.api.disk_free(self.m)
            lib().icoreg_struct_delete(self.m)
            self.m = None
        if self.pf:
            self.dev.api.pth_close(self.pf)
            lib().icoreg_struct_delete(self.pf)
            self.pf = None

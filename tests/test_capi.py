# SPDX-License-Identifier: Unlicense
"""CPU: the C-ABI library is built for gfx950, loads without a GPU, and
exports every function that include/*.h declares (no compute calls)."""

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
INCLUDE = ROOT / "include"

# A C function declaration at file scope in our headers: return type,
# name, '('. Macros, typedefs and struct bodies are skipped.
DECL = re.compile(r"^(?:const\s+)?(?:struct\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*"
                  r"\**([a-z][a-z0-9_]*)\s*\(", re.M)


def declared_functions():
    names = set()
    for h in sorted(INCLUDE.glob("*.h")):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for line in text.splitlines():
            if line.startswith((" ", "\t", "#", "typedef")):
                continue
            m = DECL.match(line)
            if m:
                names.add(m.group(1))
    return names


def test_headers_declare_the_reference_api():
    names = declared_functions()
    # ops.h:41-164 of the reference, every entry point but ops_run (no
    # kernel objects on this path).
    for f in ("ops_mat", "ops_bmat", "ops_init", "ops_free", "ops_report",
              "ops_gemm", "ops_linear", "ops_conv1x1", "ops_geom", "ops_conv_out",
              "ops_conv2d", "ops_chan_stats", "ops_chan_affine", "ops_prelu",
              "ops_act", "ops_layernorm", "ops_softmax_rows", "ops_attention",
              "ops_rope", "ops_resize", "ops_grid_sample", "ops_unfold",
              "ops_avgpool2", "ops_pool2d", "ops_transpose", "ops_axpby",
              "ops_fold_bn"):
        assert f in names, f
    # ocl_backend.h:36-61 of the reference, plus the copy / fill entry
    # points that replace the drivers' raw cl* calls.
    for f in ("ocl_init", "ocl_free", "ocl_errstr", "ocl_check", "ocl_alloc",
              "ocl_upload", "ocl_write", "ocl_read", "ocl_release", "ocl_copy",
              "ocl_copy_rect", "ocl_fill"):
        assert f in names, f


def test_library_exports_every_declared_function(ic):
    lib = ic.lib()
    missing = [f for f in sorted(declared_functions()) if not hasattr(lib, f)]
    assert not missing, missing


def test_library_is_gfx950_only(ic):
    """The offload bundle of our own build names gfx950 and nothing else."""
    data = Path(ic.library_path()).read_bytes()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa-[-a-z]*gfx[0-9a-z]+", data))
    assert targets == {b"amdgcn-amd-amdhsa--gfx950"}, targets


def test_binding_covers_exports(ic):
    lib = ic.lib()
    for name in ic.exported_symbols():
        assert hasattr(lib, name), name


def test_binding_struct_layouts_match(ic):
    """The ctypes mirrors of struct ocl_backend and struct ops have the C
    sizes (a field added on one side only would shift every later one)."""
    lib = ic.lib()
    assert C.sizeof(ic.OclBackend) == lib.icoreg_sizeof_backend()
    assert C.sizeof(ic.Ops) == lib.icoreg_sizeof_ops()


def test_fatal_errors_are_recorded_not_fatal(ic):
    """With the record mode of the binding, a host-side error (here: an
    invalid device option, found before any device call) raises instead of
    ending the process, naming the cause."""
    api = ic.api()
    be = ic.OclBackend()
    with pytest.raises(ic.IcoregError, match="cpu"):
        api.ocl_init(C.byref(be), b"cpu", None)
    with pytest.raises(ic.IcoregError, match="Invalid device option"):
        api.ocl_init(C.byref(be), b"bogus", None)


def test_bounds_checks_reject_out_of_range_views(ic):
    """ops_* check every access against the buffer sizes before a launch:
    a wrapped 64-byte buffer cannot hold a 5 x 5 GEMM operand."""
    api = ic.api()
    lib = ic.lib()
    buf = lib.ocl_wrap(None, 64)
    ops = ic.Ops()
    be = ic.OclBackend()
    ops.ocl = C.pointer(be)
    m = ic.Opnd(buf, 0, 5, 0, 0)
    with pytest.raises(ic.IcoregError, match="ops_gemm: A"):
        api.ops_gemm(C.byref(ops), 5, 5, 5, m, m, 0, m, 1, 1, None, 0, None, 0,
                     1.0, 0, 0.0)
    with pytest.raises(ic.IcoregError, match="exceeds 2\\^31"):
        api.ops_act(C.byref(ops), buf, buf, 1 << 31, 0, 0.0)
    with pytest.raises(ic.IcoregError, match="head dimension 129"):
        api.ops_attention(C.byref(ops), m, m, m, m, 1, 1, 1, 129, 1.0, None)
    with pytest.raises(ic.IcoregError, match="ops_attention_batch: Q"):
        api.ops_attention_batch(C.byref(ops), 2, m, 4, m, 0, m, 0, m, 0, 1, 1, 1, 1,
                                1.0, None)
    g = ic.geom(3, 3, 1, 1, 1, 1, 1, 1, 2)
    with pytest.raises(ic.IcoregError, match="3 -> 4 channels in 2 groups"):
        api.ops_conv2d(C.byref(ops), buf, 3, 4, 4, buf, None, 4, C.byref(g), None,
                       None, None, 0, 0.0, buf)
    lib.ocl_release(C.byref(buf))


def test_roma_kernels_reject_bad_sizes(ic):
    """RoMa launchers refuse sizes their LDS staging cannot hold (C above
    1024 or r above 7 for local correlation) and views beyond a buffer,
    on the host before any launch."""
    api = ic.api()
    lib = ic.lib()
    buf = lib.ocl_wrap(None, 64)
    ops = ic.Ops()
    be = ic.OclBackend()
    ops.ocl = C.pointer(be)
    with pytest.raises(ic.IcoregError, match="roma_local_corr: invalid sizes C=1025"):
        api.roma_local_corr(C.byref(ops), buf, buf, 1025, 1, 1, 1, buf, buf, 0)
    with pytest.raises(ic.IcoregError, match="roma_local_corr: invalid sizes C=4 r=8"):
        api.roma_local_corr(C.byref(ops), buf, buf, 4, 1, 1, 8, buf, buf, 0)
    with pytest.raises(ic.IcoregError, match="roma_warp_sample"):
        api.roma_warp_sample(C.byref(ops), buf, 4, 4, 4, buf, buf, 0)
    with pytest.raises(ic.IcoregError, match="roma_cls_to_flow"):
        api.roma_cls_to_flow(C.byref(ops), buf, 64, 64, 8, 1, buf, buf)
    lib.ocl_release(C.byref(buf))
    # The fused refiner block's input and output maps (8 x 4 x 4 floats =
    # 512 bytes) may not overlap, also as views into one allocation at
    # different offsets. The addresses are never dereferenced: the check
    # runs before any launch.
    base = 1 << 20
    a = lib.ocl_wrap(C.c_void_p(base), 1 << 16)
    for off in (0, 64, 508):
        b = lib.ocl_wrap(C.c_void_p(base + off), 1 << 16)
        with pytest.raises(ic.IcoregError, match="roma_dwpw_small: in and out must not overlap"):
            api.roma_dwpw_small(C.byref(ops), a, 8, 4, 4, a, a, a, a, b)
        with pytest.raises(ic.IcoregError, match="roma_dwpw_small: in and out must not overlap"):
            api.roma_dwpw_small(C.byref(ops), b, 8, 4, 4, a, a, a, a, a)
        lib.ocl_release(C.byref(b))
    lib.ocl_release(C.byref(a))

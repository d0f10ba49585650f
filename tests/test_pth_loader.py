# SPDX-License-Identifier: Unlicense
"""CPU: the checkpoint reader (include/pth_loader.h) on the formats the
reference's pth_loader.c reads (pth_loader.c:463-1146): torch.save zip
archives and legacy pickle streams, written here by torch itself, against
the safetensors copy of the same tensors (bit-identical) and against torch's
own values for views, half types and wrapped state_dicts."""

import ctypes as C
import io
import sys
import zipfile
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "i.coregistration.opencl_amd"))
import synth  # noqa: E402

torch = pytest.importorskip("torch")

_free = C.CDLL(None).free
_free.argtypes = [C.c_void_p]


class PthTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("ndim", C.c_int), ("shape", C.c_long * 8),
                ("stride", C.c_long * 8), ("storage_offset", C.c_long), ("dtype", C.c_int),
                ("data_offset", C.c_long), ("storage_bytes", C.c_size_t)]


class PthFile(C.Structure):
    _fields_ = [("fp", C.c_void_p), ("path", C.c_char_p), ("ntensors", C.c_int),
                ("tensors", C.POINTER(PthTensor))]


def load(ic, path, prefix=None):
    """Every tensor of the checkpoint as float32 arrays through pth_open /
    pth_read_f32, plus pth_bytes of the whole file."""
    api = ic.api()
    pf = PthFile()
    api.pth_open(C.byref(pf), str(path).encode())
    try:
        if prefix:
            api.pth_strip_prefix(C.byref(pf), prefix.encode())
        out = {}
        for i in range(pf.ntensors):
            t = pf.tensors[i]
            shape = tuple(t.shape[d] for d in range(t.ndim))
            p = api.pth_read_f32(C.byref(pf), C.byref(t))
            n = int(np.prod(shape)) if shape else 1
            out[t.name.decode()] = np.ctypeslib.as_array(p, (n,)).copy().reshape(shape)
            _free(C.cast(p, C.c_void_p))
        nbytes = api.pth_bytes(C.byref(pf), b"")
    finally:
        api.pth_close(C.byref(pf))
    return out, nbytes


def assert_same(a, b):
    assert sorted(a) == sorted(b)
    for k in a:
        assert a[k].shape == b[k].shape, k
        assert a[k].dtype == b[k].dtype == np.float32
        assert np.array_equal(a[k].view(np.uint32), b[k].view(np.uint32)), k


@pytest.mark.parametrize("legacy", [False, True])
def test_model_weights_torch_save_equal_safetensors(ic, tmp_path, legacy):
    """The ELoFTR and DISK weight sets written by torch.save read back bit
    for bit as from safetensors."""
    for name, w in (("eloftr", synth.eloftr_weights()), ("disk", synth.disk_weights())):
        st = synth.save_safetensors(w, tmp_path / f"{name}.safetensors")
        pt = synth.save_torch(w, tmp_path / f"{name}.pth", legacy=legacy)
        a, na = load(ic, st)
        b, nb = load(ic, pt)
        assert_same(a, b)
        assert na == nb == sum(v.size * 4 for v in w.values())


def _zoo():
    """Tensors torch.save writes in unusual ways: views of shared storages
    (offset slices, transposes, expanded strides), half types, parameters,
    0-d tensors and integer buffers (left out by the reader)."""
    g = torch.Generator().manual_seed(5)
    base = torch.randn(6, 10, generator=g)
    lin = torch.nn.Linear(7, 3)
    bn = torch.nn.BatchNorm2d(4)
    sd = {
        "base": base,
        "row": base[2],                     # storage offset 20
        "cols": base[:, 3:7],               # strided rows
        "t": base.t(),                      # transposed
        "half": torch.randn(3, 5, generator=g).half(),
        "bf16": torch.randn(4, 2, generator=g).bfloat16(),
        "half_t": torch.randn(5, 3, generator=g).half().t(),
        "scalar": torch.tensor(2.5),
        "param": torch.nn.Parameter(torch.randn(2, 3, generator=g)),
        "steps": torch.tensor(11),          # int64: not indexed
        "mask": torch.ones(3, dtype=torch.bool),
    }
    for k, v in lin.state_dict().items():
        sd[f"lin.{k}"] = v
    for k, v in bn.state_dict().items():
        sd[f"bn.{k}"] = v
    return sd


def _expected(sd, prefix=""):
    return {prefix + k: v.detach().float().contiguous().numpy().astype(np.float32)
            for k, v in sd.items() if v.is_floating_point()}


@pytest.mark.parametrize("legacy", [False, True])
@pytest.mark.parametrize("wrap", [None, "state_dict", "model", "extractor"])
def test_views_half_types_and_wrappers(ic, tmp_path, legacy, wrap):
    sd = _zoo()
    obj = sd if wrap is None else {wrap: sd, "epoch": 3, "note": "x",
                                   "cfg": {"lr": 0.1, "steps": [1, 2]}}
    p = tmp_path / "zoo.pth"
    torch.save(obj, str(p), _use_new_zipfile_serialization=not legacy)
    got, _ = load(ic, p)
    want = _expected(sd)
    assert "steps" not in got and "mask" not in got and "bn.num_batches_tracked" not in got
    assert_same(got, want)


def test_module_state_dict_and_prefix(ic, tmp_path):
    """An nn.Module state_dict (an OrderedDict carrying _metadata) saved
    under a wrapper prefix, stripped with pth_strip_prefix as roma.c:409
    strips "matcher.model."."""
    m = torch.nn.Sequential(torch.nn.Conv2d(3, 4, 3), torch.nn.BatchNorm2d(4),
                            torch.nn.Linear(4, 2))
    sd = {"matcher.model." + k: v for k, v in m.state_dict().items()}
    p = tmp_path / "mod.pth"
    torch.save(m.state_dict(), str(p))
    got, _ = load(ic, p)
    assert_same(got, _expected(m.state_dict()))
    torch.save(sd, str(p))
    got, _ = load(ic, p, prefix="matcher.model.")
    assert_same(got, _expected(m.state_dict()))


def test_shared_storage_across_tensors_is_read_once_each(ic, tmp_path):
    """Two names over one storage (tied weights) read the same values."""
    w = torch.randn(4, 4)
    p = tmp_path / "tied.pth"
    torch.save({"a": w, "b": w, "c": w[1:3].t()}, str(p))
    got, nbytes = load(ic, p)
    assert np.array_equal(got["a"], got["b"])
    assert np.array_equal(got["c"], w[1:3].t().contiguous().numpy())
    assert nbytes == (16 + 16 + 8) * 4


def _raises(ic, path, match):
    api = ic.api()
    pf = PthFile()
    with pytest.raises(ic.IcoregError, match=match):
        api.pth_open(C.byref(pf), str(path).encode())


def test_bad_files_are_fatal_with_a_reason(ic, tmp_path):
    _raises(ic, tmp_path / "missing.pth", "Unable to open")
    p = tmp_path / "junk.bin"
    p.write_bytes(b"\x01\x02\x03" * 100)
    _raises(ic, p, "neither")
    # A zip archive without data.pkl.
    p = tmp_path / "nodata.zip"
    with zipfile.ZipFile(p, "w", zipfile.ZIP_STORED) as z:
        z.writestr("archive/version", "3")
    _raises(ic, p, "no data.pkl")
    # A torch archive re-packed with compression.
    src = tmp_path / "ok.pth"
    torch.save({"a": torch.randn(8)}, str(src))
    p = tmp_path / "deflated.pth"
    with zipfile.ZipFile(src) as zi, zipfile.ZipFile(p, "w", zipfile.ZIP_DEFLATED) as zo:
        for info in zi.infolist():
            zo.writestr(info.filename, zi.read(info.filename))
    _raises(ic, p, "compressed")
    # A legacy stream cut inside the storage data.
    src = tmp_path / "legacy.pth"
    torch.save({"a": torch.randn(64)}, str(src), _use_new_zipfile_serialization=False)
    p = tmp_path / "cut.pth"
    p.write_bytes(src.read_bytes()[:-40])
    _raises(ic, p, "truncated")
    # A pickle whose root holds no tensors.
    p = tmp_path / "notensors.pth"
    torch.save({"epoch": 1, "cfg": {"a": 2}}, str(p))
    _raises(ic, p, "no state_dict")


def _craft_zip(path, size, stride, nfloats=8):
    """A torch.save-style zip archive written by hand: data.pkl holds
    {"w": _rebuild_tensor_v2(storage "0" of nfloats floats, offset 0,
    size, stride)}; the shape and strides are whatever is given."""
    import collections
    import pickle

    class Storage:
        pass

    class Tensor:
        def __reduce__(self):
            return (torch._utils._rebuild_tensor_v2,
                    (Storage(), 0, tuple(size), tuple(stride), False,
                     collections.OrderedDict()))

    class Pickler(pickle.Pickler):
        def persistent_id(self, obj):
            if isinstance(obj, Storage):
                return ("storage", torch.FloatStorage, "0", "cpu", nfloats)
            return None

    b = io.BytesIO()
    Pickler(b, protocol=2).dump({"w": Tensor()})
    with zipfile.ZipFile(path, "w", zipfile.ZIP_STORED) as z:
        z.writestr("archive/data.pkl", b.getvalue())
        z.writestr("archive/data/0", np.arange(nfloats, dtype=np.float32).tobytes())
        z.writestr("archive/version", "3\n")
    return path


def test_overflowing_shape_and_stride_are_rejected(ic, tmp_path):
    """Extents computed from a file's shape and strides are checked for
    overflow: 4 x (2^62 + 1) wraps to 4 in 64-bit arithmetic, which would
    pass the storage bound (5 floats of 8) and then index far outside it
    in the strided gather. A well-formed hand-written archive reads."""
    ok = _craft_zip(tmp_path / "ok.pth", (2, 4), (1, 2))
    got, _ = load(ic, ok)
    assert np.array_equal(got["w"], np.arange(8, dtype=np.float32).reshape(4, 2).T)
    _raises(ic, _craft_zip(tmp_path / "wrap.pth", (5,), (2 ** 62 + 1,)), "exceeds its storage")
    _raises(ic, _craft_zip(tmp_path / "numel.pth", (2 ** 32, 2 ** 32), (0, 0)),
            "exceeds its storage")


def test_require_checks_shapes(ic, tmp_path):
    api = ic.api()
    p = synth.save_torch({"w": np.zeros((4, 3, 5, 5), np.float32)}, tmp_path / "w.pth")
    pf = PthFile()
    api.pth_open(C.byref(pf), str(p).encode())
    try:
        ok = (C.c_long * 4)(4, -1, 5, 5)
        assert api.pth_require(C.byref(pf), b"w", 4, ok)
        bad = (C.c_long * 4)(4, 3, 3, 3)
        with pytest.raises(ic.IcoregError, match="dimension 2 is 5, 3 expected"):
            api.pth_require(C.byref(pf), b"w", 4, bad)
        with pytest.raises(ic.IcoregError, match="not found"):
            api.pth_require(C.byref(pf), b"v", 4, ok)
    finally:
        api.pth_close(C.byref(pf))

# SPDX-License-Identifier: Unlicense
"""GPU: uploads beside the library's stream (ocl_write_async,
ocl_write_join, ocl_write_wait, page-locked sources from ocl_host_alloc)
and the tile loop they serve: the next pair uploads while the current one
computes, with the same matches as the blocking eloftr_match."""

import ctypes as C
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "i.coregistration.opencl_amd"))
import synth  # noqa: E402

pytestmark = pytest.mark.gpu


class Pinned:
    """n float32 of page-locked host memory as a numpy view."""

    def __init__(self, dev, n):
        self.dev = dev
        self.ptr = dev.api.ocl_host_alloc(dev.pb, 4 * n)
        assert self.ptr
        self.a = np.ctypeslib.as_array((C.c_float * n).from_address(self.ptr))

    def free(self):
        if self.ptr:
            self.dev.api.ocl_host_free(self.ptr)
            self.ptr = None


def test_write_async_join_wait(dev, ic):
    """Two copies into two buffers, joined on the stream before a device
    copy reads them; the source is rewritten only after ocl_write_wait."""
    print("[async] write/join/wait", flush=True)
    a = dev.api
    n = 1 << 20
    rng = np.random.default_rng(3)
    x0 = rng.standard_normal(n).astype(np.float32)
    x1 = rng.standard_normal(n).astype(np.float32)
    h = Pinned(dev, n)
    try:
        d0, d1, e = dev.alloc(4 * n), dev.alloc(4 * n), dev.alloc(8 * n)
        h.a[:] = x0
        t0 = a.ocl_write_async(dev.pb, d0.mem, 0, h.ptr, 4 * n)
        a.ocl_write_wait(dev.pb, t0)
        h.a[:] = x1
        t1 = a.ocl_write_async(dev.pb, d1.mem, 0, h.ptr, 4 * n)
        assert t1 == t0 + 1
        a.ocl_write_join(dev.pb, t0)
        a.ocl_write_join(dev.pb, t1)
        a.ocl_copy(dev.pb, d0.mem, 0, e.mem, 0, 4 * n)
        a.ocl_copy(dev.pb, d1.mem, 0, e.mem, 4 * n, 4 * n)
        got = dev.read(e, 2 * n)
        assert np.array_equal(got[:n], x0) and np.array_equal(got[n:], x1)
        # A byte offset and a ragged size.
        t2 = a.ocl_write_async(dev.pb, d0.mem, 12, h.ptr, 4 * 1001)
        a.ocl_write_join(dev.pb, t2)
        got = dev.read(d0, n)
        assert np.array_equal(got[3:1004], x1[:1001])
        assert np.array_equal(got[:3], x0[:3]) and np.array_equal(got[1004:], x0[1004:])
    finally:
        h.free()


def test_write_async_errors(dev, ic):
    """Out-of-range destinations, unknown and expired tickets, and a copy
    while a graph is being recorded are refused."""
    print("[async] errors", flush=True)
    a = dev.api
    h = Pinned(dev, 64)
    try:
        d = dev.alloc(256)
        with pytest.raises(ic.IcoregError, match="ocl_write_async"):
            a.ocl_write_async(dev.pb, d.mem, 200, h.ptr, 64)
        t = a.ocl_write_async(dev.pb, d.mem, 0, h.ptr, 256)
        with pytest.raises(ic.IcoregError, match="ticket"):
            a.ocl_write_join(dev.pb, t + 1)
        with pytest.raises(ic.IcoregError, match="ticket"):
            a.ocl_write_wait(dev.pb, -1)
        for _ in range(64):
            a.ocl_write_async(dev.pb, d.mem, 0, h.ptr, 4)
        with pytest.raises(ic.IcoregError, match="ticket"):
            a.ocl_write_join(dev.pb, t)
        a.ocl_write_wait(dev.pb, t + 64)
        a.ocl_graph_begin(dev.pb)
        try:
            a.ocl_fill(dev.pb, d.mem, 0, 64, 0.0)
            with pytest.raises(ic.IcoregError, match="graph is being recorded"):
                a.ocl_write_async(dev.pb, d.mem, 0, h.ptr, 4)
        finally:
            g = a.ocl_graph_end(dev.pb)
            a.ocl_graph_free(g)
    finally:
        h.free()


def test_eloftr_tile_loop_overlapped(dev, ic, tmp_path):
    """Three pairs through the overlapped loop (pair t + 1 uploads into the
    other device slot while pair t computes) give the matches of the
    blocking eloftr_match, bit for bit."""
    print("[async] eloftr tile loop", flush=True)
    H, W = 128, 160
    wf = synth.eloftr_weights_file(tmp_path / "w.safetensors")
    net = ic.Eloftr(dev, wf, H, W)
    a = dev.api
    pairs = [synth.eloftr_noise_pair(H, W, shift=(8, 16), seed=s, noise=0.05)
             for s in (1, 2, 3)]
    try:
        ref = [net.match(g0, g1) for g0, g1 in pairs]
        assert sum(r["nm"] for r in ref) > 0
        n = H * W
        host = [Pinned(dev, 2 * n) for _ in range(2)]
        slots = [(dev.alloc(4 * n), dev.alloc(4 * n)) for _ in range(2)]
        tickets = [None, None]

        def upload(t):
            s = t % 2
            if tickets[s] is not None:
                a.ocl_write_wait(dev.pb, tickets[s][1])
            host[s].a[:n] = pairs[t][0].ravel()
            host[s].a[n:] = pairs[t][1].ravel()
            tickets[s] = (a.ocl_write_async(dev.pb, slots[s][0].mem, 0, host[s].ptr, 4 * n),
                          a.ocl_write_async(dev.pb, slots[s][1].mem, 0, host[s].ptr + 4 * n,
                                            4 * n))

        got = []
        upload(0)
        for t in range(len(pairs)):
            s = t % 2
            a.ocl_write_join(dev.pb, tickets[s][0])
            a.ocl_write_join(dev.pb, tickets[s][1])
            a.eloftr_match_enqueue(net.m, slots[s][0].mem, slots[s][1].mem)
            if t + 1 < len(pairs):
                upload(t + 1)
            a.eloftr_match_collect(net.m)
            got.append(net.result())
        for r, g in zip(ref, got):
            assert r["nm"] == g["nm"]
            for k in ("mi", "mj", "mconf", "kp", "row_max", "row_arg", "col_arg"):
                assert np.array_equal(r[k], g[k]), k
        for h in host:
            h.free()
    finally:
        net.close()

# SPDX-License-Identifier: Unlicense
"""GPU: ops_attention_noalloc (the attention entry point that allocates
nothing: its key-split partials live in a fixed device array) gives the
same output as ops_attention through the C-ABI, on two calls in a row,
the second smaller than the first, and both match a float64 softmax
attention."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _run(dev, ic, fn, Q, K, V, Nq, Nk, nh, d, scale):
    O = dev.upload(np.full(Nq * nh * d, 7.0, np.float32))
    ld = nh * d
    fn(dev.po, ic.mat(Q, 0, ld), ic.mat(K, 0, ld), ic.mat(V, 0, ld), ic.mat(O, 0, ld),
       Nq, Nk, nh, d, scale, None)
    return dev.read(O, Nq * nh * d).reshape(Nq, nh, d)


def _reference(q, k, v, scale):
    s = np.einsum("qhd,khd->hqk", q.astype(np.float64), k.astype(np.float64)) * scale
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("hqk,khd->qhd", p, v.astype(np.float64))


# The ViT's shape (1601 tokens, 16 heads of 64: three key splits, 20 MB
# of partials), then ELoFTR's smaller one (400 tokens, 8 heads of 32).
@pytest.mark.parametrize("Nq,Nk,nh,d", [(1601, 1601, 16, 64), (400, 400, 8, 32)])
def test_noalloc_matches_ops_attention(dev, ic, Nq, Nk, nh, d):
    print(f"[noalloc] attention Nq={Nq} Nk={Nk} nh={nh} d={d}", flush=True)
    rng = np.random.default_rng(Nq + d)
    q = rng.standard_normal((Nq, nh, d)).astype(np.float32)
    k = rng.standard_normal((Nk, nh, d)).astype(np.float32)
    v = rng.standard_normal((Nk, nh, d)).astype(np.float32)
    Q, K, V = dev.upload(q), dev.upload(k), dev.upload(v)
    scale = float(1.0 / np.sqrt(d))
    want = _run(dev, ic, dev.api.ops_attention, Q, K, V, Nq, Nk, nh, d, scale)
    got = _run(dev, ic, dev.api.ops_attention_noalloc, Q, K, V, Nq, Nk, nh, d, scale)
    assert np.array_equal(got, want)
    ref = _reference(q, k, v, scale)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 2e-3


def test_noalloc_rejects_partials_beyond_the_array(dev, ic):
    """10 heads of 128 over 2176 queries and 1024 keys take 6 key splits,
    64.7 MiB of partials, more than the 24 MiB array: rejected on the
    host before any launch."""
    print("[noalloc] oversize rejection", flush=True)
    Nq, Nk, nh, d = 2176, 1024, 10, 128
    Q, K, V = dev.zeros(Nq * nh * d), dev.zeros(Nk * nh * d), dev.zeros(Nk * nh * d)
    O = dev.zeros(Nq * nh * d)
    ld = nh * d
    with pytest.raises(ic.IcoregError, match="exceed the 25165824-byte scratch array"):
        dev.api.ops_attention_noalloc(dev.po, ic.mat(Q, 0, ld), ic.mat(K, 0, ld),
                                      ic.mat(V, 0, ld), ic.mat(O, 0, ld), Nq, Nk, nh, d,
                                      0.1, None)

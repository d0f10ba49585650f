# SPDX-License-Identifier: Unlicense
"""GPU: ops_gemm on shapes that take the small-product kernel (few output
tiles, K <= 256 and a multiple of 16, rows 16-byte aligned) and on their
neighbours that do not, against the oracle's gemm (the reference's
gemm contract, ops.cl:39-284 of i.coregistration.opencl) at the reference
bar of 2e-5 of the largest magnitude."""

import ctypes as C

import numpy as np
import pytest

import opcases
from oracle_lib import fp

pytestmark = pytest.mark.gpu

GEMM_SHAPES = [
    # (M, N, K, transb, nb, act, residual, biasrow): aggregated-attention
    # projections (400 and 800 tokens, K = 256) and o_proj (B transposed,
    # two images), ragged tiles, K = 16 and 48, both bias layouts; the
    # next two have K = 272 and N % 4 != 0 (main kernel).
    (400, 256, 256, 1, 1, 0, 0, 0),
    (800, 512, 256, 1, 1, 0, 0, 1),
    (256, 400, 256, 1, 2, 0, 0, 0),
    (37, 44, 48, 0, 3, 4, 1, 0),
    (33, 36, 16, 1, 1, 2, 1, 1),
    (96, 100, 256, 0, 2, 3, 0, 1),
    (64, 64, 272, 0, 1, 1, 0, 0),
    (50, 30, 64, 0, 1, 1, 1, 0),
    # LDS-DMA kernel (B given K x N, M <= 256, K >= 256): the MLP's second
    # layer, ragged rows and columns, K not a multiple of 32.
    (256, 1600, 512, 0, 2, 0, 1, 1),
    (200, 300, 292, 0, 1, 3, 0, 0),
    # Main kernel with tiles cut over K on 256 CUs (one batch, under 4
    # tiles per CU): 288 tiles (256 whole, 32 in 8 pieces) with in-place
    # residual and bias; 64 tiles in 4 pieces each, ragged edges, K not a
    # multiple of 16.
    (1100, 1024, 512, 1, 1, 4, 1, 0),
    (500, 500, 520, 1, 1, 1, 0, 1),
]


@pytest.mark.parametrize("shape", GEMM_SHAPES, ids=[str(s) for s in GEMM_SHAPES])
def test_gemm_shapes(shape, dev, ic, orc):
    M, N, K, transb, nb, act, residual, biasrow = shape
    print(f"[gemm] {shape}", flush=True)
    rng = np.random.default_rng(7 + M + N + K)
    a = rng.uniform(-1, 1, nb * M * K).astype(np.float32)
    b = rng.uniform(-1, 1, nb * N * K).astype(np.float32)
    bias = rng.uniform(-1, 1, M if biasrow else N).astype(np.float32)
    r = rng.uniform(-1, 1, nb * M * N).astype(np.float32)
    ldb = K if transb else N
    ref = r.copy() if residual else np.zeros(nb * M * N, np.float32)
    orc.orc_gemm(M, N, K, fp(a), 0, K, M * K, 0, fp(b), 0, ldb, N * K, 0, transb,
                 fp(ref), 0, N, M * N, 0, nb, 1, fp(bias), biasrow,
                 fp(ref) if residual else None, 0, C.c_float(0.5), act, C.c_float(0.1))
    A, B, Bi = dev.upload(a), dev.upload(b), dev.upload(bias)
    out = dev.upload(r) if residual else dev.zeros(nb * M * N)
    dev.api.ops_gemm(dev.po, M, N, K, ic.bmat(A, 0, K, M * K, 0),
                     ic.bmat(B, 0, ldb, N * K, 0), transb, ic.bmat(out, 0, N, M * N, 0),
                     nb, 1, ic.mem(Bi), biasrow, ic.mem(out) if residual else None, 0, 0.5,
                     act, 0.1)
    got = dev.read(out, nb * M * N)
    err = opcases.rel_err(got, ref)
    assert err <= opcases.TOL, f"{shape}: {err:.2e}"

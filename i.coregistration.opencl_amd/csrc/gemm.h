/* SPDX-License-Identifier: Unlicense */

/* The fp32 MFMA GEMM kernel family behind ops_gemm, ops_linear,
 * ops_conv1x1 and the one-group ops_conv2d (implicit GEMM). */

#ifndef ICOREG_GEMM_H
#define ICOREG_GEMM_H

#include <hip/hip_runtime.h>

/* Source of the B operand. */
enum gemm_bmode {
    GEMM_B_KN = 0,   /* B(k, n) = B[k * ldb + n]. */
    GEMM_B_NK = 1,   /* B(k, n) = B[n * ldb + k] (transb). */
    GEMM_B_CONV = 2, /* B(k, n) = im2col of a (C, H, W) input, gathered. */
};

struct gemm_args {
    int M, N, K;
    const float *A;
    long long lda, sa0, sa1;
    const float *B;
    long long ldb, sb0, sb1;
    float *C;
    long long ldc, sc0, sc1;
    const float *R; /* Already offset by roff; C's layout. */
    int nb1;
    const float *bias;
    int biasrow;
    float alpha;
    int act;
    float slope;
    /* GEMM_B_CONV: input (C, H, W), window, output width; optional
     * input normalisation and PReLU gate per input channel. */
    int cc, ch, cw, kh, kw, sy, sx, py, px, dy, dx, wo;
    const float *mean, *rstd, *gate;
    /* rup = 2 or 4: R is not in C's layout but (nb0 batches rs0 floats
     * apart) M rows of rh x rw planes, and C's column n = y * rwo + x
     * receives R's rup x bilinear resize at (y, x) (ops_resize with scale
     * rup, pixel centres: source step rsc = 1 / rup), sampled on the fly.
     * rpre: R is added before the activation instead of after it. */
    int rup, rh, rw, rwo, rpre;
    float rsc;
    long long rs0;
    /* Small-product kernel only: rotary encoding of output columns
     * 0..rcols-1 (ops_rope with one head of rd columns, interleaved pairs,
     * table row r % rnpos of rope for output row r). */
    const float2 *rope;
    int rcols, rd, rnpos;
    /* Main kernel, one batch: tiles nfull.. are cut into split pieces
     * over K whose partial sums go to part (4096 floats a piece) and are
     * added by a second kernel (gemm_split_floats; split <= 1: none). */
    int nfull, split;
    float *part;
};

/* True if the kernel takes these leading dimensions: each at least its
 * row length and below 4 Mi floats. */
bool gemm_shape_ok(const gemm_args &g, int bmode);

/* Launch on stream s over nb batches on a device of cus CUs. va/vb:
 * 16-byte vector loads allowed for A / B (every row start aligned). */
void gemm_launch(const gemm_args &g, int bmode, int nb, bool va, bool vb,
                 int cus, hipStream_t s);

/* Floats of part that gemm_launch's main kernel needs for g (0: it
 * runs without pieces). */
size_t gemm_split_floats(const gemm_args &g, int bmode, int nb, bool va, bool vb, int cus);

/* True if gemm_launch would run g on the small-product kernel. */
bool gemm_smallk_ok(const gemm_args &g, int bmode, int nb, bool va, bool vb, int cus);

/* Two products that both pass gemm_smallk_ok with B given N x K and one
 * batch, in one launch of the small-product kernel. */
void gemm_launch_smallk2(const gemm_args &g1, const gemm_args &g2, hipStream_t s);

#include "ops.h"

/* Y1 (rows x n1) = X1 (rows x in) W1^T and Y2 (rows x n2) = X2 W2^T, both
 * token-major with no bias (two ops_linear calls), followed by the rotary
 * encoding ops_rope(Y, 0, n, rows, 1, rd, npos, cs, 1) of the first rc1 /
 * rc2 columns (0: none): one launch when both products are small,
 * otherwise the separate calls. */
void ops_linear2_rope(struct ops *o, int rows, int in, cl_mem X1, cl_mem W1, cl_mem Y1, int n1,
                      int rc1, cl_mem X2, cl_mem W2, cl_mem Y2, int n2, int rc2, cl_mem cs,
                      int rd, int npos);

/* C (M x N, nb batches C.s0 apart) = act(A (M x K) B (K x N, not
 * transposed)) + the up x bilinear resize (ops_resize with scale up) of R
 * to H x W = N, R holding nb batches (M, rh, rw) rstride floats apart;
 * pre: the resize is added before the activation. A product whose
 * residual or addend is an upsampled map (ops_resize, then ops_gemm with
 * the map), without writing the upsampled map. */
void ops_gemm_upres(struct ops *o, int M, int N, int K, struct opnd A,
                    struct opnd B, struct opnd C, int nb, cl_mem R,
                    long rstride, int rh, int rw, int H, int W, int up, int pre,
                    int act, float slope);

#endif /* ICOREG_GEMM_H */

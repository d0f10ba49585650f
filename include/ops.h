/* SPDX-License-Identifier: Unlicense */

/* Generic tensor operations of the matcher networks, on one MI355X.
 *
 * The API is the reference's (ops.h:8-164 of i.coregistration.opencl),
 * signature for signature, so that the model drivers and the kernel
 * check call it unchanged; behind it are hand-written gfx950 kernels
 * (fp32 MFMA GEMM and implicit-GEMM convolution, flash attention,
 * wave-reduction norms, vectorised element-wise kernels).
 *
 * Tensors are float32, channel-major (C, H, W) for image-like data and
 * token-major (tokens, channels) for sequences. Offsets are in floats.
 * Every call checks on the host that each element it will touch lies
 * inside its buffers (cl_mem carries the byte size) and that element
 * counts passed to kernels stay below 2^31; a violation is a fatal
 * error naming the operation, before anything is launched. */

#ifndef ICOREG_OPS_H
#define ICOREG_OPS_H

#include "hip_backend.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Activations, applied after the bias (ops.h:8-13). */
#define ACT_NONE 0
#define ACT_GELU 1 /* Exact (erf) GELU. */
#define ACT_RELU 2
#define ACT_LEAKY 3 /* LeakyReLU with the given negative slope. */
#define ACT_GELU_TANH 4

/* Largest attention head dimension of ops_attention (ops.h:16). */
#define OPS_MAX_HEAD_DIM 128

/* ops.h:21-30. No kernel objects: every operation launches a typed HIP
 * kernel. scratch / scratch_bytes / im2col_bytes are kept for the
 * callers that read them; the implicit-GEMM convolution needs no
 * unfold scratch, so im2col_bytes bounds nothing here. */
struct ops {
    struct ocl_backend *ocl;
    cl_mem scratch;
    size_t scratch_bytes, im2col_bytes;
};

/* One GEMM operand: buffer, element offset, leading dimension and the
 * two batch strides (ops.h:34-39). Batch b of nb = nb0 * nb1 uses
 * (b / nb1) * s0 + (b % nb1) * s1. */
struct opnd {
    cl_mem buf;
    cl_long off;
    cl_int ld;
    cl_long s0, s1;
};

struct opnd ops_mat(cl_mem buf, long off, int ld);
struct opnd ops_bmat(cl_mem buf, long off, int ld, long s0, long s1);

void ops_init(struct ops *o, struct ocl_backend *ocl);
void ops_free(struct ops *o);

/* Per-name kernel times accumulated when ocl->profile is set (HIP events
 * around every launch, the stream synchronised after each), printed by
 * ops_report (ops.c:25-67). */
void ops_report(void);

/* Batched C = act(alpha * A * op(B) + bias) + R over nb = nb0 * nb1
 * products; bias per column, or per row with biasrow set; R NULL for no
 * residual, else it has C's layout (ldc, strides) from element offset
 * roff and may alias C. transb: B stored N x K (PyTorch Linear weight),
 * else K x N. ops.h:54-60. */
void ops_gemm(struct ops *o, int M, int N, int K, struct opnd A, struct opnd B,
              int transb, struct opnd C, int nb, int nb1, cl_mem bias,
              int biasrow, cl_mem R, long roff, float alpha, int act,
              float slope);

/* Token-major Y[rows, out] = act(X[rows, in] W^T + b) (+ Y when
 * residual), W the PyTorch [out, in] weight. ops.h:64-66. */
void ops_linear(struct ops *o, int rows, int in, int out, cl_mem X, long xoff,
                cl_mem W, cl_mem b, cl_mem Y, long yoff, int act, float slope,
                int residual);

/* 1x1 convolution: W (K, C) times X (C, HW) into Y (K, HW), bias per
 * output channel. ops.h:70-71. */
void ops_conv1x1(struct ops *o, cl_mem X, long xoff, int C, int HW, cl_mem W,
                 cl_mem b, int K, cl_mem Y, long yoff, int act, float slope);

/* Geometry of a 2D convolution or pooling window (ops.h:74-76). */
struct conv_geom {
    int kh, kw, sy, sx, py, px, dy, dx, groups;
};

/* Square kernel k, stride s, padding p, dilation 1, one group. */
struct conv_geom ops_geom(int k, int s, int p);

/* Output size of a convolution along one axis. */
int ops_conv_out(int n, int k, int s, int p, int d);

/* in (C, H, W) into out (K, Ho, Wo), weights (K, C / groups, kh, kw).
 * mean/rstd/alpha (NULL for none) normalise and gate every input value,
 * prelu((x - mean[c]) * rstd[c], alpha[c]), before the zero padding, as
 * DISK's blocks (ops.h:84-92). One group, 3 x 3 or 5 x 5, stride 1
 * or 2: direct fp32 MFMA kernel on LDS input patches; other one-group
 * geometries: implicit-GEMM fp32 MFMA kernel; grouped: a direct
 * kernel. */
void ops_conv2d(struct ops *o, cl_mem in, int C, int H, int W, cl_mem w,
                cl_mem b, int K, const struct conv_geom *g, cl_mem mean,
                cl_mem rstd, cl_mem alpha, int act, float slope, cl_mem out);

/* Extension with no counterpart in the reference: ops_conv2d over nb
 * images stored in_stride / out_stride floats apart (the two images of
 * a tile pair), in one launch; the same weights, bias and input
 * normalisation for every image. */
void ops_conv2d_batch(struct ops *o, int nb, cl_mem in, long in_stride, int C,
                      int H, int W, cl_mem w, cl_mem b, int K,
                      const struct conv_geom *g, cl_mem mean, cl_mem rstd,
                      cl_mem alpha, int act, float slope, cl_mem out,
                      long out_stride);

/* Instance statistics of (C, HW): mean and 1 / sqrt(biased var + eps)
 * per channel. ops.h:96-97. */
void ops_chan_stats(struct ops *o, cl_mem x, int C, int HW, float eps,
                    cl_mem mean, cl_mem rstd);

/* Y = act((X - mean) * rstd * g + b) per channel; mean (with rstd), g, b
 * may each be NULL. Y may alias X. ops.h:101-103. */
void ops_chan_affine(struct ops *o, cl_mem X, cl_mem Y, int C, int HW,
                     cl_mem mean, cl_mem rstd, cl_mem g, cl_mem b, int act,
                     float slope);

void ops_prelu(struct ops *o, cl_mem X, cl_mem Y, int C, int HW, cl_mem alpha);
void ops_act(struct ops *o, cl_mem X, cl_mem Y, long n, int act, float slope);

/* Row LayerNorm of rows x C (token-major), g/b NULL for none; Y may
 * alias X. ops.h:109-110. */
void ops_layernorm(struct ops *o, long rows, int C, cl_mem X, cl_mem Y,
                   cl_mem g, cl_mem b, float eps, int act, float slope);

/* In-place softmax(scale * x) over rows of L. ops.h:113. */
void ops_softmax_rows(struct ops *o, cl_mem S, long rows, int L, float scale);

/* O = softmax(scale Q K^T) V per head, nh heads of d <= 128 channels,
 * head h at columns h * d of token-major rows; kmask (Nk bytes, 0 =
 * ignore the key) may be NULL; a query with no key left gets zeros.
 * ops.h:119-121. */
void ops_attention(struct ops *o, struct opnd Q, struct opnd K, struct opnd V,
                   struct opnd O, int Nq, int Nk, int nh, int d, float scale,
                   cl_mem kmask);

/* ops_attention that allocates nothing: the key-split partials go to a
 * fixed 24 MiB device array (one per GPU, held until the process ends)
 * instead of the ops work buffer, which ops_attention grows with
 * hipMalloc. No counterpart in the reference; for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops). Same results as ops_attention. A problem whose partials
 * exceed 24 MiB is a fatal error (RoMa's ViT attention, the largest on
 * the path, needs 20.3 MB). The array costs 24 MiB of device memory per
 * process on every GPU where the library is loaded, called or not.
 * Every call on one GPU shares the array: calls that overlap on one GPU
 * (other streams or threads) race. */
void ops_attention_noalloc(struct ops *o, struct opnd Q, struct opnd K,
                           struct opnd V, struct opnd O, int Nq, int Nk, int nh,
                           int d, float scale, cl_mem kmask);

/* ops_attention on nb independent problems in one launch, problem i's Q,
 * K, V and O starting bq, bk, bv, bo floats after problem i - 1's (kmask
 * shared). No counterpart in the reference, which loops over the images
 * of a pair with one attention launch each (eloftr.c:405-449,
 * roma.c:692-713). */
void ops_attention_batch(struct ops *o, int nb, struct opnd Q, long bq,
                         struct opnd K, long bk, struct opnd V, long bv,
                         struct opnd O, long bo, int Nq, int Nk, int nh, int d,
                         float scale, cl_mem kmask);

/* Rotary encoding in place on rows x (nh heads of d) of X (row stride
 * ld, offset off), row r at table row r % npos of cs (npos x d / 2
 * (cos, sin) pairs). interleaved: pairs (2f, 2f + 1), else (f, f + d/2).
 * ops.h:127-128. */
void ops_rope(struct ops *o, cl_mem X, long off, int ld, long rows, int nh,
              int d, int npos, cl_mem cs, int interleaved);

/* Bilinear resampling of in (C, h, w) into channels coff.. of out
 * (*, H, W). align_corners 0: scale > 0 gives source step 1 / scale,
 * scale 0 the size ratio. ops.h:133-134. */
void ops_resize(struct ops *o, cl_mem in, int C, int h, int w, cl_mem out,
                int H, int W, int coff, int align_corners, float scale);

/* Bilinear sampling of in (C, H, W) at n normalised (x, y) points of
 * grid into out (C, n), zero padding. ops.h:138-139. */
void ops_grid_sample(struct ops *o, cl_mem in, int C, int H, int W, cl_mem grid,
                     int n, int align_corners, cl_mem out);

/* F.unfold of in (C, H, W) into out (C * kh * kw, Ho * Wo). */
void ops_unfold(struct ops *o, cl_mem in, int C, int H, int W,
                const struct conv_geom *g, cl_mem out);

/* 2x2 / stride 2 average pooling. */
void ops_avgpool2(struct ops *o, cl_mem in, int C, int H, int W, cl_mem out);

/* k x k pooling, stride s, padding p: maximum (padding ignored) or
 * average (padding counted). */
void ops_pool2d(struct ops *o, cl_mem in, int C, int H, int W, int k, int s,
                int p, int max, cl_mem out);

/* (B, R, C) to (B, C, R). */
void ops_transpose(struct ops *o, cl_mem in, cl_mem out, int B, int R, int C);

/* out = alpha * a + beta * b[i % bmod] (b NULL: alpha * a); out may alias
 * a. */
void ops_axpby(struct ops *o, cl_mem out, cl_mem a, float alpha, cl_mem b,
               float beta, long n, long bmod);

/* Fold an eval-mode BatchNorm into the preceding convolution's weights w
 * (K x per) and bias b (K floats, in: the convolution's bias or zeros),
 * in double precision on the host. ops.h:162-164. */
void ops_fold_bn(float *w, float *b, int K, long per, const float *gamma,
                 const float *beta, const float *mean, const float *var,
                 float eps);

#ifdef __cplusplus
}
#endif

#endif /* ICOREG_OPS_H */

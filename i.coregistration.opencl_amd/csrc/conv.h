/* SPDX-License-Identifier: Unlicense */

/* The fast paths of ops_conv2d on the fp32 matrix cores: Winograd
 * F(2 x 2, 3 x 3) for same-size 3 x 3 convolutions, and the direct k x k
 * convolution (LDS input patches) for one group, dilation 1, k = 3 or 5,
 * stride 1 or 2. */

#ifndef ICOREG_CONV_H
#define ICOREG_CONV_H

#include <hip/hip_runtime.h>

#include "ops.h"

struct conv_args {
    const float *in;  /* (nb, C, H, W) with image stride in_stride */
    const float *w;   /* (K, C, ks, ks) */
    const float *bias; /* K or NULL */
    float *out;       /* (nb, K, Ho, Wo) with image stride out_stride */
    long long in_stride, out_stride;
    int C, H, W, K, Ho, Wo, pad;
    const float *mean, *rstd, *gate; /* optional input normalisation */
    int act;
    float slope;
    /* Direct kernel only: split > 1 cuts the input channels into split
     * pieces (grid z = piece + split * image) whose partial sums go to
     * part (split x nb x K x Ho x Wo floats), added by a second pass. */
    int split;
    float *part;
};

/* True if the direct kernel handles this geometry. */
bool conv_direct_supported(int kh, int kw, int sy, int sx, int dy, int dx,
                           int groups);

/* True if the tensors are small enough for the kernel's 32-bit buffer
 * offsets (per-image input and the weights below 2 GiB). */
bool conv_direct_fits(long long in_floats, long long w_floats);

/* Bytes of the partial sums conv_direct_launch needs for a (0: none);
 * the caller passes that much memory as a.part. */
size_t conv_direct_part_bytes(const conv_args &a, int ks, int stride, int nb, int cus);

void conv_direct_launch(const conv_args &a, int ks, int stride, int nb,
                        int cus, hipStream_t s);

/* Winograd F(2 x 2, 3 x 3) path (conv_wino.hip): 3 x 3, stride 1,
 * padding 1, one group, K % 4 == 0, at least 32 channels in and out, an
 * Ho x Wo output of at most 65535 blocks of 8 x 16 pixels. */
bool conv_wino_supported(int kh, int kw, int sy, int sx, int py, int px,
                         int dy, int dx, int groups, int C, int K, int Ho,
                         int Wo);
/* Floats of the transformed filters U for a convolution with (norm) or
 * without input normalisation: MFMA fragment order when C % 8 == 0 and no
 * normalisation, else [16][C][K]. */
size_t conv_wino_weight_floats(int K, int C, bool norm);
/* U from w (K, C, 3, 3), in the order conv_wino_weight_floats names. */
void conv_wino_weights(const float *w, int K, int C, bool norm, float *U, hipStream_t s);
/* Work split of the row-split Winograd kernel. A unit is one block's
 * output: 32 channels (nkb channel blocks) x 32 tiles (ntb tile blocks) of
 * one image. Units 0..nfull-1 run whole; each later unit is cut into
 * split pieces over its input channels, which write partial sums to part
 * (split x 4096 floats per unit), added up by a second kernel. */
struct wino_split {
    int nkb, ntb, nfull, split;
    /* Units are ordered (channel group, image, tile block, channel block
     * of the group); whole units go to the XCDs in contiguous bands of
     * that order, so an XCD holds the filters of kgroups-th of the
     * channel blocks and the inputs of its own tiles. */
    int kgroups, nb;
    float *part;
};

/* The split for nb images on cus CUs: the units left over after an equal
 * whole number per CU are cut so that every CU gets about one piece. */
wino_split conv_wino_plan(const conv_args &a, int nb, int cus);
/* Floats of part that the plan needs (0 without split). */
size_t conv_wino_part_floats(const conv_args &a, int nb, const wino_split &sp);

/* The convolution of a (a.w unused) with filters U from conv_wino_weights
 * with norm = (a.mean != NULL), nb images, split sp (conv_wino_plan, part
 * set). */
void conv_wino_launch(const conv_args &a, const float *U, int nb, const wino_split &sp,
                      hipStream_t s);

/* Winograd F(4 x 4, 3 x 3) path (conv_wino4.hip): the F(2 x 2) path's
 * shapes with C % 4 == 0, K >= 16 and no input normalisation. Filters in
 * the kernel's operand order, conv_wino4_weight_floats(K, C) floats. */
bool conv_wino4_ok(int C, int K, bool norm);
size_t conv_wino4_weight_floats(int K, int C);
void conv_wino4_weights(const float *w, int K, int C, float *U, hipStream_t s);
/* Blocks of a launch: 32 output channels x 32 tiles of 4 x 4 pixels. */
long long conv_wino4_units(int K, int Ho, int Wo, int nb);
void conv_wino4_launch(const conv_args &a, const float *U, int nb, hipStream_t s);

/* Filters of a 3 x 3 convolution without input normalisation transformed
 * once (a new buffer), for callers that run the same weights many times:
 * the F(2 x 2) form, followed, where conv_wino4_ok, by the F(4 x 4) form
 * at float offset conv_wino4_offset(K, C). */
cl_mem conv_wino_prepare(struct ops *o, cl_mem w, int K, int C);
size_t conv_wino4_offset(int K, int C);
/* ops_conv2d_batch for 3 x 3, stride 1, padding 1, one group, with U
 * from conv_wino_prepare (w is used only when the Winograd path does not
 * take the shape). */
void conv3x3_wino_batch(struct ops *o, int nb, cl_mem in, long in_stride,
                        int C, int H, int W, cl_mem w, cl_mem U, cl_mem b,
                        int K, int act, float slope, cl_mem out,
                        long out_stride);

#endif /* ICOREG_CONV_H */

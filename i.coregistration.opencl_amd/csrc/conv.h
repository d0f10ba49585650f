/* SPDX-License-Identifier: Unlicense */

/* Direct k x k convolution on the fp32 matrix cores (LDS input patches):
 * the fast path of ops_conv2d for one group, dilation 1, k = 3 or 5,
 * stride 1 or 2. */

#ifndef ICOREG_CONV_H
#define ICOREG_CONV_H

#include <hip/hip_runtime.h>

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
};

/* True if the direct kernel handles this geometry. */
bool conv_direct_supported(int kh, int kw, int sy, int sx, int dy, int dx,
                           int groups);

/* True if the tensors are small enough for the kernel's 32-bit buffer
 * offsets (per-image input and the weights below 2 GiB). */
bool conv_direct_fits(long long in_floats, long long w_floats);

void conv_direct_launch(const conv_args &a, int ks, int stride, int nb,
                        int cus, hipStream_t s);

#endif /* ICOREG_CONV_H */

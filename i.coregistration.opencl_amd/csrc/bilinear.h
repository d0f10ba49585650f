/* SPDX-License-Identifier: Unlicense */

/* The bilinear arithmetic of ops_resize (ops.cl:718-760 of
 * i.coregistration.opencl: source coordinate, clamped taps, weights),
 * shared by every kernel that reads a resized map, so that a value
 * sampled on the fly is bit for bit the value the resize kernel stores. */

#ifndef ICOREG_BILINEAR_H
#define ICOREG_BILINEAR_H

#include <hip/hip_runtime.h>

/* Taps i0, i1 of source length n and weight f of i1 for output index o of
 * an output of length N: align_corners maps the end points onto each
 * other, otherwise pixel centres with scale s (source / output). */
static __device__ __forceinline__ void bl_taps(int o, int N, int n, int align, float s,
                                               int &i0, int &i1, float &f)
{
    float u;

    if (align)
        u = N > 1 ? (float)o * (float)(n - 1) / (float)(N - 1) : 0.0f;
    else
        u = fmaxf(((float)o + 0.5f) * s - 0.5f, 0.0f);
    i0 = min((int)u, n - 1);
    i1 = min(i0 + 1, n - 1);
    f = u - i0;
}

/* Interpolated value from source rows r0 (row y0) and r1 (row y1). The
 * order of the operations is fixed (explicit fma), so every caller rounds
 * alike. */
static __device__ __forceinline__ float bl_mix(const float *r0, const float *r1, int x0, int x1,
                                               float fx, float fy)
{
    const float top = fmaf(fx, r0[x1], (1.0f - fx) * r0[x0]);
    const float bot = fmaf(fx, r1[x1], (1.0f - fx) * r1[x0]);

    return fmaf(fy, bot, (1.0f - fy) * top);
}

/* Value at output (y, x) of a resize with pixel centres and source step
 * s (1 / scale) of plane p (h x w). */
static __device__ __forceinline__ float bl_up(const float *p, int h, int w, float s, int y,
                                              int x)
{
    int y0, y1, x0, x1;
    float fy, fx;

    bl_taps(y, 0, h, 0, s, y0, y1, fy);
    bl_taps(x, 0, w, 0, s, x0, x1, fx);
    return bl_mix(p + (long long)y0 * w, p + (long long)y1 * w, x0, x1, fx, fy);
}

/* The 2x resize (scale 2, source step 1 / 2). */
static __device__ __forceinline__ float bl_up2(const float *p, int h, int w, int y, int x)
{
    return bl_up(p, h, w, 0.5f, y, x);
}

#endif /* ICOREG_BILINEAR_H */

/* SPDX-License-Identifier: Unlicense */

/* DISK's own kernels on gfx950: the 5 x 5 non-maxima suppression of the
 * heatmap and the descriptor gather. Contracts of disk_kernels.cl:8-60
 * (i.coregistration.opencl).
 *
 *  - NMS: 32 x 8 output cells per block, the (12 x 36) heat patch staged
 *    in LDS once, so each heat value is read from HBM about 1.6 times
 *    instead of 25;
 *  - gather: one wave64 per keypoint, lanes over the descriptor
 *    channels, the squared norm by a cross-lane reduction, coalesced
 *    descriptor rows. */

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdlib.h>

#include "common.h"
#include "icoreg_kernels.h"
#include "reduce.h"

using namespace icoreg;

#define NMS_TX 32
#define NMS_TY 8

__global__ void __launch_bounds__(256)
    nms5x5_kernel(const float *__restrict__ heat, int W, int h, int w,
                  float thresh, unsigned char *__restrict__ mask)
{
    __shared__ float t[NMS_TY + 4][NMS_TX + 5];
    const int lx = threadIdx.x & (NMS_TX - 1), ly = threadIdx.x / NMS_TX;
    const int x0 = blockIdx.x * NMS_TX, y0 = blockIdx.y * NMS_TY;
    const int x = x0 + lx, y = y0 + ly;

    for (int e = threadIdx.x; e < (NMS_TY + 4) * (NMS_TX + 4); e += 256) {
        const int yy = y0 - 2 + e / (NMS_TX + 4), xx = x0 - 2 + e % (NMS_TX + 4);

        t[e / (NMS_TX + 4)][e % (NMS_TX + 4)] =
            yy >= 0 && yy < h && xx >= 0 && xx < w
                ? heat[(long long)yy * W + xx]
                : -INFINITY;
    }
    __syncthreads();
    if (x >= w || y >= h)
        return;
    if (x < 2 || y < 2 || x >= w - 2 || y >= h - 2) {
        mask[(long long)y * w + x] = 0;
        return;
    }
    {
        const float v = t[ly + 2][lx + 2];
        bool keep = v > thresh;

#pragma unroll
        for (int dy = 0; dy < 5; dy++)
#pragma unroll
            for (int dx = 0; dx < 5; dx++)
                if (dy != 2 || dx != 2)
                    keep = keep && v > t[ly + dy][lx + dx];
        mask[(long long)y * w + x] = keep ? 1 : 0;
    }
}

__global__ void __launch_bounds__(256)
    gather_desc_kernel(const float *__restrict__ feat, long long plane,
                       int D, const int *__restrict__ xy, int n, int W,
                       float *__restrict__ desc)
{
    const int lane = threadIdx.x & 63;
    const int k = blockIdx.x * 4 + (threadIdx.x >> 6);
    long long off;
    float ss = 0.0f, inv;

    if (k >= n)
        return;
    off = (long long)xy[2 * k + 1] * W + xy[2 * k];
    for (int d = lane; d < D; d += 64) {
        const float v = feat[d * plane + off];

        ss = fmaf(v, v, ss);
    }
    ss = wave_sum(ss);
    inv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
    for (int d = lane; d < D; d += 64)
        desc[(long long)k * D + d] = feat[d * plane + off] * inv;
}

extern "C" void disk_nms5x5(struct ops *o, cl_mem heat, long off, int W, int h,
                            int w, float thresh, cl_mem mask)
{
    ICOREG_API_BEGIN
    const char *op = "disk_nms5x5";

    if (h < 0 || w < 0 || W < w || off < 0)
        icoreg_fatal("%s: invalid crop %d x %d of width %d", op, h, w, W);
    if ((long long)h * w == 0)
        return;
    need_floats(heat, off, (long long)(h - 1) * W + w, op, "heat");
    need_bytes(mask, 0, (long long)h * w, op, "mask");
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(nms5x5_kernel,
                       dim3((unsigned)((w + NMS_TX - 1) / NMS_TX),
                            (unsigned)((h + NMS_TY - 1) / NMS_TY)),
                       dim3(256), 0, stream_of(o->ocl), cfptr(heat) + off, W, h,
                       w, thresh, (unsigned char *)mask->ptr);
    launch_check(op);
    ICOREG_API_END
}

extern "C" void disk_gather_desc(struct ops *o, cl_mem feat, int H, int W,
                                 int D, cl_mem xy, int n, cl_mem desc)
{
    ICOREG_API_BEGIN
    const char *op = "disk_gather_desc";
    const long long plane = (long long)H * W;

    if (H < 1 || W < 1 || D < 1 || n < 0)
        icoreg_fatal("%s: invalid sizes H=%d W=%d D=%d n=%d", op, H, W, D, n);
    if (n == 0)
        return;
    need_floats(feat, 0, (long long)D * plane, op, "feat");
    need_bytes(xy, 0, 8LL * n, op, "xy");
    need_floats(desc, 0, (long long)n * D, op, "desc");
    {
        /* Keypoint coordinates are host data the caller uploaded: check
         * them before they index the feature planes. */
        int *h_xy = (int *)malloc(8 * (size_t)n);

        ocl_read(o->ocl, xy, 0, h_xy, 8 * (size_t)n);
        for (int k = 0; k < n; k++)
            if (h_xy[2 * k] < 0 || h_xy[2 * k] >= W || h_xy[2 * k + 1] < 0 ||
                h_xy[2 * k + 1] >= H) {
                const int x = h_xy[2 * k], y = h_xy[2 * k + 1];

                free(h_xy);
                icoreg_fatal("%s: keypoint %d at (%d, %d) outside %d x %d", op,
                             k, x, y, W, H);
            }
        free(h_xy);
    }
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(gather_desc_kernel, dim3((unsigned)((n + 3) / 4)),
                       dim3(256), 0, stream_of(o->ocl), cfptr(feat), plane, D,
                       (const int *)xy->ptr, n, W, fptr(desc));
    launch_check(op);
    ICOREG_API_END
}

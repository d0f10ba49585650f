/* SPDX-License-Identifier: Unlicense */

/* RoMa's input preparation and result epilogue on gfx950, the host steps
 * of roma.c:1106-1186 (Pillow-style antialiased bicubic resampling and
 * ImageNet normalisation) and roma.c:1328-1349,1413-1429 (certainty
 * sigmoid and bounds, v2's standard deviation). The images cross the bus
 * once per match, unresized; only the warp and certainty come back.
 *
 *  - prep_taps_kernel: per output index of one axis, the first input
 *    index, the tap count and the normalised weights of the filter
 *    (Keys' cubic with a = -0.5, support scaled by the reduction), in
 *    double with contraction off, so they are the host formula's to the
 *    bit; stored tap-major so that neighbouring outputs read adjacent
 *    words.
 *  - prep_rows_kernel / prep_cols_kernel: the separable passes, width
 *    first, each sum in double in tap order and rounded to float once
 *    (as the host does); the column pass applies the normalisation.
 *  - prep_copy_kernel: same-size pass (the fine pass), normalisation
 *    only.
 *  - epilogue and sd kernels: one thread per cell. */

#include <hip/hip_runtime.h>

#include <math.h>

#include "common.h"
#include "icoreg_kernels.h"

using namespace icoreg;

#define PREP_KMAX 64 /* taps per output: reductions up to 15.5x */

__constant__ float prep_mean[3] = {0.485f, 0.456f, 0.406f};
__constant__ float prep_std[3] = {0.229f, 0.224f, 0.225f};

/* Keys' cubic convolution kernel, a = -0.5 (Pillow's bicubic). */
__device__ double keys_cubic(double x)
{
#pragma clang fp contract(off)
    const double a = -0.5;

    x = fabs(x);
    if (x < 1)
        return ((a + 2) * x - (a + 3)) * x * x + 1;
    if (x < 2)
        return (((x - 5) * x + 8) * x - 4) * a;
    return 0;
}

__global__ void __launch_bounds__(256)
    prep_taps_kernel(int n_in, int n_out, int *__restrict__ lo, int *__restrict__ cnt,
                     double *__restrict__ k)
{
#pragma clang fp contract(off)
    const int o = blockIdx.x * 256 + threadIdx.x;

    if (o >= n_out)
        return;
    const double scale = (double)n_in / n_out, fs = scale > 1 ? scale : 1;
    const double support = 2 * fs, center = (o + 0.5) * scale;
    int first = (int)(center - support + 0.5), last = (int)(center + support + 0.5);
    double sum = 0;

    if (first < 0)
        first = 0;
    if (last > n_in)
        last = n_in;
    const int n = min(last - first, PREP_KMAX);
    for (int t = 0; t < n; t++)
        sum += keys_cubic((t + first - center + 0.5) / fs);
    for (int t = 0; t < n; t++)
        k[(long long)t * n_out + o] =
            sum != 0 ? keys_cubic((t + first - center + 0.5) / fs) / sum : 0;
    lo[o] = first;
    cnt[o] = n;
}

/* in (planes, H, W) -> tmp (planes, H, w). */
__global__ void __launch_bounds__(256)
    prep_rows_kernel(const float *__restrict__ in, int H, int W, int w,
                     const int *__restrict__ lo, const int *__restrict__ cnt,
                     const double *__restrict__ k, float *__restrict__ tmp)
{
#pragma clang fp contract(off)
    const int o = blockIdx.x * 256 + threadIdx.x, y = blockIdx.y, pl = blockIdx.z;

    if (o >= w)
        return;
    const float *src = in + ((long long)pl * H + y) * W + lo[o];
    const int n = cnt[o];
    double s = 0;

    for (int t = 0; t < n; t++)
        s += k[(long long)t * w + o] * (double)src[t];
    tmp[((long long)pl * H + y) * w + o] = (float)s;
}

/* tmp (planes, H, w) -> out (planes, h, w), normalised per channel
 * (plane % 3) when imagenet is set. */
__global__ void __launch_bounds__(256)
    prep_cols_kernel(const float *__restrict__ tmp, int H, int w, int h,
                     const int *__restrict__ lo, const int *__restrict__ cnt,
                     const double *__restrict__ k, int imagenet, float *__restrict__ out)
{
#pragma clang fp contract(off)
    const int x = blockIdx.x * 256 + threadIdx.x, oy = blockIdx.y, pl = blockIdx.z;

    if (x >= w)
        return;
    const float *src = tmp + ((long long)pl * H + lo[oy]) * w + x;
    const int n = cnt[oy];
    double s = 0;
    float v;

    for (int t = 0; t < n; t++)
        s += k[(long long)t * h + oy] * (double)src[(long long)t * w];
    v = (float)s;
    if (imagenet)
        v = (v - prep_mean[pl % 3]) / prep_std[pl % 3];
    out[((long long)pl * h + oy) * w + x] = v;
}

__global__ void __launch_bounds__(256)
    prep_copy_kernel(const float *__restrict__ in, long long plane, int imagenet,
                     float *__restrict__ out)
{
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    const int pl = blockIdx.y;
    float v;

    if (i >= plane)
        return;
    v = in[pl * plane + i];
    if (imagenet)
        v = (v - prep_mean[pl % 3]) / prep_std[pl % 3];
    out[pl * plane + i] = v;
}

__global__ void __launch_bounds__(256)
    epilogue_kernel(float *__restrict__ flow, float *__restrict__ cert,
                    const float *__restrict__ low, long long hw)
{
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;

    if (i >= hw)
        return;
    const float fx = flow[i], fy = flow[hw + i];
    float c = cert[i];

    if (low && low[i] < 0)
        c = c - 0.5f * low[i];
    c = 1.0f / (1.0f + expf(-c));
    if (fabsf(fx) > 1 || fabsf(fy) > 1)
        c = 0;
    flow[i] = fx < -1 ? -1.0f : fx > 1 ? 1.0f : fx;
    flow[hw + i] = fy < -1 ? -1.0f : fy > 1 ? 1.0f : fy;
    cert[i] = c;
}

__global__ void __launch_bounds__(256)
    sd_kernel(const float *__restrict__ prec, float *__restrict__ sd, long long hw)
{
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;

    if (i >= hw)
        return;
    const double det = (double)prec[i] * prec[2 * hw + i] - (double)prec[hw + i] * prec[hw + i];

    sd[i] = det > 0 ? (float)pow(det, -0.25) : NAN;
}

static size_t round256(size_t b) { return (b + 255) / 256 * 256; }

extern "C" void roma_prepare(struct ops *o, cl_mem in, int nimg, int H, int W, cl_mem out,
                             int h, int w, int imagenet)
{
    ICOREG_API_BEGIN
    const char *op = "roma_prepare";
    hipStream_t st = stream_of(o->ocl);
    const int planes = 3 * nimg;

    if (nimg <= 0 || H <= 0 || W <= 0 || h <= 0 || w <= 0)
        icoreg_fatal("%s: invalid sizes nimg=%d %dx%d -> %dx%d", op, nimg, H, W, h, w);
    if ((double)W / w > 15.5 || (double)H / h > 15.5)
        icoreg_fatal("%s: %dx%d -> %dx%d reduces more than 15.5 times", op, H, W, h, w);
    if (planes > 65535 || h > 65535 || H > 65535)
        icoreg_fatal("%s: sizes beyond the grid", op);
    count32((long long)planes * H * W, op);
    count32((long long)planes * h * w, op);
    need_floats(in, 0, (long long)planes * H * W, op, "in");
    need_floats(out, 0, (long long)planes * h * w, op, "out");
    prof_scope ps(o->ocl, op);
    if (H == h && W == w) {
        const long long plane = (long long)h * w;

        hipLaunchKernelGGL(prep_copy_kernel, dim3((unsigned)((plane + 255) / 256), planes),
                           dim3(256), 0, st, cfptr(in), plane, imagenet, fptr(out));
    }
    else {
        const size_t tmp_b = round256((size_t)planes * H * w * 4);
        const size_t kx_b = round256((size_t)PREP_KMAX * w * 8);
        const size_t ky_b = round256((size_t)PREP_KMAX * h * 8);
        const size_t ix_b = round256((size_t)2 * w * 4);
        cl_mem sc = scratch_get(o, tmp_b + kx_b + ky_b + ix_b + round256((size_t)2 * h * 4));
        char *base = (char *)sc->ptr;
        float *tmp = (float *)base;
        double *kx = (double *)(base + tmp_b), *ky = (double *)(base + tmp_b + kx_b);
        int *ix = (int *)(base + tmp_b + kx_b + ky_b), *iy = (int *)(base + tmp_b + kx_b + ky_b + ix_b);

        hipLaunchKernelGGL(prep_taps_kernel, dim3((unsigned)((w + 255) / 256)), dim3(256), 0, st,
                           W, w, ix, ix + w, kx);
        hipLaunchKernelGGL(prep_taps_kernel, dim3((unsigned)((h + 255) / 256)), dim3(256), 0, st,
                           H, h, iy, iy + h, ky);
        hipLaunchKernelGGL(prep_rows_kernel, dim3((unsigned)((w + 255) / 256), H, planes),
                           dim3(256), 0, st, cfptr(in), H, W, w, (const int *)ix,
                           (const int *)(ix + w), (const double *)kx, tmp);
        hipLaunchKernelGGL(prep_cols_kernel, dim3((unsigned)((w + 255) / 256), h, planes),
                           dim3(256), 0, st, (const float *)tmp, H, w, h, (const int *)iy,
                           (const int *)(iy + h), (const double *)ky, imagenet, fptr(out));
    }
    launch_check(op);
    ICOREG_API_END
}

extern "C" void roma_epilogue(struct ops *o, cl_mem flow, cl_mem cert, cl_mem low, long hw)
{
    ICOREG_API_BEGIN
    const char *op = "roma_epilogue";

    if (hw < 0)
        icoreg_fatal("%s: invalid size %ld", op, hw);
    if (hw == 0)
        return;
    need_floats(flow, 0, 2LL * hw, op, "flow");
    need_floats(cert, 0, hw, op, "cert");
    if (low)
        need_floats(low, 0, hw, op, "low");
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(epilogue_kernel, dim3((unsigned)((hw + 255) / 256)), dim3(256), 0,
                       stream_of(o->ocl), fptr(flow), fptr(cert), cfptr(low), (long long)hw);
    launch_check(op);
    ICOREG_API_END
}

extern "C" void roma_sd(struct ops *o, cl_mem prec, long poff, cl_mem sd, long hw)
{
    ICOREG_API_BEGIN
    const char *op = "roma_sd";

    if (hw < 0 || poff < 0)
        icoreg_fatal("%s: invalid size %ld", op, hw);
    if (hw == 0)
        return;
    need_floats(prec, poff, 3LL * hw, op, "prec");
    need_floats(sd, 0, hw, op, "sd");
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(sd_kernel, dim3((unsigned)((hw + 255) / 256)), dim3(256), 0,
                       stream_of(o->ocl), cfptr(prec) + poff, fptr(sd), (long long)hw);
    launch_check(op);
    ICOREG_API_END
}

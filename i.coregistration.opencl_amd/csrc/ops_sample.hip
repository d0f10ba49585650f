/* SPDX-License-Identifier: Unlicense */

/* Resampling and pooling: bilinear resize into a channel offset,
 * grid_sample (bilinear, zero padding), unfold, 2 x 2 average pooling
 * and k x k max / average pooling. Contracts of the reference's
 * ops.cl:718-860 with the host checks of ops.c:496-578
 * (i.coregistration.opencl); one thread per output value, consecutive
 * threads along the output row so that stores are coalesced. */

#include <hip/hip_runtime.h>

#include <math.h>

#include "bilinear.h"
#include "common.h"
#include "ops.h"

using namespace icoreg;

/* ---- bilinear resize --------------------------------------------------- */

/* Four consecutive outputs of one row per thread: the row's source rows
 * and weight are found once for the four, and with W % 4 == 0 (and an
 * aligned output) the four go out as one 16-byte store. */
__global__ void __launch_bounds__(256)
    resize_kernel(const float *__restrict__ in, int h, int w,
                  float *__restrict__ out, int H, int W, int coff, int align,
                  float sy, float sx, int C, int X4, int vec)
{
    const long long item = (long long)blockIdx.x * 256 + threadIdx.x;
    int it, x4, row, y, c, y0, y1;
    float fy, v[4];
    const float *r0, *r1;
    float *o;

    if (item >= (long long)C * H * X4)
        return;
    it = (int)item;
    row = it / X4;
    x4 = it - row * X4;
    c = row / H;
    y = row - c * H;
    bl_taps(y, H, h, align, sy, y0, y1, fy);
    r0 = in + ((long long)c * h + y0) * w;
    r1 = in + ((long long)c * h + y1) * w;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int x = min(4 * x4 + k, W - 1);
        float fx;
        int x0, x1;

        bl_taps(x, W, w, align, sx, x0, x1, fx);
        v[k] = bl_mix(r0, r1, x0, x1, fx, fy);
    }
    o = out + ((long long)(c + coff) * H + y) * W + 4 * x4;
    if (vec) {
        *(float4 *)o = make_float4(v[0], v[1], v[2], v[3]);
        return;
    }
#pragma unroll
    for (int k = 0; k < 4; k++)
        if (4 * x4 + k < W)
            o[k] = v[k];
}

extern "C" void ops_resize(struct ops *o, cl_mem in, int C, int h, int w,
                           cl_mem out, int H, int W, int coff,
                           int align_corners, float scale)
{
    ICOREG_API_BEGIN
    const char *op = "ops_resize";
    float sy = scale > 0 ? 1.0f / scale : (float)h / H;
    float sx = scale > 0 ? 1.0f / scale : (float)w / W;
    long long total = (long long)C * H * W;

    if (C < 0 || h < 1 || w < 1 || H < 1 || W < 1 || coff < 0)
        icoreg_fatal("%s: invalid sizes C=%d %dx%d -> %dx%d coff=%d", op, C, h,
                     w, H, W, coff);
    if (total == 0)
        return;
    count32((long long)(C + coff) * H * W, "resize output");
    need_floats(in, 0, (long long)C * h * w, op, "in");
    need_floats(out, (long long)coff * H * W, total, op, "out");
    {
        const int X4 = (W + 3) / 4;
        const long long items = (long long)C * H * X4;
        const int vec = W % 4 == 0 && ((uintptr_t)fptr(out) & 15) == 0;

        prof_scope ps(o->ocl, "resize_bilinear");
        hipLaunchKernelGGL(resize_kernel,
                           dim3((unsigned)((items + 255) / 256)), dim3(256),
                           0, stream_of(o->ocl), cfptr(in), h, w, fptr(out),
                           H, W, coff, align_corners, sy, sx, C, X4, vec);
    }
    launch_check("resize_bilinear");
    ICOREG_API_END
}

/* ---- grid_sample -------------------------------------------------------- */

/* One thread per (point, group of CG channels): the point's taps and
 * weights are computed once for its group, the group's planes read at
 * the same offsets with all loads in flight together, and each channel's
 * stores are 256 consecutive points, non-temporal (written once, read by
 * the next kernel). A block takes 256 points of one channel group, so
 * that a few thousand points still fill the GPU; CG is 8, or 4 when that
 * leaves fewer idle channel slots. */
template <int CG>
__global__ void __launch_bounds__(256)
    grid_sample_kernel(const float *__restrict__ in, int C, int H, int W,
                       const float2 *__restrict__ grid, int n, int align,
                       float *__restrict__ out)
{
    /* Block L -> (channel group, point block), point blocks fastest, in
     * contiguous bands per XCD (L % 8): neighbouring point blocks of a
     * smooth grid share input rows, fetched once into that XCD's L2. */
    const int npb = (n + 255) / 256, total = gridDim.x;
    const int q = total >> 3, rem = total & 7, xc = blockIdx.x & 7, idx = blockIdx.x >> 3;
    const int ord = (xc < rem ? xc * (q + 1) : rem * (q + 1) + (xc - rem) * q) + idx;
    const int i = (ord % npb) * 256 + threadIdx.x, c0 = (ord / npb) * CG;
    const long long plane = (long long)H * W;
    float2 g;
    float ix, iy, fx = 0.0f, fy = 0.0f, v[CG][4];
    int x0 = 0, y0 = 0, o[4] = {0, 0, 0, 0};
    bool ok, in4[4];

    if (i >= n)
        return;
    g = grid[i];
    if (align) {
        ix = (g.x + 1.0f) * 0.5f * (W - 1);
        iy = (g.y + 1.0f) * 0.5f * (H - 1);
    }
    else {
        ix = ((g.x + 1.0f) * W - 1.0f) * 0.5f;
        iy = ((g.y + 1.0f) * H - 1.0f) * 0.5f;
    }
    /* Coordinates far outside are clamped first (all four taps stay
     * outside, so the value is still 0), which keeps the integer
     * conversion defined; non-finite ones give 0. */
    ok = isfinite(ix) && isfinite(iy);
    if (ok) {
        ix = fminf(fmaxf(ix, -2.0f), (float)W + 1.0f);
        iy = fminf(fmaxf(iy, -2.0f), (float)H + 1.0f);
        x0 = (int)floorf(ix);
        y0 = (int)floorf(iy);
        fx = ix - x0;
        fy = iy - y0;
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int xx = x0 + (q & 1), yy = y0 + (q >> 1);

        in4[q] = ok && xx >= 0 && xx < W && yy >= 0 && yy < H;
        o[q] = in4[q] ? yy * W + xx : 0;
    }
#pragma unroll
    for (int k = 0; k < CG; k++) {
        const float *p = in + (long long)min(c0 + k, C - 1) * plane;

#pragma unroll
        for (int q = 0; q < 4; q++)
            v[k][q] = in4[q] ? p[o[q]] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < CG; k++)
        if (c0 + k < C)
            __builtin_nontemporal_store(
                ok ? (1.0f - fy) * ((1.0f - fx) * v[k][0] + fx * v[k][1]) +
                         fy * ((1.0f - fx) * v[k][2] + fx * v[k][3])
                   : 0.0f,
                &out[(long long)(c0 + k) * n + i]);
}

extern "C" void ops_grid_sample(struct ops *o, cl_mem in, int C, int H, int W,
                                cl_mem grid, int n, int align_corners,
                                cl_mem out)
{
    ICOREG_API_BEGIN
    const char *op = "ops_grid_sample";

    if (C < 0 || H < 1 || W < 1 || n < 0)
        icoreg_fatal("%s: invalid sizes C=%d H=%d W=%d n=%d", op, C, H, W, n);
    if (C == 0 || n == 0)
        return;
    count32((long long)C * H * W, "grid_sample input");
    count32((long long)C * n, "grid_sample output");
    need_floats(in, 0, (long long)C * H * W, op, "in");
    need_floats(grid, 0, 2LL * n, op, "grid");
    need_floats(out, 0, (long long)C * n, op, "out");
    prof_scope ps(o->ocl, "grid_sample");
    {
        const int cg = sample_cg(C);
        const long long blocks = (long long)((n + 255) / 256) * ((C + cg - 1) / cg);

        if (blocks >= (1LL << 31))
            icoreg_fatal("%s: grid too large", op);
        if (cg == 4)
            hipLaunchKernelGGL(grid_sample_kernel<4>, dim3((unsigned)blocks), dim3(256), 0,
                               stream_of(o->ocl), cfptr(in), C, H, W,
                               (const float2 *)cfptr(grid), n, align_corners, fptr(out));
        else
            hipLaunchKernelGGL(grid_sample_kernel<8>, dim3((unsigned)blocks), dim3(256), 0,
                               stream_of(o->ocl), cfptr(in), C, H, W,
                               (const float2 *)cfptr(grid), n, align_corners, fptr(out));
    }
    launch_check("grid_sample");
    ICOREG_API_END
}

/* ---- unfold ----------------------------------------------------------------- */

__global__ void __launch_bounds__(256)
    unfold_kernel(const float *__restrict__ in, int C, int H, int W, int kh,
                  int kw, int sy, int sx, int py, int px, int Ho, int Wo,
                  float *__restrict__ out)
{
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long L = (long long)Ho * Wo, total = (long long)C * kh * kw * L;
    int row, c, i, j, iy, ix;
    long long t;

    if (idx >= total)
        return;
    t = idx % L;
    row = (int)(idx / L);
    c = row / (kh * kw);
    i = (row / kw) % kh;
    j = row % kw;
    iy = (int)(t / Wo) * sy - py + i;
    ix = (int)(t % Wo) * sx - px + j;
    out[idx] = iy >= 0 && iy < H && ix >= 0 && ix < W
                   ? in[((long long)c * H + iy) * W + ix]
                   : 0.0f;
}

extern "C" void ops_unfold(struct ops *o, cl_mem in, int C, int H, int W,
                           const struct conv_geom *g, cl_mem out)
{
    ICOREG_API_BEGIN
    const char *op = "ops_unfold";
    int Ho = ops_conv_out(H, g->kh, g->sy, g->py, 1);
    int Wo = ops_conv_out(W, g->kw, g->sx, g->px, 1);
    long long total = (long long)C * g->kh * g->kw * Ho * Wo;

    if (Ho < 1 || Wo < 1 || C < 1)
        icoreg_fatal("%s: empty output", op);
    count32(total, "unfold output");
    need_floats(in, 0, (long long)C * H * W, op, "in");
    need_floats(out, 0, total, op, "out");
    prof_scope ps(o->ocl, "unfold");
    hipLaunchKernelGGL(unfold_kernel, dim3((unsigned)((total + 255) / 256)),
                       dim3(256), 0, stream_of(o->ocl), cfptr(in), C, H, W,
                       g->kh, g->kw, g->sy, g->sx, g->py, g->px, Ho, Wo,
                       fptr(out));
    launch_check("unfold");
    ICOREG_API_END
}

/* ---- pooling ------------------------------------------------------------- */

__global__ void __launch_bounds__(256)
    avgpool2_kernel(const float *__restrict__ in, int H, int W, int C,
                    float *__restrict__ out)
{
    const int w = W / 2, h = H / 2;
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long total = (long long)C * h * w;
    int x, y, c;
    const float *p;

    if (idx >= total)
        return;
    x = (int)(idx % w);
    y = (int)((idx / w) % h);
    c = (int)(idx / ((long long)w * h));
    p = in + ((long long)c * H + 2 * y) * W + 2 * x;
    out[idx] = 0.25f * (p[0] + p[1] + p[W] + p[W + 1]);
}

extern "C" void ops_avgpool2(struct ops *o, cl_mem in, int C, int H, int W,
                             cl_mem out)
{
    ICOREG_API_BEGIN
    const char *op = "ops_avgpool2";
    long long total = (long long)C * (H / 2) * (W / 2);

    if (C < 0 || H < 2 || W < 2)
        icoreg_fatal("%s: invalid sizes C=%d H=%d W=%d", op, C, H, W);
    if (total == 0)
        return;
    count32((long long)C * H * W, "avgpool2 input");
    need_floats(in, 0, (long long)C * H * W, op, "in");
    need_floats(out, 0, total, op, "out");
    prof_scope ps(o->ocl, "avgpool2");
    hipLaunchKernelGGL(avgpool2_kernel, dim3((unsigned)((total + 255) / 256)),
                       dim3(256), 0, stream_of(o->ocl), cfptr(in), H, W, C,
                       fptr(out));
    launch_check("avgpool2");
    ICOREG_API_END
}

__global__ void __launch_bounds__(256)
    pool2d_kernel(const float *__restrict__ in, int H, int W, int Ho, int Wo,
                  int k, int s, int pad, int ismax, int C,
                  float *__restrict__ out)
{
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long total = (long long)C * Ho * Wo;
    int x, y, c;
    const float *p;
    float acc;

    if (idx >= total)
        return;
    x = (int)(idx % Wo);
    y = (int)((idx / Wo) % Ho);
    c = (int)(idx / ((long long)Wo * Ho));
    p = in + (long long)c * H * W;
    acc = ismax ? -INFINITY : 0.0f;
    for (int i = 0; i < k; i++) {
        const int iy = y * s - pad + i;

        if (iy < 0 || iy >= H)
            continue;
        for (int j = 0; j < k; j++) {
            const int ix = x * s - pad + j;

            if (ix < 0 || ix >= W)
                continue;
            acc = ismax ? fmaxf(acc, p[iy * W + ix]) : acc + p[iy * W + ix];
        }
    }
    out[idx] = ismax ? acc : acc / (k * k);
}

extern "C" void ops_pool2d(struct ops *o, cl_mem in, int C, int H, int W,
                           int ks, int s, int p, int max, cl_mem out)
{
    ICOREG_API_BEGIN
    const char *op = "ops_pool2d";
    int Ho, Wo;
    long long total;

    if (ks < 1 || s < 1 || p < 0 || C < 0)
        icoreg_fatal("%s: invalid window k=%d s=%d p=%d", op, ks, s, p);
    Ho = ops_conv_out(H, ks, s, p, 1);
    Wo = ops_conv_out(W, ks, s, p, 1);
    if (Ho < 1 || Wo < 1)
        icoreg_fatal("%s: empty output", op);
    total = (long long)C * Ho * Wo;
    if (total == 0)
        return;
    count32((long long)C * H * W, "pool2d input");
    need_floats(in, 0, (long long)C * H * W, op, "in");
    need_floats(out, 0, total, op, "out");
    prof_scope ps(o->ocl, max ? "maxpool" : "avgpool");
    hipLaunchKernelGGL(pool2d_kernel, dim3((unsigned)((total + 255) / 256)),
                       dim3(256), 0, stream_of(o->ocl), cfptr(in), H, W, Ho, Wo,
                       ks, s, p, max, C, fptr(out));
    launch_check("pool2d");
    ICOREG_API_END
}

/* SPDX-License-Identifier: Unlicense */

/* RoMa's own kernels on gfx950: Gaussian-process kernel pieces, the
 * coarse warp from the anchor classes, warp sampling, local correlation,
 * displacement input, warp / certainty updates (v1, v2) and the
 * refiners' depthwise 5 x 5. Contracts of roma_kernels.cl:9-284
 * (i.coregistration.opencl).
 *
 * Design points:
 *  - row norms and cls_to_flow: one wave64 per row, cross-lane
 *    reductions (the reference: work-groups of 256 with LDS trees);
 *  - warp sampling: one thread per cell for all channels, the bilinear
 *    taps and weights computed once per cell and reused across channels
 *    (the reference recomputes them per (cell, channel));
 *  - local correlation: one wave per cell with the lanes over the
 *    (2 r + 2)^2 whole cells of the window (consecutive lanes on
 *    consecutive columns, so each channel's reads of a window row are
 *    contiguous), looping over channels against the cell's own feature
 *    vector broadcast from LDS; the (2 r + 1)^2 correlations are then
 *    the bilinear combinations of those whole-cell dot products, as the
 *    reference forms them;
 *  - depthwise 5 x 5: 32 x 8 output tiles, the (36 x 12) input patch in
 *    LDS, 16-byte-free scalar loads coalesced along rows. */

#include <hip/hip_runtime.h>

#include <math.h>

#include "common.h"
#include "icoreg_kernels.h"
#include "reduce.h"

using namespace icoreg;

/* ---- GP pieces --------------------------------------------------------------- */

__global__ void __launch_bounds__(256)
    row_norm_kernel(const float *__restrict__ X, int rows, int C,
                    float *__restrict__ out)
{
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    const float *x;
    float s = 0.0f;

    if (r >= rows)
        return;
    x = X + (long long)r * C;
    for (int c = lane; c < C; c += 64)
        s = fmaf(x[c], x[c], s);
    s = wave_sum(s);
    if (lane == 0)
        out[r] = sqrtf(s);
}

__global__ void __launch_bounds__(256)
    cos_exp_kernel(float *__restrict__ S, const float *__restrict__ nx,
                   const float *__restrict__ ny, int N, int M, float T,
                   float eps)
{
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    int i, j;
    float c;

    if (idx >= (long long)N * M)
        return;
    i = (int)(idx / M);
    j = (int)(idx % M);
    c = S[idx] / (nx[i] * ny[j] + eps);
    S[idx] = expf((c - 1.0f) / T);
}

/* ---- coarse warp from the anchor classes ----------------------------------- */

__global__ void __launch_bounds__(256)
    cls_to_flow_kernel(const float *__restrict__ L, int ld, int C, int res,
                       int n, float *__restrict__ flow,
                       float *__restrict__ cert)
{
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    const float *p;
    float m = -INFINITY, s = 0.0f;
    int arg = 0;

    if (t >= n)
        return;
    p = L + (long long)t * ld;
    for (int j = lane; j < C; j += 64)
        if (p[j] > m) {
            m = p[j];
            arg = j;
        }
    wave_argmax(m, arg);
    for (int j = lane; j < C; j += 64)
        s += expf(p[j] - m);
    s = wave_sum(s);
    if (lane == 0) {
        const int nb[5] = {arg - 1, arg, arg + 1, arg - res, arg + res};
        float fx = 0.0f, fy = 0.0f, tot = 0.0f;

        for (int k = 0; k < 5; k++) {
            const int c = min(max(nb[k], 0), C - 1);
            const float pr = expf(p[c] - m) / s;

            fx += pr * (-1.0f + (2 * (c % res) + 1) / (float)res);
            fy += pr * (-1.0f + (2 * (c / res) + 1) / (float)res);
            tot += pr;
        }
        flow[t] = fx / tot;
        flow[n + t] = fy / tot;
        cert[t] = p[C];
    }
}

/* ---- warp sampling ---------------------------------------------------------------- */

/* Pixel coordinates of a normalised warp (align_corners = 0) and the
 * bilinear setup; ok false for non-finite coordinates. Coordinates more
 * than margin + 2 cells outside the image are clamped to that distance
 * first (which keeps the integer conversion defined): every tap of a
 * window reaching margin cells around the point then stays outside, as
 * it was, so the sampled values (zeros) do not change. */
struct bil {
    int x0, y0;
    float fx, fy;
    bool ok;
};

__device__ __forceinline__ bil bilinear_setup(float x, float y, int H, int W,
                                              int margin = 0)
{
    bil b;
    float ix = ((x + 1.0f) * W - 1.0f) * 0.5f;
    float iy = ((y + 1.0f) * H - 1.0f) * 0.5f;

    b.ok = isfinite(ix) && isfinite(iy);
    if (!b.ok) {
        b.x0 = b.y0 = 0;
        b.fx = b.fy = 0.0f;
        return b;
    }
    ix = fminf(fmaxf(ix, -2.0f - margin), (float)(W + 1 + margin));
    iy = fminf(fmaxf(iy, -2.0f - margin), (float)(H + 1 + margin));
    b.x0 = (int)floorf(ix);
    b.y0 = (int)floorf(iy);
    b.fx = ix - b.x0;
    b.fy = iy - b.y0;
    return b;
}

__global__ void __launch_bounds__(256)
    warp_sample_kernel(const float *__restrict__ in, int C, int H, int W,
                       const float *__restrict__ flow, float *__restrict__ out,
                       int coff)
{
    const int i = blockIdx.x * 256 + threadIdx.x, n = H * W;
    bil b;
    bool in00, in01, in10, in11;
    int o00, o01, o10, o11;

    if (i >= n)
        return;
    b = bilinear_setup(flow[i], flow[n + i], H, W);
    in00 = b.ok && b.x0 >= 0 && b.x0 < W && b.y0 >= 0 && b.y0 < H;
    in01 = b.ok && b.x0 + 1 >= 0 && b.x0 + 1 < W && b.y0 >= 0 && b.y0 < H;
    in10 = b.ok && b.x0 >= 0 && b.x0 < W && b.y0 + 1 >= 0 && b.y0 + 1 < H;
    in11 = b.ok && b.x0 + 1 >= 0 && b.x0 + 1 < W && b.y0 + 1 >= 0 &&
           b.y0 + 1 < H;
    o00 = b.y0 * W + b.x0;
    o01 = o00 + 1;
    o10 = o00 + W;
    o11 = o10 + 1;
    for (int c = 0; c < C; c++) {
        const float *p = in + (long long)c * n;
        const float v00 = in00 ? p[o00] : 0.0f, v01 = in01 ? p[o01] : 0.0f;
        const float v10 = in10 ? p[o10] : 0.0f, v11 = in11 ? p[o11] : 0.0f;

        out[(long long)(coff + c) * n + i] =
            b.ok ? (1.0f - b.fy) * ((1.0f - b.fx) * v00 + b.fx * v01) +
                       b.fy * ((1.0f - b.fx) * v10 + b.fx * v11)
                 : 0.0f;
    }
}

/* ---- local correlation ------------------------------------------------------------- */

#define CORR_MAXC 1024

__global__ void __launch_bounds__(256)
    local_corr_kernel(const float *__restrict__ f1,
                      const float *__restrict__ f2, int C, int H, int W, int r,
                      const float *__restrict__ flow, float *__restrict__ out,
                      int coff)
{
    __shared__ float a1[4][CORR_MAXC];
    __shared__ float S[4][256];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int i = blockIdx.x * 4 + w, n = H * W;
    const int side = 2 * r + 1, ps = 2 * r + 2, np = ps * ps;
    const float rc = 1.0f / sqrtf((float)C);
    const bool active = i < n;
    bil b;

    if (active) {
        for (int c = lane; c < C; c += 64)
            a1[w][c] = f1[(long long)c * n + i] * rc;
        b = bilinear_setup(flow[i], flow[n + i], H, W, r);
    }
    else
        b = bilinear_setup(0.0f, 0.0f, H, W);
    __syncthreads();
    /* Whole-cell dot products of the (2 r + 2)^2 window, lanes over the
     * window cells (up to 4 per lane at r = 7). */
    if (active) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        int off[4];
        bool ok[4];

#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int e = lane + 64 * q;
            const int yy = b.y0 - r + e / ps, xx = b.x0 - r + e % ps;

            ok[q] = e < np && b.ok && xx >= 0 && xx < W && yy >= 0 && yy < H;
            off[q] = ok[q] ? yy * W + xx : 0;
        }
        for (int c = 0; c < C; c++) {
            const float a = a1[w][c];
            const float *p = f2 + (long long)c * n;

#pragma unroll
            for (int q = 0; q < 4; q++)
                if (ok[q])
                    acc[q] = fmaf(a, p[off[q]], acc[q]);
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int e = lane + 64 * q;

            if (e < np)
                S[w][e] = acc[q];
        }
    }
    __syncthreads();
    if (!active)
        return;
    for (int k = lane; k < side * side; k += 64) {
        const int e0 = (k / side) * ps + k % side, e1 = e0 + ps;
        const float *s = S[w];

        out[(long long)(coff + k) * n + i] =
            (1.0f - b.fy) * ((1.0f - b.fx) * s[e0] + b.fx * s[e0 + 1]) +
            b.fy * ((1.0f - b.fx) * s[e1] + b.fx * s[e1 + 1]);
    }
}

/* ---- displacement and updates ------------------------------------------------------- */

__global__ void __launch_bounds__(256)
    disp_kernel(const float *__restrict__ flow, int H, int W, float fx,
                float fy, float *__restrict__ out)
{
    const int i = blockIdx.x * 256 + threadIdx.x, n = H * W;
    float gx, gy;

    if (i >= n)
        return;
    gx = -1.0f + 1.0f / W + (i % W) * (2.0f - 2.0f / W) / (W - 1);
    gy = -1.0f + 1.0f / H + (i / W) * (2.0f - 2.0f / H) / (H - 1);
    out[i] = fx * (flow[i] - gx);
    out[n + i] = fy * (flow[n + i] - gy);
}

__global__ void __launch_bounds__(256)
    update_kernel(float *__restrict__ flow, float *__restrict__ cert,
                  const float *__restrict__ d, int n, float scale, float Wf,
                  float Hf)
{
    const int i = blockIdx.x * 256 + threadIdx.x;

    if (i >= n)
        return;
    flow[i] += scale * (d[i] / (4.0f * Wf));
    flow[n + i] += scale * (d[n + i] / (4.0f * Hf));
    cert[i] += d[2 * n + i];
}

__device__ __forceinline__ float softplus20(float x)
{
    return x > 20.0f ? x : log1pf(expf(x));
}

__global__ void __launch_bounds__(256)
    update2_kernel(float *__restrict__ flow, float *__restrict__ conf,
                   const float *__restrict__ d, int n, float W, float H)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    float l00, l10, l11;

    if (i >= n)
        return;
    flow[i] += d[i] / (4.0f * W);
    flow[n + i] += d[n + i] / (4.0f * H);
    l00 = softplus20(d[3 * n + i]) + 1e-6f;
    l10 = d[4 * n + i];
    l11 = softplus20(d[5 * n + i]) + 1e-6f;
    conf[i] += d[2 * n + i];
    conf[n + i] += l00 * l00;
    conf[2 * n + i] += l00 * l10;
    conf[3 * n + i] += l10 * l10 + l11 * l11;
}

/* ---- depthwise 5 x 5 + bias + ReLU ----------------------------------------------------- */

#define DW_TX 32
#define DW_TY 8

__global__ void __launch_bounds__(256)
    dwconv5_kernel(const float *__restrict__ in, int H, int W,
                   const float *__restrict__ wt, const float *__restrict__ bias,
                   float *__restrict__ out)
{
    __shared__ float t[DW_TY + 4][DW_TX + 5];
    const int lx = threadIdx.x & (DW_TX - 1), ly = threadIdx.x / DW_TX;
    const int x0 = blockIdx.x * DW_TX, y0 = blockIdx.y * DW_TY;
    const int c = blockIdx.z, x = x0 + lx, y = y0 + ly;
    const float *p = in + (long long)c * H * W;
    const float *w = wt + c * 25;
    float acc;

    for (int e = threadIdx.x; e < (DW_TY + 4) * (DW_TX + 4); e += 256) {
        const int yy = y0 - 2 + e / (DW_TX + 4), xx = x0 - 2 + e % (DW_TX + 4);

        t[e / (DW_TX + 4)][e % (DW_TX + 4)] =
            yy >= 0 && yy < H && xx >= 0 && xx < W ? p[(long long)yy * W + xx]
                                                   : 0.0f;
    }
    __syncthreads();
    if (x >= W || y >= H)
        return;
    acc = bias[c];
#pragma unroll
    for (int i = 0; i < 5; i++)
#pragma unroll
        for (int j = 0; j < 5; j++)
            acc = fmaf(t[ly + i][lx + j], w[i * 5 + j], acc);
    out[((long long)c * H + y) * W + x] = fmaxf(acc, 0.0f);
}

/* ---- launchers -------------------------------------------------------------------------- */

static unsigned nblk(long long n, int per) { return (unsigned)((n + per - 1) / per); }

extern "C" void roma_row_norm(struct ops *o, cl_mem X, int rows, int C,
                              cl_mem out)
{
    ICOREG_API_BEGIN
    const char *op = "roma_row_norm";

    if (rows < 0 || C < 1)
        icoreg_fatal("%s: invalid sizes rows=%d C=%d", op, rows, C);
    if (rows == 0)
        return;
    need_floats(X, 0, (long long)rows * C, op, "X");
    need_floats(out, 0, rows, op, "out");
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(row_norm_kernel, dim3(nblk(rows, 4)), dim3(256), 0,
                       stream_of(o->ocl), cfptr(X), rows, C, fptr(out));
    launch_check(op);
    ICOREG_API_END
}

extern "C" void roma_cos_exp(struct ops *o, cl_mem S, cl_mem nx, cl_mem ny,
                             int N, int M, float T, float eps)
{
    ICOREG_API_BEGIN
    const char *op = "roma_cos_exp";

    if (N < 0 || M < 0)
        icoreg_fatal("%s: invalid sizes N=%d M=%d", op, N, M);
    if ((long long)N * M == 0)
        return;
    need_floats(S, 0, (long long)N * M, op, "S");
    need_floats(nx, 0, N, op, "nx");
    need_floats(ny, 0, M, op, "ny");
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(cos_exp_kernel, dim3(nblk((long long)N * M, 256)),
                       dim3(256), 0, stream_of(o->ocl), fptr(S), cfptr(nx),
                       cfptr(ny), N, M, T, eps);
    launch_check(op);
    ICOREG_API_END
}

extern "C" void roma_cls_to_flow(struct ops *o, cl_mem L, int ld, int C,
                                 int res, int n, cl_mem flow, cl_mem cert)
{
    ICOREG_API_BEGIN
    const char *op = "roma_cls_to_flow";

    if (n < 0 || C < 1 || res < 1 || ld < C + 1)
        icoreg_fatal("%s: invalid sizes n=%d C=%d res=%d ld=%d", op, n, C, res,
                     ld);
    if (n == 0)
        return;
    need_floats(L, 0, (long long)(n - 1) * ld + C + 1, op, "L");
    need_floats(flow, 0, 2LL * n, op, "flow");
    need_floats(cert, 0, n, op, "cert");
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(cls_to_flow_kernel, dim3(nblk(n, 4)), dim3(256), 0,
                       stream_of(o->ocl), cfptr(L), ld, C, res, n, fptr(flow),
                       fptr(cert));
    launch_check(op);
    ICOREG_API_END
}

extern "C" void roma_warp_sample(struct ops *o, cl_mem in, int C, int H, int W,
                                 cl_mem flow, cl_mem out, int coff)
{
    ICOREG_API_BEGIN
    const char *op = "roma_warp_sample";
    long long n = (long long)H * W;

    if (C < 0 || H < 1 || W < 1 || coff < 0)
        icoreg_fatal("%s: invalid sizes C=%d H=%d W=%d", op, C, H, W);
    if (C == 0)
        return;
    count32((long long)(coff + C) * n, op);
    need_floats(in, 0, (long long)C * n, op, "in");
    need_floats(flow, 0, 2 * n, op, "flow");
    need_floats(out, (long long)coff * n, (long long)C * n, op, "out");
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(warp_sample_kernel, dim3(nblk(n, 256)), dim3(256), 0,
                       stream_of(o->ocl), cfptr(in), C, H, W, cfptr(flow),
                       fptr(out), coff);
    launch_check(op);
    ICOREG_API_END
}

extern "C" void roma_local_corr(struct ops *o, cl_mem f1, cl_mem f2, int C,
                                int H, int W, int r, cl_mem flow, cl_mem out,
                                int coff)
{
    ICOREG_API_BEGIN
    const char *op = "roma_local_corr";
    long long n = (long long)H * W;

    if (C < 1 || C > CORR_MAXC || r < 0 || r > 7 || H < 1 || W < 1 ||
        coff < 0)
        icoreg_fatal("%s: invalid sizes C=%d r=%d (C <= %d, r <= 7)", op, C, r,
                     CORR_MAXC);
    count32((long long)(coff + (2 * r + 1) * (2 * r + 1)) * n, op);
    need_floats(f1, 0, (long long)C * n, op, "f1");
    need_floats(f2, 0, (long long)C * n, op, "f2");
    need_floats(flow, 0, 2 * n, op, "flow");
    need_floats(out, (long long)coff * n, (long long)(2 * r + 1) * (2 * r + 1) * n,
                op, "out");
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(local_corr_kernel, dim3(nblk(n, 4)), dim3(256), 0,
                       stream_of(o->ocl), cfptr(f1), cfptr(f2), C, H, W, r,
                       cfptr(flow), fptr(out), coff);
    launch_check(op);
    ICOREG_API_END
}

extern "C" void roma_disp(struct ops *o, cl_mem flow, int H, int W, float fx,
                          float fy, cl_mem out)
{
    ICOREG_API_BEGIN
    const char *op = "roma_disp";
    long long n = (long long)H * W;

    if (H < 2 || W < 2)
        icoreg_fatal("%s: grid %d x %d too small", op, H, W);
    need_floats(flow, 0, 2 * n, op, "flow");
    need_floats(out, 0, 2 * n, op, "out");
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(disp_kernel, dim3(nblk(n, 256)), dim3(256), 0,
                       stream_of(o->ocl), cfptr(flow), H, W, fx, fy, fptr(out));
    launch_check(op);
    ICOREG_API_END
}

extern "C" void roma_update(struct ops *o, cl_mem flow, cl_mem cert, cl_mem d,
                            int n, float scale, float Wf, float Hf)
{
    ICOREG_API_BEGIN
    const char *op = "roma_update";

    if (n < 0)
        icoreg_fatal("%s: n=%d", op, n);
    if (n == 0)
        return;
    need_floats(flow, 0, 2LL * n, op, "flow");
    need_floats(cert, 0, n, op, "cert");
    need_floats(d, 0, 3LL * n, op, "d");
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(update_kernel, dim3(nblk(n, 256)), dim3(256), 0,
                       stream_of(o->ocl), fptr(flow), fptr(cert), cfptr(d), n,
                       scale, Wf, Hf);
    launch_check(op);
    ICOREG_API_END
}

extern "C" void roma2_update(struct ops *o, cl_mem flow, cl_mem conf, cl_mem d,
                             int n, float W, float H)
{
    ICOREG_API_BEGIN
    const char *op = "roma2_update";

    if (n < 0)
        icoreg_fatal("%s: n=%d", op, n);
    if (n == 0)
        return;
    need_floats(flow, 0, 2LL * n, op, "flow");
    need_floats(conf, 0, 4LL * n, op, "conf");
    need_floats(d, 0, 6LL * n, op, "d");
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(update2_kernel, dim3(nblk(n, 256)), dim3(256), 0,
                       stream_of(o->ocl), fptr(flow), fptr(conf), cfptr(d), n,
                       W, H);
    launch_check(op);
    ICOREG_API_END
}

extern "C" void roma_dwconv5(struct ops *o, cl_mem in, int C, int H, int W,
                             cl_mem w, cl_mem bias, cl_mem out)
{
    ICOREG_API_BEGIN
    const char *op = "roma_dwconv5";

    if (C < 1 || H < 1 || W < 1 || C > 65535)
        icoreg_fatal("%s: invalid sizes C=%d H=%d W=%d", op, C, H, W);
    count32((long long)C * H * W, op);
    need_floats(in, 0, (long long)C * H * W, op, "in");
    need_floats(w, 0, 25LL * C, op, "w");
    need_floats(bias, 0, C, op, "bias");
    need_floats(out, 0, (long long)C * H * W, op, "out");
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(dwconv5_kernel,
                       dim3(nblk(W, DW_TX), nblk(H, DW_TY), (unsigned)C),
                       dim3(256), 0, stream_of(o->ocl), cfptr(in), H, W,
                       cfptr(w), cfptr(bias), fptr(out));
    launch_check(op);
    ICOREG_API_END
}

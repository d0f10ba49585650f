/* SPDX-License-Identifier: Unlicense */

/* Memory-bound generic operations: instance statistics, per-channel
 * affine, PReLU, activation, LayerNorm, row softmax, RoPE, axpby and
 * transpose. Contracts of the reference's ops.cl:450-602, 689-716,
 * 862-893 (i.coregistration.opencl) with its host checks (ops.c:338-494,
 * 580-610); kernels written for wave64: one wave per row with
 * cross-lane reductions, 16-byte accesses where rows allow. */

#include <hip/hip_runtime.h>

#include <math.h>

#include "act.h"
#include "common.h"
#include "ops.h"
#include "reduce.h"

using namespace icoreg;

static unsigned blocks_for(long long n, int per_block, long long cap = 1 << 20)
{
    long long b = (n + per_block - 1) / per_block;

    if (b < 1)
        b = 1;
    return (unsigned)(b > cap ? cap : b);
}

/* ---- instance statistics -------------------------------------------- */

/* Per-channel mean and 1 / sqrt(biased variance + eps), two passes as
 * the reference's chan_stats (ops.cl:453-492): the mean first, then the
 * squared deviations from it. Each channel is cut into segments of whole
 * 1024-float chunks so that a handful of channels still fill the GPU
 * (DISK's last level: 80 channels of 512 x 512); each pass writes one
 * partial per (channel, segment), and every block that needs a channel's
 * mean or variance adds that channel's partials itself, in segment
 * order, so the result does not depend on the schedule. Float4 loads
 * when HW % 4 == 0. */
#define CS_MAXSEG 64

__device__ __forceinline__ float cs_seg_sum(const float *__restrict__ p, int HW, int s0,
                                            int s1, float m, bool dev, bool v4)
{
    float acc = 0.0f;

    if (v4) {
        const float4 *q = (const float4 *)p;

        for (int i = s0 / 4 + threadIdx.x; i < s1 / 4; i += 256) {
            const float4 v = q[i];

            if (dev) {
                acc = fmaf(v.x - m, v.x - m, acc);
                acc = fmaf(v.y - m, v.y - m, acc);
                acc = fmaf(v.z - m, v.z - m, acc);
                acc = fmaf(v.w - m, v.w - m, acc);
            }
            else
                acc += (v.x + v.y) + (v.z + v.w);
        }
    }
    else
        for (int i = s0 + threadIdx.x; i < s1; i += 256) {
            const float v = p[i];

            acc = dev ? fmaf(v - m, v - m, acc) : acc + v;
        }
    return acc;
}

__device__ __forceinline__ float cs_total(const float *__restrict__ part, int nseg)
{
    float t = 0.0f;

    for (int k = 0; k < nseg; k++)
        t += part[k];
    return t;
}

/* Pass 1 (dev = 0): part_s = sum of the segment. Pass 2 (dev = 1): part_d
 * = sum of squared deviations from the channel's mean. */
__global__ void __launch_bounds__(256)
    chan_stats_part_kernel(const float *__restrict__ x, int HW, int seg, int nseg,
                           const float *__restrict__ part_s, float *__restrict__ out,
                           int dev)
{
    __shared__ float red[4];
    const int c = blockIdx.y, k = blockIdx.x;
    const int s0 = k * seg, s1 = min(HW, s0 + seg);
    const float m = dev ? cs_total(part_s + (long long)c * nseg, nseg) / HW : 0.0f;
    float acc = cs_seg_sum(x + (long long)c * HW, HW, s0, s1, m, dev != 0, (HW & 3) == 0);

    acc = block_sum<4>(acc, red);
    if (threadIdx.x == 0)
        out[(long long)c * nseg + k] = acc;
}

__global__ void __launch_bounds__(256)
    chan_stats_final_kernel(const float *__restrict__ part_s,
                            const float *__restrict__ part_d, int C, int HW, int nseg,
                            float eps, float *__restrict__ mean, float *__restrict__ rstd)
{
    const int c = blockIdx.x * 256 + threadIdx.x;

    if (c >= C)
        return;
    mean[c] = cs_total(part_s + (long long)c * nseg, nseg) / HW;
    rstd[c] = 1.0f / sqrtf(cs_total(part_d + (long long)c * nseg, nseg) / HW + eps);
}

extern "C" void ops_chan_stats(struct ops *o, cl_mem x, int C, int HW,
                               float eps, cl_mem mean, cl_mem rstd)
{
    ICOREG_API_BEGIN
    const char *op = "ops_chan_stats";

    if (C < 1 || HW < 1)
        icoreg_fatal("%s: empty tensor (%d x %d)", op, C, HW);
    count32((long long)C * HW, "chan_stats");
    need_floats(x, 0, (long long)C * HW, op, "x");
    need_floats(mean, 0, C, op, "mean");
    need_floats(rstd, 0, C, op, "rstd");
    {
        /* Segments of whole 1024-float chunks: about 2048 blocks in all. */
        const long long chunks = (HW + 1023) / 1024;
        long long want = (2048 + C - 1) / C;
        int nseg, seg;

        want = want < 1 ? 1 : want > CS_MAXSEG ? CS_MAXSEG : want;
        want = want > chunks ? chunks : want;
        seg = (int)((chunks + want - 1) / want) * 1024;
        nseg = (int)((HW + seg - 1) / seg);
        cl_mem sc = scratch_get(o, 2 * (size_t)C * nseg * sizeof(float));
        float *ps = (float *)sc->ptr, *pd = ps + (size_t)C * nseg;
        hipStream_t st = stream_of(o->ocl);

        prof_scope pr(o->ocl, "chan_stats");
        hipLaunchKernelGGL(chan_stats_part_kernel, dim3(nseg, C), dim3(256), 0, st,
                           cfptr(x), HW, seg, nseg, (const float *)ps, ps, 0);
        hipLaunchKernelGGL(chan_stats_part_kernel, dim3(nseg, C), dim3(256), 0, st,
                           cfptr(x), HW, seg, nseg, (const float *)ps, pd, 1);
        hipLaunchKernelGGL(chan_stats_final_kernel, dim3((C + 255) / 256), dim3(256), 0, st,
                           (const float *)ps, (const float *)pd, C, HW, nseg, eps, fptr(mean),
                           fptr(rstd));
    }
    launch_check("chan_stats");
    ICOREG_API_END
}

/* ---- per-channel affine, PReLU, activation ---------------------------- */

__global__ void __launch_bounds__(256)
    chan_affine_kernel(const float *X, float *Y, int HW, int total,
                       const float *__restrict__ mean,
                       const float *__restrict__ rstd,
                       const float *__restrict__ g, const float *__restrict__ b,
                       int act, float slope)
{
    for (int i = blockIdx.x * 256 + threadIdx.x; i < total;
         i += gridDim.x * 256) {
        const int c = i / HW;
        float v = X[i];

        if (mean)
            v = (v - mean[c]) * rstd[c];
        if (g)
            v *= g[c];
        if (b)
            v += b[c];
        Y[i] = icoreg_act(v, act, slope);
    }
}

extern "C" void ops_chan_affine(struct ops *o, cl_mem X, cl_mem Y, int C,
                                int HW, cl_mem mean, cl_mem rstd, cl_mem g,
                                cl_mem b, int act, float slope)
{
    ICOREG_API_BEGIN
    const char *op = "ops_chan_affine";
    int n = count32((long long)C * HW, "chan_affine");

    if (n == 0)
        return;
    need_floats(X, 0, n, op, "X");
    need_floats(Y, 0, n, op, "Y");
    if (mean) {
        need_floats(mean, 0, C, op, "mean");
        need_floats(rstd, 0, C, op, "rstd");
    }
    if (g)
        need_floats(g, 0, C, op, "g");
    if (b)
        need_floats(b, 0, C, op, "b");
    prof_scope ps(o->ocl, "chan_affine");
    hipLaunchKernelGGL(chan_affine_kernel, dim3(blocks_for(n, 256, 65536)),
                       dim3(256), 0, stream_of(o->ocl), cfptr(X), fptr(Y), HW,
                       n, cfptr(mean), cfptr(rstd), cfptr(g), cfptr(b), act,
                       slope);
    launch_check("chan_affine");
    ICOREG_API_END
}

__global__ void __launch_bounds__(256)
    prelu_kernel(const float *X, float *Y, int HW, int total,
                 const float *__restrict__ alpha)
{
    for (int i = blockIdx.x * 256 + threadIdx.x; i < total;
         i += gridDim.x * 256) {
        const float v = X[i];

        Y[i] = v >= 0.0f ? v : alpha[i / HW] * v;
    }
}

extern "C" void ops_prelu(struct ops *o, cl_mem X, cl_mem Y, int C, int HW,
                          cl_mem alpha)
{
    ICOREG_API_BEGIN
    const char *op = "ops_prelu";
    int n = count32((long long)C * HW, "prelu");

    if (n == 0)
        return;
    need_floats(X, 0, n, op, "X");
    need_floats(Y, 0, n, op, "Y");
    need_floats(alpha, 0, C, op, "alpha");
    prof_scope ps(o->ocl, "prelu");
    hipLaunchKernelGGL(prelu_kernel, dim3(blocks_for(n, 256, 65536)), dim3(256),
                       0, stream_of(o->ocl), cfptr(X), fptr(Y), HW, n,
                       cfptr(alpha));
    launch_check("prelu");
    ICOREG_API_END
}

__global__ void __launch_bounds__(256)
    act_kernel(const float *X, float *Y, int total, int act, float slope)
{
    for (int i = blockIdx.x * 256 + threadIdx.x; i < total;
         i += gridDim.x * 256)
        Y[i] = icoreg_act(X[i], act, slope);
}

extern "C" void ops_act(struct ops *o, cl_mem X, cl_mem Y, long n, int act,
                        float slope)
{
    ICOREG_API_BEGIN
    const char *op = "ops_act";
    int cn = count32(n, "act");

    if (act < ACT_NONE || act > ACT_GELU_TANH)
        icoreg_fatal("%s: unknown activation %d", op, act);
    if (cn == 0)
        return;
    need_floats(X, 0, cn, op, "X");
    need_floats(Y, 0, cn, op, "Y");
    prof_scope ps(o->ocl, "act");
    hipLaunchKernelGGL(act_kernel, dim3(blocks_for(cn, 256, 65536)), dim3(256),
                       0, stream_of(o->ocl), cfptr(X), fptr(Y), cn, act, slope);
    launch_check("act");
    ICOREG_API_END
}

/* ---- axpby -------------------------------------------------------------- */

__global__ void __launch_bounds__(256)
    axpby_kernel(float *out, const float *a, float alpha, const float *b,
                 float beta, int n, int bmod)
{
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256)
        out[i] = alpha * a[i] + (b ? beta * b[i % bmod] : 0.0f);
}

/* Same with 16-byte accesses (n, bmod multiples of 4, aligned). */
__global__ void __launch_bounds__(256)
    axpby4_kernel(float4 *out, const float4 *a, float alpha, const float4 *b,
                  float beta, int n4, int bmod4)
{
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n4; i += gridDim.x * 256) {
        float4 x = a[i], r;

        if (b) {
            const float4 y = b[bmod4 == n4 ? i : i % bmod4];

            r.x = alpha * x.x + beta * y.x;
            r.y = alpha * x.y + beta * y.y;
            r.z = alpha * x.z + beta * y.z;
            r.w = alpha * x.w + beta * y.w;
        }
        else {
            r.x = alpha * x.x + 0.0f;
            r.y = alpha * x.y + 0.0f;
            r.z = alpha * x.z + 0.0f;
            r.w = alpha * x.w + 0.0f;
        }
        out[i] = r;
    }
}

extern "C" void ops_axpby(struct ops *o, cl_mem out, cl_mem a, float alpha,
                          cl_mem b, float beta, long n, long bmod)
{
    ICOREG_API_BEGIN
    const char *op = "ops_axpby";
    int cn = count32(n, "axpby"), cm = bmod > 0 ? count32(bmod, "axpby") : 1;

    if (cn == 0)
        return;
    need_floats(out, 0, cn, op, "out");
    need_floats(a, 0, cn, op, "a");
    if (b)
        need_floats(b, 0, cn < cm ? cn : cm, op, "b");
    prof_scope ps(o->ocl, "axpby");
    if (cn % 4 == 0 && cm % 4 == 0 && ((uintptr_t)out->ptr & 15) == 0 &&
        ((uintptr_t)a->ptr & 15) == 0 &&
        (!b || ((uintptr_t)b->ptr & 15) == 0))
        hipLaunchKernelGGL(axpby4_kernel, dim3(blocks_for(cn / 4, 256, 8192)),
                           dim3(256), 0, stream_of(o->ocl), (float4 *)fptr(out),
                           (const float4 *)cfptr(a), alpha,
                           (const float4 *)cfptr(b), beta, cn / 4, cm / 4);
    else
        hipLaunchKernelGGL(axpby_kernel, dim3(blocks_for(cn, 256, 8192)),
                           dim3(256), 0, stream_of(o->ocl), fptr(out), cfptr(a),
                           alpha, cfptr(b), beta, cn, cm);
    launch_check("axpby");
    ICOREG_API_END
}

/* ---- LayerNorm ---------------------------------------------------------- */

/* One wave per row; VPL values per lane cached in registers (C <= 64
 * VPL), or VPL = 0: three passes over the row in memory. */
template <int VPL>
__global__ void __launch_bounds__(256)
    layernorm_kernel(const float *X, float *Y, const float *__restrict__ g,
                     const float *__restrict__ bt, int C, long long rows,
                     float eps, int act, float slope)
{
    const int lane = threadIdx.x & 63;
    const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const float *x;
    float *y;
    float s = 0.0f, mean, var, r;

    if (row >= rows)
        return;
    x = X + row * C;
    y = Y + row * C;
    if (VPL > 0) {
        float v[VPL > 0 ? VPL : 1];

#pragma unroll
        for (int t = 0; t < VPL; t++) {
            const int c = lane + 64 * t;

            v[t] = c < C ? x[c] : 0.0f;
            s += v[t];
        }
        mean = wave_sum(s) / C;
        s = 0.0f;
#pragma unroll
        for (int t = 0; t < VPL; t++) {
            const int c = lane + 64 * t;
            const float d = v[t] - mean;

            if (c < C)
                s = fmaf(d, d, s);
        }
        var = wave_sum(s) / C;
        r = 1.0f / sqrtf(var + eps);
#pragma unroll
        for (int t = 0; t < VPL; t++) {
            const int c = lane + 64 * t;
            float u;

            if (c >= C)
                continue;
            u = (v[t] - mean) * r;
            if (g)
                u *= g[c];
            if (bt)
                u += bt[c];
            y[c] = icoreg_act(u, act, slope);
        }
        return;
    }
    for (int c = lane; c < C; c += 64)
        s += x[c];
    mean = wave_sum(s) / C;
    s = 0.0f;
    for (int c = lane; c < C; c += 64) {
        const float d = x[c] - mean;

        s = fmaf(d, d, s);
    }
    var = wave_sum(s) / C;
    r = 1.0f / sqrtf(var + eps);
    for (int c = lane; c < C; c += 64) {
        float u = (x[c] - mean) * r;

        if (g)
            u *= g[c];
        if (bt)
            u += bt[c];
        y[c] = icoreg_act(u, act, slope);
    }
}

static inline bool aligned16(cl_mem m)
{
    return ((uintptr_t)m->ptr & 15) == 0;
}

/* The same for C % 4 == 0 and 16-byte aligned rows: lane l holds the
 * float4 groups l + 64 t (t < NV), all of them (and the matching gamma
 * and beta groups) loaded before the first reduction, so a row costs one
 * memory round trip; DPP wave sums. */
template <int NV>
__global__ void __launch_bounds__(256)
    layernorm4_kernel(const float4 *X, float4 *Y, const float4 *__restrict__ g,
                      const float4 *__restrict__ bt, int C, long long rows,
                      float eps, int act, float slope)
{
    const int lane = threadIdx.x & 63, C4 = C >> 2;
    const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const float4 *x;
    float4 *y, v[NV], gv[NV], bv[NV];
    float s = 0.0f, mean, r;

    if (row >= rows)
        return;
    x = X + row * C4;
    y = Y + row * C4;
#pragma unroll
    for (int t = 0; t < NV; t++) {
        const int c = lane + 64 * t;
        const float4 one = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);

        v[t] = c < C4 ? x[c] : zero;
        gv[t] = g && c < C4 ? g[c] : one;
        bv[t] = bt && c < C4 ? bt[c] : zero;
    }
#pragma unroll
    for (int t = 0; t < NV; t++)
        s += (v[t].x + v[t].y) + (v[t].z + v[t].w);
    mean = wave_sum_full(s) / C;
    s = 0.0f;
#pragma unroll
    for (int t = 0; t < NV; t++)
        if (lane + 64 * t < C4) {
            const float d0 = v[t].x - mean, d1 = v[t].y - mean;
            const float d2 = v[t].z - mean, d3 = v[t].w - mean;

            s = fmaf(d0, d0, s);
            s = fmaf(d1, d1, s);
            s = fmaf(d2, d2, s);
            s = fmaf(d3, d3, s);
        }
    r = 1.0f / sqrtf(wave_sum_full(s) / C + eps);
#pragma unroll
    for (int t = 0; t < NV; t++) {
        const int c = lane + 64 * t;
        float u[4] = {(v[t].x - mean) * r, (v[t].y - mean) * r,
                      (v[t].z - mean) * r, (v[t].w - mean) * r};

        if (c >= C4)
            continue;
        if (g) {
            u[0] *= gv[t].x;
            u[1] *= gv[t].y;
            u[2] *= gv[t].z;
            u[3] *= gv[t].w;
        }
        if (bt) {
            u[0] += bv[t].x;
            u[1] += bv[t].y;
            u[2] += bv[t].z;
            u[3] += bv[t].w;
        }
        y[c] = make_float4(icoreg_act(u[0], act, slope),
                           icoreg_act(u[1], act, slope),
                           icoreg_act(u[2], act, slope),
                           icoreg_act(u[3], act, slope));
    }
}

extern "C" void ops_layernorm(struct ops *o, long rows, int C, cl_mem X,
                              cl_mem Y, cl_mem g, cl_mem b, float eps, int act,
                              float slope)
{
    ICOREG_API_BEGIN
    const char *op = "ops_layernorm";
    dim3 grid, block(256);

    if (rows < 0 || C < 1)
        icoreg_fatal("%s: invalid sizes rows=%ld C=%d", op, rows, C);
    if (rows == 0)
        return;
    need_floats(X, 0, (long long)rows * C, op, "X");
    need_floats(Y, 0, (long long)rows * C, op, "Y");
    if (g)
        need_floats(g, 0, C, op, "g");
    if (b)
        need_floats(b, 0, C, op, "b");
    if ((rows + 3) / 4 > 0x7fffffffLL)
        icoreg_fatal("%s: %ld rows", op, rows);
    grid = dim3((unsigned)((rows + 3) / 4));
    prof_scope ps(o->ocl, "layernorm");
#define LN(V)                                                                  \
    hipLaunchKernelGGL(layernorm_kernel<V>, grid, block, 0, stream_of(o->ocl), \
                       cfptr(X), fptr(Y), cfptr(g), cfptr(b), C,               \
                       (long long)rows, eps, act, slope)
#define LN4(V)                                                                 \
    hipLaunchKernelGGL(layernorm4_kernel<V>, grid, block, 0,                   \
                       stream_of(o->ocl), (const float4 *)cfptr(X),            \
                       (float4 *)fptr(Y), (const float4 *)cfptr(g),            \
                       (const float4 *)cfptr(b), C, (long long)rows, eps, act, \
                       slope)
    const bool v4 = C % 4 == 0 && C <= 2048 && aligned16(X) && aligned16(Y) &&
                    (!g || aligned16(g)) && (!b || aligned16(b));

    if (v4 && C <= 256)
        LN4(1);
    else if (v4 && C <= 512)
        LN4(2);
    else if (v4 && C <= 1024)
        LN4(4);
    else if (v4)
        LN4(8);
    else if (C <= 256)
        LN(4);
    else if (C <= 512)
        LN(8);
    else if (C <= 1024)
        LN(16);
    else if (C <= 2048)
        LN(32);
    else
        LN(0);
#undef LN
#undef LN4
    launch_check("layernorm");
    ICOREG_API_END
}

/* ---- row softmax ---------------------------------------------------------- */

__global__ void __launch_bounds__(256)
    softmax_rows_kernel(float *S, int L, long long rows, float scale)
{
    const int lane = threadIdx.x & 63;
    const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    float *s;
    float m = -INFINITY, sum = 0.0f, inv;

    if (row >= rows)
        return;
    s = S + row * L;
    for (int j = lane; j < L; j += 64)
        m = fmaxf(m, s[j] * scale);
    m = wave_max(m);
    for (int j = lane; j < L; j += 64) {
        const float v = expf(s[j] * scale - m);

        s[j] = v;
        sum += v;
    }
    inv = 1.0f / wave_sum(sum);
    for (int j = lane; j < L; j += 64)
        s[j] *= inv;
}

extern "C" void ops_softmax_rows(struct ops *o, cl_mem S, long rows, int L,
                                 float scale)
{
    ICOREG_API_BEGIN
    const char *op = "ops_softmax_rows";

    if (rows < 0 || L < 1)
        icoreg_fatal("%s: invalid sizes rows=%ld L=%d", op, rows, L);
    if (rows == 0)
        return;
    need_floats(S, 0, (long long)rows * L, op, "S");
    prof_scope ps(o->ocl, "softmax_rows");
    hipLaunchKernelGGL(softmax_rows_kernel, dim3((unsigned)((rows + 3) / 4)),
                       dim3(256), 0, stream_of(o->ocl), fptr(S), L,
                       (long long)rows, scale);
    launch_check("softmax_rows");
    ICOREG_API_END
}

/* ---- RoPE ----------------------------------------------------------------- */

__global__ void __launch_bounds__(256)
    rope_kernel(float *X, int ld, int nh, int d, int npos,
                const float2 *__restrict__ cs, int interleaved, int total)
{
    const int gid = blockIdx.x * 256 + threadIdx.x, nf = d / 2;
    int f, h, r, i0, i1;
    float *x;
    float2 rot;
    float a, b;

    if (gid >= total)
        return;
    f = gid % nf;
    h = (gid / nf) % nh;
    r = gid / (nf * nh);
    x = X + (long long)r * ld + h * d;
    rot = cs[(r % npos) * nf + f];
    i0 = interleaved ? 2 * f : f;
    i1 = interleaved ? 2 * f + 1 : f + nf;
    a = x[i0];
    b = x[i1];
    icoreg_rope_pair(a, b, rot, x[i0], x[i1]);
}

extern "C" void ops_rope(struct ops *o, cl_mem X, long off, int ld, long rows,
                         int nh, int d, int npos, cl_mem cs, int interleaved)
{
    ICOREG_API_BEGIN
    const char *op = "ops_rope";
    int n;

    if (rows < 0 || nh < 1 || d < 2 || d % 2 || npos < 1 || ld < nh * d ||
        off < 0)
        icoreg_fatal("%s: invalid sizes rows=%ld nh=%d d=%d npos=%d ld=%d", op,
                     rows, nh, d, npos, ld);
    n = count32((long long)rows * nh * (d / 2), "rope");
    if (n == 0)
        return;
    need_floats(X, off, (long long)(rows - 1) * ld + (long long)nh * d, op,
                "X");
    need_floats(cs, 0, (long long)(rows < npos ? rows : npos) * d, op,
                "table");
    prof_scope ps(o->ocl, "rope");
    hipLaunchKernelGGL(rope_kernel, dim3(blocks_for(n, 256)), dim3(256), 0,
                       stream_of(o->ocl), fptr(X) + off, ld, nh, d, npos,
                       (const float2 *)cfptr(cs), interleaved, n);
    launch_check("rope");
    ICOREG_API_END
}

/* ---- transpose ------------------------------------------------------------ */

/* (B, R, C) -> (B, C, R) by 32 x 32 tiles through LDS (padded rows). */
__global__ void __launch_bounds__(256)
    transpose_kernel(const float *__restrict__ in, float *__restrict__ out,
                     int R, int C)
{
    __shared__ float t[32][33];
    const long long base = (long long)blockIdx.z * R * C;
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;

#pragma unroll
    for (int k = 0; k < 32; k += 8) {
        const int r = r0 + ty + k, c = c0 + tx;

        if (r < R && c < C)
            t[ty + k][tx] = in[base + (long long)r * C + c];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 32; k += 8) {
        const int c = c0 + ty + k, r = r0 + tx;

        if (r < R && c < C)
            out[base + (long long)c * R + r] = t[tx][ty + k];
    }
}

extern "C" void ops_transpose(struct ops *o, cl_mem in, cl_mem out, int B,
                              int R, int C)
{
    ICOREG_API_BEGIN
    const char *op = "ops_transpose";
    long long n = (long long)B * R * C;

    if (B < 0 || R < 0 || C < 0 || B > 65535)
        icoreg_fatal("%s: invalid sizes B=%d R=%d C=%d", op, B, R, C);
    count32(n, "transpose");
    if (n == 0)
        return;
    need_floats(in, 0, n, op, "in");
    need_floats(out, 0, n, op, "out");
    prof_scope ps(o->ocl, "transpose");
    hipLaunchKernelGGL(transpose_kernel,
                       dim3((unsigned)((C + 31) / 32), (unsigned)((R + 31) / 32),
                            (unsigned)B),
                       dim3(256), 0, stream_of(o->ocl), cfptr(in), fptr(out), R,
                       C);
    launch_check("transpose");
    ICOREG_API_END
}

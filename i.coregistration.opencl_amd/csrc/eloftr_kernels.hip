/* SPDX-License-Identifier: Unlicense */

/* ELoFTR's own kernels on gfx950: the coarse dual-softmax statistics and
 * argmaxes over a block of score rows, and the two-stage fine matching.
 * Contracts of eloftr_kernels.cl:10-295 (i.coregistration.opencl).
 *
 * Row kernels: one wave64 per score row, 16-byte loads, cross-lane
 * reductions. Column kernels: the reference walks each column over all
 * rows of the block with one work-item per column (n = 6400 work-items,
 * a few percent of 256 CUs); here the rows are cut into chunks of 64,
 * one thread per (column, chunk) with coalesced row reads, and a second
 * kernel merges the chunk results per column in increasing row order,
 * so that the running statistics and the first-argmax rule are those of
 * the sequential scan. Argmax merges break ties to the lowest index.
 *
 * Fine matching: one block per match; both feature windows (8 x 8 of
 * image 0, 10 x 10 of image 1, 64 channels) staged in LDS once, the
 * 64 x 100 first-stage scores computed on the matrix cores
 * (v_mfma_f32_32x32x2f32, 8 output tiles over 4 waves), the softmax
 * statistics, argmax and the 3 x 3 second stage read from LDS. */

#include <climits>
#include <hip/hip_runtime.h>

#include <math.h>

#include "bilinear.h"
#include "common.h"
#include "eloftr_fused.h"
#include "icoreg_kernels.h"
#include "reduce.h"

using namespace icoreg;

typedef float floatx16 __attribute__((ext_vector_type(16)));

#define COL_CHUNK 64
/* Column merges: MERGE_C columns per block, MERGE_G thread groups per
 * column splitting the chunks. */
#define MERGE_C 16
#define MERGE_G 16

/* ---- rows ----------------------------------------------------------------- */

/* One wave per row, one pass over it: each lane keeps a running
 * (max, sum of exp(x - max)) over its elements, taken 4 at a time (one
 * rescale per 4), and the lanes are merged at the end. */
__global__ void __launch_bounds__(256)
    row_lse_kernel(const float *__restrict__ S, int rows, int N, int r0,
                   float *__restrict__ lse)
{
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    const float *s;
    float m = -INFINITY, sum = 0.0f, mw, sw;

    if (r >= rows)
        return;
    s = S + (long long)r * N;
    for (int j0 = 4 * lane; j0 < N; j0 += 256) {
        float v[4], cm = -INFINITY;

#pragma unroll
        for (int u = 0; u < 4; u++) {
            v[u] = j0 + u < N ? s[j0 + u] : -INFINITY;
            cm = fmaxf(cm, v[u]);
        }
        if (cm > m) {
            sum = m == -INFINITY ? 0.0f : sum * expf(m - cm);
            m = cm;
        }
#pragma unroll
        for (int u = 0; u < 4; u++)
            sum += v[u] == -INFINITY ? 0.0f : expf(v[u] - m);
    }
    mw = wave_max(m);
    sw = wave_sum(m == -INFINITY ? 0.0f : sum * expf(m - mw));
    if (lane == 0)
        lse[r0 + r] = mw + logf(sw);
}

/* lc[j] = cm[j] + log(cs[j]): the column log-sum-exp, as dual_conf
 * (eloftr_kernels.cl:69-72) forms it. */
__global__ void __launch_bounds__(256)
    col_logz_kernel(const float *__restrict__ cm, const float *__restrict__ cs,
                    int N, float *__restrict__ lc)
{
    const int j = blockIdx.x * 256 + threadIdx.x;

    if (j < N)
        lc[j] = cm[j] + logf(cs[j]);
}

__device__ __forceinline__ float dual_conf(float s, float lr, float lc)
{
    return expf(s - lr) * expf(s - lc);
}

__global__ void __launch_bounds__(256)
    conf_row_kernel(const float *__restrict__ S, int rows, int N, int r0,
                    const float *__restrict__ lse, const float *__restrict__ lc,
                    float *__restrict__ rmax, int *__restrict__ rarg)
{
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    const float *s;
    float best = -1.0f, lr;
    int bi = 0;

    if (r >= rows)
        return;
    s = S + (long long)r * N;
    lr = lse[r0 + r];
    for (int j = lane; j < N; j += 64) {
        const float c = dual_conf(s[j], lr, lc[j]);

        if (c > best) {
            best = c;
            bi = j;
        }
    }
    wave_argmax(best, bi);
    if (lane == 0) {
        rmax[r0 + r] = best;
        rarg[r0 + r] = bi;
    }
}

/* ---- columns ---------------------------------------------------------------- */

/* Chunk c of the block's rows: column maximum and sum of exp(x - max),
 * the chunk's values read once into registers. */
__global__ void __launch_bounds__(256)
    col_lse_part_kernel(const float *__restrict__ S, int R, int N,
                        float2 *__restrict__ part)
{
    const int j = blockIdx.x * 256 + threadIdx.x, c = blockIdx.y;
    const int ra = c * COL_CHUNK, nr = min(R - ra, COL_CHUNK);
    float v[COL_CHUNK], m = -INFINITY, s = 0.0f;

    if (j >= N)
        return;
#pragma unroll
    for (int r = 0; r < COL_CHUNK; r++) {
        v[r] = r < nr ? S[(long long)(ra + r) * N + j] : -INFINITY;
        m = fmaxf(m, v[r]);
    }
#pragma unroll
    for (int r = 0; r < COL_CHUNK; r++)
        s += r < nr ? expf(v[r] - m) : 0.0f;
    part[(long long)c * N + j] = make_float2(m, s);
}

/* Chunks merged into the block's (max, sum): group g of a column's
 * threads takes chunks g, g + MERGE_G, ... in two passes (the maximum of
 * the chunk maxima, then the rescaled sums: independent loads, no serial
 * chain), the groups are combined in order, and the result goes into the
 * running (cm, cs) as eloftr_col_lse does (eloftr_kernels.cl:62-65);
 * first: there is no running state yet (the first row block). */
__global__ void __launch_bounds__(256)
    col_lse_merge_kernel(const float2 *__restrict__ part, int nchunks, int N,
                         float *__restrict__ cm, float *__restrict__ cs, int first)
{
    __shared__ float2 red[MERGE_G][MERGE_C];
    const int cl = threadIdx.x % MERGE_C, g = threadIdx.x / MERGE_C;
    const int j = blockIdx.x * MERGE_C + cl;
    float m = -INFINITY, s = 0.0f, mo, mn;

    if (j < N) {
        for (int c = g; c < nchunks; c += MERGE_G)
            m = fmaxf(m, part[(long long)c * N + j].x);
        if (m != -INFINITY)
            for (int c = g; c < nchunks; c += MERGE_G) {
                const float2 p = part[(long long)c * N + j];

                s += p.x == -INFINITY ? 0.0f : p.y * expf(p.x - m);
            }
    }
    red[g][cl] = make_float2(m, s);
    __syncthreads();
    if (g != 0 || j >= N)
        return;
    m = -INFINITY;
    s = 0.0f;
    for (int q = 0; q < MERGE_G; q++)
        m = fmaxf(m, red[q][cl].x);
    if (m != -INFINITY)
        for (int q = 0; q < MERGE_G; q++)
            s += red[q][cl].x == -INFINITY ? 0.0f : red[q][cl].y * expf(red[q][cl].x - m);
    if (first) {
        cm[j] = m;
        cs[j] = m == -INFINITY ? 0.0f : s;
        return;
    }
    mo = cm[j];
    mn = fmaxf(mo, m);
    if (mn == -INFINITY)
        return;
    cs[j] = (mo == -INFINITY ? 0.0f : cs[j] * expf(mo - mn)) +
            (m == -INFINITY ? 0.0f : s * expf(m - mn));
    cm[j] = mn;
}

/* Chunk c: column maximum of the confidence and its first row. */
__global__ void __launch_bounds__(256)
    conf_col_part_kernel(const float *__restrict__ S, int R, int N, int r0,
                         const float *__restrict__ lse,
                         const float *__restrict__ lc, float *__restrict__ pv,
                         int *__restrict__ pi)
{
    const int j = blockIdx.x * 256 + threadIdx.x, c = blockIdx.y;
    const int ra = c * COL_CHUNK, rb = min(R, ra + COL_CHUNK);
    float best = -1.0f, l;
    int bi = -1;

    if (j >= N)
        return;
    l = lc[j];
    for (int r = ra; r < rb; r++) {
        const float v = dual_conf(S[(long long)r * N + j], lse[r0 + r], l);

        if (v > best) {
            best = v;
            bi = r0 + r;
        }
    }
    pv[(long long)c * N + j] = best;
    pi[(long long)c * N + j] = bi;
}

/* Chunks merged from the running state (cmax, carg): group g of a
 * column's threads scans chunks g, g + MERGE_G, ... in increasing order
 * with a strict comparison, and the groups' results are merged with ties
 * to the lowest row. Rows of the running state precede the block's, so
 * the first row reaching the maximum wins, as in the sequential scan of
 * eloftr_conf_col. first: no running state yet, start from (-1, -1). */
__global__ void __launch_bounds__(256)
    conf_col_merge_kernel(const float *__restrict__ pv,
                          const int *__restrict__ pi, int nchunks, int N,
                          float *__restrict__ cmax, int *__restrict__ carg, int first)
{
    __shared__ float rv[MERGE_G][MERGE_C];
    __shared__ int ri[MERGE_G][MERGE_C];
    const int cl = threadIdx.x % MERGE_C, g = threadIdx.x / MERGE_C;
    const int j = blockIdx.x * MERGE_C + cl;
    float best = -INFINITY;
    int bi = INT_MAX;

    if (j < N)
        for (int c = g; c < nchunks; c += MERGE_G) {
            const float v = pv[(long long)c * N + j];

            if (v > best) {
                best = v;
                bi = pi[(long long)c * N + j];
            }
        }
    rv[g][cl] = best;
    ri[g][cl] = bi;
    __syncthreads();
    if (g != 0 || j >= N)
        return;
    best = first ? -1.0f : cmax[j];
    bi = first ? -1 : carg[j];
    for (int q = 0; q < MERGE_G; q++) {
        const float v = rv[q][cl];

        if (v > best || (v == best && ri[q][cl] < bi && v != -INFINITY)) {
            best = v;
            bi = ri[q][cl];
        }
    }
    cmax[j] = best;
    carg[j] = bi;
}

/* ---- launchers --------------------------------------------------------------- */

static void check_block(cl_mem S, int rows, int N, const char *op)
{
    if (rows < 0 || N < 1)
        icoreg_fatal("%s: invalid sizes rows=%d N=%d", op, rows, N);
    need_floats(S, 0, (long long)rows * N, op, "S");
}

extern "C" void eloftr_row_lse(struct ops *o, cl_mem S, int rows, int N,
                               int r0, cl_mem lse)
{
    ICOREG_API_BEGIN
    const char *op = "eloftr_row_lse";

    check_block(S, rows, N, op);
    if (rows == 0)
        return;
    need_floats(lse, r0, rows, op, "lse");
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(row_lse_kernel, dim3((rows + 3) / 4), dim3(256), 0,
                       stream_of(o->ocl), cfptr(S), rows, N, r0, fptr(lse));
    launch_check(op);
    ICOREG_API_END
}

extern "C" void eloftr_col_lse(struct ops *o, cl_mem S, int R, int N,
                               cl_mem cm, cl_mem cs)
{
    ICOREG_API_BEGIN
    const char *op = "eloftr_col_lse";
    int nch = (R + COL_CHUNK - 1) / COL_CHUNK;
    cl_mem part;

    check_block(S, R, N, op);
    if (R == 0)
        return;
    need_floats(cm, 0, N, op, "cm");
    need_floats(cs, 0, N, op, "cs");
    part = scratch_get(o, (size_t)nch * N * sizeof(float2));
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(col_lse_part_kernel, dim3((N + 255) / 256, nch),
                       dim3(256), 0, stream_of(o->ocl), cfptr(S), R, N,
                       (float2 *)part->ptr);
    hipLaunchKernelGGL(col_lse_merge_kernel, dim3((N + MERGE_C - 1) / MERGE_C), dim3(256),
                       0, stream_of(o->ocl), (const float2 *)part->ptr, nch, N,
                       fptr(cm), fptr(cs), 0);
    launch_check(op);
    ICOREG_API_END
}

extern "C" void eloftr_conf_row(struct ops *o, cl_mem S, int rows, int N,
                                int r0, cl_mem lse, cl_mem cm, cl_mem cs,
                                cl_mem rmax, cl_mem rarg)
{
    ICOREG_API_BEGIN
    const char *op = "eloftr_conf_row";
    cl_mem lc;

    check_block(S, rows, N, op);
    if (rows == 0)
        return;
    need_floats(lse, r0, rows, op, "lse");
    need_floats(cm, 0, N, op, "cm");
    need_floats(cs, 0, N, op, "cs");
    need_floats(rmax, r0, rows, op, "rmax");
    need_bytes(rarg, 4LL * r0, 4LL * rows, op, "rarg");
    lc = scratch_get(o, (size_t)N * sizeof(float));
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(col_logz_kernel, dim3((N + 255) / 256), dim3(256), 0,
                       stream_of(o->ocl), cfptr(cm), cfptr(cs), N, fptr(lc));
    hipLaunchKernelGGL(conf_row_kernel, dim3((rows + 3) / 4), dim3(256), 0,
                       stream_of(o->ocl), cfptr(S), rows, N, r0, cfptr(lse),
                       cfptr(lc), fptr(rmax), (int *)rarg->ptr);
    launch_check(op);
    ICOREG_API_END
}

extern "C" void eloftr_conf_col(struct ops *o, cl_mem S, int R, int N, int r0,
                                cl_mem lse, cl_mem cm, cl_mem cs, cl_mem cmax,
                                cl_mem carg)
{
    ICOREG_API_BEGIN
    const char *op = "eloftr_conf_col";
    int nch = (R + COL_CHUNK - 1) / COL_CHUNK;
    size_t lc_bytes, pv_bytes;
    cl_mem sc;
    char *base;

    check_block(S, R, N, op);
    if (R == 0)
        return;
    need_floats(lse, r0, R, op, "lse");
    need_floats(cm, 0, N, op, "cm");
    need_floats(cs, 0, N, op, "cs");
    need_floats(cmax, 0, N, op, "cmax");
    need_bytes(carg, 0, 4LL * N, op, "carg");
    lc_bytes = ((size_t)N * 4 + 255) & ~(size_t)255;
    pv_bytes = ((size_t)nch * N * 4 + 255) & ~(size_t)255;
    sc = scratch_get(o, lc_bytes + 2 * pv_bytes);
    base = (char *)sc->ptr;
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(col_logz_kernel, dim3((N + 255) / 256), dim3(256), 0,
                       stream_of(o->ocl), cfptr(cm), cfptr(cs), N,
                       (float *)base);
    hipLaunchKernelGGL(conf_col_part_kernel, dim3((N + 255) / 256, nch),
                       dim3(256), 0, stream_of(o->ocl), cfptr(S), R, N, r0,
                       cfptr(lse), (const float *)base,
                       (float *)(base + lc_bytes),
                       (int *)(base + lc_bytes + pv_bytes));
    hipLaunchKernelGGL(conf_col_merge_kernel, dim3((N + MERGE_C - 1) / MERGE_C), dim3(256),
                       0, stream_of(o->ocl), (const float *)(base + lc_bytes),
                       (const int *)(base + lc_bytes + pv_bytes), nch, N,
                       fptr(cmax), (int *)carg->ptr, 0);
    launch_check(op);
    ICOREG_API_END
}

/* ---- the two passes, each in one read of S ---------------------------------- */

/* The driver's form of the four passes above: a block of R rows of S is
 * read once for both row and column log-sum-exps, and once more for both
 * confidence maxima. Tile: 64 rows (one column chunk, 16 per wave) x 256
 * columns (one band, 4 per lane, 16-byte loads). Rows are reduced across
 * the wave into one partial per (row, band), columns within the lane and
 * then across the block's waves in row order into one partial per
 * (chunk, column); the column partials are merged by the kernels above,
 * the row partials band by band in increasing order. N % 4 == 0. */
#define TB_RPW 16 /* rows per wave */

/* The exponentials are the full-precision expf of the reference's
 * dual_conf (eloftr_kernels.cl:68-72): these passes decide the row and
 * column argmaxes and the 0.2 threshold, so no fast exp2 form is used. */

__global__ void __launch_bounds__(256)
    lse_tile_kernel(const float *__restrict__ S, int R, int N, int nbands,
                    float2 *__restrict__ rpart, float2 *__restrict__ cpart)
{
    __shared__ float2 cp[4][256];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int b = blockIdx.x, c = blockIdx.y, j0 = b * 256 + 4 * lane;
    const int rb = c * COL_CHUNK + TB_RPW * w;
    float4 v[TB_RPW];

#pragma unroll
    for (int i = 0; i < TB_RPW; i++)
        v[i] = rb + i < R && j0 < N ? *(const float4 *)(S + (long long)(rb + i) * N + j0)
                                     : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
#pragma unroll
    for (int i = 0; i < TB_RPW; i++) {
        const float m = wave_max_full(fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
        float e = 0.0f;

        if (m != -INFINITY)
            e = expf(v[i].x - m) + expf(v[i].y - m) + expf(v[i].z - m) + expf(v[i].w - m);
        e = wave_sum_full(e);
        if (lane == 0 && rb + i < R)
            rpart[(long long)(rb + i) * nbands + b] = make_float2(m, e);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float m = -INFINITY, e = 0.0f;

#pragma unroll
        for (int i = 0; i < TB_RPW; i++)
            m = fmaxf(m, ((const float *)&v[i])[k]);
        if (m != -INFINITY)
#pragma unroll
            for (int i = 0; i < TB_RPW; i++)
                e += expf(((const float *)&v[i])[k] - m);
        cp[w][4 * lane + k] = make_float2(m, e);
    }
    __syncthreads();
    {
        const int j = b * 256 + tid;
        float m = -INFINITY, e = 0.0f;

        if (j >= N)
            return;
#pragma unroll
        for (int q = 0; q < 4; q++)
            m = fmaxf(m, cp[q][tid].x);
        if (m != -INFINITY)
#pragma unroll
            for (int q = 0; q < 4; q++)
                e += cp[q][tid].x == -INFINITY ? 0.0f : cp[q][tid].y * expf(cp[q][tid].x - m);
        cpart[(long long)c * N + j] = make_float2(m, e);
    }
}

/* lse[r0 + r] from the band partials of row r: MERGE_C lanes per row
 * split the bands, combined with lane exchanges in a fixed order. */
__global__ void __launch_bounds__(256)
    lse_row_merge_kernel(const float2 *__restrict__ rpart, int R, int nbands, int r0,
                         float *__restrict__ lse)
{
    const int r = blockIdx.x * (256 / MERGE_C) + threadIdx.x / MERGE_C;
    const int q0 = threadIdx.x % MERGE_C;
    const float2 *p = rpart + (long long)min(r, R - 1) * nbands;
    float m = -INFINITY, e = 0.0f, mt;

    for (int q = q0; q < nbands; q += MERGE_C)
        m = fmaxf(m, p[q].x);
    mt = m;
#pragma unroll
    for (int o = MERGE_C / 2; o > 0; o >>= 1)
        mt = fmaxf(mt, __shfl_xor(mt, o, MERGE_C));
    if (mt != -INFINITY)
        for (int q = q0; q < nbands; q += MERGE_C)
            e += p[q].x == -INFINITY ? 0.0f : p[q].y * expf(p[q].x - mt);
#pragma unroll
    for (int o = MERGE_C / 2; o > 0; o >>= 1)
        e += __shfl_xor(e, o, MERGE_C);
    if (r < R && q0 == 0)
        lse[r0 + r] = mt + logf(e);
}

/* Confidence maxima of the tile: per (row, band) and per (chunk, column),
 * first index on ties as in the sequential scans. */
__global__ void __launch_bounds__(256)
    conf_tile_kernel(const float *__restrict__ S, int R, int N, int r0, int nbands,
                     const float *__restrict__ lse, const float *__restrict__ lc,
                     float *__restrict__ rpv, int *__restrict__ rpi,
                     float *__restrict__ cpv, int *__restrict__ cpi)
{
    __shared__ float cv[4][256];
    __shared__ int ci[4][256];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int b = blockIdx.x, c = blockIdx.y, j0 = b * 256 + 4 * lane;
    const int rb = c * COL_CHUNK + TB_RPW * w;
    const bool jon = j0 < N;
    float4 v[TB_RPW];
    float4 l4 = jon ? *(const float4 *)(lc + j0) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float cb[4] = {-1.0f, -1.0f, -1.0f, -1.0f};
    int cbi[4] = {-1, -1, -1, -1};

#pragma unroll
    for (int i = 0; i < TB_RPW; i++)
        v[i] = rb + i < R && jon ? *(const float4 *)(S + (long long)(rb + i) * N + j0)
                                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int i = 0; i < TB_RPW; i++) {
        const int r = rb + i;
        const float lr = r < R ? lse[r0 + r] : 0.0f;
        float best = -1.0f;
        int bi = 0;

#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float x = dual_conf(((const float *)&v[i])[k], lr, ((const float *)&l4)[k]);

            if (jon && r < R) {
                if (x > best) {
                    best = x;
                    bi = j0 + k;
                }
                if (x > cb[k]) {
                    cb[k] = x;
                    cbi[k] = r0 + r;
                }
            }
        }
        wave_argmax_full(best, bi);
        if (lane == 0 && r < R) {
            rpv[(long long)r * nbands + b] = best;
            rpi[(long long)r * nbands + b] = bi;
        }
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        cv[w][4 * lane + k] = cb[k];
        ci[w][4 * lane + k] = cbi[k];
    }
    __syncthreads();
    {
        const int j = b * 256 + tid;
        float best = -1.0f;
        int bi = -1;

        if (j >= N)
            return;
        /* Waves in row order, strict comparison: the first row wins. */
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (cv[q][tid] > best) {
                best = cv[q][tid];
                bi = ci[q][tid];
            }
        cpv[(long long)c * N + j] = best;
        cpi[(long long)c * N + j] = bi;
    }
}

/* rmax / rarg from the band partials in increasing band order. */
__global__ void __launch_bounds__(256)
    conf_row_merge_kernel(const float *__restrict__ rpv, const int *__restrict__ rpi, int R,
                          int nbands, int r0, float *__restrict__ rmax, int *__restrict__ rarg)
{
    const int r = blockIdx.x * 256 + threadIdx.x;
    float best = -1.0f;
    int bi = 0;

    if (r >= R)
        return;
    for (int q = 0; q < nbands; q++) {
        const float x = rpv[(long long)r * nbands + q];

        if (x > best) {
            best = x;
            bi = rpi[(long long)r * nbands + q];
        }
    }
    rmax[r0 + r] = best;
    rarg[r0 + r] = bi;
}

bool eloftr_tiles_ok(cl_mem S, int N)
{
    return N % 4 == 0 && ((uintptr_t)S->ptr & 15) == 0;
}

void eloftr_lse_tiles(struct ops *o, cl_mem S, int R, int N, int r0, cl_mem lse, cl_mem cm,
                      cl_mem cs)
{
    const char *op = "eloftr_lse_tiles";
    const int nch = (R + COL_CHUNK - 1) / COL_CHUNK, nbands = (N + 255) / 256;
    size_t rb;
    cl_mem sc;

    check_block(S, R, N, op);
    if (R == 0)
        return;
    if (!eloftr_tiles_ok(S, N))
        icoreg_fatal("%s: N %% 4 and 16-byte alignment required", op);
    need_floats(lse, r0, R, op, "lse");
    need_floats(cm, 0, N, op, "cm");
    need_floats(cs, 0, N, op, "cs");
    rb = ((size_t)R * nbands * sizeof(float2) + 255) & ~(size_t)255;
    sc = scratch_get(o, rb + (size_t)nch * N * sizeof(float2));
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(lse_tile_kernel, dim3(nbands, nch), dim3(256), 0, stream_of(o->ocl),
                       cfptr(S), R, N, nbands, (float2 *)sc->ptr,
                       (float2 *)((char *)sc->ptr + rb));
    hipLaunchKernelGGL(lse_row_merge_kernel, dim3((R + 256 / MERGE_C - 1) / (256 / MERGE_C)), dim3(256), 0,
                       stream_of(o->ocl), (const float2 *)sc->ptr, R, nbands, r0, fptr(lse));
    hipLaunchKernelGGL(col_lse_merge_kernel, dim3((N + MERGE_C - 1) / MERGE_C), dim3(256), 0,
                       stream_of(o->ocl), (const float2 *)((char *)sc->ptr + rb), nch, N,
                       fptr(cm), fptr(cs), r0 == 0);
    launch_check(op);
}

void eloftr_conf_tiles(struct ops *o, cl_mem S, int R, int N, int r0, cl_mem lse, cl_mem cm,
                       cl_mem cs, cl_mem rmax, cl_mem rarg, cl_mem cmax, cl_mem carg)
{
    const char *op = "eloftr_conf_tiles";
    const int nch = (R + COL_CHUNK - 1) / COL_CHUNK, nbands = (N + 255) / 256;
    size_t lcb, rpb, cpb;
    cl_mem sc;
    char *base;

    check_block(S, R, N, op);
    if (R == 0)
        return;
    if (!eloftr_tiles_ok(S, N))
        icoreg_fatal("%s: N %% 4 and 16-byte alignment required", op);
    need_floats(lse, r0, R, op, "lse");
    need_floats(cm, 0, N, op, "cm");
    need_floats(cs, 0, N, op, "cs");
    need_floats(rmax, r0, R, op, "rmax");
    need_bytes(rarg, 4LL * r0, 4LL * R, op, "rarg");
    need_floats(cmax, 0, N, op, "cmax");
    need_bytes(carg, 0, 4LL * N, op, "carg");
    lcb = ((size_t)N * 4 + 255) & ~(size_t)255;
    rpb = ((size_t)R * nbands * 4 + 255) & ~(size_t)255;
    cpb = ((size_t)nch * N * 4 + 255) & ~(size_t)255;
    sc = scratch_get(o, lcb + 2 * rpb + 2 * cpb);
    base = (char *)sc->ptr;
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(col_logz_kernel, dim3((N + 255) / 256), dim3(256), 0,
                       stream_of(o->ocl), cfptr(cm), cfptr(cs), N, (float *)base);
    hipLaunchKernelGGL(conf_tile_kernel, dim3(nbands, nch), dim3(256), 0, stream_of(o->ocl),
                       cfptr(S), R, N, r0, nbands, cfptr(lse), (const float *)base,
                       (float *)(base + lcb), (int *)(base + lcb + rpb),
                       (float *)(base + lcb + 2 * rpb), (int *)(base + lcb + 2 * rpb + cpb));
    hipLaunchKernelGGL(conf_row_merge_kernel, dim3((R + 255) / 256), dim3(256), 0,
                       stream_of(o->ocl), (const float *)(base + lcb),
                       (const int *)(base + lcb + rpb), R, nbands, r0, fptr(rmax),
                       (int *)rarg->ptr);
    hipLaunchKernelGGL(conf_col_merge_kernel, dim3((N + MERGE_C - 1) / MERGE_C), dim3(256), 0,
                       stream_of(o->ocl), (const float *)(base + lcb + 2 * rpb),
                       (const int *)(base + lcb + 2 * rpb + cpb), nch, N, fptr(cmax),
                       (int *)carg->ptr, r0 == 0);
    launch_check(op);
}

/* ---- fine matching ------------------------------------------------------------ */

#define FW 8           /* window of image 0 */
#define FW1 10         /* window of image 1 (one cell of padding) */
#define FC 64          /* fine channels */
#define FS 8           /* second-stage channels (the last ones) */
#define NP (FW * FW)   /* 64 positions in image 0 */
#define NQ (FW1 * FW1) /* 100 positions in image 1 */
#define WP (FC + 1)    /* LDS row pitch of the windows */
#define SP (NQ + 1)    /* LDS row pitch of the scores */

/* UP2: f0 and f1 hold the features at half resolution (H / 2 x W / 2)
 * and each window value is their 2x bilinear resize (bl_up2, the resize
 * kernel's arithmetic), so the full-resolution maps need not exist. */
template <bool UP2>
__global__ void __launch_bounds__(256)
    fine_kernel(const float *__restrict__ f0, const float *__restrict__ f1,
                int H, int W, const int4 *__restrict__ cells, int M, float T,
                float4 *__restrict__ out, const int *__restrict__ mcount)
{
    __shared__ float A[NP * WP];
    __shared__ float B[NQ * WP];
    __shared__ float sc[NP * SP];
    __shared__ float pm[NQ], ps[NQ], qm[NP], qs[NP];
    __shared__ float rv[4], s2[9];
    __shared__ int ri[4];
    const int k = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int wave = tid >> 6, half = lane >> 5, col = lane & 31;
    const long long plane = UP2 ? (long long)(H / 2) * (W / 2) : (long long)H * W;
    int4 cl;

    if (mcount)
        M = min(M, *mcount);
    if (k >= M)
        return;
    cl = cells[k];

    /* Windows into LDS, [position][channel], zero outside the image. */
    for (int e = tid; e < FC * NP; e += 256) {
        const int c = e / NP, p = e % NP;
        const int x = cl.x * FW + p % FW, y = cl.y * FW + p / FW;

        A[p * WP + c] = (x >= 0 && y >= 0 && x < W && y < H)
                            ? (UP2 ? bl_up2(f0 + c * plane, H / 2, W / 2, y, x)
                                   : f0[c * plane + (long long)y * W + x])
                            : 0.0f;
    }
    for (int e = tid; e < FC * NQ; e += 256) {
        const int c = e / NQ, q = e % NQ;
        const int x = cl.z * FW - 1 + q % FW1, y = cl.w * FW - 1 + q / FW1;

        B[q * WP + c] = (x >= 0 && y >= 0 && x < W && y < H)
                            ? (UP2 ? bl_up2(f1 + c * plane, H / 2, W / 2, y, x)
                                   : f1[c * plane + (long long)y * W + x])
                            : 0.0f;
    }
    __syncthreads();

    /* First-stage scores on the first FC - FS channels / FC: wave w owns
     * image-0 rows (w / 2) * 32.. and image-1 columns (w % 2) * 64.. as
     * two 32 x 32 MFMA tiles (columns past NQ are zero). */
    {
        const int pt = wave >> 1, qb = (wave & 1) * 64;
        floatx16 acc[2];

        for (int j = 0; j < 2; j++)
            for (int r = 0; r < 16; r++)
                acc[j][r] = 0.0f;
#pragma unroll 4
        for (int st = 0; st < (FC - FS) / 2; st++) {
            const int c = 2 * st + half;
            const float a = A[(pt * 32 + col) * WP + c];

#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int q = qb + j * 32 + col;
                const float b = q < NQ ? B[q * WP + c] : 0.0f;

                acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[j], 0,
                                                              0, 0);
            }
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int q = qb + j * 32 + col;

            if (q >= NQ)
                continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int p = pt * 32 + (r >> 2) * 8 + half * 4 + (r & 3);

                sc[p * SP + q] = acc[j][r] * (1.0f / FC);
            }
        }
    }
    __syncthreads();

    /* Softmax statistics over image 0's positions (per q) and over image
     * 1's positions (per p). */
    if (tid < NQ) {
        const int q = tid;
        float m = -INFINITY, s = 0.0f;

        for (int p = 0; p < NP; p++)
            m = fmaxf(m, sc[p * SP + q]);
        for (int p = 0; p < NP; p++)
            s += expf(sc[p * SP + q] - m);
        pm[q] = m;
        ps[q] = s;
    }
    else if (tid >= 128 && tid < 128 + NP) {
        const int p = tid - 128;
        float m = -INFINITY, s = 0.0f;

        for (int q = 0; q < NQ; q++)
            m = fmaxf(m, sc[p * SP + q]);
        for (int q = 0; q < NQ; q++)
            s += expf(sc[p * SP + q] - m);
        qm[p] = m;
        qs[p] = s;
    }
    __syncthreads();

    /* First argmax over (p, inner 8 x 8 of image 1) in the flattened
     * order p * 64 + i * 8 + j. */
    {
        float best = -1.0f;
        int bi = 0;

        for (int e = tid; e < NP * FW * FW; e += 256) {
            const int pp = e / (FW * FW), ii = (e / FW) % FW, jj = e % FW;
            const int qq = (ii + 1) * FW1 + jj + 1;
            const float s = sc[pp * SP + qq];
            const float v =
                expf(s - pm[qq]) / ps[qq] * (expf(s - qm[pp]) / qs[pp]);

            if (v > best) {
                best = v;
                bi = e;
            }
        }
        wave_argmax(best, bi);
        if (lane == 0) {
            rv[wave] = best;
            ri[wave] = bi;
        }
    }
    __syncthreads();
    {
        float best = rv[0];
        int bi = ri[0];

        for (int w = 1; w < 4; w++)
            argmax_merge(best, bi, rv[w], ri[w]);
        {
            const int bp = bi / (FW * FW), bq = bi % (FW * FW);
            const int qi = bq / FW, qj = bq % FW;

            /* Second stage: 3 x 3 around the 10 x 10 indices (qi, qj),
             * index -1 wrapping to 9 as the reference. */
            if (tid < 9) {
                const int ii = (qi + tid / 3 - 1 + FW1) % FW1;
                const int jj = (qj + tid % 3 - 1 + FW1) % FW1;
                const float *a = A + bp * WP, *b = B + (ii * FW1 + jj) * WP;
                float d = 0.0f;

                for (int c = FC - FS; c < FC; c++)
                    d = fmaf(a[c], b[c], d);
                s2[tid] = d * (1.0f / sqrtf((float)FS)) / T;
            }
            __syncthreads();
            if (tid == 0) {
                float m = -INFINITY, s = 0.0f, ex = 0.0f, ey = 0.0f;

                for (int t = 0; t < 9; t++)
                    m = fmaxf(m, s2[t]);
                for (int t = 0; t < 9; t++)
                    s += expf(s2[t] - m);
                for (int t = 0; t < 9; t++) {
                    const float w = expf(s2[t] - m) / s;

                    ex += w * (t % 3 - 1);
                    ey += w * (t / 3 - 1);
                }
                out[k] = make_float4(cl.x * FW + bp % FW - (FW / 2 - 0.5f),
                                     cl.y * FW + bp / FW - (FW / 2 - 0.5f),
                                     cl.z * FW + qj - (FW / 2 - 0.5f) + ex,
                                     cl.w * FW + qi - (FW / 2 - 0.5f) + ey);
            }
        }
    }
}

extern "C" void eloftr_fine(struct ops *o, cl_mem f0, cl_mem f1, int H, int W,
                            cl_mem cells, int M, float T, cl_mem out)
{
    ICOREG_API_BEGIN
    const char *op = "eloftr_fine";

    if (M < 0 || H < 1 || W < 1)
        icoreg_fatal("%s: invalid sizes M=%d H=%d W=%d", op, M, H, W);
    if (M == 0)
        return;
    need_floats(f0, 0, (long long)FC * H * W, op, "f0");
    need_floats(f1, 0, (long long)FC * H * W, op, "f1");
    need_bytes(cells, 0, 16LL * M, op, "cells");
    need_floats(out, 0, 4LL * M, op, "out");
    if (((uintptr_t)cells->ptr & 15) || ((uintptr_t)out->ptr & 15))
        icoreg_fatal("%s: cells and out must be 16-byte aligned", op);
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(fine_kernel<false>, dim3(M), dim3(256), 0, stream_of(o->ocl),
                       cfptr(f0), cfptr(f1), H, W, (const int4 *)cells->ptr, M,
                       T, (float4 *)out->ptr, nullptr);
    launch_check(op);
    ICOREG_API_END
}

extern "C" void eloftr_fine_half(struct ops *o, cl_mem f0, cl_mem f1, int H, int W,
                                 cl_mem cells, int M, float T, cl_mem out)
{
    ICOREG_API_BEGIN
    const char *op = "eloftr_fine_half";

    if (M < 0 || H < 2 || W < 2 || H % 2 || W % 2)
        icoreg_fatal("%s: invalid sizes M=%d H=%d W=%d", op, M, H, W);
    if (M == 0)
        return;
    need_floats(f0, 0, (long long)FC * (H / 2) * (W / 2), op, "f0");
    need_floats(f1, 0, (long long)FC * (H / 2) * (W / 2), op, "f1");
    need_bytes(cells, 0, 16LL * M, op, "cells");
    need_floats(out, 0, 4LL * M, op, "out");
    if (((uintptr_t)cells->ptr & 15) || ((uintptr_t)out->ptr & 15))
        icoreg_fatal("%s: cells and out must be 16-byte aligned", op);
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(fine_kernel<true>, dim3(M), dim3(256), 0, stream_of(o->ocl),
                       cfptr(f0), cfptr(f1), H, W, (const int4 *)cells->ptr, M, T,
                       (float4 *)out->ptr, nullptr);
    launch_check(op);
    ICOREG_API_END
}

extern "C" void eloftr_fine_half_count(struct ops *o, cl_mem f0, cl_mem f1, int H, int W,
                                       cl_mem cells, cl_mem count, int nmax, float T,
                                       cl_mem out)
{
    ICOREG_API_BEGIN
    const char *op = "eloftr_fine_half_count";

    if (nmax < 0 || H < 2 || W < 2 || H % 2 || W % 2)
        icoreg_fatal("%s: invalid sizes nmax=%d H=%d W=%d", op, nmax, H, W);
    if (nmax == 0)
        return;
    need_floats(f0, 0, (long long)FC * (H / 2) * (W / 2), op, "f0");
    need_floats(f1, 0, (long long)FC * (H / 2) * (W / 2), op, "f1");
    need_bytes(cells, 0, 16LL * nmax, op, "cells");
    need_bytes(count, 0, 4, op, "count");
    need_floats(out, 0, 4LL * nmax, op, "out");
    if (((uintptr_t)cells->ptr & 15) || ((uintptr_t)out->ptr & 15))
        icoreg_fatal("%s: cells and out must be 16-byte aligned", op);
    prof_scope ps(o->ocl, "eloftr_fine_half");
    hipLaunchKernelGGL(fine_kernel<true>, dim3(nmax), dim3(256), 0, stream_of(o->ocl),
                       cfptr(f0), cfptr(f1), H, W, (const int4 *)cells->ptr, nmax, T,
                       (float4 *)out->ptr, (const int *)count->ptr);
    launch_check(op);
    ICOREG_API_END
}

/* ---- mutual nearest-neighbour selection of the coarse matches ---------- */

/* The host loop of eloftr.c:606-636 on the device: cell i of image 0 is
 * kept with j = its row argmax when its best confidence exceeds thr, j's
 * column argmax is i, and both cells are at least border cells from the
 * edges. One block of 1024 threads: each thread takes a contiguous run
 * of cells, counts, the counts are scanned, and the kept matches are
 * written in raster order (i, j, confidence, and the cells' (x, y) for
 * fine matching). count[0] = the number kept; count[1] = 1 if a row
 * argmax was out of range (the host raises the error). */
#define MU_T 1024
__global__ void __launch_bounds__(MU_T)
    mutual_kernel(const float *__restrict__ rmax, const int *__restrict__ rarg,
                  const int *__restrict__ carg, int h, int w, int border, float thr,
                  int *__restrict__ mi, int *__restrict__ mj, float *__restrict__ mconf,
                  int4 *__restrict__ cells, int *__restrict__ count)
{
    __shared__ int wsum[MU_T / 64];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n = h * w, per = (n + MU_T - 1) / MU_T;
    const int i0 = min(n, tid * per), i1 = min(n, i0 + per);
    int cnt = 0, bad = 0, off;

    auto keep = [&](int i, int &j) {
        j = rarg[i];
        if (j < 0 || j >= n) {
            bad = 1;
            return false;
        }
        const int xi = i % w, yi = i / w, xj = j % w, yj = j / w;

        return rmax[i] > thr && carg[j] == i && xi >= border && yi >= border &&
               xi < w - border && yi < h - border && xj >= border && yj >= border &&
               xj < w - border && yj < h - border;
    };
    for (int i = i0; i < i1; i++) {
        int j;

        cnt += keep(i, j) ? 1 : 0;
    }
    /* Exclusive scan of the counts over the block. */
    {
        int x = cnt;

#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int y = __shfl_up(x, d);

            if (lane >= d)
                x += y;
        }
        if (lane == 63)
            wsum[wv] = x;
        __syncthreads();
        if (wv == 0) {
            int t = lane < MU_T / 64 ? wsum[lane] : 0;

#pragma unroll
            for (int d = 1; d < MU_T / 64; d <<= 1) {
                const int y = __shfl_up(t, d);

                if (lane >= d)
                    t += y;
            }
            if (lane < MU_T / 64)
                wsum[lane] = t;
        }
        __syncthreads();
        off = x - cnt + (wv > 0 ? wsum[wv - 1] : 0);
        if (tid == MU_T - 1)
            count[0] = wsum[MU_T / 64 - 1];
    }
    for (int i = i0; i < i1; i++) {
        int j;

        if (keep(i, j)) {
            mi[off] = i;
            mj[off] = j;
            mconf[off] = rmax[i];
            cells[off] = make_int4(i % w, i / w, j % w, j / w);
            off++;
        }
    }
    bad = __syncthreads_or(bad);
    if (tid == 0)
        count[1] = bad;
}

extern "C" void eloftr_mutual(struct ops *o, cl_mem row_max, cl_mem row_arg, cl_mem col_arg,
                              int h, int w, int border, float thr, cl_mem mi, cl_mem mj,
                              cl_mem mconf, cl_mem cells, cl_mem count)
{
    ICOREG_API_BEGIN
    const char *op = "eloftr_mutual";
    const long long n = (long long)h * w;

    if (h < 1 || w < 1)
        icoreg_fatal("%s: invalid sizes h=%d w=%d", op, h, w);
    count32(n, op);
    need_floats(row_max, 0, n, op, "row_max");
    need_bytes(row_arg, 0, 4 * n, op, "row_arg");
    need_bytes(col_arg, 0, 4 * n, op, "col_arg");
    need_bytes(mi, 0, 4 * n, op, "mi");
    need_bytes(mj, 0, 4 * n, op, "mj");
    need_floats(mconf, 0, n, op, "mconf");
    need_bytes(cells, 0, 16 * n, op, "cells");
    need_bytes(count, 0, 8, op, "count");
    if ((uintptr_t)cells->ptr & 15)
        icoreg_fatal("%s: cells must be 16-byte aligned", op);
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(mutual_kernel, dim3(1), dim3(MU_T), 0, stream_of(o->ocl),
                       cfptr(row_max), (const int *)row_arg->ptr, (const int *)col_arg->ptr, h,
                       w, border, thr, (int *)mi->ptr, (int *)mj->ptr, fptr(mconf),
                       (int4 *)cells->ptr, (int *)count->ptr);
    launch_check(op);
    ICOREG_API_END
}

/* ---- MLP output LayerNorm + residual on channel-major maps -------------- */

/* X[b][c][j] += LayerNorm over c of M[b][c][j] (gain g, bias bt): the end
 * of an aggregated-attention block (eloftr.c:445-448: LayerNorm of the
 * MLP output per token, then x + message), on channel-major maps so that
 * neither operand is transposed. A block takes 64 tokens, one per lane;
 * its LNR_NW waves split the C <= 256 channels, each lane holding its
 * token's share in registers, so M is read once; the per-token sums are
 * combined across the waves in LDS. Reads of one channel row are 256
 * contiguous bytes per wave. T (or NULL) also receives the result
 * token-major, T[b][j][c]. */
#define LNR_MAXC 256
#define LNR_NW 16
__global__ void __launch_bounds__(64 * LNR_NW)
    chan_ln_add_kernel(const float *__restrict__ Mm, float *__restrict__ X,
                       const float *__restrict__ g,
                       const float *__restrict__ bt, int C, int n, float eps,
                       float *__restrict__ T)
{
    constexpr int CPW = LNR_MAXC / LNR_NW;
    __shared__ float part[2][LNR_NW][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = blockIdx.x * 64 + lane;
    const int cw = (C + LNR_NW - 1) / LNR_NW, c0 = wave * cw;
    const int nc = max(0, min(cw, C - c0));
    const long long base = (long long)blockIdx.y * C * n;
    const bool on = j < n;
    float v[CPW], xv[CPW];
    float s = 0.0f, mean, r;

    /* The residual's values load with the MLP output's: one round trip. */
#pragma unroll
    for (int k = 0; k < CPW; k++) {
        const bool in = on && k < nc;

        v[k] = in ? Mm[base + (long long)(c0 + k) * n + j] : 0.0f;
        xv[k] = in ? X[base + (long long)(c0 + k) * n + j] : 0.0f;
        s += v[k];
    }
    part[0][wave][lane] = s;
    __syncthreads();
    s = 0.0f;
#pragma unroll
    for (int w = 0; w < LNR_NW; w++)
        s += part[0][w][lane];
    mean = s / C;
    s = 0.0f;
#pragma unroll
    for (int k = 0; k < CPW; k++) {
        const float d = v[k] - mean;

        if (k < nc)
            s = fmaf(d, d, s);
    }
    part[1][wave][lane] = s;
    __syncthreads();
    s = 0.0f;
#pragma unroll
    for (int w = 0; w < LNR_NW; w++)
        s += part[1][w][lane];
    r = 1.0f / sqrtf(s / C + eps);
    if (!on)
        return;
#pragma unroll
    for (int k = 0; k < CPW; k++) {
        if (k < nc) {
            const int c = c0 + k;
            float u = (v[k] - mean) * r;

            u = u * g[c] + bt[c];
            xv[k] += u;
            X[base + (long long)c * n + j] = xv[k];
        }
    }
    if (T) {
        /* C % 64 == 0: every wave's channel share is whole float4s. */
        float4 *t = (float4 *)(T + base + (long long)j * C + c0);

#pragma unroll
        for (int q = 0; q < CPW / 4; q++)
            if (4 * q < nc)
                t[q] = make_float4(xv[4 * q], xv[4 * q + 1], xv[4 * q + 2], xv[4 * q + 3]);
    }
}

void eloftr_ln_residual(struct ops *o, cl_mem M, int nb, int C, int n,
                        cl_mem g, cl_mem b, float eps, cl_mem X, cl_mem T)
{
    const char *op = "eloftr_ln_residual";

    if (nb < 1 || nb > 65535 || C < 1 || C > LNR_MAXC || n < 1)
        icoreg_fatal("%s: invalid sizes nb=%d C=%d n=%d", op, nb, C, n);
    count32((long long)C * n, "channel map");
    need_floats(M, 0, (long long)nb * C * n, op, "M");
    need_floats(X, 0, (long long)nb * C * n, op, "X");
    need_floats(g, 0, C, op, "g");
    need_floats(b, 0, C, op, "b");
    if (T) {
        need_floats(T, 0, (long long)nb * C * n, op, "T");
        if (C % 64 || ((uintptr_t)T->ptr & 15))
            icoreg_fatal("%s: token-major copy needs C %% 64 == 0 and 16-byte alignment", op);
    }
    prof_scope ps(o->ocl, "ln_residual");
    hipLaunchKernelGGL(chan_ln_add_kernel, dim3((n + 63) / 64, nb),
                       dim3(64 * LNR_NW), 0, stream_of(o->ocl), cfptr(M), fptr(X),
                       cfptr(g), cfptr(b), C, n, eps, T ? fptr(T) : nullptr);
    launch_check(op);
}

/* ---- token aggregation of an attention block ------------------------- */

/* For tokens p = (ay, ax) of image b and channels c:
 *   q[p][c]  = sum_{i,j<4} wq[c][i][j] X[b][c][4 ay + i][4 ax + j]
 *   kv[p][c] = max_{i,j<4}          Y[b][c][4 ay + i][4 ax + j]
 * then each row LayerNorm over the channels (gain g, bias bt), written
 * token-major: eloftr.c:411-423 (depthwise 4 x 4 aggregation, 4 x 4 max
 * pooling, transposes to tokens, LayerNorm) in one launch. A block takes
 * AGG_T = 4 consecutive tokens and all 256 channels: (channel, token)
 * pair p of the block is c = p / 4, token p % 4, so the four lanes of a
 * channel read one 64-byte run of each window row (when the four tokens
 * share an aggregated row) and a wave instruction touches 16 runs, not
 * 64 scattered 16-byte pieces. The filters are staged in LDS,
 * the values go to LDS token-major, and wave t normalises token t of both
 * outputs. */
#define AGG_D 256
#define AGG_T 4
#define AGG_NT 1024 /* threads: one (channel, token) pair each */
__global__ void __launch_bounds__(AGG_NT)
    aggregate_kernel(const float *__restrict__ X, const float *__restrict__ Y,
                     long long img, const float *__restrict__ wq,
                     const float *__restrict__ g, const float *__restrict__ bt,
                     int h, int w, int aw, float eps, float *__restrict__ Q,
                     float *__restrict__ KV)
{
    static_assert(AGG_D / 64 == AGG_T, "one wave per token");
    __shared__ float sv[2][AGG_T][AGG_D];
    __shared__ __align__(16) float ws[AGG_D * 16];
    const int tid = threadIdx.x, b = blockIdx.y, na = (h / 4) * aw;
    const int p0 = blockIdx.x * AGG_T;
    constexpr int PP = AGG_D * AGG_T / AGG_NT; /* pairs per thread */
    float q[PP], kv[PP];

    *(float4 *)&ws[tid * 4] = *(const float4 *)(wq + tid * 4);
    {
        float4 xr[PP][4], yr[PP][4];

#pragma unroll
        for (int r = 0; r < PP; r++) {
            const int pr = tid + AGG_NT * r, c = pr / AGG_T, t = pr % AGG_T;
            const int p = min(p0 + t, na - 1), ay = p / aw, ax = p - ay * aw;
            const long long base = (long long)b * img + (long long)c * h * w +
                                   (long long)(4 * ay) * w + 4 * ax;

            /* Rows of a window are 16-byte aligned (w % 4 == 0). */
#pragma unroll
            for (int i = 0; i < 4; i++) {
                xr[r][i] = *(const float4 *)(X + base + i * w);
                yr[r][i] = *(const float4 *)(Y + base + i * w);
            }
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < PP; r++) {
            const int pr = tid + AGG_NT * r, c = pr / AGG_T;

            q[r] = 0.0f;
            kv[r] = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 wr = *(const float4 *)&ws[c * 16 + i * 4];

                q[r] = fmaf(wr.x, xr[r][i].x, q[r]);
                q[r] = fmaf(wr.y, xr[r][i].y, q[r]);
                q[r] = fmaf(wr.z, xr[r][i].z, q[r]);
                q[r] = fmaf(wr.w, xr[r][i].w, q[r]);
                kv[r] = fmaxf(kv[r], fmaxf(fmaxf(yr[r][i].x, yr[r][i].y),
                                           fmaxf(yr[r][i].z, yr[r][i].w)));
            }
        }
    }
#pragma unroll
    for (int r = 0; r < PP; r++) {
        const int pr = tid + AGG_NT * r, c = pr / AGG_T, t = pr % AGG_T;

        sv[0][t][c] = q[r];
        sv[1][t][c] = kv[r];
    }
    __syncthreads();
    if (tid < 64 * AGG_T && p0 + (tid >> 6) < na) {
        const int lane = tid & 63, t = tid >> 6;
        const long long row = (long long)b * na + p0 + t;

#pragma unroll
        for (int k = 0; k < 2; k++) {
            float v[AGG_D / 64], s = 0.0f, mean, r;

#pragma unroll
            for (int u = 0; u < AGG_D / 64; u++) {
                v[u] = sv[k][t][lane + 64 * u];
                s += v[u];
            }
            mean = wave_sum(s) / AGG_D;
            s = 0.0f;
#pragma unroll
            for (int u = 0; u < AGG_D / 64; u++) {
                v[u] -= mean;
                s = fmaf(v[u], v[u], s);
            }
            r = 1.0f / sqrtf(wave_sum(s) / AGG_D + eps);
#pragma unroll
            for (int u = 0; u < AGG_D / 64; u++) {
                const int cc = lane + 64 * u;

                (k ? KV : Q)[row * AGG_D + cc] = v[u] * r * g[cc] + bt[cc];
            }
        }
    }
}

void eloftr_aggregate(struct ops *o, cl_mem X, cl_mem Y, int nb, int C, int h,
                      int w, cl_mem wq, cl_mem g, cl_mem b, float eps,
                      cl_mem Q, cl_mem KV)
{
    const char *op = "eloftr_aggregate";
    const int ah = h / 4, aw = w / 4;
    const long long img = (long long)C * h * w;

    if (C != AGG_D || nb < 1 || nb > 65535 || h < 4 || w < 4 || h % 4 ||
        w % 4)
        icoreg_fatal("%s: invalid sizes C=%d nb=%d %dx%d", op, C, nb, h, w);
    if (((uintptr_t)X->ptr | (uintptr_t)Y->ptr | (uintptr_t)wq->ptr) & 15)
        icoreg_fatal("%s: X, Y and wq must be 16-byte aligned", op);
    need_floats(X, 0, nb * img, op, "X");
    need_floats(Y, 0, nb * img, op, "Y");
    need_floats(wq, 0, (long long)C * 16, op, "wq");
    need_floats(g, 0, C, op, "g");
    need_floats(b, 0, C, op, "b");
    need_floats(Q, 0, (long long)nb * ah * aw * C, op, "Q");
    need_floats(KV, 0, (long long)nb * ah * aw * C, op, "KV");
    prof_scope ps(o->ocl, "aggregate");
    hipLaunchKernelGGL(aggregate_kernel, dim3((ah * aw + AGG_T - 1) / AGG_T, nb),
                       dim3(AGG_NT), 0,
                       stream_of(o->ocl), cfptr(X), cfptr(Y), img, cfptr(wq),
                       cfptr(g), cfptr(b), h, w, aw, eps, fptr(Q), fptr(KV));
    launch_check(op);
}

extern "C" void eloftr_lse_block(struct ops *o, cl_mem S, int R, int N, int r0, cl_mem lse,
                                 cl_mem cm, cl_mem cs)
{
    ICOREG_API_BEGIN
    eloftr_lse_tiles(o, S, R, N, r0, lse, cm, cs);
    ICOREG_API_END
}

extern "C" void eloftr_conf_block(struct ops *o, cl_mem S, int R, int N, int r0, cl_mem lse,
                                  cl_mem cm, cl_mem cs, cl_mem rmax, cl_mem rarg, cl_mem cmax,
                                  cl_mem carg)
{
    ICOREG_API_BEGIN
    eloftr_conf_tiles(o, S, R, N, r0, lse, cm, cs, rmax, rarg, cmax, carg);
    ICOREG_API_END
}

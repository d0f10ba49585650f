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
 *  - warp sampling: one thread per (cell, group of 8 channels), the
 *    bilinear taps and weights computed once per group (the reference
 *    recomputes them per (cell, channel)), grid y over the groups;
 *  - local correlation: 4 x 4 cell patches; the products of the patch's
 *    cells with the union box of their windows on the matrix cores when
 *    the box is small (a per-cell path otherwise), then the bilinear
 *    combinations of those whole-cell products, as the reference forms
 *    them;
 *  - depthwise 5 x 5: 64 x 32 output tiles, 8 rows per thread, the
 *    (68 x 36) input patch loaded at once and staged in LDS, each
 *    thread's neighbourhood in registers. */

#include <hip/hip_runtime.h>

#include <limits.h>
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

/* One thread per (cell, group of channels): the cell's taps and weights
 * are computed once for its group, the group's channel planes read at
 * the same offsets (all loads of the group in flight together), and the
 * stores of a channel are 256 consecutive cells. The grid's y dimension
 * runs over the channel groups, so that a few thousand cells still fill
 * the GPU (11 664 cells x 512 channels at 1/8 of 864 x 864: 2944 blocks
 * instead of 46). */
#define WS_CG 8 /* channels per thread */

__global__ void __launch_bounds__(256)
    warp_sample_kernel(const float *__restrict__ in, int C, int H, int W,
                       const float *__restrict__ flow, float *__restrict__ out,
                       int coff)
{
    /* Block L -> (cell block, channel group), channel groups fastest; the
     * XCDs (L % 8) get contiguous bands of that order, so that the input
     * rows two neighbouring cell blocks share are fetched into one L2. */
    const int ng = (C + WS_CG - 1) / WS_CG, total = gridDim.x;
    const int q = total >> 3, rem = total & 7, x = blockIdx.x & 7, idx = blockIdx.x >> 3;
    const int ord = (x < rem ? x * (q + 1) : rem * (q + 1) + (x - rem) * q) + idx;
    const int n = H * W, i = (ord / ng) * 256 + threadIdx.x;
    const int c0 = (ord % ng) * WS_CG;
    bil b;
    bool in00, in01, in10, in11;
    int o00, o01, o10, o11;
    float v[WS_CG][4];

    if (i >= n)
        return;
    b = bilinear_setup(flow[i], flow[n + i], H, W);
    in00 = b.ok && b.x0 >= 0 && b.x0 < W && b.y0 >= 0 && b.y0 < H;
    in01 = b.ok && b.x0 + 1 >= 0 && b.x0 + 1 < W && b.y0 >= 0 && b.y0 < H;
    in10 = b.ok && b.x0 >= 0 && b.x0 < W && b.y0 + 1 >= 0 && b.y0 + 1 < H;
    in11 = b.ok && b.x0 + 1 >= 0 && b.x0 + 1 < W && b.y0 + 1 >= 0 &&
           b.y0 + 1 < H;
    o00 = in00 ? b.y0 * W + b.x0 : 0;
    o01 = in01 ? b.y0 * W + b.x0 + 1 : 0;
    o10 = in10 ? (b.y0 + 1) * W + b.x0 : 0;
    o11 = in11 ? (b.y0 + 1) * W + b.x0 + 1 : 0;
#pragma unroll
    for (int k = 0; k < WS_CG; k++) {
        const float *p = in + (long long)min(c0 + k, C - 1) * n;

        v[k][0] = in00 ? p[o00] : 0.0f;
        v[k][1] = in01 ? p[o01] : 0.0f;
        v[k][2] = in10 ? p[o10] : 0.0f;
        v[k][3] = in11 ? p[o11] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < WS_CG; k++)
        if (c0 + k < C)
            out[(long long)(coff + c0 + k) * n + i] =
                b.ok ? (1.0f - b.fy) * ((1.0f - b.fx) * v[k][0] + b.fx * v[k][1]) +
                           b.fy * ((1.0f - b.fx) * v[k][2] + b.fx * v[k][3])
                     : 0.0f;
}

/* ---- local correlation ------------------------------------------------------------- */

/* out[k, i] for the (2 r + 1)^2 offsets k of cell i is the bilinear
 * combination (at the warp's fractional position) of whole-cell dot
 * products S[e] = sum_c f1[c, i] / sqrt(C) * f2[c, e] over the cells e of
 * the (2 r + 2)^2 window at the warp's integer position (zero outside
 * the image), roma_kernels.cl:143-192.
 *
 * A block takes a 4 x 4 patch of cells. Neighbouring cells of a smooth
 * warp have overlapping windows, so the union of the patch's windows
 * (clipped to the image) is a box of about (4 + 2 r + 1)^2 cells instead
 * of 16 (2 r + 2)^2 reads. When the box holds at most LC_NB cells, the
 * block forms every patch-cell x box-cell product on the matrix cores
 * (v_mfma_f32_16x16x4f32: 16 cells x 16 box cells x 4 channels, box
 * tiles shared out over the 4 waves), each wave streaming its operands
 * from memory straight into registers with no LDS staging and no
 * barriers (32 channels of loads in flight per wave). Each cell then
 * reads its window's products from the box. Patches whose windows
 * scatter (far-off or broken warps) take the per-cell path instead: one
 * wave per cell, lanes over the window cells, channels in order.
 * Patches go to the XCDs in contiguous bands, so that neighbouring
 * patches share their f2 rows in one L2.
 *
 * Measured at 864 x 864 (1/8: C = 512, r = 3; 1/4: C = 256, r = 2) the
 * kernel is bound by L1 misses (each 4 x 4 patch touches its box rows
 * channel by channel, 16-44 bytes of every 128-byte line), not by HBM or
 * the matrix cores. */
#define CORR_MAXC 1024 /* channels accepted (the reference's kernel: 512) */
#define LC_T 16        /* cells of a patch (4 x 4) */
#define LC_NB 256      /* box cells on the matrix-core path */
#define LC_GS 260      /* LDS row pitch of the products */

typedef float lc_f4 __attribute__((ext_vector_type(4)));

/* Any patch counted by local_corr_scan_kernel (nc block counts). */
__device__ __forceinline__ bool lc_any_scattered(const int *__restrict__ counts, int nc)
{
    int any = 0;

    for (int i = 0; i < nc; i++)
        any |= counts[i];
    return any != 0;
}

/* Block L of T to a tile: the 8 XCDs (blocks L, L + 8, ... on XCD L % 8)
 * each get a contiguous band of tiles. */
__device__ __forceinline__ int lc_xcd_tile(int L, int T)
{
    const int q = T >> 3, rem = T & 7, x = L & 7, idx = L >> 3;

    return (x < rem ? x * (q + 1) : rem * (q + 1) + (x - rem) * q) + idx;
}

/* f1, f2 channel-major (C x n). t1, t2 (or NULL): the same maps
 * cell-major (n x C, C % 4 == 0), read by the per-cell path, whose window
 * reads then run along each window cell's own channel row. */
__global__ void __launch_bounds__(256)
    local_corr_kernel(const float *__restrict__ f1,
                      const float *__restrict__ f2, int C, int H, int W, int r,
                      const float *__restrict__ flow, float *__restrict__ out,
                      int coff, const float *__restrict__ t1,
                      const float *__restrict__ t2, const int *__restrict__ tcounts,
                      int tnc)
{
    __shared__ float G[LC_T * LC_GS]; /* products of the patch's cells */
    __shared__ int cid[LC_T], ox[LC_T], oy[LC_T], okc[LC_T];
    __shared__ float cfx[LC_T], cfy[LC_T];
    __shared__ int box[4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tiles_x = (W + 3) >> 2, ntiles = tiles_x * ((H + 3) >> 2);
    const int tile_id = lc_xcd_tile(blockIdx.x, ntiles);
    const int px0 = (tile_id % tiles_x) * 4, py0 = (tile_id / tiles_x) * 4;
    const int n = H * W, ps = 2 * r + 2, side = 2 * r + 1;
    const float rc = 1.0f / sqrtf((float)C);

    /* The patch's cells: window origins and the box of their windows. */
    if (tid < 64) {
        const int x = px0 + (tid & 3), y = py0 + ((tid >> 2) & 3);
        int lo_x = INT_MAX, lo_y = INT_MAX, hi_x = INT_MIN, hi_y = INT_MIN;

        if (tid < LC_T) {
            bil b = bilinear_setup(0.0f, 0.0f, H, W);
            int ci = -1;

            if (x < W && y < H) {
                ci = y * W + x;
                b = bilinear_setup(flow[ci], flow[n + ci], H, W, r);
            }
            cid[tid] = ci;
            okc[tid] = ci >= 0 && b.ok;
            ox[tid] = b.x0 - r;
            oy[tid] = b.y0 - r;
            cfx[tid] = b.fx;
            cfy[tid] = b.fy;
            if (ci >= 0 && b.ok) {
                lo_x = b.x0 - r;
                lo_y = b.y0 - r;
                hi_x = b.x0 - r + ps - 1;
                hi_y = b.y0 - r + ps - 1;
            }
        }
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) {
            lo_x = min(lo_x, __shfl_xor(lo_x, o, 16));
            lo_y = min(lo_y, __shfl_xor(lo_y, o, 16));
            hi_x = max(hi_x, __shfl_xor(hi_x, o, 16));
            hi_y = max(hi_y, __shfl_xor(hi_y, o, 16));
        }
        if (tid == 0) {
            lo_x = max(lo_x, 0);
            lo_y = max(lo_y, 0);
            hi_x = min(hi_x, W - 1);
            hi_y = min(hi_y, H - 1);
            box[0] = lo_x;
            box[1] = lo_y;
            box[2] = hi_x >= lo_x ? hi_x - lo_x + 1 : 0;
            box[3] = hi_y >= lo_y ? hi_y - lo_y + 1 : 0;
        }
    }
    __syncthreads();
    const int bx0 = box[0], by0 = box[1], bw = box[2], bh = box[3];
    const int nb = bw * bh;
    const bool tiled = nb <= LC_NB;

    if (tiled && nb > 0) {
        /* Each wave streams its box tiles' operands straight from memory
         * into registers (no LDS, no barriers): per step of 4 channels,
         * lane l reads f1 of patch cell l % 16 and f2 of box cell
         * 16 t + l % 16 of each of its tiles t, channel l / 16 of the step. */
        const int nt = (nb + 15) >> 4;
        const int acell = cid[lane & 15], kq = lane >> 4;
        unsigned boff[4];
        bool bon[4];
        lc_f4 acc[4];

#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int j = (wv + 4 * t) * 16 + (lane & 15);

            bon[t] = j < nb;
            boff[t] = bon[t] ? (unsigned)((by0 + j / bw) * W + bx0 + j % bw) : 0u;
            acc[t] = (lc_f4){0.0f, 0.0f, 0.0f, 0.0f};
        }
        const bool aon = acell >= 0;
        const unsigned aoff = aon ? (unsigned)acell : 0u;
        const int ntw = nt > wv ? (nt - wv + 3) >> 2 : 0; /* tiles of this wave */
        const int cmain = C & ~31;

        auto step = [&](int c, bool tail) {
            const bool cok = !tail || c < C;
            const long long base = (long long)c * n;
            const float a = aon && cok ? f1[base + aoff] * rc : 0.0f;
            float b[4];

#pragma unroll
            for (int t = 0; t < 4; t++)
                b[t] = t < ntw && bon[t] && cok ? f2[base + boff[t]] : 0.0f;
#pragma unroll
            for (int t = 0; t < 4; t++)
                if (t < ntw)
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b[t], acc[t], 0, 0, 0);
        };
        for (int c0 = 0; c0 < cmain; c0 += 32) {
#pragma unroll
            for (int s = 0; s < 8; s++)
                step(c0 + 4 * s + kq, false);
        }
        for (int c0 = cmain; c0 < C; c0 += 4)
            step(c0 + kq, true);
        /* Products to LDS: lane l holds rows 4 (l / 16) + v of the tile's
         * 16 x 16 block, column l % 16. */
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int tile = wv + 4 * t;

            if (tile < nt)
#pragma unroll
                for (int v = 0; v < 4; v++)
                    G[(4 * (lane >> 4) + v) * LC_GS + tile * 16 + (lane & 15)] = acc[t][v];
        }
    }
    else if (!tiled) {
        /* Per-cell path: wave wv takes cells wv, wv + 4, ...; S of cell m
         * over its own window goes to row m of G. */
        for (int m = wv; m < LC_T; m += 4) {
            const int i = cid[m];
            float a4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            int off[4];
            bool ok[4];

            if (i < 0 || !okc[m])
                continue;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int e = lane + 64 * q;
                const int yy = oy[m] + e / ps, xx = ox[m] + e % ps;

                ok[q] = e < ps * ps && xx >= 0 && xx < W && yy >= 0 && yy < H;
                off[q] = ok[q] ? yy * W + xx : 0;
            }
            if (t1 && lc_any_scattered(tcounts, tnc)) {
                /* Lane by lane along each window cell's own channel row
                 * (the copies exist: this patch was counted). */
                const float *pa = t1 + (long long)i * C;

                for (int c = 0; c < C; c += 4) {
                    const lc_f4 a = *(const lc_f4 *)(pa + c) * rc;

#pragma unroll
                    for (int q = 0; q < 4; q++)
                        if (ok[q]) {
                            const lc_f4 b = *(const lc_f4 *)(t2 + (long long)off[q] * C + c);

                            a4[q] = fmaf(a[0], b[0], a4[q]);
                            a4[q] = fmaf(a[1], b[1], a4[q]);
                            a4[q] = fmaf(a[2], b[2], a4[q]);
                            a4[q] = fmaf(a[3], b[3], a4[q]);
                        }
                }
            }
            else
                for (int c = 0; c < C; c++) {
                    const float a = f1[(long long)c * n + i] * rc;
                    const float *p = f2 + (long long)c * n;

#pragma unroll
                    for (int q = 0; q < 4; q++)
                        if (ok[q])
                            a4[q] = fmaf(a, p[off[q]], a4[q]);
                }
#pragma unroll
            for (int q = 0; q < 4; q++)
                if (lane + 64 * q < ps * ps)
                    G[m * LC_GS + lane + 64 * q] = a4[q];
        }
    }
    __syncthreads();
    /* Outputs: consecutive threads take consecutive cells of one offset. */
    for (int idx = tid; idx < LC_T * side * side; idx += 256) {
        const int m = idx & 15, k = idx >> 4;
        const int i = cid[m];

        if (i < 0)
            continue;
        float v = 0.0f;

        if (okc[m]) {
            const int ky = k / side, kx = k - ky * side;
            const int yy = oy[m] + ky, xx = ox[m] + kx;
            const float fx = cfx[m], fy = cfy[m];
            float s[4];

#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int y = yy + (q >> 1), x = xx + (q & 1);

                if (tiled)
                    s[q] = x >= bx0 && x < bx0 + bw && y >= by0 && y < by0 + bh
                               ? G[m * LC_GS + (y - by0) * bw + (x - bx0)]
                               : 0.0f;
                else
                    s[q] = G[m * LC_GS + (ky + (q >> 1)) * ps + kx + (q & 1)];
            }
            v = (1.0f - fy) * ((1.0f - fx) * s[0] + fx * s[1]) +
                fy * ((1.0f - fx) * s[2] + fx * s[3]);
        }
        out[(long long)(coff + k) * n + i] = v;
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

/* Depthwise 5 x 5 (+ bias, ReLU) of one channel plane per block tile:
 * 64 columns x 32 rows, one column per lane and 8 rows per thread. The
 * (36 x 68) input patch (1.2 times the tile, against 1.7 for a 32 x 8
 * tile) is loaded with every load issued before any is used, staged in
 * LDS, and each thread keeps the 12 x 5 neighbourhood of its 8 outputs in
 * registers, so each patch value is read from LDS about 1.2 times. Sums
 * in tap order, as the reference. */
#define DW_TW 64
#define DW_RPT 8
#define DW_TH (256 / DW_TW * DW_RPT)
#define DW_PW (DW_TW + 4)
#define DW_PH (DW_TH + 4)
#define DW_NL ((DW_PW * DW_PH + 255) / 256)

__global__ void __launch_bounds__(256)
    dwconv5_kernel(const float *__restrict__ in, int H, int W,
                   const float *__restrict__ wt, const float *__restrict__ bias,
                   float *__restrict__ out)
{
    __shared__ float t[DW_PH][DW_PW + 1];
    const int lx = threadIdx.x % DW_TW, g = threadIdx.x / DW_TW;
    const int x0 = blockIdx.x * DW_TW, y0 = blockIdx.y * DW_TH, c = blockIdx.z;
    const float *p = in + (long long)c * H * W;
    const float *w = wt + c * 25;
    float v[DW_NL], nb[DW_RPT + 4][5], wk[25];

#pragma unroll
    for (int q = 0; q < DW_NL; q++) {
        const int e = threadIdx.x + 256 * q, yy = y0 - 2 + e / DW_PW, xx = x0 - 2 + e % DW_PW;
        const bool ok = e < DW_PW * DW_PH && yy >= 0 && yy < H && xx >= 0 && xx < W;

        v[q] = p[ok ? (long long)yy * W + xx : 0];
        v[q] = ok ? v[q] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < 25; k++)
        wk[k] = w[k];
#pragma unroll
    for (int q = 0; q < DW_NL; q++) {
        const int e = threadIdx.x + 256 * q;

        if (e < DW_PW * DW_PH)
            t[e / DW_PW][e % DW_PW] = v[q];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < DW_RPT + 4; r++)
#pragma unroll
        for (int j = 0; j < 5; j++)
            nb[r][j] = t[g * DW_RPT + r][lx + j];
    {
        const int x = x0 + lx;
        const float b = bias[c];

#pragma unroll
        for (int r = 0; r < DW_RPT; r++) {
            const int y = y0 + g * DW_RPT + r;
            float acc = b;

#pragma unroll
            for (int i = 0; i < 5; i++)
#pragma unroll
                for (int j = 0; j < 5; j++)
                    acc = fmaf(nb[r + i][j], wk[i * 5 + j], acc);
            if (x < W && y < H)
                out[((long long)c * H + y) * W + x] = fmaxf(acc, 0.0f);
        }
    }
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
    if ((long long)nblk(n, 256) * nblk(C, WS_CG) >= (1LL << 31))
        icoreg_fatal("%s: grid too large", op);
    hipLaunchKernelGGL(warp_sample_kernel, dim3(nblk(n, 256) * nblk(C, WS_CG)), dim3(256),
                       0, stream_of(o->ocl), cfptr(in), C, H, W, cfptr(flow),
                       fptr(out), coff);
    launch_check(op);
    ICOREG_API_END
}

/* Patches whose windows do not fit one LC_NB-cell box (the per-cell path
 * of local_corr_kernel), counted per block of 256 patches into
 * counts[blockIdx.x]: one thread per 4 x 4 patch, the box formed as the
 * kernel forms it. */
__global__ void __launch_bounds__(256)
    local_corr_scan_kernel(const float *__restrict__ flow, int H, int W, int r,
                           int *__restrict__ counts)
{
    const int tiles_x = (W + 3) >> 2, ntiles = tiles_x * ((H + 3) >> 2);
    const int t = blockIdx.x * 256 + threadIdx.x, n = H * W, ps = 2 * r + 2;
    const int px0 = (t % tiles_x) * 4, py0 = (t / tiles_x) * 4;
    int lo_x = INT_MAX, lo_y = INT_MAX, hi_x = INT_MIN, hi_y = INT_MIN;

    for (int c = 0; c < LC_T && t < ntiles; c++) {
        const int x = px0 + (c & 3), y = py0 + (c >> 2);

        if (x < W && y < H) {
            const int ci = y * W + x;
            const bil b = bilinear_setup(flow[ci], flow[n + ci], H, W, r);

            if (b.ok) {
                lo_x = min(lo_x, b.x0 - r);
                lo_y = min(lo_y, b.y0 - r);
                hi_x = max(hi_x, b.x0 - r + ps - 1);
                hi_y = max(hi_y, b.y0 - r + ps - 1);
            }
        }
    }
    lo_x = max(lo_x, 0);
    lo_y = max(lo_y, 0);
    hi_x = min(hi_x, W - 1);
    hi_y = min(hi_y, H - 1);
    {
        const int bw = hi_x >= lo_x ? hi_x - lo_x + 1 : 0, bh = hi_y >= lo_y ? hi_y - lo_y + 1 : 0;
        const int nsc = __syncthreads_count(t < ntiles && bw * bh > LC_NB);

        if (threadIdx.x == 0)
            counts[blockIdx.x] = nsc;
    }
}


/* (C x n) to (n x C) for both maps, 32 x 32 tiles through LDS, the grid
 * striding over the tiles of both; nothing when no patch scatters (then
 * the launch costs a few microseconds). */
__global__ void __launch_bounds__(256)
    lc_transpose_kernel(const float *__restrict__ f1, const float *__restrict__ f2,
                        float *__restrict__ o1, float *__restrict__ o2, int C, int n,
                        const int *__restrict__ counts, int nc)
{
    __shared__ float t[32][33];
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    const int tiles_i = (n + 31) / 32, tiles = tiles_i * ((C + 31) / 32);

    if (!lc_any_scattered(counts, nc))
        return;
    for (int u = blockIdx.x; u < 2 * tiles; u += gridDim.x) {
        const int z = u >= tiles, v = u - z * tiles;
        const int i0 = (v % tiles_i) * 32, c0 = (v / tiles_i) * 32;
        const float *in = z ? f2 : f1;
        float *out = z ? o2 : o1;

        __syncthreads();
#pragma unroll
        for (int k = 0; k < 32; k += 8) {
            const int c = c0 + ty + k, i = i0 + tx;

            if (c < C && i < n)
                t[ty + k][tx] = in[(long long)c * n + i];
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 32; k += 8) {
            const int i = i0 + ty + k, c = c0 + tx;

            if (c < C && i < n)
                out[(long long)i * C + c] = t[tx][ty + k];
        }
    }
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
    /* Byte offsets inside a 16-channel chunk stay below 2^31. */
    if (n >= (1LL << 25))
        icoreg_fatal("%s: %lld cells (at most 2^25)", op, n);
    need_floats(f1, 0, (long long)C * n, op, "f1");
    need_floats(f2, 0, (long long)C * n, op, "f2");
    need_floats(flow, 0, 2 * n, op, "flow");
    need_floats(out, (long long)coff * n, (long long)(2 * r + 1) * (2 * r + 1) * n,
                op, "out");
    {
        const int tiles = ((W + 3) / 4) * ((H + 3) / 4);
        const dim3 grid((unsigned)tiles);
        hipStream_t st = stream_of(o->ocl);

        prof_scope ps(o->ocl, op);
        if (C % 4 == 0) {
            /* Cell-major copies for the per-cell path, made only when a
             * patch scatters (counted first on the device). */
            const size_t cn = (size_t)C * n;
            const int nc = (tiles + 255) / 256;
            cl_mem sc = scratch_get(o, 2 * cn * sizeof(float) + (size_t)nc * sizeof(int));
            float *t1 = (float *)sc->ptr, *t2 = t1 + cn;
            int *counts = (int *)(t2 + cn);
            const long long ttiles = 2LL * ((n + 31) / 32) * ((C + 31) / 32);
            const dim3 tg((unsigned)(ttiles < 2048 ? ttiles : 2048));

            hipLaunchKernelGGL(local_corr_scan_kernel, dim3((unsigned)nc), dim3(256), 0, st,
                               cfptr(flow), H, W, r, counts);
            hipLaunchKernelGGL(lc_transpose_kernel, tg, dim3(256), 0, st, cfptr(f1), cfptr(f2),
                               t1, t2, C, (int)n, (const int *)counts, nc);
            hipLaunchKernelGGL(local_corr_kernel, grid, dim3(256), 0, st, cfptr(f1),
                               cfptr(f2), C, H, W, r, cfptr(flow), fptr(out), coff,
                               (const float *)t1, (const float *)t2, (const int *)counts, nc);
        }
        else
            hipLaunchKernelGGL(local_corr_kernel, grid, dim3(256), 0, st, cfptr(f1),
                               cfptr(f2), C, H, W, r, cfptr(flow), fptr(out), coff, nullptr,
                               nullptr, nullptr, 0);
    }
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
                       dim3(nblk(W, DW_TW), nblk(H, DW_TH), (unsigned)C),
                       dim3(256), 0, stream_of(o->ocl), cfptr(in), H, W,
                       cfptr(w), cfptr(bias), fptr(out));
    launch_check(op);
    ICOREG_API_END
}

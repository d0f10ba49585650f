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
 *  - warp sampling: one thread per (cell, group of 4 or 8 channels), the
 *    bilinear taps and weights computed once per group (the reference
 *    recomputes them per (cell, channel)), blocks over the groups;
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

/* One thread per (cell, group of CG channels): the cell's taps and
 * weights are computed once for its group, the group's channel planes
 * read at the same offsets (all loads of the group in flight together),
 * and the stores of a channel are 256 consecutive cells, non-temporal
 * (the map is written once and read by the next kernel). A block takes
 * 256 cells of one channel group, so that a few thousand cells still fill
 * the GPU (11 664 cells x 512 channels at 1/8 of 864 x 864: 2944 blocks
 * instead of 46). CG is 8, or 4 when that leaves fewer idle channel slots;
 * maps of up to 16 channels (the 1/1 refiner's 9) take one thread per
 * cell (CG 16), so that the flow and taps of a cell are read and formed
 * once. Slots past C issue no loads (the test is the same for the whole
 * block). */
template <int CG>
__global__ void __launch_bounds__(256)
    warp_sample_kernel(const float *__restrict__ in, int C, int H, int W,
                       const float *__restrict__ flow, float *__restrict__ out,
                       int coff)
{
    /* Block L -> (channel group, cell block), cell blocks fastest; the
     * XCDs (L % 8) get contiguous bands of that order, so that the input
     * rows two neighbouring cell blocks share are fetched into one L2. */
    const int n = H * W, ncb = (n + 255) / 256, total = gridDim.x;
    const int q = total >> 3, rem = total & 7, x = blockIdx.x & 7, idx = blockIdx.x >> 3;
    const int ord = (x < rem ? x * (q + 1) : rem * (q + 1) + (x - rem) * q) + idx;
    const int i = (ord % ncb) * 256 + threadIdx.x;
    const int c0 = (ord / ncb) * CG;
    bil b;
    bool in00, in01, in10, in11;
    int o00, o01, o10, o11;
    float v[CG][4];

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
    for (int k = 0; k < CG; k++) {
        if (c0 + k >= C)
            break;
        const float *p = in + (long long)(c0 + k) * n;

        v[k][0] = in00 ? p[o00] : 0.0f;
        v[k][1] = in01 ? p[o01] : 0.0f;
        v[k][2] = in10 ? p[o10] : 0.0f;
        v[k][3] = in11 ? p[o11] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < CG; k++)
        if (c0 + k < C)
            __builtin_nontemporal_store(
                b.ok ? (1.0f - b.fy) * ((1.0f - b.fx) * v[k][0] + b.fx * v[k][1]) +
                           b.fy * ((1.0f - b.fx) * v[k][2] + b.fx * v[k][3])
                     : 0.0f,
                &out[(long long)(coff + c0 + k) * n + i]);
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
 * of 16 (2 r + 2)^2 reads. When the box holds at most LC_NB cells
 * (LC_NB2 in the cell-major kernel), the
 * block forms every patch-cell x box-cell product on the matrix cores
 * (v_mfma_f32_16x16x4f32: 16 cells x 16 box cells x 4 channels), each
 * wave streaming its operands from memory straight into registers with
 * no LDS staging and no barriers. Each cell then reads its window's
 * products from the box. Patches whose windows scatter (far-off or
 * broken warps) take a per-cell path instead. Patches go to the XCDs in
 * contiguous bands, so that neighbouring patches share their f2 rows in
 * one L2.
 *
 * Two forms:
 *  - cell-major (C % 4 == 0, local_corr_cm_kernel): f2 is first
 *    transposed to (n x C), so that a box cell's channels are one
 *    contiguous row: every box operand load is 16 bytes of a lane's own
 *    4 channels, and a 16-channel chunk of a cell is one 64-byte piece;
 *    f1 (16 cells a patch, each read once) stays channel-major, four
 *    4-byte loads for a lane's 4 channels.
 *    Each of the 4 waves takes all box tiles over a quarter of the
 *    channels (so a patch or box row is loaded once per block), and the
 *    quarters' products meet in LDS. The per-cell path puts 16
 *    lanes on each window cell (4 window cells per load instruction,
 *    256 contiguous bytes each) and sums the 16 lanes by DPP;
 *  - channel-major (other C, local_corr_kernel): operands read straight
 *    from the (C x n) maps, 4-byte loads of 4 channels x 16 cells per
 *    instruction (16-44 bytes of every 128-byte line: bound by L1
 *    misses), the box tiles shared out over the 4 waves; per-cell path:
 *    one wave per cell, lanes over the window cells, channels in order. */
#define CORR_MAXC 1024 /* channels accepted (the reference's kernel: 512) */
#define LC_T 16        /* cells of a patch (4 x 4) */
#define LC_NB 256      /* box cells on the matrix-core path */
#define LC_GS 260      /* LDS row pitch of the products */
#define LC_PG 148      /* LDS row pitch of a channel-quarter plane (<= 144 box cells) */
/* The cell-major kernel's limits: boxes of up to 25 tiles stay on the
 * matrix cores (radius 7 on a smooth warp: 19 x 19 = 361 cells), rows of
 * its products LC_GS2 floats apart (4 LC_GS2 = 16 mod 64 banks, as for
 * LC_GS). */
#define LC_NB2 400
#define LC_GS2 404

typedef float lc_f4 __attribute__((ext_vector_type(4)));

/* Block L of T to a tile: the 8 XCDs (blocks L, L + 8, ... on XCD L % 8)
 * each get a contiguous band of tiles. */
__device__ __forceinline__ int lc_xcd_tile(int L, int T)
{
    const int q = T >> 3, rem = T & 7, x = L & 7, idx = L >> 3;

    return (x < rem ? x * (q + 1) : rem * (q + 1) + (x - rem) * q) + idx;
}

/* A patch's cells (index, or -1 outside the map; whether the warp is
 * finite; window origin; bilinear fractions) and the box of their
 * windows clipped to the map (x0, y0, width, height). */
struct lc_patch {
    int cid[LC_T], ox[LC_T], oy[LC_T], okc[LC_T];
    float cfx[LC_T], cfy[LC_T];
    int box[4];
};

/* Fills p for the 4 x 4 patch at (px0, py0) from threads 0..63; the
 * caller's barrier follows. */
__device__ __forceinline__ void lc_setup(lc_patch &p, const float *__restrict__ flow, int H,
                                         int W, int r, int px0, int py0, int tid)
{
    const int n = H * W, ps = 2 * r + 2;

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
            p.cid[tid] = ci;
            p.okc[tid] = ci >= 0 && b.ok;
            p.ox[tid] = b.x0 - r;
            p.oy[tid] = b.y0 - r;
            p.cfx[tid] = b.fx;
            p.cfy[tid] = b.fy;
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
            p.box[0] = lo_x;
            p.box[1] = lo_y;
            p.box[2] = hi_x >= lo_x ? hi_x - lo_x + 1 : 0;
            p.box[3] = hi_y >= lo_y ? hi_y - lo_y + 1 : 0;
        }
    }
}

/* The outputs of the patch: out[coff + k, i] for its cells i and the
 * (2 r + 1)^2 offsets k, the bilinear combination of the cell's window
 * products. Tiled: np partial planes G + j pstride (rows gs apart, row m
 * x box cell) added in order j = 0 .. np - 1; else G row m (gs
 * apart) holds cell m's (2 r + 2)^2 window. Consecutive threads take
 * consecutive cells of one offset. */
__device__ __forceinline__ void lc_outputs(const lc_patch &p, const float *G, int np, int pstride,
                                           int gs, bool tiled, int r, int n,
                                           float *__restrict__ out, int coff, int tid)
{
    const int ps = 2 * r + 2, side = 2 * r + 1;
    const int bx0 = p.box[0], by0 = p.box[1], bw = p.box[2], bh = p.box[3];

    for (int idx = tid; idx < LC_T * side * side; idx += 256) {
        const int m = idx & 15, k = idx >> 4;
        const int i = p.cid[m];

        if (i < 0)
            continue;
        float v = 0.0f;

        if (p.okc[m]) {
            const int ky = k / side, kx = k - ky * side;
            const int yy = p.oy[m] + ky, xx = p.ox[m] + kx;
            const float fx = p.cfx[m], fy = p.cfy[m];
            float s[4];

#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int y = yy + (q >> 1), x = xx + (q & 1);

                if (tiled) {
                    const int e = m * gs + (y - by0) * bw + (x - bx0);
                    const bool in = x >= bx0 && x < bx0 + bw && y >= by0 && y < by0 + bh;
                    float v2 = 0.0f;

                    if (in) {
                        v2 = G[e];
                        for (int j = 1; j < np; j++)
                            v2 += G[e + j * pstride];
                    }
                    s[q] = v2;
                }
                else
                    s[q] = G[m * gs + (ky + (q >> 1)) * ps + kx + (q & 1)];
            }
            v = (1.0f - fy) * ((1.0f - fx) * s[0] + fx * s[1]) +
                fy * ((1.0f - fx) * s[2] + fx * s[3]);
        }
        out[(long long)(coff + k) * n + i] = v;
    }
}

/* Channel-major form: f1, f2 (C x n). */
__global__ void __launch_bounds__(256)
    local_corr_kernel(const float *__restrict__ f1,
                      const float *__restrict__ f2, int C, int H, int W, int r,
                      const float *__restrict__ flow, float *__restrict__ out,
                      int coff)
{
    __shared__ float G[LC_T * LC_GS]; /* products of the patch's cells */
    __shared__ lc_patch pt;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tiles_x = (W + 3) >> 2, ntiles = tiles_x * ((H + 3) >> 2);
    const int tile_id = lc_xcd_tile(blockIdx.x, ntiles);
    const int n = H * W, ps = 2 * r + 2;
    const float rc = 1.0f / sqrtf((float)C);
    const int *cid = pt.cid, *okc = pt.okc, *ox = pt.ox, *oy = pt.oy;

    lc_setup(pt, flow, H, W, r, (tile_id % tiles_x) * 4, (tile_id / tiles_x) * 4, tid);
    __syncthreads();
    const int *box = pt.box;
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
    lc_outputs(pt, G, 1, 0, LC_GS, tiled, r, n, out, coff, tid);
}

/* Sum over the 16 lanes of each DPP row (every lane of the row gets it). */
__device__ __forceinline__ float lc_row_sum(float v)
{
    v += dpp_f(v, 0xB1);
    v += dpp_f(v, 0x4E);
    v += dpp_f(v, 0x141);
    v += dpp_f(v, 0x140);
    return v;
}

/* Loads at or past this byte offset of a buffer window return zeros. */
#define LC_OOB 0x80000000u

/* Raw buffer window over bytes bytes from p (< 2^31). */
__device__ __forceinline__ __amdgpu_buffer_rsrc_t lc_rsrc(const float *p, unsigned bytes)
{
    /* Word 3: 32-bit data, the gfx9-family raw buffer format. */
    return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ lc_f4 lc_load4(__amdgpu_buffer_rsrc_t r, unsigned off)
{
    return __builtin_bit_cast(lc_f4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

/* Four channels of one cell of a channel-major map: floats at byte
 * offsets off, off + ps, off + 2 ps, off + 3 ps (ps: a channel plane's
 * bytes); LC_OOB gives zeros. */
__device__ __forceinline__ lc_f4 lc_load_planes4(__amdgpu_buffer_rsrc_t r, unsigned off,
                                                 unsigned ps)
{
    lc_f4 v;

#pragma unroll
    for (int s = 0; s < 4; s++)
        v[s] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)(off == LC_OOB ? LC_OOB
                                                                             : off + s * ps),
                                                        0, 0));
    return v;
}

/* NQ box tiles of the cell-major tiled path for one wave: the 16-channel
 * chunks kw, kw + 4, ... (nch chunks in all) into acc[t]. ra: window
 * over f1 (channel-major), ao: byte offset of the lane's patch cell in
 * its first channel's plane (channel 4 kq; LC_OOB: none), ps: a plane's
 * bytes; rb: window over the cell-major f2, bo[t]: byte offset of the
 * lane's box cell row of tile t (LC_OOB: none) plus 16 (4 kq) for its
 * channels. A chunk past C or a missing cell loads zeros from past the
 * window's end, so that the loop has no branches and two chunks load
 * while two multiply. */
template <int NQ>
__device__ __forceinline__ void lc_cm_tiles(__amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb,
                                            unsigned ao, unsigned ps, const unsigned (&bo)[9],
                                            int kw, int nch, int C, int kq, float rc,
                                            lc_f4 (&acc)[9])
{
    auto load = [&](int q, lc_f4 &a, lc_f4 (&b)[NQ]) {
        const int c = q * 16 + 4 * kq;
        const bool cok = q < nch && c < C;
        const unsigned cb = 64u * q;

        a = lc_load_planes4(ra, cok && ao != LC_OOB ? ao + 16u * q * ps : LC_OOB, ps) * rc;
#pragma unroll
        for (int t = 0; t < NQ; t++)
            b[t] = lc_load4(rb, cok && bo[t] != LC_OOB ? bo[t] + cb : LC_OOB);
    };
    auto mul = [&](const lc_f4 &a, const lc_f4 (&b)[NQ]) {
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int t = 0; t < NQ; t++)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[t][s], acc[t], 0, 0, 0);
    };
    lc_f4 a0, a1, b0[NQ], b1[NQ];

    /* The scheduling barriers keep this order: the compiler would
     * otherwise gather both chunks' loads at the end of the body and wait
     * for all of them at its top. */
    load(kw, a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    load(kw + 4, a1, b1);
    __builtin_amdgcn_sched_barrier(0);
    for (int q = kw; q < nch; q += 8) {
        mul(a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        load(q + 8, a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        mul(a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        load(q + 12, a1, b1);
        __builtin_amdgcn_sched_barrier(0);
    }
}

/* LDS of a cell-major block: the staging ring's two buffers, or
 * afterwards the product planes. A ring buffer holds one 32-channel
 * chunk: 20 rows of 8 box cells (128 bytes a cell, its eight 4-channel
 * groups in slots swizzled by the cell: slot p holds group p ^ ((cell /
 * 2) % 8), so that the 16 cells an operand read takes spread over the
 * banks), then the patch's 16 cells x 32 channels (channel c of cell m at
 * 16 (8 (c % 4) + c / 4) + m, so that the four channels one MFMA step
 * reads fall into different banks). */
#define LC_RBOX 5120
#define LC_RBUF (LC_RBOX + 512)
#define LC_SM (2 * LC_RBUF > 2 * LC_T * LC_GS2 ? 2 * LC_RBUF : 2 * LC_T * LC_GS2)

/* The staged path of the cell-major kernel for one wave's NTW box tiles
 * (tw, tw + 2, ...) over its half h of every chunk's channels. Chunk q
 * (channels 32 q ..) is loaded into registers two chunks ahead (load: 6
 * 16-byte loads a lane), written to ring buffer q % 2 a chunk ahead
 * (store), one barrier a chunk; the wave's products accumulate into acc.
 * In MFMA step s a lane's k index kq stands for channel 16 h + 4 kq + s
 * of the chunk in both operands; the box operand is one 16-byte LDS read
 * of the lane's cell (its group 4 h + kq), the patch operand one 4-byte
 * read a step, times rc = 1 / sqrt(C) as the reference scales f1. */
template <int NTW, typename Load, typename Store>
__device__ __forceinline__ void lc_ring_tiles(float *sm, int nq, int h, int tw, int lane, float rc,
                                              Load &&load, Store &&store, lc_f4 (&acc)[5])
{
    const int m = lane & 15, kq = lane >> 4;
    const int ao = LC_RBOX + 16 * (4 * h + kq) + m;
    const int bo = 32 * m + 4 * ((4 * h + kq) ^ (m >> 1)) + 512 * tw;
    lc_f4 st[6];

    load(0, st);
    store(st, sm);
    load(1, st);
    for (int q = 0; q < nq; q++) {
        const float *buf = sm + (q & 1) * LC_RBUF;

        /* Buffer q % 2 is written; the other one is read by no wave. */
        __syncthreads();
        store(st, sm + ((q + 1) & 1) * LC_RBUF);
        load(q + 2, st);
        float a[4];
        lc_f4 b[NTW > 0 ? NTW : 1];

#pragma unroll
        for (int s = 0; s < 4; s++)
            a[s] = buf[ao + 128 * s] * rc;
#pragma unroll
        for (int i = 0; i < NTW; i++)
            b[i] = *(const lc_f4 *)(buf + bo + 1024 * i);
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int i = 0; i < NTW; i++)
                acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[i][s], acc[i], 0, 0, 0);
    }
    __syncthreads();
}

/* Cell-major form: f1 (C x n) as it is, t2 is f2 as (n x C) with rows
 * ld floats apart (C % 4 == 0, ld % 4 == 0, t2 16-byte aligned, C n 4 and
 * n ld 4 below 2^31). The patch's own cells are 16 of n, read a channel
 * plane at a time; the box cells, read (2 r + 2)^2-fold over the
 * patches, are the ones worth a contiguous channel row. */
__global__ void __launch_bounds__(256)
    local_corr_cm_kernel(const float *__restrict__ f1, const float *__restrict__ t2, int C,
                         int ld, int H, int W, int r, const float *__restrict__ flow,
                         float *__restrict__ out, int coff, int ring)
{
    /* The staging ring (ring path), then the products of the patch's
     * cells: two planes LC_T x LC_PG (ring path), four planes LC_T x LC_PG
     * (tiled path, at most 144 box cells), two planes LC_T x LC_GS2 (tiled
     * path, more), or LC_T rows LC_GS2 apart (per-cell path's windows). */
    __shared__ __align__(16) float sm[LC_SM];
    float *const G = sm;
    __shared__ lc_patch pt;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tiles_x = (W + 3) >> 2, ntiles = tiles_x * ((H + 3) >> 2);
    const int tile_id = lc_xcd_tile(blockIdx.x, ntiles);
    const int n = H * W, ps = 2 * r + 2;
    const float rc = 1.0f / sqrtf((float)C);
    const int m = lane & 15, kq = lane >> 4;

    lc_setup(pt, flow, H, W, r, (tile_id % tiles_x) * 4, (tile_id / tiles_x) * 4, tid);
    __syncthreads();
    const int bx0 = pt.box[0], by0 = pt.box[1], bw = pt.box[2], bh = pt.box[3];
    const int nb = bw * bh;
    const bool tiled = nb <= LC_NB2;

    if (ring && nb > 0 && nb <= 144) {
        /* Boxes of up to 9 tiles with C % 32 == 0 and W % 4 == 0: both
         * operands staged through LDS a 32-channel chunk at a time (box
         * rows 128 bytes a cell from the cell-major map, the patch's rows
         * of 4 cells from the channel planes, each loaded once per block),
         * the next chunk's loads in flight during this chunk's products.
         * Wave wv takes the tiles wv / 2, wv / 2 + 2, ... over half wv % 2
         * of the channels; the halves meet in two planes. */
        const int nt = (nb + 15) >> 4, h = wv & 1, tw = wv >> 1;
        const int ntw = nt > tw ? (nt - tw + 1) >> 1 : 0;
        const int nq = C >> 5;
        const unsigned pbytes = (unsigned)n * 4u;
        const __amdgpu_buffer_rsrc_t ra = lc_rsrc(f1, (unsigned)C * pbytes);
        const __amdgpu_buffer_rsrc_t rb = lc_rsrc(t2, (unsigned)n * (unsigned)ld * 4u);
        const int px0 = (tile_id % tiles_x) * 4, py0 = (tile_id / tiles_x) * 4;
        /* Box rows wv + 4 j: lane l loads cell 8 (wv + 4 j) + l / 8,
         * channel group (l % 8) ^ ((cell / 2) % 8); past the box, zeros. */
        unsigned boff[5];

#pragma unroll
        for (int j = 0; j < 5; j++) {
            const int e = 8 * (wv + 4 * j) + (lane >> 3);
            const int g = (lane & 7) ^ ((e >> 1) & 7);

            boff[j] = e < nb ? ((unsigned)((by0 + e / bw) * W + bx0 + e % bw) * (unsigned)ld +
                                4u * (unsigned)g) *
                                   4u
                             : LC_OOB;
        }
        /* Patch row wv % 2 (waves 2, 3 repeat the rows of 0, 1): lane l
         * loads slot 64 (wv % 2) + l, 4 cells of row y = l % 4 of channel
         * 4 (c' % 8) + c' / 8, c' = slot / 4. */
        const int fsl = 64 * (wv & 1) + lane, fcp = fsl >> 2, fy = fsl & 3;
        const int fc = 4 * (fcp & 7) + (fcp >> 3);
        const unsigned foff =
            py0 + fy < H ? ((unsigned)fc * (unsigned)n + (unsigned)((py0 + fy) * W + px0)) * 4u
                         : LC_OOB;
        /* Chunk q's 6 loads of this lane (past C: zeros), and their LDS
         * slots: box row wv + 4 j at 256 (wv + 4 j) + 4 l floats, patch
         * row wv % 2 at LC_RBOX + 256 (wv % 2) + 4 l (waves 2, 3 write
         * the same values as 0, 1). */
        auto load = [&](int q, lc_f4 (&st)[6]) {
            const bool in = q < nq;
            const unsigned cb = 128u * (unsigned)q, fb = 32u * (unsigned)q * pbytes;

#pragma unroll
            for (int j = 0; j < 5; j++)
                st[j] = lc_load4(rb, in && boff[j] != LC_OOB ? boff[j] + cb : LC_OOB);
            st[5] = lc_load4(ra, in && foff != LC_OOB ? foff + fb : LC_OOB);
        };
        auto store = [&](const lc_f4 (&st)[6], float *buf) {
#pragma unroll
            for (int j = 0; j < 5; j++)
                *(lc_f4 *)(buf + 256 * (wv + 4 * j) + 4 * lane) = st[j];
            *(lc_f4 *)(buf + LC_RBOX + 256 * (wv & 1) + 4 * lane) = st[5];
        };
        lc_f4 acc[5];

#pragma unroll
        for (int i = 0; i < 5; i++)
            acc[i] = (lc_f4){0.0f, 0.0f, 0.0f, 0.0f};
        switch (ntw) {
        case 0:
            lc_ring_tiles<0>(sm, nq, h, tw, lane, rc, load, store, acc);
            break;
        case 1:
            lc_ring_tiles<1>(sm, nq, h, tw, lane, rc, load, store, acc);
            break;
        case 2:
            lc_ring_tiles<2>(sm, nq, h, tw, lane, rc, load, store, acc);
            break;
        case 3:
            lc_ring_tiles<3>(sm, nq, h, tw, lane, rc, load, store, acc);
            break;
        case 4:
            lc_ring_tiles<4>(sm, nq, h, tw, lane, rc, load, store, acc);
            break;
        default:
            lc_ring_tiles<5>(sm, nq, h, tw, lane, rc, load, store, acc);
        }
        /* Lane l holds rows 4 (l / 16) + v of each tile's 16 x 16 block,
         * column l % 16; plane h. */
        {
            const int m = lane & 15, kq = lane >> 4;
            float *Gh = G + h * LC_T * LC_PG;

#pragma unroll
            for (int i = 0; i < 5; i++)
                if (i < ntw)
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        Gh[(4 * kq + v) * LC_PG + (tw + 2 * i) * 16 + m] = acc[i][v];
        }
        __syncthreads();
        lc_outputs(pt, G, 2, LC_T * LC_PG, LC_PG, true, r, n, out, coff, tid);
        return;
    }
    if (tiled) {
        /* Wave wv takes the 16-channel chunks wv, wv + 4, ... of all box
         * tiles (up to nine at a time), so that each patch and box row is loaded
         * once per block. Per chunk lane l reads channels 4 (l / 16) .. + 3
         * of patch cell l % 16 and of box cell 16 t + l % 16 of each tile t
         * as one 16-byte load; in MFMA step s the lane's k index (l / 16)
         * stands for channel 4 (l / 16) + s of the chunk, the same channel
         * in both operands. The four channel quarters' products meet in
         * LDS in a fixed order: with at most 9 tiles each wave stores into
         * its own plane (LC_PG pitch) and the outputs add the four planes;
         * with more, per 8 tiles waves 2 and 3 store into two planes
         * (LC_GS2 pitch), waves 0 and 1 add theirs after a barrier, and the
         * outputs add the two planes. */
        const int nt = (nb + 15) >> 4, nch = (C + 15) >> 4;
        const int acell = pt.cid[m];
        const unsigned pb = (unsigned)n * 4u; /* bytes of a channel plane */
        const __amdgpu_buffer_rsrc_t ra = lc_rsrc(f1, (unsigned)C * pb);
        const __amdgpu_buffer_rsrc_t rb = lc_rsrc(t2, (unsigned)n * (unsigned)ld * 4u);
        const unsigned ao = acell >= 0 ? (4u * kq * (unsigned)n + (unsigned)acell) * 4u : LC_OOB;
        const bool four = nt <= 9;
        const int gp = four ? LC_PG : LC_GS2, gsz = four ? 9 : 8;
        float *Gw = G + (four ? wv : (wv & 1)) * LC_T * gp;

        for (int u0 = 0; u0 < nt; u0 += gsz) {
            const int nq = nt - u0 < gsz ? nt - u0 : gsz;
            unsigned bo[9];
            lc_f4 acc[9];

#pragma unroll
            for (int t = 0; t < 9; t++) {
                const int j = (u0 + t) * 16 + m;

                bo[t] = t < nq && j < nb
                            ? ((unsigned)((by0 + j / bw) * W + bx0 + j % bw) * ld + 4 * kq) * 4u
                            : LC_OOB;
                acc[t] = (lc_f4){0.0f, 0.0f, 0.0f, 0.0f};
            }
            switch (nq) {
            case 1:
                lc_cm_tiles<1>(ra, rb, ao, pb, bo, wv, nch, C, kq, rc, acc);
                break;
            case 2:
                lc_cm_tiles<2>(ra, rb, ao, pb, bo, wv, nch, C, kq, rc, acc);
                break;
            case 3:
                lc_cm_tiles<3>(ra, rb, ao, pb, bo, wv, nch, C, kq, rc, acc);
                break;
            case 4:
                lc_cm_tiles<4>(ra, rb, ao, pb, bo, wv, nch, C, kq, rc, acc);
                break;
            case 5:
                lc_cm_tiles<5>(ra, rb, ao, pb, bo, wv, nch, C, kq, rc, acc);
                break;
            case 6:
                lc_cm_tiles<6>(ra, rb, ao, pb, bo, wv, nch, C, kq, rc, acc);
                break;
            case 7:
                lc_cm_tiles<7>(ra, rb, ao, pb, bo, wv, nch, C, kq, rc, acc);
                break;
            case 8:
                lc_cm_tiles<8>(ra, rb, ao, pb, bo, wv, nch, C, kq, rc, acc);
                break;
            default:
                lc_cm_tiles<9>(ra, rb, ao, pb, bo, wv, nch, C, kq, rc, acc);
            }
            /* Lane l holds rows 4 (l / 16) + v of the tile's 16 x 16 block,
             * column l % 16. */
            if (four || wv >= 2)
#pragma unroll
                for (int t = 0; t < 9; t++)
                    if (t < nq)
#pragma unroll
                        for (int v = 0; v < 4; v++)
                            Gw[(4 * kq + v) * gp + (u0 + t) * 16 + m] = acc[t][v];
            if (!four) {
                __syncthreads();
                if (wv < 2)
#pragma unroll
                    for (int t = 0; t < 9; t++)
                        if (t < nq)
#pragma unroll
                            for (int v = 0; v < 4; v++)
                                Gw[(4 * kq + v) * gp + (u0 + t) * 16 + m] += acc[t][v];
            }
        }
    }
    else {
        /* Per-cell path: wave wv takes cells wv, wv + 4, ...; 16 window
         * cells e = e0 + 4 u + (l / 16) at a time, lane l summing channels
         * 4 (l % 16) .. + 3 of every 64 of its window cells, the 16 lanes
         * of a row then added by DPP; S of cell mm over its window goes to
         * row mm of G. */
        const int np2 = ps * ps;
        const unsigned pb = (unsigned)n * 4u;
        const __amdgpu_buffer_rsrc_t ra = lc_rsrc(f1, (unsigned)C * pb);
        const __amdgpu_buffer_rsrc_t rb = lc_rsrc(t2, (unsigned)n * (unsigned)ld * 4u);

        for (int mm = wv; mm < LC_T; mm += 4) {
            const int i = pt.cid[mm];

            if (i < 0 || !pt.okc[mm])
                continue;
            const unsigned ao = (unsigned)i * 4u;

            for (int e0 = 0; e0 < np2; e0 += 16) {
                unsigned bo[4];
                float sum[4];

#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int e = e0 + 4 * u + kq;
                    const int yy = pt.oy[mm] + e / ps, xx = pt.ox[mm] + e % ps;
                    const bool ok = e < np2 && xx >= 0 && xx < W && yy >= 0 && yy < H;

                    bo[u] = ok ? (unsigned)(yy * W + xx) * ld * 4u : LC_OOB;
                    sum[u] = 0.0f;
                }
                for (int c = 4 * m; c < C; c += 64) {
                    const lc_f4 a = lc_load_planes4(ra, ao + (unsigned)c * pb, pb) * rc;

#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const lc_f4 b = lc_load4(rb, bo[u] == LC_OOB ? LC_OOB : bo[u] + 4u * c);

                        sum[u] = fmaf(a[0], b[0], sum[u]);
                        sum[u] = fmaf(a[1], b[1], sum[u]);
                        sum[u] = fmaf(a[2], b[2], sum[u]);
                        sum[u] = fmaf(a[3], b[3], sum[u]);
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int e = e0 + 4 * u + kq;
                    const float v = lc_row_sum(sum[u]);

                    if (m == 0 && e < np2)
                        G[mm * LC_GS2 + e] = v;
                }
            }
        }
    }
    __syncthreads();
    {
        const bool four = ((nb + 15) >> 4) <= 9;

        lc_outputs(pt, G, four ? 4 : 2, LC_T * (four ? LC_PG : LC_GS2), four ? LC_PG : LC_GS2,
                   tiled, r, n, out, coff, tid);
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

/* Depthwise 5 x 5 (+ bias, ReLU) over a block tile of 64 columns x 32
 * rows, one column per lane and 8 rows per thread, for DW_CPB consecutive
 * channel planes in turn. The (36 x 68) input patch (1.2 times the tile,
 * against 1.7 for a 32 x 8 tile) is staged in LDS, and each thread keeps
 * the 12 x 5 neighbourhood of its 8 outputs in registers, so each patch
 * value is read from LDS about 1.2 times. The next channel's patch is
 * loaded into registers while the current one is computed (prefetching
 * two channels ahead needs 164 registers a thread and measured slower).
 * Sums in tap order, as the reference. */
#define DW_TW 64
#define DW_RPT 8
#define DW_TH (256 / DW_TW * DW_RPT)
#define DW_PW (DW_TW + 4)
#define DW_PH (DW_TH + 4)
#define DW_NL ((DW_PW * DW_PH + 255) / 256)
#define DW_CPB 4

__global__ void __launch_bounds__(256)
    dwconv5_kernel(const float *__restrict__ in, int C, int H, int W,
                   const float *__restrict__ wt, const float *__restrict__ bias,
                   float *__restrict__ out)
{
    __shared__ float t[DW_PH][DW_PW + 1];
    const int lx = threadIdx.x % DW_TW, g = threadIdx.x / DW_TW;
    const int x0 = blockIdx.x * DW_TW, y0 = blockIdx.y * DW_TH;
    const int cb = blockIdx.z * DW_CPB, ce = min(C, cb + DW_CPB);
    const long long HW = (long long)H * W;
    const int x = x0 + lx;
    float v[DW_NL], nb[DW_RPT + 4][5];
    /* This thread's patch elements: offset in a channel plane, -1 outside
     * the map. */
    int so[DW_NL];

#pragma unroll
    for (int q = 0; q < DW_NL; q++) {
        const int e = threadIdx.x + 256 * q, yy = y0 - 2 + e / DW_PW, xx = x0 - 2 + e % DW_PW;
        const bool ok = e < DW_PW * DW_PH && yy >= 0 && yy < H && xx >= 0 && xx < W;

        so[q] = ok ? yy * W + xx : -1;
    }
    auto fetch = [&](int c) {
        const float *p = in + c * HW;

#pragma unroll
        for (int q = 0; q < DW_NL; q++)
            v[q] = so[q] >= 0 ? p[so[q]] : 0.0f;
    };
    fetch(cb);
    for (int c = cb; c < ce; c++) {
        if (c > cb)
            __syncthreads();
#pragma unroll
        for (int q = 0; q < DW_NL; q++) {
            const int e = threadIdx.x + 256 * q;

            if (e < DW_PW * DW_PH)
                t[e / DW_PW][e % DW_PW] = v[q];
        }
        __syncthreads();
        if (c + 1 < ce)
            fetch(c + 1);
#pragma unroll
        for (int r = 0; r < DW_RPT + 4; r++)
#pragma unroll
            for (int j = 0; j < 5; j++)
                nb[r][j] = t[g * DW_RPT + r][lx + j];

        const float *w = wt + c * 25;
        const float b = bias[c];

#pragma unroll
        for (int r = 0; r < DW_RPT; r++) {
            const int y = y0 + g * DW_RPT + r;
            float acc = b;

#pragma unroll
            for (int i = 0; i < 5; i++)
#pragma unroll
                for (int j = 0; j < 5; j++)
                    acc = fmaf(nb[r + i][j], w[i * 5 + j], acc);
            if (x < W && y < H)
                out[c * HW + (long long)y * W + x] = fmaxf(acc, 0.0f);
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
    {
        const int cg = C <= 16 ? 16 : sample_cg(C);

        if ((long long)nblk(n, 256) * nblk(C, cg) >= (1LL << 31))
            icoreg_fatal("%s: grid too large", op);
        if (cg == 16)
            hipLaunchKernelGGL(warp_sample_kernel<16>, dim3(nblk(n, 256)), dim3(256), 0,
                               stream_of(o->ocl), cfptr(in), C, H, W, cfptr(flow), fptr(out),
                               coff);
        else if (cg == 4)
            hipLaunchKernelGGL(warp_sample_kernel<4>, dim3(nblk(n, 256) * nblk(C, 4)), dim3(256),
                               0, stream_of(o->ocl), cfptr(in), C, H, W, cfptr(flow), fptr(out),
                               coff);
        else
            hipLaunchKernelGGL(warp_sample_kernel<8>, dim3(nblk(n, 256) * nblk(C, 8)), dim3(256),
                               0, stream_of(o->ocl), cfptr(in), C, H, W, cfptr(flow), fptr(out),
                               coff);
    }
    launch_check(op);
    ICOREG_API_END
}

/* (C x n) to (n x C), output rows ld floats apart: one 64-cell x
 * 64-channel tile per block through LDS. VEC (n % 4 == 0, C % 4 == 0,
 * ld % 4 == 0, the input 16-byte aligned): 16-byte loads along the cells
 * and 16-byte stores along the channels. */
template <bool VEC>
__global__ void __launch_bounds__(256)
    lc_transpose_kernel(const float *__restrict__ in, float *__restrict__ out, int C, int ld,
                        int n)
{
    __shared__ float t[64][65];
    const int tid = threadIdx.x;
    const int tiles_i = (n + 63) / 64, v = blockIdx.x;
    const int i0 = (v % tiles_i) * 64, c0 = (v / tiles_i) * 64;

    if (VEC) {
        const int j4 = (tid & 15) * 4, row = tid >> 4;
        lc_f4 x[4];

#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int c = c0 + row + 16 * k, i = i0 + j4;

            x[k] = c < C && i < n ? *(const lc_f4 *)(in + (long long)c * n + i)
                                  : (lc_f4){0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                t[row + 16 * k][j4 + e] = x[k][e];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = i0 + row + 16 * k, c = c0 + j4;

            if (i < n && c < C)
                *(lc_f4 *)(out + (long long)i * ld + c) =
                    (lc_f4){t[j4][row + 16 * k], t[j4 + 1][row + 16 * k],
                            t[j4 + 2][row + 16 * k], t[j4 + 3][row + 16 * k]};
        }
    }
    else {
        const int tx = tid & 63, ty = tid >> 6;

        for (int k = 0; k < 64; k += 4) {
            const int c = c0 + ty + k, i = i0 + tx;

            if (c < C && i < n)
                t[ty + k][tx] = in[(long long)c * n + i];
        }
        __syncthreads();
        for (int k = 0; k < 64; k += 4) {
            const int i = i0 + ty + k, c = c0 + tx;

            if (c < C && i < n)
                out[(long long)i * ld + c] = t[tx][ty + k];
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
        /* Cell-major row pitch: whole 256-byte units, an odd number of
         * them, so that the 16 rows one load instruction reads at the same
         * channel offset fall into different memory channels (a pitch of
         * 2^k bytes sends them all to one or two); rows under 256 bytes
         * are left unpadded. */
        long long ld = C;

        if (C >= 64) {
            ld = (C + 63) / 64 * 64;
            if ((ld / 64) % 2 == 0)
                ld += 64;
        }
        if (C % 4 == 0 && ld * n * 4 < (1LL << 31)) {
            /* f2 cell-major into the scratch buffer (its start is 256-byte
             * aligned, and ld % 4 == 0 keeps every row 16-byte aligned),
             * then the cell-major kernel (its buffer windows take byte
             * offsets below 2^31; C n 4 <= ld n 4). */
            const size_t cn = (size_t)ld * n;
            cl_mem sc = scratch_get(o, cn * sizeof(float));
            float *t2 = (float *)sc->ptr;
            const long long ttiles = ((n + 63) / 64) * ((C + 63) / 64);
            const bool vec = n % 4 == 0 && ((uintptr_t)cfptr(f2) & 15) == 0;

            if (ttiles >= (1LL << 31))
                icoreg_fatal("%s: transpose grid too large", op);
            if (vec)
                hipLaunchKernelGGL(lc_transpose_kernel<true>, dim3((unsigned)ttiles), dim3(256),
                                   0, st, cfptr(f2), t2, C, (int)ld, (int)n);
            else
                hipLaunchKernelGGL(lc_transpose_kernel<false>, dim3((unsigned)ttiles), dim3(256),
                                   0, st, cfptr(f2), t2, C, (int)ld, (int)n);
            /* The staging ring takes whole 32-channel chunks and rows of
             * 4 patch cells that are wholly inside or outside the map. */
            const int ring = C % 32 == 0 && W % 4 == 0;

            hipLaunchKernelGGL(local_corr_cm_kernel, grid, dim3(256), 0, st, cfptr(f1),
                               (const float *)t2, C, (int)ld, H, W, r, cfptr(flow), fptr(out),
                               coff, ring);
        }
        else
            hipLaunchKernelGGL(local_corr_kernel, grid, dim3(256), 0, st, cfptr(f1),
                               cfptr(f2), C, H, W, r, cfptr(flow), fptr(out), coff);
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

/* A refiner block on C <= 32 channels (C % 8 == 0) in one pass: the
 * depthwise 5 x 5 + bias + ReLU of dwconv5_kernel (same tap order), then
 * the 1 x 1 convolution (pw: C x C, row k for output channel k; pb) that
 * follows it, the depthwise results kept in registers instead of a
 * C x H x W map written and read back. A block takes 64 columns (one a
 * lane) x 8 rows (two a thread); the input patch goes through LDS four
 * channels at a time, the next four loaded into registers meanwhile; the
 * weights are uniform across the block (scalar loads). */
#define DP_TW 64
#define DP_TH 8
#define DP_CC 4
template <int C>
__global__ void __launch_bounds__(256)
    dwpw_small_kernel(const float *__restrict__ in, int H, int W,
                      const float *__restrict__ dw, const float *__restrict__ db,
                      const float *__restrict__ pw, const float *__restrict__ pb,
                      float *__restrict__ out)
{
    constexpr int TR = 2, PR = DP_TH + 4, PC = DP_TW + 4, PN = DP_CC * PR * PC;
    constexpr int NP = (PN + 255) / 256;
    static_assert(C % DP_CC == 0 && C <= 32, "channels");
    __shared__ float patch[DP_CC][PR][PC + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int x0 = blockIdx.x * DP_TW, y0 = blockIdx.y * DP_TH, ry = wave * TR;
    const long long HW = (long long)H * W;
    float acc[TR][C], rp[NP];
    /* This thread's patch elements: offset from channel c0's plane (cc HW
     * + pixel), -1 outside the map; the same for every chunk. */
    int so[NP];

#pragma unroll
    for (int p = 0; p < TR; p++)
#pragma unroll
        for (int k = 0; k < C; k++)
            acc[p][k] = 0.0f;
#pragma unroll
    for (int q = 0; q < NP; q++) {
        const int e = tid + 256 * q, cc = e / (PR * PC), rem = e - cc * (PR * PC);
        const int r = rem / PC, col = rem - r * PC;
        const int gy = y0 + r - 2, gx = x0 + col - 2;
        const bool ok = e < PN && gy >= 0 && gy < H && gx >= 0 && gx < W;

        so[q] = ok ? (int)(cc * HW + (long long)gy * W + gx) : -1;
    }
    /* The patch of channels c0 .. c0 + 3 into registers (zero outside the
     * map). */
    auto fetch = [&](int c0) {
        const float *base = in + c0 * HW;

#pragma unroll
        for (int q = 0; q < NP; q++)
            rp[q] = so[q] >= 0 ? base[so[q]] : 0.0f;
    };
    fetch(0);
    for (int c0 = 0; c0 < C; c0 += DP_CC) {
#pragma unroll
        for (int q = 0; q < NP; q++) {
            const int e = tid + 256 * q, cc = e / (PR * PC), rem = e - cc * (PR * PC);

            if (e < PN)
                patch[cc][rem / PC][rem % PC] = rp[q];
        }
        __syncthreads();
        if (c0 + DP_CC < C)
            fetch(c0 + DP_CC);
#pragma unroll
        for (int cc = 0; cc < DP_CC; cc++) {
            const int c = c0 + cc;
            float win[TR + 4][5];

#pragma unroll
            for (int i = 0; i < TR + 4; i++)
#pragma unroll
                for (int j = 0; j < 5; j++)
                    win[i][j] = patch[cc][ry + i][lane + j];
#pragma unroll
            for (int p = 0; p < TR; p++) {
                float a = db[c];

#pragma unroll
                for (int i = 0; i < 5; i++)
#pragma unroll
                    for (int j = 0; j < 5; j++)
                        a = fmaf(win[p + i][j], dw[c * 25 + i * 5 + j], a);
                a = fmaxf(a, 0.0f);
#pragma unroll
                for (int k = 0; k < C; k++)
                    acc[p][k] = fmaf(pw[k * C + c], a, acc[p][k]);
            }
        }
        __syncthreads();
    }
    const int x = x0 + lane;

#pragma unroll
    for (int p = 0; p < TR; p++) {
        const int yy = y0 + ry + p;

        if (x < W && yy < H)
#pragma unroll
            for (int k = 0; k < C; k++)
                out[k * HW + (long long)yy * W + x] = acc[p][k] + pb[k];
    }
}

extern "C" void roma_dwpw_small(struct ops *o, cl_mem in, int C, int H, int W, cl_mem dw,
                                cl_mem db, cl_mem pw, cl_mem pb, cl_mem out)
{
    ICOREG_API_BEGIN
    const char *op = "roma_dwpw_small";

    if (C < 8 || C > 32 || C % 8 != 0 || H < 1 || W < 1)
        icoreg_fatal("%s: invalid sizes C=%d H=%d W=%d (C one of 8, 16, 24, 32)", op, C, H, W);
    count32((long long)C * H * W, op);
    need_floats(in, 0, (long long)C * H * W, op, "in");
    need_floats(dw, 0, 25LL * C, op, "dw");
    need_floats(db, 0, C, op, "db");
    need_floats(pw, 0, (long long)C * C, op, "pw");
    need_floats(pb, 0, C, op, "pb");
    need_floats(out, 0, (long long)C * H * W, op, "out");
    {
        /* Blocks read their input patches while others write: the two
         * maps' byte ranges must be disjoint (views of one buffer too). */
        const char *a = (const char *)in->ptr, *b = (const char *)out->ptr;
        const size_t nb = (size_t)C * H * W * sizeof(float);

        if (a < b + nb && b < a + nb)
            icoreg_fatal("%s: in and out must not overlap", op);
    }
    if ((long long)DP_CC * H * W >= (1LL << 31))
        icoreg_fatal("%s: %d x %d map too large", op, H, W);
    prof_scope ps(o->ocl, op);
    const dim3 grid(nblk(W, DP_TW), nblk(H, DP_TH));
    hipStream_t s = stream_of(o->ocl);

    switch (C) {
    case 8:
        hipLaunchKernelGGL(dwpw_small_kernel<8>, grid, dim3(256), 0, s, cfptr(in), H, W,
                           cfptr(dw), cfptr(db), cfptr(pw), cfptr(pb), fptr(out));
        break;
    case 16:
        hipLaunchKernelGGL(dwpw_small_kernel<16>, grid, dim3(256), 0, s, cfptr(in), H, W,
                           cfptr(dw), cfptr(db), cfptr(pw), cfptr(pb), fptr(out));
        break;
    case 24:
        hipLaunchKernelGGL(dwpw_small_kernel<24>, grid, dim3(256), 0, s, cfptr(in), H, W,
                           cfptr(dw), cfptr(db), cfptr(pw), cfptr(pb), fptr(out));
        break;
    default:
        hipLaunchKernelGGL(dwpw_small_kernel<32>, grid, dim3(256), 0, s, cfptr(in), H, W,
                           cfptr(dw), cfptr(db), cfptr(pw), cfptr(pb), fptr(out));
        break;
    }
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
                       dim3(nblk(W, DW_TW), nblk(H, DW_TH), nblk(C, DW_CPB)),
                       dim3(256), 0, stream_of(o->ocl), cfptr(in), C, H, W,
                       cfptr(w), cfptr(bias), fptr(out));
    launch_check(op);
    ICOREG_API_END
}

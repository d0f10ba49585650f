/* SPDX-License-Identifier: Unlicense */

/* fp32 GEMM on the CDNA4 matrix cores: C = act(alpha A op(B) + bias) + R.
 *
 * The contract is the reference's gemm / gemm_big (ops.cl:39-284 of
 * i.coregistration.opencl): batched over nb = nb0 * nb1 with two batch
 * strides per operand, B either K x N or N x K, bias per row or column,
 * activation, residual that may alias C. The design is gfx950's own:
 *
 *  - 4, 8 or 16 wave64s in a WGM x WGN arrangement; each wave owns a
 *    (BM/WGM) x (BN/WGN) block of the output as 32 x 32 tiles
 *    accumulated by v_mfma_f32_32x32x2f32 (4096 flop per instruction,
 *    full fp32 matrix rate);
 *  - BK = 16 or 32 slices of A and B staged through LDS, double-buffered: the
 *    next slice is fetched from HBM/L2 into registers (16-byte loads
 *    when rows are aligned) while the matrix cores work on the current
 *    one, then written to the other LDS buffer two MFMA steps before
 *    the slice ends; one barrier per slice;
 *  - operands are read through buffer windows over the tile's rows, so
 *    rows and columns past the matrix edge read 0 from the window's
 *    range check instead of a branch per load, and the per-thread
 *    offsets are computed once;
 *  - LDS operand reads run two MFMA steps ahead of their use;
 *  - LDS holds both operands k-major ([k][m], [k][n]) so that the 32
 *    lanes of an MFMA operand read 32 consecutive floats;
 *  - the B operand of a convolution is gathered from the (C, H, W) input
 *    on the fly (implicit GEMM): no unfold buffer, one pass over the
 *    input per output tile, the optional DISK normalisation and PReLU
 *    gate applied while gathering;
 *  - output tiles are assigned so that each of the 8 XCDs (one L2 each)
 *    works on a contiguous band of tiles, which share A rows in its L2. */

#include <algorithm>
#include <hip/hip_runtime.h>

#include "act.h"
#include "bilinear.h"
#include "gemm.h"

typedef float floatx16 __attribute__((ext_vector_type(16)));

#define GEMM_PAD 4

/* Offset past the end of every window: the load reads 0. */
#define GEMM_OOB 0x80000000u
/* gfx9 s_waitcnt immediate: vmcnt(0), expcnt and lgkmcnt not waited on. */
#define GEMM_WAIT_VM0 0x0F70

/* Word 3 of a raw buffer resource on gfx9-family parts: 32-bit data. */
#define GEMM_RSRC_FLAGS 0x00020000

/* Buffer window of `bytes` bytes from p: loads at byte offsets at or past
 * its end return 0. */
static __device__ __forceinline__ __amdgpu_buffer_rsrc_t
gemm_rsrc(const float *p, long long bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0,
                                             (int)(unsigned)bytes,
                                             GEMM_RSRC_FLAGS);
}

/* Four consecutive floats at byte offset off of window r: one 16-byte
 * load (VEC: the four are either all inside the window or all past its
 * end), else four 4-byte loads. */
template <bool VEC>
__device__ __forceinline__ float4 gemm_load4(__amdgpu_buffer_rsrc_t r,
                                             unsigned off)
{
    if (VEC)
        return __builtin_bit_cast(
            float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
    float4 v;

    v.x = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
    v.y = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off + 4, 0, 0));
    v.z = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off + 8, 0, 0));
    v.w = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off + 12, 0, 0));
    return v;
}

/* Components i of v with lo + i >= hi set to 0. */
__device__ __forceinline__ float4 mask4(float4 v, int lo, int hi)
{
    v.x = lo < hi ? v.x : 0.0f;
    v.y = lo + 1 < hi ? v.y : 0.0f;
    v.z = lo + 2 < hi ? v.z : 0.0f;
    v.w = lo + 3 < hi ? v.w : 0.0f;
    return v;
}

/* Most pieces a cut GEMM tile is split into. */
#define GEMM_MAX_SPLIT 8

/* Output tile of linear block id L among T tiles: blocks are dealt to
 * the 8 XCDs round-robin (L % 8), so give XCD x the x-th contiguous
 * band of tiles. A bijection of 0..T-1. */
__device__ __forceinline__ int xcd_tile(int L, int T)
{
    const int q = T >> 3, rem = T & 7, x = L & 7, idx = L >> 3;

    return (x < rem ? x * (q + 1) : rem * (q + 1) + (x - rem) * q) + idx;
}

/* C = act(alpha acc + bias) + R for the TM x TN 32 x 32 tiles of a wave
 * whose block of C starts at (r0, c0), batch (b0, b1). Register r of a
 * tile holds row (r / 4) * 8 + (lane / 32) * 4 + r % 4, column lane % 32. */
template <int TM, int TN>
__device__ __forceinline__ void gemm_epilogue(const gemm_args &g, const floatx16 (&acc)[TM][TN],
                                              long long b0, long long b1, int r0, int c0,
                                              int lane)
{
    float *C = g.C + b0 * g.sc0 + b1 * g.sc1;
    const float *R =
        g.R ? (g.rup ? g.R + b0 * g.rs0 : g.R + b0 * g.sc0 + b1 * g.sc1) : nullptr;

#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int col = c0 + j * 32 + (lane & 31);
            const int ry = g.rup ? col / g.rwo : 0, rx = g.rup ? col - ry * g.rwo : 0;

            if (col >= g.N)
                continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = r0 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                float v;

                if (row >= g.M)
                    continue;
                v = g.alpha * acc[i][j][r];
                if (g.bias)
                    v += g.bias[g.biasrow ? row : col];
                if (R && g.rpre)
                    v += bl_up(R + (long long)row * g.rh * g.rw, g.rh, g.rw, g.rsc, ry, rx);
                v = icoreg_act(v, g.act, g.slope);
                if (R && !g.rpre)
                    v += g.rup ? bl_up(R + (long long)row * g.rh * g.rw, g.rh, g.rw, g.rsc, ry,
                                       rx)
                               : R[(long long)row * g.ldc + col];
                C[(long long)row * g.ldc + col] = v;
            }
        }
}

/* BM x BN output tile, BK slice, WGM x WGN waves (each a
 * BM / WGM x BN / WGN block of 32 x 32 MFMA tiles). */
template <int BM, int BN, int BK, int MODE, bool VA, bool VB, int WGM = 2,
          int WGN = 2>
__global__ void __launch_bounds__(64 * WGM * WGN) gemm_mfma(const gemm_args g)
{
    constexpr int NTH = 64 * WGM * WGN;
    constexpr int LDSA = BM + GEMM_PAD, LDSB = BN + GEMM_PAD;
    constexpr int TM = BM / WGM / 32, TN = BN / WGN / 32;
    constexpr int KQ = BK / 4;            /* float4 per row of a slice */
    constexpr int A4 = BM * BK / 4 / NTH; /* float4 loads of A per thread */
    constexpr int B4 = BN * BK / 4 / NTH; /* dense B */
    constexpr int BE = BN * BK / NTH;     /* gathered B elements */
    constexpr int NS = BK / 2;            /* MFMA steps per slice */
    constexpr int PF = 2;                 /* LDS reads run PF steps ahead */
    static_assert(A4 >= 1 && BM * BK % (4 * NTH) == 0 &&
                      BN * BK % (4 * NTH) == 0 && NTH % BN == 0,
                  "tile shape");
    __shared__ float As[2][BK * LDSA];
    __shared__ float Bs[2][BK * LDSB];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int tiles_n = (g.N + BN - 1) / BN;
    const int tiles = tiles_n * ((g.M + BM - 1) / BM);
    const int nk = (g.K + BK - 1) / BK;
    /* Unit (tile) L; units from nfull on are cut into pieces over the
     * k slices. */
    int L = blockIdx.x, piece = -1, kt0 = 0, kt1 = nk;

    if (g.split > 1 && L >= g.nfull) {
        const int p = L - g.nfull;

        piece = p % g.split;
        L = g.nfull + p / g.split;
        kt0 = piece * nk / g.split;
        kt1 = (piece + 1) * nk / g.split;
    }
    const int tile = xcd_tile(L, tiles);
    const int m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;
    const long long bt = blockIdx.y, b0 = bt / g.nb1, b1 = bt % g.nb1;
    const float *A = g.A + b0 * g.sa0 + b1 * g.sa1;
    const float *B = g.B + b0 * g.sb0 + b1 * g.sb1;
    const int M = g.M, N = g.N, K = g.K;
    const long long lda = g.lda, ldb = g.ldb;
    /* Rows of A and columns of B inside the matrix for this tile. */
    const int rows_a = min(BM, M - m0), cols_b = min(BN, N - n0);
    const float *Ablk = A + m0 * lda;

    float4 ra[A4], rb[B4 > 0 ? B4 : 1];
    float rg[MODE == GEMM_B_CONV ? BE : 1];
    unsigned aoff[A4], boff[B4 > 0 ? B4 : 1];
    floatx16 acc[TM][TN];

    /* Byte offsets inside the windows, the same for every slice: A rows
     * past rows_a (and B rows past cols_b for B given N x K) land past
     * the window's end and read 0. */
#pragma unroll
    for (int e = 0; e < A4; e++) {
        const int q = tid + NTH * e, row = q / KQ, kq = (q % KQ) * 4;

        aoff[e] = (unsigned)((row * lda + kq) * 4);
    }
    if (MODE == GEMM_B_NK) {
#pragma unroll
        for (int e = 0; e < B4; e++) {
            const int q = tid + NTH * e, row = q / KQ, kq = (q % KQ) * 4;

            boff[e] = (unsigned)((row * ldb + kq) * 4);
        }
    }
    else if (MODE == GEMM_B_KN) {
#pragma unroll
        for (int e = 0; e < B4; e++) {
            const int q = tid + NTH * e, kk = q / (BN / 4);
            const int nq = (q % (BN / 4)) * 4;

            boff[e] = (unsigned)((kk * ldb + nq) * 4);
        }
    }

    /* Convolution gather: this thread's output column is fixed. */
    const int cn = tid % BN, ck0 = tid / BN;
    int cy = 0, cx = 0;
    bool cvalid = false;
    if (MODE == GEMM_B_CONV) {
        const int p = n0 + cn;

        cvalid = p < N;
        cy = cvalid ? (p / g.wo) * g.sy - g.py : 0;
        cx = cvalid ? (p % g.wo) * g.sx - g.px : 0;
    }

    for (int i = 0; i < TM; i++)
        for (int j = 0; j < TN; j++)
            for (int r = 0; r < 16; r++)
                acc[i][j][r] = 0.0f;

    auto fetch = [&](int k0) {
        const bool ktail = k0 + BK > K;
        const __amdgpu_buffer_rsrc_t wa =
            gemm_rsrc(Ablk + k0, ((rows_a - 1) * lda + K - k0) * 4);

#pragma unroll
        for (int e = 0; e < A4; e++)
            ra[e] = gemm_load4<VA>(wa, aoff[e]);
        if (MODE == GEMM_B_NK) {
            const __amdgpu_buffer_rsrc_t wb = gemm_rsrc(
                B + n0 * ldb + k0, ((cols_b - 1) * ldb + K - k0) * 4);

#pragma unroll
            for (int e = 0; e < B4; e++)
                rb[e] = gemm_load4<VB>(wb, boff[e]);
        }
        else if (MODE == GEMM_B_KN) {
            const float *Bk = B + (long long)k0 * ldb;
            const int kv = min(BK, K - k0);
            const __amdgpu_buffer_rsrc_t wb =
                gemm_rsrc(Bk + n0, ((kv - 1) * ldb + cols_b) * 4);

#pragma unroll
            for (int e = 0; e < B4; e++)
                rb[e] = gemm_load4<VB>(wb, boff[e]);
            if (cols_b < BN) {
                /* Columns past N of rows before the window's last read
                 * the next row: zero them. */
#pragma unroll
                for (int e = 0; e < B4; e++) {
                    const int q = tid + NTH * e, nq = (q % (BN / 4)) * 4;

                    rb[e] = mask4(rb[e], nq, cols_b);
                }
            }
        }
        else {
            const int khw = g.kh * g.kw;
#pragma unroll
            for (int e = 0; e < BE; e++) {
                const int r = k0 + ck0 + e * (NTH / BN);
                float v = 0.0f;

                if (cvalid && r < K) {
                    const int c = r / khw, rem = r - c * khw;
                    const int i = rem / g.kw, j = rem - i * g.kw;
                    const int iy = cy + i * g.dy, ix = cx + j * g.dx;

                    if (iy >= 0 && iy < g.ch && ix >= 0 && ix < g.cw) {
                        v = B[((long long)c * g.ch + iy) * g.cw + ix];
                        if (g.mean) {
                            v = (v - g.mean[c]) * g.rstd[c];
                            if (g.gate)
                                v = v >= 0.0f ? v : g.gate[c] * v;
                        }
                    }
                }
                rg[e] = v;
            }
        }
        if (ktail) {
            /* Last slice of a K that BK does not divide: columns past K
             * of rows before the window's last read the next row. */
#pragma unroll
            for (int e = 0; e < A4; e++) {
                const int q = tid + NTH * e, kq = (q % KQ) * 4;

                ra[e] = mask4(ra[e], k0 + kq, K);
            }
            if (MODE == GEMM_B_NK) {
#pragma unroll
                for (int e = 0; e < B4; e++) {
                    const int q = tid + NTH * e, kq = (q % KQ) * 4;

                    rb[e] = mask4(rb[e], k0 + kq, K);
                }
            }
        }
    };

    auto stash = [&](int buf) {
        float *as = As[buf], *bs = Bs[buf];

#pragma unroll
        for (int e = 0; e < A4; e++) {
            const int q = tid + NTH * e, row = q / KQ, kq = (q % KQ) * 4;

            as[(kq + 0) * LDSA + row] = ra[e].x;
            as[(kq + 1) * LDSA + row] = ra[e].y;
            as[(kq + 2) * LDSA + row] = ra[e].z;
            as[(kq + 3) * LDSA + row] = ra[e].w;
        }
        if (MODE == GEMM_B_NK) {
#pragma unroll
            for (int e = 0; e < B4; e++) {
                const int q = tid + NTH * e, row = q / KQ, kq = (q % KQ) * 4;

                bs[(kq + 0) * LDSB + row] = rb[e].x;
                bs[(kq + 1) * LDSB + row] = rb[e].y;
                bs[(kq + 2) * LDSB + row] = rb[e].z;
                bs[(kq + 3) * LDSB + row] = rb[e].w;
            }
        }
        else if (MODE == GEMM_B_KN) {
#pragma unroll
            for (int e = 0; e < B4; e++) {
                const int q = tid + NTH * e, kk = q / (BN / 4);
                const int nq = (q % (BN / 4)) * 4;

                *(float4 *)&bs[kk * LDSB + nq] = rb[e];
            }
        }
        else {
#pragma unroll
            for (int e = 0; e < BE; e++)
                bs[(ck0 + e * (NTH / BN)) * LDSB + cn] = rg[e];
        }
    };

    if (kt0 < kt1) {
        fetch(kt0 * BK);
        stash(0);
    }
    __syncthreads();
    for (int kt = kt0; kt < kt1; kt++) {
        const int cur = (kt - kt0) & 1;

        if (kt + 1 < kt1)
            fetch((kt + 1) * BK);
        {
            const float *as = As[cur] + wm * (BM / WGM) + (lane & 31);
            const float *bs = Bs[cur] + wn * (BN / WGN) + (lane & 31);
            const int kh = lane >> 5;
            auto operands = [&](int ks, float *a, float *b) {
                const int kr = 2 * ks + kh;

#pragma unroll
                for (int i = 0; i < TM; i++)
                    a[i] = as[kr * LDSA + i * 32];
#pragma unroll
                for (int j = 0; j < TN; j++)
                    b[j] = bs[kr * LDSB + j * 32];
            };
            float a[PF + 1][TM], b[PF + 1][TN];

            /* The scheduling barriers keep the LDS reads of step ks + PF
             * ahead of the MFMAs of step ks; the next slice goes to the
             * other LDS buffer two steps before the end. */
#pragma unroll
            for (int ks = 0; ks < PF; ks++)
                operands(ks, a[ks], b[ks]);
#pragma unroll
            for (int ks = 0; ks < NS; ks++) {
                constexpr int NB = PF + 1;

                if (ks + PF < NS)
                    operands(ks + PF, a[(ks + PF) % NB], b[(ks + PF) % NB]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            a[ks % NB][i], b[ks % NB][j], acc[i][j], 0, 0, 0);
                if (ks == NS - 2 && kt + 1 < kt1)
                    stash(cur ^ 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __syncthreads();
    }

    if (piece >= 0) {
        /* Raw partial sums of the piece, [row][col] of the BM x BN tile. */
        float *pp = g.part + ((long long)(L - g.nfull) * g.split + piece) * (BM * BN);

#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = wm * (BM / WGM) + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 +
                                    (r & 3);
                    const int col = wn * (BN / WGN) + j * 32 + (lane & 31);

                    pp[row * BN + col] = acc[i][j][r];
                }
        return;
    }
    gemm_epilogue<TM, TN>(g, acc, b0, b1, m0 + wm * (BM / WGM), n0 + wn * (BN / WGN), lane);
}

/* The cut tiles of gemm_mfma<64, 64, ...> (one batch): one thread per
 * output adds the pieces' partial sums in piece order (all loads issued
 * first), then alpha, bias, activation and residual as gemm_epilogue. */
__global__ void __launch_bounds__(256) gemm_pieces_kernel(const gemm_args g, int tail)
{
    constexpr int BM = 64, BN = 64;
    const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
    const int t = (int)(e / (BM * BN)), w = (int)(e % (BM * BN));

    if (t >= tail)
        return;
    const int tiles_n = (g.N + BN - 1) / BN;
    const int tiles = tiles_n * ((g.M + BM - 1) / BM);
    const int tile = xcd_tile(g.nfull + t, tiles);
    const int row = (tile / tiles_n) * BM + w / BN, col = (tile % tiles_n) * BN + w % BN;
    const float *q = g.part + (long long)t * g.split * (BM * BN) + w;
    float p[GEMM_MAX_SPLIT], v;

    if (row >= g.M || col >= g.N)
        return;
#pragma unroll
    for (int pc = 0; pc < GEMM_MAX_SPLIT; pc++)
        if (pc < g.split)
            p[pc] = q[(long long)pc * (BM * BN)];
    v = p[0];
#pragma unroll
    for (int pc = 1; pc < GEMM_MAX_SPLIT; pc++)
        if (pc < g.split)
            v += p[pc];
    v *= g.alpha;
    if (g.bias)
        v += g.bias[g.biasrow ? row : col];
    v = icoreg_act(v, g.act, g.slope);
    if (g.R)
        v += g.R[(long long)row * g.ldc + col];
    g.C[(long long)row * g.ldc + col] = v;
}



/* Small products (few output tiles, K <= 256): one 32 x 32 output tile per
 * block of 8 waves. Both operand panels (32 x K of A, K x 32 of B) are
 * loaded to LDS at once, the 8 waves split K into eighths and their
 * partial tiles are summed through LDS. For the q / kv / o projections of
 * aggregated attention (a few hundred tokens, K = 256) the main kernel
 * leaves most CUs idle and waits on 16 dependent slice loads per tile;
 * here every block has one load round trip and K / 16 MFMA steps. */
#define GEMM_SK_MAXK 256

template <int MODE, bool DIRECT>
__global__ void __launch_bounds__(512)
    gemm_smallk(const gemm_args g1, const gemm_args g2, int nblk1)
{
    constexpr int NTH = 512, T = 32;
    /* Row-major panels as loaded (no transposing stores): A [m][k] and B
     * given N x K as [n][k], K + 2 floats a row, so the 32 lanes of an
     * MFMA operand (32 rows, one k) fall in 32 different even banks and
     * lanes 32-63 (k + 1) in the odd ones; B given K x N as [k][n].
     * DIRECT (K % 64 == 0): no panels; LDS holds only the 8 partial
     * tiles. */
    constexpr int P = GEMM_SK_MAXK + 2;
    __shared__ __align__(16) float lds[DIRECT ? 8 * T * T : 2 * T * P];
    float *const As = lds, *const Bs = lds + (DIRECT ? 0 : T * P);

    /* Blocks nblk1.. run the second product. */
    const bool second = (int)blockIdx.x >= nblk1;
    const gemm_args &g = second ? g2 : g1;
    const int bx = second ? (int)blockIdx.x - nblk1 : (int)blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tiles_n = (g.N + T - 1) / T;
    const int m0 = (bx / tiles_n) * T, n0 = (bx % tiles_n) * T;
    const long long bt = blockIdx.y, b0 = bt / g.nb1, b1 = bt % g.nb1;
    const float *A = g.A + b0 * g.sa0 + b1 * g.sa1;
    const float *B = g.B + b0 * g.sb0 + b1 * g.sb1;
    const int M = g.M, N = g.N, K = g.K, KQ = K / 4, pk = K + 2;
    const int rows_a = min(T, M - m0), cols_b = min(T, N - n0);
    const long long lda = g.lda, ldb = g.ldb;
    floatx16 acc;

    for (int r = 0; r < 16; r++)
        acc[r] = 0.0f;
    if constexpr (DIRECT) {
        /* Wave w takes k in [w kw, (w + 1) kw), kw = K / 8, lane half h
         * the half [w kw + h kw / 2, + kw / 2): MFMA step s pairs k =
         * w kw + s (lanes 0-31) with w kw + kw / 2 + s (lanes 32-63) for
         * both operands. Each lane reads its row's kw / 2 floats straight
         * into registers through windows ending at the last row inside
         * the matrix (rows past it read 0). */
        constexpr int KH = GEMM_SK_MAXK / 16; /* most k per lane */
        const int kh = K / 16, c = lane & 31;
        const int kb = wave * (K / 8) + (lane >> 5) * kh;
        const __amdgpu_buffer_rsrc_t wa =
            gemm_rsrc(A + m0 * lda, ((rows_a - 1) * lda + K) * 4);
        const __amdgpu_buffer_rsrc_t wb =
            MODE == GEMM_B_NK ? gemm_rsrc(B + n0 * ldb, ((cols_b - 1) * ldb + K) * 4)
                              : gemm_rsrc(B + n0, ((K - 1) * ldb + cols_b) * 4);
        float av[KH], bv[KH];

#pragma unroll
        for (int q = 0; q < KH / 4; q++)
            if (4 * q < kh) {
                const float4 t = gemm_load4<true>(wa, (unsigned)((c * lda + kb + 4 * q) * 4));

                av[4 * q] = t.x;
                av[4 * q + 1] = t.y;
                av[4 * q + 2] = t.z;
                av[4 * q + 3] = t.w;
                if (MODE == GEMM_B_NK) {
                    const float4 u = gemm_load4<true>(wb, (unsigned)((c * ldb + kb + 4 * q) * 4));

                    bv[4 * q] = u.x;
                    bv[4 * q + 1] = u.y;
                    bv[4 * q + 2] = u.z;
                    bv[4 * q + 3] = u.w;
                }
                else {
                    /* Columns past N of rows before the window's last
                     * read the next row: zeroed. */
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float v = __builtin_bit_cast(
                            float, __builtin_amdgcn_raw_buffer_load_b32(
                                       wb, (int)(((kb + 4 * q + e) * ldb + c) * 4), 0, 0));

                        bv[4 * q + e] = c < cols_b ? v : 0.0f;
                    }
                }
            }
#pragma unroll
        for (int q = 0; q < KH; q++)
            if (q < kh)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q], bv[q], acc, 0, 0, 0);
    }
    else {
        /* Panels: 16-byte loads through windows ending at the last row inside
         * the matrix (rows past it read 0), all issued before the first LDS
         * store. At most 32 x 256 / 4 / 512 = 4 per thread and operand. */
        {
            constexpr int NL = GEMM_SK_MAXK * T / 4 / NTH;
            const __amdgpu_buffer_rsrc_t wa =
                gemm_rsrc(A + m0 * lda, ((rows_a - 1) * lda + K) * 4);
            const __amdgpu_buffer_rsrc_t wb =
                MODE == GEMM_B_NK ? gemm_rsrc(B + n0 * ldb, ((cols_b - 1) * ldb + K) * 4)
                                  : gemm_rsrc(B + n0, ((K - 1) * ldb + cols_b) * 4);
            const int nq4 = T * KQ; /* float4 groups per panel */
            float4 va[NL], vb[NL];

#pragma unroll
            for (int i = 0; i < NL; i++) {
                const int q = tid + i * NTH, row = q / KQ, kq = (q % KQ) * 4;

                va[i] = q < nq4 ? gemm_load4<true>(wa, (unsigned)((row * lda + kq) * 4))
                                : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (MODE == GEMM_B_NK) {
                    vb[i] = q < nq4 ? gemm_load4<true>(wb, (unsigned)((row * ldb + kq) * 4))
                                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
                else {
                    const int kk = q / (T / 4), nq = (q % (T / 4)) * 4;

                    /* Columns past N of rows before the window's last read
                     * the next row. */
                    vb[i] = q < nq4 ? mask4(gemm_load4<true>(wb, (unsigned)((kk * ldb + nq) * 4)),
                                            nq, cols_b)
                                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
            }
#pragma unroll
            for (int i = 0; i < NL; i++) {
                const int q = tid + i * NTH, row = q / KQ, kq = (q % KQ) * 4;

                if (q >= nq4)
                    continue;
                *(float2 *)&As[row * pk + kq] = make_float2(va[i].x, va[i].y);
                *(float2 *)&As[row * pk + kq + 2] = make_float2(va[i].z, va[i].w);
                if (MODE == GEMM_B_NK) {
                    *(float2 *)&Bs[row * pk + kq] = make_float2(vb[i].x, vb[i].y);
                    *(float2 *)&Bs[row * pk + kq + 2] = make_float2(vb[i].z, vb[i].w);
                }
                else {
                    const int kk = q / (T / 4), nq = (q % (T / 4)) * 4;

                    *(float4 *)&Bs[kk * T + nq] = vb[i];
                }
            }
        }
        __syncthreads();

        /* Wave w: k in [w K / 8, (w + 1) K / 8). */
        {
            const int kw = K / 8, kb = wave * kw, kh = lane >> 5, c = lane & 31;

            for (int ks = 0; ks < kw; ks += 2) {
                const int kr = kb + ks + kh;
                const float bvl = MODE == GEMM_B_NK ? Bs[c * pk + kr] : Bs[kr * T + c];

                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(As[c * pk + kr], bvl, acc, 0, 0, 0);
            }
        }
        __syncthreads();
    }
    /* Partial tiles [w][row][col] over the A panel, then the sum of the 8
     * per output in the fixed order w = 0..7. */
    {
        float *Ps = As;

#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);

            Ps[(wave * T + row) * T + (lane & 31)] = acc[r];
        }
    }
    __syncthreads();
    {
        float *C = g.C + b0 * g.sc0 + b1 * g.sc1;
        const float *R = g.R ? g.R + b0 * g.sc0 + b1 * g.sc1 : nullptr;
        /* Output (row, col) of the tile: the 8 partials in order, then
         * alpha, bias, activation, residual. */
        auto value = [&](int row, int col) {
            const int gr = m0 + row, gc = n0 + col;
            float v = 0.0f;

#pragma unroll
            for (int w = 0; w < 8; w++)
                v += As[(w * T + row) * T + col];
            v *= g.alpha;
            if (g.bias)
                v += g.bias[g.biasrow ? gr : gc];
            v = icoreg_act(v, g.act, g.slope);
            if (R)
                v += R[(long long)gr * g.ldc + gc];
            return v;
        };

        for (int e = tid; e < T * T; e += NTH) {
            const int row = e / T, col = e % T, gr = m0 + row, gc = n0 + col;
            float v;

            if (gr >= M || gc >= N)
                continue;
            v = value(row, col);
            if (g.rope && gc < g.rcols) {
                /* The pair (gc & ~1, gc | 1) lies in the tile (n0 is a
                 * multiple of 32, rcols even and at most N). */
                const float vp = value(row, col ^ 1);
                const float2 rot =
                    g.rope[(long long)(gr % g.rnpos) * (g.rd / 2) + (gc % g.rd) / 2];
                float x0, x1;

                if (col & 1) {
                    icoreg_rope_pair(vp, v, rot, x0, x1);
                    v = x1;
                }
                else {
                    icoreg_rope_pair(v, vp, rot, x0, x1);
                    v = x0;
                }
            }
            C[(long long)gr * g.ldc + gc] = v;
        }
    }
}

/* Products with 16-byte aligned rows: operands by LDS DMA. Each thread
 * loads 16-byte chunks of the A and B panels straight into LDS
 * (buffer_load ... lds: no register staging, no transposing stores), 32
 * k per slice, two slices in flight, one barrier per slice. Rows of the
 * [row][k] panels (A, and B given N x K) hold their eight chunks in the
 * order chunk ^ (row / 2 % 8), so that the 32 rows an MFMA operand reads
 * spread over the banks; a K x N panel of B swaps the two halves of every
 * odd k row for the same reason. The MFMA steps take k in the order
 * 4 g + 2 h + j (lane half h, step j of group g) for both operands, so a
 * lane reads its two k of a group with one 8-byte load. */
template <int BM, int BN, int WM, int WN, int MODE>
__global__ void __launch_bounds__(64 * WM * WN) gemm_dma(const gemm_args g)
{
    constexpr int NT = 64 * WM * WN, BK = 32;
    constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
    constexpr int ASZ = BM * BK, BSZ = BN * BK; /* floats per slice */
    constexpr int AL = ASZ / 4 / NT, BL = BSZ / 4 / NT; /* chunks per thread */
    static_assert(AL >= 1 && BL >= 1 && ASZ % (4 * NT) == 0 && BSZ % (4 * NT) == 0 &&
                      BN >= 64,
                  "tile shape");
    __shared__ __align__(16) float lds[2 * (ASZ + BSZ)];
    float *const A0 = lds, *const B0 = lds + ASZ, *const A1 = lds + ASZ + BSZ,
                 *const B1 = lds + 2 * ASZ + BSZ;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN, h = lane >> 5, r32 = lane & 31;
    const int tiles_n = (g.N + BN - 1) / BN;
    const int tiles = tiles_n * ((g.M + BM - 1) / BM);
    const int tile = xcd_tile(blockIdx.x, tiles);
    const int m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;
    const long long bt = blockIdx.y, b0 = bt / g.nb1, b1 = bt % g.nb1;
    const float *A = g.A + b0 * g.sa0 + b1 * g.sa1;
    const float *B = g.B + b0 * g.sb0 + b1 * g.sb1;
    const int M = g.M, N = g.N, K = g.K;
    const long long lda = g.lda, ldb = g.ldb;
    /* Windows over whole operands (their byte offsets fit in 31 bits). */
    const long long abytes = ((long long)(M - 1) * lda + K) * 4;
    const long long bbytes = MODE == GEMM_B_NK ? ((long long)(N - 1) * ldb + K) * 4
                                               : ((long long)(K - 1) * ldb + N) * 4;
    int arow[AL], ak[AL], brow[BL], bk[BL];
    floatx16 acc[TM][TN];

#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                acc[i][j][r] = 0.0f;
    /* Chunk slot s of this thread (LDS floats 4 s .. 4 s + 3): A (and B
     * given N x K) row s / 8, its chunk (s % 8) ^ (row / 2 % 8); B given
     * K x N: k row s / (BN / 4), columns 4 ((s % (BN / 4)) ^ 8 (k & 1)). */
#pragma unroll
    for (int q = 0; q < AL; q++) {
        const int sl = tid + NT * q, row = sl / 8;

        arow[q] = row;
        ak[q] = 4 * ((sl % 8) ^ ((row >> 1) & 7));
    }
#pragma unroll
    for (int q = 0; q < BL; q++) {
        const int sl = tid + NT * q;

        if (MODE == GEMM_B_NK) {
            const int row = sl / 8;

            brow[q] = row;
            bk[q] = 4 * ((sl % 8) ^ ((row >> 1) & 7));
        }
        else {
            const int kr = sl / (BN / 4);

            brow[q] = kr;
            bk[q] = 4 * ((sl % (BN / 4)) ^ ((kr & 1) ? 8 : 0));
        }
    }

    auto load = [&](int k0, float *__restrict__ As, float *__restrict__ Bs) {
        const __amdgpu_buffer_rsrc_t ra = gemm_rsrc(A, abytes);
        const __amdgpu_buffer_rsrc_t rb = gemm_rsrc(B, bbytes);

#pragma unroll
        for (int q = 0; q < AL; q++) {
            const int gm = m0 + arow[q], gk = k0 + ak[q];
            const unsigned off = gm < M && gk < K ? (unsigned)((gm * lda + gk) * 4) : GEMM_OOB;

            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void *)(As + 4 * (NT * q + 64 * wave)), 16,
                (int)off, 0, 0, 0);
        }
#pragma unroll
        for (int q = 0; q < BL; q++) {
            unsigned off;

            if (MODE == GEMM_B_NK) {
                const int gn = n0 + brow[q], gk = k0 + bk[q];

                off = gn < N && gk < K ? (unsigned)((gn * ldb + gk) * 4) : GEMM_OOB;
            }
            else {
                const int gk = k0 + brow[q], gn = n0 + bk[q];

                off = gk < K && gn < N ? (unsigned)((gk * ldb + gn) * 4) : GEMM_OOB;
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (__attribute__((address_space(3))) void *)(Bs + 4 * (NT * q + 64 * wave)), 16,
                (int)off, 0, 0, 0);
        }
    };
    auto compute = [&](const float *__restrict__ As, const float *__restrict__ Bs) {
#pragma unroll
        for (int gq = 0; gq < BK / 4; gq++) {
            float2 a[TM], b[TN];

#pragma unroll
            for (int i = 0; i < TM; i++) {
                const int row = wm * (BM / WM) + i * 32 + r32;

                a[i] = *(const float2 *)(As + row * BK + 4 * (gq ^ ((row >> 1) & 7)) + 2 * h);
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = wn * (BN / WN) + j * 32 + r32;

                if (MODE == GEMM_B_NK) {
                    b[j] = *(const float2 *)(Bs + n * BK + 4 * (gq ^ ((n >> 1) & 7)) + 2 * h);
                }
                else {
                    const int k = 4 * gq + 2 * h;

                    b[j].x = Bs[k * BN + n];
                    b[j].y = Bs[(k + 1) * BN + (((n >> 2) ^ 8) << 2) + (n & 3)];
                }
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] =
                        __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].x, b[j].x, acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] =
                        __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].y, b[j].y, acc[i][j], 0, 0, 0);
        }
    };

    const int nk = (K + BK - 1) / BK;
    /* Slice kt from (Ac, Bc) while slice kt + 1 loads into (An, Bn); the
     * loads have landed (LDS DMA counts in vmcnt) and everyone's reads of
     * (Ac, Bc) are done at the barrier. */
    auto step = [&](int kt, const float *__restrict__ Ac, const float *__restrict__ Bc,
                    float *__restrict__ An, float *__restrict__ Bn) {
        if (kt + 1 < nk)
            load((kt + 1) * BK, An, Bn);
        compute(Ac, Bc);
        __builtin_amdgcn_s_waitcnt(GEMM_WAIT_VM0);
        __syncthreads();
    };

    load(0, A0, B0);
    __builtin_amdgcn_s_waitcnt(GEMM_WAIT_VM0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt += 2) {
        step(kt, A0, B0, A1, B1);
        if (kt + 1 < nk)
            step(kt + 1, A1, B1, A0, B0);
    }
    gemm_epilogue<TM, TN>(g, acc, b0, b1, m0 + wm * (BM / WM), n0 + wn * (BN / WN), lane);
}

template <int BM, int BN, int BK, int WGM, int WGN, int MODE>
static void launch_mode(const gemm_args &g, int nb, bool va, bool vb,
                        hipStream_t s, int blocks)
{
    const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
    dim3 grid(blocks > 0 ? blocks : tiles, nb), block(64 * WGM * WGN);

#define GEMM_LAUNCH(VA_, VB_)                                                  \
    hipLaunchKernelGGL((gemm_mfma<BM, BN, BK, MODE, VA_, VB_, WGM, WGN>),      \
                       grid, block, 0, s, g)
    if (MODE == GEMM_B_CONV) {
        if (va)
            GEMM_LAUNCH(true, false);
        else
            GEMM_LAUNCH(false, false);
    }
    else if (va && vb)
        GEMM_LAUNCH(true, true);
    else if (va)
        GEMM_LAUNCH(true, false);
    else if (vb)
        GEMM_LAUNCH(false, true);
    else
        GEMM_LAUNCH(false, false);
#undef GEMM_LAUNCH
}

template <int BM, int BN, int BK, int WGM, int WGN>
static void launch_cfg(const gemm_args &g, int bmode, int nb, bool va,
                       bool vb, hipStream_t s, int blocks)
{
    switch (bmode) {
    case GEMM_B_KN:
        launch_mode<BM, BN, BK, WGM, WGN, GEMM_B_KN>(g, nb, va, vb, s, blocks);
        break;
    case GEMM_B_NK:
        launch_mode<BM, BN, BK, WGM, WGN, GEMM_B_NK>(g, nb, va, vb, s, blocks);
        break;
    default:
        launch_mode<BM, BN, BK, WGM, WGN, GEMM_B_CONV>(g, nb, va, vb, s, blocks);
        break;
    }
}

bool gemm_shape_ok(const gemm_args &g, int bmode)
{
    /* Buffer windows span at most 128 rows of an operand (32-bit byte
     * offsets below 2 GiB), and rows must not overlap. */
    const long long lim = (1LL << 31) / (4 * 128);

    if (g.lda < g.K || g.lda >= lim)
        return false;
    if (bmode == GEMM_B_NK)
        return g.ldb >= g.K && g.ldb < lim;
    if (bmode == GEMM_B_KN)
        return g.ldb >= g.N && g.ldb < lim;
    return true;
}

bool gemm_smallk_ok(const gemm_args &g, int bmode, int nb, bool va, bool vb, int cus)
{
    /* Small products that would fill under half of the CUs with 64 x 64
     * tiles: the one-shot small-K kernel. */
    const long long tiles64 = (long long)((g.M + 63) / 64) * ((g.N + 63) / 64) * nb;

    va = va && g.K % 4 == 0;
    vb = vb && (bmode == GEMM_B_KN ? g.N % 4 == 0 : g.K % 4 == 0);
    return bmode != GEMM_B_CONV && va && vb && g.K <= GEMM_SK_MAXK && g.K % 16 == 0 &&
           g.rup == 0 && 2 * tiles64 <= cus;
}

void gemm_launch_smallk2(const gemm_args &g1, const gemm_args &g2, hipStream_t s)
{
    const int n1 = ((g1.M + 31) / 32) * ((g1.N + 31) / 32);
    const int n2 = ((g2.M + 31) / 32) * ((g2.N + 31) / 32);

    if (g1.K % 64 == 0 && g2.K % 64 == 0)
        hipLaunchKernelGGL((gemm_smallk<GEMM_B_NK, true>), dim3(n1 + n2, 1), dim3(512), 0, s, g1,
                           g2, n1);
    else
        hipLaunchKernelGGL((gemm_smallk<GEMM_B_NK, false>), dim3(n1 + n2, 1), dim3(512), 0, s,
                           g1, g2, n1);
}

/* The LDS-DMA kernel: in the ELoFTR and RoMa pipelines it is faster only
 * for products with few output rows (M <= 256, B given K x N, K >= 256:
 * the MLP's second layer); on larger grids the main kernel's smaller LDS
 * footprint (more blocks per CU) wins, and on K <= 128 its shorter
 * slices do. It addresses whole operands with 31-bit byte offsets. va,
 * vb as adjusted by gemm_launch. */
static bool gemm_dma_ok(const gemm_args &g, int bmode, bool va, bool vb)
{
    const long long lim = 1LL << 31;

    if (!(bmode == GEMM_B_KN && va && vb && g.M <= 256 && g.K >= 256))
        return false;
    return ((long long)(g.M - 1) * g.lda + g.K) * 4 < lim &&
           ((long long)(g.K - 1) * g.ldb + g.N) * 4 < lim;
}

/* Main-kernel work split over cus CUs, for one-batch grids of under 4
 * tiles per CU with plain epilogues: the tiles from nfull on are cut over
 * K into split pieces of at least 4 k slices. Either the tiles left over
 * after an equal whole number per CU are cut (about one piece per CU), or
 * all of them; the choice with the smallest per-CU load (in tiles) is
 * taken when it is at least 10 % below the uncut grid's, which pays for
 * the second launch. */
static bool gemm_plan(const gemm_args &g, int bmode, int nb, int cus, int &nfull, int &split)
{
    const int tiles = ((g.M + 63) / 64) * ((g.N + 63) / 64);
    const int nk = (g.K + 15) / 16;
    const int smax = std::min(nk / 4, GEMM_MAX_SPLIT);
    const int rem = cus > 0 ? tiles % cus : 0;
    double best;

    nfull = tiles;
    split = 1;
    if (nb != 1 || g.nb1 != 1 || bmode == GEMM_B_CONV || g.rup || cus < 1 ||
        tiles >= 4 * cus || smax < 2)
        return false;
    best = 0.9 * (double)((tiles + cus - 1) / cus);
    for (int s = 2; s <= smax; s++) {
        /* All tiles cut. */
        const double all = (double)(((long long)tiles * s + cus - 1) / cus) / s;
        /* Only the leftover tiles cut. */
        const double left =
            rem ? (double)(tiles - rem) / cus + (double)((rem * s + cus - 1) / cus) / s : 1e30;

        if (left < best) {
            best = left;
            nfull = tiles - rem;
            split = s;
        }
        if (all < best) {
            best = all;
            nfull = 0;
            split = s;
        }
    }
    return split > 1;
}

size_t gemm_split_floats(const gemm_args &g, int bmode, int nb, bool va, bool vb, int cus)
{
    int nfull, split;

    va = va && g.K % 4 == 0;
    vb = vb && (bmode == GEMM_B_KN ? g.N % 4 == 0 : g.K % 4 == 0);
    if (gemm_smallk_ok(g, bmode, nb, va, vb, cus) || gemm_dma_ok(g, bmode, va, vb) ||
        !gemm_plan(g, bmode, nb, cus, nfull, split))
        return 0;
    return (size_t)(((g.M + 63) / 64) * ((g.N + 63) / 64) - nfull) * split * 4096;
}

void gemm_launch(const gemm_args &g, int bmode, int nb, bool va, bool vb,
                 int cus, hipStream_t s)
{
    /* 16-byte loads need every four-float group wholly inside or wholly
     * past the matrix edge: K (A, and B given N x K) or N (B given
     * K x N) a multiple of 4. */
    va = va && g.K % 4 == 0;
    vb = vb && (bmode == GEMM_B_KN ? g.N % 4 == 0 : g.K % 4 == 0);
    /* 64 x 64 tiles, 4 waves, BK = 16 at every shape: 17 KB of LDS and
     * few registers keep up to 8 waves per SIMD in flight. In isolated
     * sweeps 64 x 128 (8 waves, BK = 32) and 128 x 128 (16 waves) tiles
     * ran some ViT shapes up to 15 % faster, but inside the RoMa and
     * ELoFTR pipelines (operands fresh from the previous kernel) they
     * were 5-70 % slower on the same shapes, so the kernel's WGM x WGN
     * generality is not used here. */
    if (gemm_smallk_ok(g, bmode, nb, va, vb, cus)) {
        const int nblk = ((g.M + 31) / 32) * ((g.N + 31) / 32);
        const dim3 grid(nblk, nb);

        const bool direct = g.K % 64 == 0;

        if (bmode == GEMM_B_NK && direct)
            hipLaunchKernelGGL((gemm_smallk<GEMM_B_NK, true>), grid, dim3(512), 0, s, g, g, nblk);
        else if (bmode == GEMM_B_NK)
            hipLaunchKernelGGL((gemm_smallk<GEMM_B_NK, false>), grid, dim3(512), 0, s, g, g, nblk);
        else if (direct)
            hipLaunchKernelGGL((gemm_smallk<GEMM_B_KN, true>), grid, dim3(512), 0, s, g, g, nblk);
        else
            hipLaunchKernelGGL((gemm_smallk<GEMM_B_KN, false>), grid, dim3(512), 0, s, g, g, nblk);
        return;
    }
    /* The LDS-DMA kernel: in the ELoFTR and RoMa pipelines it is faster
     * only for products with few output rows (M <= 256, B given K x N,
     * K >= 256: the MLP's second layer); on larger grids the main
     * kernel's smaller LDS footprint (more blocks per CU) wins, and on
     * K <= 128 its shorter slices do. It addresses whole operands with
     * 31-bit byte offsets. */
    if (gemm_dma_ok(g, bmode, va, vb)) {
        const int tiles = ((g.M + 63) / 64) * ((g.N + 63) / 64);
        const dim3 grid(tiles, nb);

        if (bmode == GEMM_B_NK)
            hipLaunchKernelGGL((gemm_dma<64, 64, 2, 2, GEMM_B_NK>), grid, dim3(256), 0, s, g);
        else
            hipLaunchKernelGGL((gemm_dma<64, 64, 2, 2, GEMM_B_KN>), grid, dim3(256), 0, s, g);
        return;
    }
    {
        int nfull, split;

        if (g.part && gemm_plan(g, bmode, nb, cus, nfull, split)) {
            gemm_args gs = g;
            const int tiles = ((g.M + 63) / 64) * ((g.N + 63) / 64);
            const long long tail = tiles - nfull;

            gs.nfull = nfull;
            gs.split = split;
            launch_cfg<64, 64, 16, 2, 2>(gs, bmode, nb, va, vb, s, nfull + (int)tail * split);
            hipLaunchKernelGGL(gemm_pieces_kernel, dim3((unsigned)((tail * 4096 + 255) / 256)),
                               dim3(256), 0, s, gs, (int)tail);
            return;
        }
    }
    launch_cfg<64, 64, 16, 2, 2>(g, bmode, nb, va, vb, s, 0);
}

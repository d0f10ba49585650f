/* SPDX-License-Identifier: Unlicense */

/* fp32 GEMM on the CDNA4 matrix cores: C = act(alpha A op(B) + bias) + R.
 *
 * The contract is the reference's gemm / gemm_big (ops.cl:39-284 of
 * i.coregistration.opencl): batched over nb = nb0 * nb1 with two batch
 * strides per operand, B either K x N or N x K, bias per row or column,
 * activation, residual that may alias C. The design is gfx950's own:
 *
 *  - 256 threads = 4 wave64s in a 2 x 2 arrangement; each wave owns a
 *    (BM/2) x (BN/2) block of the output as 32 x 32 tiles accumulated by
 *    v_mfma_f32_32x32x2f32 (4096 flop per instruction, full fp32 matrix
 *    rate), so the accumulators live in the matrix unit's registers;
 *  - BK = 16 slices of A and B staged through LDS, double-buffered: the
 *    next slice is fetched from HBM/L2 into registers (16-byte loads
 *    when rows are aligned) while the matrix cores work on the current
 *    one, then written to the other LDS buffer; one barrier per slice;
 *  - LDS holds both operands k-major ([k][m], [k][n]) so that the 32
 *    lanes of an MFMA operand read 32 consecutive floats;
 *  - the B operand of a convolution is gathered from the (C, H, W) input
 *    on the fly (implicit GEMM): no unfold buffer, one pass over the
 *    input per output tile, the optional DISK normalisation and PReLU
 *    gate applied while gathering;
 *  - output tiles are assigned so that each of the 8 XCDs (one L2 each)
 *    works on a contiguous band of tiles, which share A rows in its L2. */

#include <hip/hip_runtime.h>

#include "act.h"
#include "gemm.h"

typedef float floatx16 __attribute__((ext_vector_type(16)));

#define GEMM_BK 16
#define GEMM_PAD 4

/* Four floats of a row at column k (k, k+1, k+2, k+3 < K), zero past K;
 * one 16-byte load when allowed and the whole vector is inside. */
template <bool VEC>
__device__ __forceinline__ float4 load_row4(const float *p, int k, int K)
{
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);

    if (VEC && k + 3 < K)
        return *(const float4 *)p;
    if (k < K)
        v.x = p[0];
    if (k + 1 < K)
        v.y = p[1];
    if (k + 2 < K)
        v.z = p[2];
    if (k + 3 < K)
        v.w = p[3];
    return v;
}

/* Output tile of linear block id L among T tiles: blocks are dealt to
 * the 8 XCDs round-robin (L % 8), so give XCD x the x-th contiguous
 * band of tiles. A bijection of 0..T-1. */
__device__ __forceinline__ int xcd_tile(int L, int T)
{
    const int q = T >> 3, rem = T & 7, x = L & 7, idx = L >> 3;

    return (x < rem ? x * (q + 1) : rem * (q + 1) + (x - rem) * q) + idx;
}

template <int BM, int BN, int MODE, bool VA, bool VB>
__global__ void __launch_bounds__(256) gemm_mfma(const gemm_args g)
{
    constexpr int BK = GEMM_BK;
    constexpr int LDSA = BM + GEMM_PAD, LDSB = BN + GEMM_PAD;
    constexpr int TM = BM / 64, TN = BN / 64;
    constexpr int A4 = BM * BK / 4 / 256; /* float4 loads of A per thread */
    constexpr int B4 = BN * BK / 4 / 256; /* dense B */
    constexpr int BE = BN * BK / 256;     /* gathered B elements */
    __shared__ float As[2][BK * LDSA];
    __shared__ float Bs[2][BK * LDSB];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int tiles_n = (g.N + BN - 1) / BN;
    const int tiles = tiles_n * ((g.M + BM - 1) / BM);
    const int tile = xcd_tile(blockIdx.x, tiles);
    const int m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;
    const long long bt = blockIdx.y, b0 = bt / g.nb1, b1 = bt % g.nb1;
    const float *A = g.A + b0 * g.sa0 + b1 * g.sa1;
    const float *B = g.B + b0 * g.sb0 + b1 * g.sb1;
    const int M = g.M, N = g.N, K = g.K;

    float4 ra[A4], rb[B4 > 0 ? B4 : 1];
    float rg[MODE == GEMM_B_CONV ? BE : 1];
    floatx16 acc[TM][TN];

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
#pragma unroll
        for (int e = 0; e < A4; e++) {
            const int q = tid + 256 * e, row = q >> 2, kq = (q & 3) * 4;
            const int gm = m0 + row;

            ra[e] = gm < M ? load_row4<VA>(A + (long long)gm * g.lda + k0 + kq,
                                           k0 + kq, K)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (MODE == GEMM_B_NK) {
#pragma unroll
            for (int e = 0; e < B4; e++) {
                const int q = tid + 256 * e, row = q >> 2, kq = (q & 3) * 4;
                const int gn = n0 + row;

                rb[e] = gn < N ? load_row4<VB>(B + (long long)gn * g.ldb + k0 +
                                                   kq,
                                               k0 + kq, K)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        else if (MODE == GEMM_B_KN) {
#pragma unroll
            for (int e = 0; e < B4; e++) {
                const int q = tid + 256 * e, kk = q / (BN / 4);
                const int nq = (q % (BN / 4)) * 4, gk = k0 + kk;

                rb[e] = gk < K ? load_row4<VB>(B + (long long)gk * g.ldb + n0 +
                                                   nq,
                                               n0 + nq, N)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        else {
            const int khw = g.kh * g.kw;
#pragma unroll
            for (int e = 0; e < BE; e++) {
                const int r = k0 + ck0 + e * (256 / BN);
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
    };

    auto stash = [&](int buf) {
        float *as = As[buf], *bs = Bs[buf];

#pragma unroll
        for (int e = 0; e < A4; e++) {
            const int q = tid + 256 * e, row = q >> 2, kq = (q & 3) * 4;

            as[(kq + 0) * LDSA + row] = ra[e].x;
            as[(kq + 1) * LDSA + row] = ra[e].y;
            as[(kq + 2) * LDSA + row] = ra[e].z;
            as[(kq + 3) * LDSA + row] = ra[e].w;
        }
        if (MODE == GEMM_B_NK) {
#pragma unroll
            for (int e = 0; e < B4; e++) {
                const int q = tid + 256 * e, row = q >> 2, kq = (q & 3) * 4;

                bs[(kq + 0) * LDSB + row] = rb[e].x;
                bs[(kq + 1) * LDSB + row] = rb[e].y;
                bs[(kq + 2) * LDSB + row] = rb[e].z;
                bs[(kq + 3) * LDSB + row] = rb[e].w;
            }
        }
        else if (MODE == GEMM_B_KN) {
#pragma unroll
            for (int e = 0; e < B4; e++) {
                const int q = tid + 256 * e, kk = q / (BN / 4);
                const int nq = (q % (BN / 4)) * 4;

                *(float4 *)&bs[kk * LDSB + nq] = rb[e];
            }
        }
        else {
#pragma unroll
            for (int e = 0; e < BE; e++)
                bs[(ck0 + e * (256 / BN)) * LDSB + cn] = rg[e];
        }
    };

    const int nk = (K + BK - 1) / BK;

    if (nk > 0) {
        fetch(0);
        stash(0);
    }
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;

        if (kt + 1 < nk)
            fetch((kt + 1) * BK);
        {
            const float *as = As[cur] + wm * (BM / 2) + (lane & 31);
            const float *bs = Bs[cur] + wn * (BN / 2) + (lane & 31);
            const int kh = lane >> 5;

#pragma unroll
            for (int ks = 0; ks < BK / 2; ks++) {
                const int kr = 2 * ks + kh;
                float a[TM], b[TN];

#pragma unroll
                for (int i = 0; i < TM; i++)
                    a[i] = as[kr * LDSA + i * 32];
#pragma unroll
                for (int j = 0; j < TN; j++)
                    b[j] = bs[kr * LDSB + j * 32];
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            a[i], b[j], acc[i][j], 0, 0, 0);
            }
        }
        if (kt + 1 < nk)
            stash(cur ^ 1);
        __syncthreads();
    }

    /* Epilogue: register r of a 32 x 32 tile holds row (r / 4) * 8 +
     * (lane / 32) * 4 + r % 4, column lane % 32. */
    {
        float *C = g.C + b0 * g.sc0 + b1 * g.sc1;
        const float *R = g.R ? g.R + b0 * g.sc0 + b1 * g.sc1 : nullptr;

#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int col = n0 + wn * (BN / 2) + j * 32 + (lane & 31);

                if (col >= N)
                    continue;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = m0 + wm * (BM / 2) + i * 32 + (r >> 2) * 8 +
                                    (lane >> 5) * 4 + (r & 3);
                    float v;

                    if (row >= M)
                        continue;
                    v = g.alpha * acc[i][j][r];
                    if (g.bias)
                        v += g.bias[g.biasrow ? row : col];
                    v = icoreg_act(v, g.act, g.slope);
                    if (R)
                        v += R[(long long)row * g.ldc + col];
                    C[(long long)row * g.ldc + col] = v;
                }
            }
    }
}

template <int BM, int BN, int MODE>
static void launch_mode(const gemm_args &g, int nb, bool va, bool vb,
                        hipStream_t s)
{
    const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
    dim3 grid(tiles, nb), block(256);

    if (MODE == GEMM_B_CONV) {
        if (va)
            hipLaunchKernelGGL((gemm_mfma<BM, BN, MODE, true, false>), grid,
                               block, 0, s, g);
        else
            hipLaunchKernelGGL((gemm_mfma<BM, BN, MODE, false, false>), grid,
                               block, 0, s, g);
        return;
    }
    if (va && vb)
        hipLaunchKernelGGL((gemm_mfma<BM, BN, MODE, true, true>), grid, block, 0,
                           s, g);
    else if (va)
        hipLaunchKernelGGL((gemm_mfma<BM, BN, MODE, true, false>), grid, block,
                           0, s, g);
    else if (vb)
        hipLaunchKernelGGL((gemm_mfma<BM, BN, MODE, false, true>), grid, block,
                           0, s, g);
    else
        hipLaunchKernelGGL((gemm_mfma<BM, BN, MODE, false, false>), grid, block,
                           0, s, g);
}

template <int BM, int BN>
static void launch_tile(const gemm_args &g, int bmode, int nb, bool va,
                        bool vb, hipStream_t s)
{
    switch (bmode) {
    case GEMM_B_KN:
        launch_mode<BM, BN, GEMM_B_KN>(g, nb, va, vb, s);
        break;
    case GEMM_B_NK:
        launch_mode<BM, BN, GEMM_B_NK>(g, nb, va, vb, s);
        break;
    default:
        launch_mode<BM, BN, GEMM_B_CONV>(g, nb, va, vb, s);
        break;
    }
}

void gemm_launch(const gemm_args &g, int bmode, int nb, int bm, int bn,
                 bool va, bool vb, hipStream_t s)
{
    if (bm == 128 && bn == 128)
        launch_tile<128, 128>(g, bmode, nb, va, vb, s);
    else if (bm == 64 && bn == 128)
        launch_tile<64, 128>(g, bmode, nb, va, vb, s);
    else
        launch_tile<64, 64>(g, bmode, nb, va, vb, s);
}

/* SPDX-License-Identifier: Unlicense */

/* Direct k x k convolution (k = 3, 5; stride 1, 2; one group) on the
 * CDNA4 matrix cores. Same contract as the reference's conv5x5 and
 * im2col + GEMM paths of ops_conv2d (ops.cl:319-387, ops.c:236-336 of
 * i.coregistration.opencl): out = act(W * in + bias), optional input
 * normalisation and PReLU gate before the zero padding.
 *
 * A block computes 128 output pixels (a 4 x 32 tile of one image) for
 * BM output channels as an implicit GEMM (M = channels, N = pixels,
 * K = C k k). The K loop walks CC input channels at a time:
 *  - the weights of the slice (BM x CC k k, contiguous per output
 *    channel) go to LDS k-major;
 *  - the input patch under the tile (CC x (4 s + k - s) x (32 s + k - s)
 *    floats, zero outside the image) goes to LDS once, normalised and
 *    gated there (once per input value rather than once per tap);
 *  - each MFMA step (v_mfma_f32_32x32x2f32, K = 2) reads its B operand
 *    straight from the patch at the tap's (channel, row, column) shift,
 *    consecutive lanes on consecutive pixels of one output row; the
 *    shifts are compile-time constants, so the inner loop has no index
 *    arithmetic beyond one select per step for the lane half.
 * Double-buffered: the next slice is fetched into registers while the
 * matrix cores work on the current one. Images of a batch run on the
 * grid's z dimension. */

#include <hip/hip_runtime.h>

#include "act.h"
#include "conv.h"

typedef float floatx16 __attribute__((ext_vector_type(16)));

#define TILE_H 4
#define TILE_W 32

template <int KS, int ST, int BM>
__global__ void __launch_bounds__(256) conv_mfma(const conv_args a)
{
    /* Input channels per K slice: 36 or 18 taps for 3 x 3, 50 for 5 x 5. */
    constexpr int CC = KS == 3 ? (BM == 128 ? 2 : 4) : 2;
    constexpr int KK = KS * KS;
    constexpr int KT = CC * KK;          /* K per slice (even) */
    constexpr int PH = (TILE_H - 1) * ST + KS;
    constexpr int PW = (TILE_W - 1) * ST + KS;
    constexpr int PWP = PW + 1;
    constexpr int PCH = PH * PWP;        /* LDS floats per patch channel */
    constexpr int LDA = BM + 4;
    constexpr int TM = BM / 64;
    constexpr int NA = (BM * KT + 255) / 256;
    constexpr int NP = (CC * PH * PW + 255) / 256;
    static_assert(KT % 2 == 0, "K slice must be even");
    __shared__ float As[2][KT * LDA];
    __shared__ float Ps[2][CC * PCH];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, half = lane >> 5, col = lane & 31;
    const int tiles_w = (a.Wo + TILE_W - 1) / TILE_W;
    const int oy0 = (blockIdx.x / tiles_w) * TILE_H;
    const int ox0 = (blockIdx.x % tiles_w) * TILE_W;
    const int m0 = blockIdx.y * BM;
    const int iy0 = oy0 * ST - a.pad, ix0 = ox0 * ST - a.pad;
    const int C = a.C, H = a.H, W = a.W, K = a.K;
    const float *in = a.in + (long long)blockIdx.z * a.in_stride;
    const long long wrow = (long long)C * KK;
    float ra[NA], rp[NP];
    floatx16 acc[TM][2];

#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                acc[i][j][r] = 0.0f;

    auto fetch = [&](int c0) {
#pragma unroll
        for (int q = 0; q < NA; q++) {
            const int e = tid + 256 * q, m = e / KT, t = e - m * KT;
            const int c = c0 + t / KK;
            float v = 0.0f;

            if (e < BM * KT && m0 + m < K && c < C)
                v = a.w[(long long)(m0 + m) * wrow + (long long)c0 * KK + t];
            ra[q] = v;
        }
#pragma unroll
        for (int q = 0; q < NP; q++) {
            const int e = tid + 256 * q, c = e / (PH * PW);
            const int rem = e - c * (PH * PW), py = rem / PW, px = rem - py * PW;
            const int iy = iy0 + py, ix = ix0 + px, cg = c0 + c;
            float v = 0.0f;

            if (e < CC * PH * PW && cg < C && iy >= 0 && iy < H && ix >= 0 &&
                ix < W) {
                v = in[((long long)cg * H + iy) * W + ix];
                if (a.mean) {
                    v = (v - a.mean[cg]) * a.rstd[cg];
                    if (a.gate)
                        v = v >= 0.0f ? v : a.gate[cg] * v;
                }
            }
            rp[q] = v;
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int q = 0; q < NA; q++) {
            const int e = tid + 256 * q, m = e / KT, t = e - m * KT;

            if (e < BM * KT)
                As[buf][t * LDA + m] = ra[q];
        }
#pragma unroll
        for (int q = 0; q < NP; q++) {
            const int e = tid + 256 * q, c = e / (PH * PW);
            const int rem = e - c * (PH * PW), py = rem / PW, px = rem - py * PW;

            if (e < CC * PH * PW)
                Ps[buf][c * PCH + py * PWP + px] = rp[q];
        }
    };

    const int nk = (C + CC - 1) / CC;

    fetch(0);
    stash(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;

        if (kt + 1 < nk)
            fetch((kt + 1) * CC);
        {
            const float *as = As[cur] + wm * (BM / 2) + col;
            const float *ps = Ps[cur] + (wn * 2 * ST) * PWP + col * ST;

#pragma unroll
            for (int s = 0; s < KT / 2; s++) {
                /* Taps t = 2 s (lane half 0) and 2 s + 1 (half 1). */
                const int t0 = 2 * s, t1 = 2 * s + 1;
                const int p0 = (t0 / KK) * PCH + ((t0 % KK) / KS) * PWP + t0 % KS;
                const int p1 = (t1 / KK) * PCH + ((t1 % KK) / KS) * PWP + t1 % KS;
                const int po = half ? p1 : p0;
                const int ao = (2 * s + half) * LDA;
                float av[TM], bv[2];

#pragma unroll
                for (int i = 0; i < TM; i++)
                    av[i] = as[ao + i * 32];
#pragma unroll
                for (int j = 0; j < 2; j++)
                    bv[j] = ps[po + j * ST * PWP];
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            av[i], bv[j], acc[i][j], 0, 0, 0);
            }
        }
        if (kt + 1 < nk)
            stash(cur ^ 1);
        __syncthreads();
    }

    {
        float *out = a.out + (long long)blockIdx.z * a.out_stride;

#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int oy = oy0 + wn * 2 + j, ox = ox0 + col;

            if (oy >= a.Ho || ox >= a.Wo)
                continue;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = m0 + wm * (BM / 2) + i * 32 + (r >> 2) * 8 +
                                  half * 4 + (r & 3);
                    float v;

                    if (m >= K)
                        continue;
                    v = acc[i][j][r];
                    if (a.bias)
                        v += a.bias[m];
                    out[((long long)m * a.Ho + oy) * a.Wo + ox] =
                        icoreg_act(v, a.act, a.slope);
                }
        }
    }
}

bool conv_direct_supported(int kh, int kw, int sy, int sx, int dy, int dx,
                           int groups)
{
    return groups == 1 && kh == kw && (kh == 3 || kh == 5) && sy == sx &&
           (sy == 1 || sy == 2) && dy == 1 && dx == 1;
}

template <int KS, int ST>
static void launch_ks(const conv_args &a, int nb, hipStream_t s)
{
    const int tiles = ((a.Wo + TILE_W - 1) / TILE_W) *
                      ((a.Ho + TILE_H - 1) / TILE_H);

    if (a.K <= 64)
        hipLaunchKernelGGL((conv_mfma<KS, ST, 64>),
                           dim3(tiles, (a.K + 63) / 64, nb), dim3(256), 0, s,
                           a);
    else
        hipLaunchKernelGGL((conv_mfma<KS, ST, 128>),
                           dim3(tiles, (a.K + 127) / 128, nb), dim3(256), 0,
                           s, a);
}

void conv_direct_launch(const conv_args &a, int ks, int stride, int nb,
                        int cus, hipStream_t s)
{
    (void)cus;
    if (ks == 3 && stride == 1)
        launch_ks<3, 1>(a, nb, s);
    else if (ks == 3)
        launch_ks<3, 2>(a, nb, s);
    else if (stride == 1)
        launch_ks<5, 1>(a, nb, s);
    else
        launch_ks<5, 2>(a, nb, s);
}

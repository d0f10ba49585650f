/* SPDX-License-Identifier: Unlicense */

/* Direct k x k convolution (k = 3, 5; stride 1, 2; one group) on the
 * CDNA4 matrix cores. Same contract as the reference's conv5x5 and
 * im2col + GEMM paths of ops_conv2d (ops.cl:319-387, ops.c:236-336 of
 * i.coregistration.opencl): out = act(W * in + bias), optional input
 * normalisation and PReLU gate before the zero padding.
 *
 * A block computes 64 or 128 output pixels (a TH x TW tile of one image,
 * 32 or 16 wide, whichever wastes less of the image) for BM output
 * channels as an implicit GEMM (M = channels, N = pixels, K = C k k). The K loop
 * walks CC input channels at a time:
 *  - the weights of the slice (BM x CC k k, contiguous per output
 *    channel) go to LDS k-major;
 *  - the input patch under the tile (CC x ((TH-1) s + k) x ((TW-1) s + k)
 *    floats, zero outside the image) goes to LDS once, normalised and
 *    gated there (once per input value rather than once per tap); at
 *    stride 2 its even and odd columns are stored apart, so that the
 *    lanes of one output row read consecutive words;
 *  - each MFMA step (v_mfma_f32_32x32x2f32, K = 2) reads its B operand
 *    straight from the patch at the tap's (channel, row, column) shift;
 *    the shifts are compile-time constants.
 * Global reads are buffer loads: the zero padding, the channel and
 * output-channel tails come from the buffer's range check (an offset
 * past the end reads 0), so a fetch is one load per value with offsets
 * computed once per thread. Double-buffered: the next slice is fetched
 * into registers while the matrix cores work on the current one. Images
 * of a batch run on the grid's z dimension. */

#include <algorithm>
#include <hip/hip_runtime.h>

#include "act.h"
#include "conv.h"

typedef float floatx16 __attribute__((ext_vector_type(16)));

/* Offset past the end of every buffer the kernel reads (each is below
 * 2 GiB): its load returns 0. */
#define CONV_OOB 0x80000000u

/* Word 3 of a raw buffer resource on gfx9-family parts: 32-bit data. */
#define CONV_RSRC_FLAGS 0x00020000

static __device__ __forceinline__ __amdgpu_buffer_rsrc_t
conv_rsrc(const float *p, unsigned long long bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0,
                                             (int)(unsigned)bytes,
                                             CONV_RSRC_FLAGS);
}

static __device__ __forceinline__ float conv_load(__amdgpu_buffer_rsrc_t r,
                                                  unsigned off)
{
    return __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}

/* KS x KS taps, stride ST, BM output channels and a TH x TW tile of
 * 64 NJ pixels per block (each wave NJ 32-pixel MFMA tiles), CC input
 * channels per K slice. */
template <int KS, int ST, int BM, int TW, int CC, int NJ>
__global__ void __launch_bounds__(256) conv_mfma(const conv_args a)
{
    constexpr int TH = 64 * NJ / TW;
    constexpr int KK = KS * KS;
    constexpr int KT = CC * KK;
    constexpr int PH = (TH - 1) * ST + KS;
    constexpr int PW = (TW - 1) * ST + KS;
    constexpr int HALF = (PW + 1) / 2;   /* stride 2: even columns first */
    constexpr int PWP = PW + 1;
    constexpr int PCH = PH * PWP;        /* LDS floats per patch channel */
    constexpr int PN = CC * PH * PW;     /* patch values per slice */
    constexpr int LDA = BM + 4;
    constexpr int TM = BM / 64;
    constexpr int NA = BM * KT / 256;
    constexpr int NP = (PN + 255) / 256;
    constexpr int RJ = 32 / TW;          /* tile rows per 32 pixels */
    static_assert(KT % 2 == 0 && BM * KT % 256 == 0, "slice shape");
    __shared__ float As[2][KT * LDA];
    __shared__ float Ps[2][CC * PCH + 1]; /* + one slot for idle lanes */

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, half = lane >> 5, col = lane & 31;
    const int tiles_w = (a.Wo + TW - 1) / TW;
    const int oy0 = (blockIdx.x / tiles_w) * TH;
    const int ox0 = (blockIdx.x % tiles_w) * TW;
    const int m0 = blockIdx.y * BM;
    const int iy0 = oy0 * ST - a.pad, ix0 = ox0 * ST - a.pad;
    const int C = a.C, H = a.H, W = a.W, K = a.K;
    const long long HW = (long long)H * W;
    const int piece = blockIdx.z % a.split, img = blockIdx.z / a.split;
    const float *in = a.in + (long long)img * a.in_stride;
    const long long wrow = (long long)C * KK;
    unsigned woff[NA], poff[NP];
    int lda_[NA], ldp[NP];
    float ra[NA], rp[NP];
    floatx16 acc[TM][NJ];

#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                acc[i][j][r] = 0.0f;

    /* Per-thread offsets, the same for every slice: weights of output
     * channel m0 + m at slice tap t; patch value (c, py, px). */
#pragma unroll
    for (int q = 0; q < NA; q++) {
        const int e = tid + 256 * q, m = e / KT, t = e - m * KT;

        woff[q] = m0 + m < K ? (unsigned)(((m0 + m) * wrow + t) * 4)
                             : CONV_OOB;
        lda_[q] = t * LDA + m;
    }
#pragma unroll
    for (int q = 0; q < NP; q++) {
        const int e = tid + 256 * q, c = e / (PH * PW);
        const int rem = e - c * (PH * PW), py = rem / PW, px = rem - py * PW;
        const int iy = iy0 + py, ix = ix0 + px;
        const int lc = ST == 1 ? px : (px & 1) * HALF + (px >> 1);

        poff[q] = e < PN && iy >= 0 && iy < H && ix >= 0 && ix < W
                      ? (unsigned)((c * HW + (long long)iy * W + ix) * 4)
                      : CONV_OOB;
        ldp[q] = e < PN ? c * PCH + py * PWP + lc : CC * PCH;
    }

    const unsigned long long wbytes = (unsigned long long)K * wrow * 4;
    const unsigned long long ibytes = (unsigned long long)C * HW * 4;

    auto fetch = [&](int c0) {
        const __amdgpu_buffer_rsrc_t rw =
            conv_rsrc(a.w + (long long)c0 * KK, wbytes - (unsigned long long)c0 * KK * 4);
        const __amdgpu_buffer_rsrc_t ri =
            conv_rsrc(in + c0 * HW, ibytes - (unsigned long long)c0 * HW * 4);

#pragma unroll
        for (int q = 0; q < NA; q++)
            ra[q] = conv_load(rw, woff[q]);
#pragma unroll
        for (int q = 0; q < NP; q++)
            rp[q] = conv_load(ri, poff[q]);
        if (c0 + CC > C) {
            /* Ragged last slice: the weight rows run on into the next
             * output channel, so mask the taps of missing channels. */
#pragma unroll
            for (int q = 0; q < NA; q++) {
                const int e = tid + 256 * q, t = e - (e / KT) * KT;

                ra[q] = c0 + t / KK < C ? ra[q] : 0.0f;
            }
        }
        if (a.mean) {
#pragma unroll
            for (int q = 0; q < NP; q++) {
                const int cg = c0 + (tid + 256 * q) / (PH * PW);
                const int cc = cg < C ? cg : C - 1;
                float v = (rp[q] - a.mean[cc]) * a.rstd[cc];

                if (a.gate)
                    v = v >= 0.0f ? v : a.gate[cc] * v;
                rp[q] = poff[q] != CONV_OOB && cg < C ? v : 0.0f;
            }
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int q = 0; q < NA; q++)
            As[buf][lda_[q]] = ra[q];
#pragma unroll
        for (int q = 0; q < NP; q++)
            Ps[buf][ldp[q]] = rp[q];
    };

    /* Slices [kt0, kt1) of CC channels: all of them, or this piece's
     * share (the host makes every piece non-empty). */
    const int nk_all = (C + CC - 1) / CC, per = (nk_all + a.split - 1) / a.split;
    const int kt0 = piece * per, nk = min(nk_all, kt0 + per);
    /* This lane's first pixel: row r of the tile, column x. */
    const int pr = (wn * 32 * NJ + col) / TW, px0 = col % TW;
    const int pbase = pr * ST * PWP + px0;

    fetch(kt0 * CC);
    stash(0);
    __syncthreads();
    for (int kt = kt0; kt < nk; kt++) {
        const int cur = (kt - kt0) & 1;

        if (kt + 1 < nk)
            fetch((kt + 1) * CC);
        {
            const float *as = As[cur] + wm * (BM / 2) + col;
            const float *ps = Ps[cur] + pbase;
            /* Operands of step s: taps t = 2 s (lane half 0) and 2 s + 1
             * (half 1). */
            auto operands = [&](int s, float *av, float *bv) {
                const int t0 = 2 * s, t1 = 2 * s + 1;
                const int c_0 = t0 / KK, y_0 = (t0 % KK) / KS, x_0 = t0 % KS;
                const int c_1 = t1 / KK, y_1 = (t1 % KK) / KS, x_1 = t1 % KS;
                const int p0 = c_0 * PCH + y_0 * PWP +
                               (ST == 1 ? x_0 : (x_0 & 1) * HALF + (x_0 >> 1));
                const int p1 = c_1 * PCH + y_1 * PWP +
                               (ST == 1 ? x_1 : (x_1 & 1) * HALF + (x_1 >> 1));
                const int po = half ? p1 : p0;
                const int ao = (2 * s + half) * LDA;

#pragma unroll
                for (int i = 0; i < TM; i++)
                    av[i] = as[ao + i * 32];
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    bv[j] = ps[po + j * RJ * ST * PWP];
            };
            constexpr int NS = KT / 2;
            /* LDS reads run PF steps ahead of the MFMAs that use them. */
            constexpr int PF = 2;
            float av[PF + 1][TM], bv[PF + 1][NJ];

            /* The scheduling barriers keep the reads of step s + PF ahead
             * of the MFMAs of step s, so their latency hides behind the
             * matrix pipe; the next slice goes to the other LDS buffer a
             * few steps before the end. */
#pragma unroll
            for (int s = 0; s < PF; s++)
                operands(s, av[s], bv[s]);
#pragma unroll
            for (int s = 0; s < NS; s++) {
                constexpr int NB = PF + 1;

                if (s + PF < NS)
                    operands(s + PF, av[(s + PF) % NB], bv[(s + PF) % NB]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < NJ; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            av[s % NB][i], bv[s % NB][j], acc[i][j], 0, 0,
                            0);
                if (s == NS - 4 && kt + 1 < nk)
                    stash(cur ^ 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __syncthreads();
    }

    {
        /* Whole: bias, activation, the output. Piece: raw partial sums
         * into part[piece][img]. */
        const bool whole = a.split == 1;
        float *out = whole ? a.out + (long long)img * a.out_stride
                           : a.part + ((long long)piece * (gridDim.z / a.split) + img) *
                                          K * a.Ho * a.Wo;

#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int oy = oy0 + pr + j * RJ, ox = ox0 + px0;

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
                    if (whole) {
                        if (a.bias)
                            v += a.bias[m];
                        v = icoreg_act(v, a.act, a.slope);
                    }
                    out[((long long)m * a.Ho + oy) * a.Wo + ox] = v;
                }
        }
    }
}

/* Sum of the split pieces' partials in piece order, bias, activation. */
__global__ void __launch_bounds__(256) conv_pieces_kernel(const conv_args a, int nb)
{
    const long long plane = (long long)a.K * a.Ho * a.Wo;
    const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
    const int img = blockIdx.y;

    if (e >= plane)
        return;
    float v = a.part[(long long)img * plane + e];

    for (int p = 1; p < a.split; p++)
        v += a.part[((long long)p * nb + img) * plane + e];
    if (a.bias)
        v += a.bias[e / ((long long)a.Ho * a.Wo)];
    a.out[(long long)img * a.out_stride + e] = icoreg_act(v, a.act, a.slope);
}

/* One input channel (ELoFTR's grey first layer): one thread per output
 * pixel holds its KS x KS taps in registers and runs over the K output
 * channels, the filters and bias staged in LDS (K KS^2 <= C1_MAXW, K <=
 * C1_MAXK); each channel's store is one contiguous run per wave. No MFMA:
 * K C KS^2 products per pixel are few, and the layer is bound by its
 * output writes. */
#define C1_MAXW 4096
#define C1_MAXK 256
template <int KS, int ST>
__global__ void __launch_bounds__(256) conv_c1_kernel(const conv_args a)
{
    __shared__ float ws[C1_MAXW], bs[C1_MAXK];
    const int HWo = a.Ho * a.Wo;
    const int p = blockIdx.x * 256 + threadIdx.x;
    const float *in = a.in + (long long)blockIdx.z * a.in_stride;
    float *out = a.out + (long long)blockIdx.z * a.out_stride;
    float t[KS * KS];

    for (int i = threadIdx.x; i < a.K * KS * KS; i += 256)
        ws[i] = a.w[i];
    for (int i = threadIdx.x; i < a.K; i += 256)
        bs[i] = a.bias ? a.bias[i] : 0.0f;
    {
        const int pc = min(p, HWo - 1);
        const int oy = pc / a.Wo, ox = pc - oy * a.Wo;
        const int iy0 = oy * ST - a.pad, ix0 = ox * ST - a.pad;

#pragma unroll
        for (int i = 0; i < KS; i++)
#pragma unroll
            for (int j = 0; j < KS; j++) {
                const int iy = iy0 + i, ix = ix0 + j;

                t[i * KS + j] = iy >= 0 && iy < a.H && ix >= 0 && ix < a.W
                                    ? in[(long long)iy * a.W + ix]
                                    : 0.0f;
            }
    }
    __syncthreads();
    if (p >= HWo)
        return;
#pragma unroll 8
    for (int k = 0; k < a.K; k++) {
        const float *wk = ws + k * KS * KS;
        float v = 0.0f;

#pragma unroll
        for (int q = 0; q < KS * KS; q++)
            v = fmaf(wk[q], t[q], v);
        out[(long long)k * HWo + p] = icoreg_act(v + bs[k], a.act, a.slope);
    }
}

/* The last few output channels (at most FK_MAXK) of a layer whose
 * channel count would leave a nearly empty MFMA block (DISK's last layer:
 * 129 = 128 + 1 channels, where a second 128-channel block would repeat
 * the whole layer's matrix work for one channel). A block takes a 16 x 32
 * output tile, each thread two vertically adjacent pixels (their windows
 * share KS - 1 rows). The patches of 4 input channels (2 at stride 2)
 * are staged in LDS per step, normalised and gated exactly as conv_mfma loads them, the
 * next step's values loaded into registers while this one is used; a
 * channel's NK filters are read from LDS once and used for both pixels.
 * The input channels can be cut into a.split pieces (grid z = image + nb
 * piece, whole steps each): a grid of a few hundred tiles then still
 * fills the CUs, each piece's raw sums going to a.part for
 * conv_fewk_sum_kernel. Filters and normalisation of the block's channels
 * sit in dynamic LDS (fewk_lds_bytes). */
#define FK_MAXK 8
#define FK_MAXW 8192
#define FK_MAXC 1024

/* Dynamic LDS of a conv_fewk_kernel block: the filters of its input
 * channels (nk cpp KK floats) and their mean, rstd and gate. */
static size_t fewk_lds_bytes(int nk, int cpp, int kk)
{
    return ((size_t)nk * cpp * kk + 3 * (size_t)cpp) * sizeof(float);
}

template <int KS, int ST, int NK>
__global__ void __launch_bounds__(256) conv_fewk_kernel(const conv_args a, int k0, int nb,
                                                        int cpp)
{
    constexpr int TW = 16, TH = 32, KK = KS * KS, FK_CC = ST == 1 ? 4 : 2;
    constexpr int PW = (TW - 1) * ST + KS, PH = (TH - 1) * ST + KS;
    constexpr int PN = FK_CC * PH * PW, NP = (PN + 255) / 256;
    static_assert(NP <= 32, "validity mask");
    /* Row pitch: at stride 1 the two rows a half-wave reads (2 pitch
     * apart) fall on disjoint banks when 2 pitch = 16 (mod 32). */
    constexpr int PP = ST == 1 ? (PW + 8) / 16 * 16 + 8 : PW + 1;
    extern __shared__ float fk_dyn[];
    __shared__ float patch[FK_CC][PH][PP];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int ox0 = blockIdx.x * TW, oy0 = blockIdx.y * TH;
    const int iy0 = oy0 * ST - a.pad, ix0 = ox0 * ST - a.pad;
    const int img = blockIdx.z % nb, piece = blockIdx.z / nb;
    /* This block's input channels [cb, ce): cpp (a multiple of FK_CC) a
     * piece. */
    const int cb = piece * cpp, ce = min(a.C, cb + cpp), cn = ce - cb;
    float *const ws = fk_dyn;              /* [NK][cn][KK] */
    float *const nm = fk_dyn + NK * cpp * KK; /* mean, rstd, gate: [3][cn] */
    const long long HW = (long long)a.H * a.W;
    const float *in = a.in + (long long)img * a.in_stride + cb * HW;
    float acc[2][NK], rp[NP];
    unsigned valid = 0;

#pragma unroll
    for (int k = 0; k < NK; k++)
        acc[0][k] = acc[1][k] = 0.0f;
    for (int i = threadIdx.x; i < NK * cn * KK; i += 256) {
        const int k = i / (cn * KK), r = i - k * cn * KK;

        ws[i] = a.w[((long long)(k0 + k) * a.C + cb) * KK + r];
    }
    if (a.mean)
        for (int c = threadIdx.x; c < cn; c += 256) {
            nm[c] = a.mean[cb + c];
            nm[cn + c] = a.rstd[cb + c];
            nm[2 * cn + c] = a.gate ? a.gate[cb + c] : 1.0f;
        }
    /* Loads only, every one issued before any is used: out-of-range
     * values read the channel's first element and are masked later. */
    auto fetch = [&](int c0) {
        valid = 0;
#pragma unroll
        for (int q = 0; q < NP; q++) {
            const int e = threadIdx.x + 256 * q, cc = e / (PH * PW), rem = e - cc * (PH * PW);
            const int py = rem / PW, px = rem - py * PW, iy = iy0 + py, ix = ix0 + px;
            const int c = min(c0 + cc, cn - 1);
            const bool ok = e < PN && c0 + cc < cn && iy >= 0 && iy < a.H && ix >= 0 &&
                            ix < a.W;

            rp[q] = in[c * HW + (ok ? (long long)iy * a.W + ix : 0)];
            valid |= ok ? 1u << q : 0u;
        }
    };
    fetch(0);
    __syncthreads();
    for (int c0 = 0; c0 < cn; c0 += FK_CC) {
#pragma unroll
        for (int q = 0; q < NP; q++) {
            const int e = threadIdx.x + 256 * q, cc = e / (PH * PW), rem = e - cc * (PH * PW);
            const int c = min(c0 + cc, cn - 1);
            float v = rp[q];

            if (a.mean) {
                v = (v - nm[c]) * nm[cn + c];
                if (a.gate)
                    v = v >= 0.0f ? v : nm[2 * cn + c] * v;
            }
            if (e < PN)
                patch[cc][rem / PW][rem % PW] = valid >> q & 1u ? v : 0.0f;
        }
        __syncthreads();
        if (c0 + FK_CC < cn)
            fetch(c0 + FK_CC);
        for (int cc = 0; cc < FK_CC && c0 + cc < cn; cc++) {
            float wk[NK][KK];

#pragma unroll
            for (int k = 0; k < NK; k++)
#pragma unroll
                for (int t = 0; t < KK; t++)
                    wk[k][t] = ws[(k * cn + c0 + cc) * KK + t];
#pragma unroll
            for (int i = 0; i < KS + ST; i++)
#pragma unroll
                for (int j = 0; j < KS; j++) {
                    const float x = patch[cc][2 * ty * ST + i][tx * ST + j];

#pragma unroll
                    for (int k = 0; k < NK; k++) {
                        if (i < KS)
                            acc[0][k] = fmaf(wk[k][i * KS + j], x, acc[0][k]);
                        if (i >= ST)
                            acc[1][k] = fmaf(wk[k][(i - ST) * KS + j], x, acc[1][k]);
                    }
                }
        }
        __syncthreads();
    }
    {
        const int ox = ox0 + tx;
        float *out = a.out + (long long)img * a.out_stride;
        /* Pieces: raw sums, planes [piece][image][k]. */
        float *pp = a.part + ((long long)piece * nb + img) * NK * a.Ho * a.Wo;

#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int oy = oy0 + 2 * ty + r;

            if (ox >= a.Wo || oy >= a.Ho)
                continue;
#pragma unroll
            for (int k = 0; k < NK; k++) {
                if (a.split > 1) {
                    pp[((long long)k * a.Ho + oy) * a.Wo + ox] = acc[r][k];
                    continue;
                }
                const float v = acc[r][k] + (a.bias ? a.bias[k0 + k] : 0.0f);

                out[((long long)(k0 + k) * a.Ho + oy) * a.Wo + ox] =
                    icoreg_act(v, a.act, a.slope);
            }
        }
    }
}

/* The pieces of conv_fewk_kernel: one thread per (image, channel, output)
 * adds them in piece order, then bias and activation. */
__global__ void __launch_bounds__(256)
    conv_fewk_sum_kernel(const conv_args a, int k0, int nk, int nb)
{
    const long long plane = (long long)nk * a.Ho * a.Wo;
    const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
    const int img = blockIdx.y;

    if (e >= plane)
        return;
    float v = a.part[(long long)img * plane + e];

    for (int p = 1; p < a.split; p++)
        v += a.part[((long long)p * nb + img) * plane + e];
    const int k = (int)(e / ((long long)a.Ho * a.Wo));

    if (a.bias)
        v += a.bias[k0 + k];
    a.out[(long long)img * a.out_stride + (long long)k0 * a.Ho * a.Wo + e] =
        icoreg_act(v, a.act, a.slope);
}

/* Pieces of the input channels for conv_fewk_kernel over nb images: about
 * eight blocks a CU, whole steps of FK_CC channels each. cpp: channels a
 * piece. */
static int fewk_split(const conv_args &a, int st, int nb, int cus, int &cpp)
{
    const int cc = st == 1 ? 4 : 2, steps = (a.C + cc - 1) / cc;
    const long long blocks = (long long)((a.Wo + 15) / 16) * ((a.Ho + 31) / 32) * nb;
    int split = blocks < 8LL * cus ? (int)((8LL * cus + blocks - 1) / blocks) : 1;

    split = std::min(std::min(split, 8), steps);
    if (nb * (long long)split > 65535)
        split = 1;
    cpp = (steps + split - 1) / split * cc;
    return (a.C + cpp - 1) / cpp;
}

template <int KS, int ST>
static void launch_fewk(const conv_args &a, int k0, int nk, int nb, int cus, hipStream_t s)
{
    int cpp;
    const int split = a.part ? fewk_split(a, ST, nb, cus, cpp) : 1;
    conv_args f = a;

    if (split == 1)
        cpp = (a.C + (ST == 1 ? 4 : 2) - 1) / (ST == 1 ? 4 : 2) * (ST == 1 ? 4 : 2);
    f.split = split;
    const dim3 grid((a.Wo + 15) / 16, (a.Ho + 31) / 32, nb * split);
    const size_t lds = fewk_lds_bytes(nk, cpp, KS * KS);

#define FK_CASE(N)                                                             \
    case N:                                                                    \
        hipLaunchKernelGGL((conv_fewk_kernel<KS, ST, N>), grid, dim3(256), lds, s, f, k0, nb, \
                           cpp);                                               \
        break;
    switch (nk) {
        FK_CASE(1)
        FK_CASE(2)
        FK_CASE(3)
        FK_CASE(4)
        FK_CASE(5)
        FK_CASE(6)
        FK_CASE(7)
        FK_CASE(8)
    }
#undef FK_CASE
    if (split > 1)
        hipLaunchKernelGGL(conv_fewk_sum_kernel,
                           dim3((unsigned)(((long long)nk * a.Ho * a.Wo + 255) / 256), nb),
                           dim3(256), 0, s, f, k0, nk, nb);
}

bool conv_direct_supported(int kh, int kw, int sy, int sx, int dy, int dx,
                           int groups)
{
    return groups == 1 && kh == kw && (kh == 3 || kh == 5) && sy == sx &&
           (sy == 1 || sy == 2) && dy == 1 && dx == 1;
}

bool conv_direct_fits(long long in_floats, long long w_floats)
{
    /* Buffer offsets are 32-bit byte offsets below the value that marks
     * padding. */
    return in_floats * 4 < 0x80000000LL && w_floats * 4 < 0x80000000LL;
}

/* Padded output area of a th x tw tiling. */
static long long tiled_area(int Ho, int Wo, int th, int tw)
{
    return (long long)((Ho + th - 1) / th) * th * ((Wo + tw - 1) / tw) * tw;
}

/* The direct kernel's configuration for a: channels per block (bm),
 * tile width (tw), the channels the MFMA kernel takes (kmain; the last
 * K - kmain go to the few-channel kernel) and the input-channel pieces. */
struct direct_plan {
    int bm, tw, kmain, split;
};

/* 3 x 3: blocks of 64 channels x 64 pixels, the fastest of the 64 / 128
 * channel x 64 / 128 pixel blocks at every ELoFTR layer measured (the
 * small block keeps the most waves per CU in flight). 5 x 5: 128 pixels,
 * and 128 channels unless that grid would leave CUs with fewer than two
 * blocks each. The tile is 2 x 32 / 4 x 32 or 4 x 16 / 8 x 16 pixels,
 * whichever pads the image less. A last block of at most FK_MAXK
 * channels goes to the few-channel kernel. Grids of fewer blocks than
 * CUs (DISK's 64 x 64 and 32 x 32 layers: 8-32 blocks) are cut over the
 * input channels into up to 16 pieces, so that about two blocks per CU
 * run, each piece at least one channel slice. */
static direct_plan plan_direct(const conv_args &a, int ks, int nb, int cus)
{
    const int nj = ks == 3 ? 1 : 2, px = 64 * nj;
    const bool narrow = tiled_area(a.Ho, a.Wo, px / 16, 16) < tiled_area(a.Ho, a.Wo, px / 32, 32);
    const int tw = narrow ? 16 : 32, th = px / tw;
    const long long tiles = (long long)((a.Wo + tw - 1) / tw) * ((a.Ho + th - 1) / th);
    direct_plan p;

    p.tw = tw;
    p.bm = ks == 5 && a.K > 64 && tiles * ((a.K + 127) / 128) * nb >= 2LL * cus ? 128 : 64;
    {
        const int rem = a.K % p.bm;

        p.kmain = a.K > p.bm && rem <= FK_MAXK && a.C <= FK_MAXC &&
                          (long long)rem * a.C * ks * ks <= FK_MAXW
                      ? a.K - rem
                      : a.K;
    }
    {
        const int cc = p.bm == 128 ? 2 : 4, nk = (a.C + cc - 1) / cc;
        const long long blocks = tiles * ((p.kmain + p.bm - 1) / p.bm) * nb;
        int split = blocks < cus ? (int)((2LL * cus + blocks - 1) / blocks) : 1;

        split = split < 16 ? split : 16;
        split = split < nk ? split : nk;
        /* Every piece non-empty: pieces of ceil(nk / split) slices. */
        if (split > 1) {
            const int per = (nk + split - 1) / split;

            split = (nk + per - 1) / per;
        }
        if (nb * (long long)split > 65535)
            split = 1;
        p.split = split;
    }
    return p;
}

size_t conv_direct_part_bytes(const conv_args &a, int ks, int stride, int nb, int cus)
{
    if (a.C == 1 && !a.mean && a.K <= C1_MAXK && a.K * ks * ks <= C1_MAXW)
        return 0;
    const direct_plan p = plan_direct(a, ks, nb, cus);
    const size_t main = p.split > 1 ? (size_t)p.split * nb * p.kmain * a.Ho * a.Wo : 0;
    size_t fewk = 0;

    if (p.kmain < a.K) {
        /* The few-channel kernel runs after the main one's pieces are
         * added, so the two share the buffer. */
        int cpp;
        const int split = fewk_split(a, stride, nb, cus, cpp);

        if (split > 1)
            fewk = (size_t)split * nb * (a.K - p.kmain) * a.Ho * a.Wo;
    }
    return std::max(main, fewk) * sizeof(float);
}

template <int KS, int ST, int BM, int TW, int NJ>
static void launch_cfg(const conv_args &a, const direct_plan &p, int nb, int cus, hipStream_t s)
{
    /* K = 100 (5 x 5) or 36 (3 x 3) per slice at 64 channels per block,
     * 50 at 128. */
    constexpr int CC = BM == 128 ? 2 : 4;
    constexpr int TH = 64 * NJ / TW;
    const int tiles = ((a.Wo + TW - 1) / TW) * ((a.Ho + TH - 1) / TH);
    conv_args m = a;

    m.K = p.kmain;
    m.split = p.split;
    hipLaunchKernelGGL((conv_mfma<KS, ST, BM, TW, CC, NJ>),
                       dim3(tiles, (m.K + BM - 1) / BM, nb * p.split), dim3(256), 0, s, m);
    if (p.split > 1)
        hipLaunchKernelGGL(conv_pieces_kernel,
                           dim3((unsigned)(((long long)m.K * a.Ho * a.Wo + 255) / 256), nb),
                           dim3(256), 0, s, m, nb);
    if (p.kmain < a.K)
        launch_fewk<KS, ST>(a, p.kmain, a.K - p.kmain, nb, cus, s);
}

template <int KS, int ST>
static void launch_ks(const conv_args &a, int nb, int cus, hipStream_t s)
{
    constexpr int NJ = KS == 3 ? 1 : 2;
    const direct_plan p = plan_direct(a, KS, nb, cus);

    if (p.bm == 128) {
        if (p.tw == 16)
            launch_cfg<KS, ST, 128, 16, NJ>(a, p, nb, cus, s);
        else
            launch_cfg<KS, ST, 128, 32, NJ>(a, p, nb, cus, s);
        return;
    }
    if (p.tw == 16)
        launch_cfg<KS, ST, 64, 16, NJ>(a, p, nb, cus, s);
    else
        launch_cfg<KS, ST, 64, 32, NJ>(a, p, nb, cus, s);
}

void conv_direct_launch(const conv_args &a, int ks, int stride, int nb,
                        int cus, hipStream_t s)
{
    if (a.C == 1 && !a.mean && a.K <= C1_MAXK && a.K * ks * ks <= C1_MAXW) {
        const dim3 grid((unsigned)(((long long)a.Ho * a.Wo + 255) / 256), 1, nb);

        if (ks == 3 && stride == 1)
            hipLaunchKernelGGL((conv_c1_kernel<3, 1>), grid, dim3(256), 0, s, a);
        else if (ks == 3)
            hipLaunchKernelGGL((conv_c1_kernel<3, 2>), grid, dim3(256), 0, s, a);
        else if (stride == 1)
            hipLaunchKernelGGL((conv_c1_kernel<5, 1>), grid, dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL((conv_c1_kernel<5, 2>), grid, dim3(256), 0, s, a);
        return;
    }
    if (ks == 3 && stride == 1)
        launch_ks<3, 1>(a, nb, cus, s);
    else if (ks == 3)
        launch_ks<3, 2>(a, nb, cus, s);
    else if (stride == 1)
        launch_ks<5, 1>(a, nb, cus, s);
    else
        launch_ks<5, 2>(a, nb, cus, s);
}

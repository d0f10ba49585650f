/* SPDX-License-Identifier: Unlicense */

/* 3 x 3, stride 1, padding 1 convolution by Winograd's F(4 x 4, 3 x 3) on
 * the CDNA4 matrix cores: the same result as the reference's direct and
 * im2col + GEMM paths of ops_conv2d (ops.cl:319-387, ops.c:236-336 of
 * i.coregistration.opencl), with 36 products per 4 x 4 output tile and
 * input channel instead of 144 (F(2 x 2, 3 x 3) of conv_wino.hip does 64
 * for the same 16 outputs).
 *
 * For a tile d (6 x 6 input values, padding zeros included) and a filter
 * g (3 x 3): V = B^T d B, U = G g G^T, Y = A^T (sum over channels of
 * U . V) A, with the interpolation points 0, 1, -1, 2, -2 and infinity:
 *   B^T = [4  0 -5  0  1  0;  0 -4 -4  1  1  0;  0  4 -4 -1  1  0;
 *          0 -2 -1  2  1  0;  0  2 -1 -2  1  0;  0  4  0 -5  0  1],
 *   G   = [1/4 0 0; -1/6 -1/6 -1/6; -1/6 1/6 -1/6; 1/24 1/12 1/6;
 *          1/24 -1/12 1/6; 0 0 1],
 *   A^T = [1 1 1 1 1 0;  0 1 -1 2 -2 0;  0 1 1 4 4 0;  0 1 -1 8 -8 1]
 * (Lavin and Gray, "Fast Algorithms for Convolutional Neural Networks",
 * 2016). fp32 error of the transform pair: about 2e-6 of the output scale
 * over 256 channels (3e-7 for F(2 x 2)), far inside the 1e-3 contraction
 * tolerance.
 *
 * The 36 positions (xi, nu) of the transform are 36 GEMMs over the input
 * channels, M(xi nu)(k, t) = sum_c U(xi nu)(k, c) V(xi nu)(c, t), run on
 * v_mfma_f32_16x16x4f32 (16 output channels x 16 tiles x 4 input
 * channels): lane l feeds the B operand with V of (channel l / 16, tile
 * l % 16), so a lane forms the transform of its (tile, channel) itself
 * from the window it reads, and the accumulators of its (4 output
 * channels, tile) hold M for those outputs, so the output transform runs
 * in registers too.
 *
 * The matrix cores and the vector ALUs of a SIMD do not run at the same
 * time for fp32 work on gfx950 (a wave interleaving 8 MFMAs with 64 VALU
 * FMAs took the sum of the two loops' times, not the larger), so the
 * transform's VALU cycles add to the MFMA cycles, and the kernel uses each
 * transformed value in as many products as the registers allow: a
 * transformed tile feeds 32 output channels (two 16-channel GEMMs a
 * position), and the 36 positions are split over two waves of the same 16
 * tiles. Wave half hf takes the rows xi = 3 hf .. 3 hf + 2 of V = B^T d B
 * (it reads five of the window's six rows, forms the three rows of B^T d
 * it needs, then their row transforms) and keeps 2 x 18 accumulators
 * (about 1.4 VALU instructions a product, against 2.5 for a wave of all
 * 36 positions and 16 channels).
 *
 * A block is four waves: two tile groups of 16 tiles (32 tiles: BTR x
 * BTC of 4 x 4 pixels) times the two halves, two blocks a CU so that one
 * block's LDS reads after its barrier overlap the other's products. The
 * block walks the input channels 4 at a time (a slice): the input patch
 * of a slice (from 16-byte aligned columns, the range check of the buffer
 * window giving the zero padding) arrives by LDS DMA (buffer_load ...
 * lds) three slices ahead into a ring of four buffers, and a wave reads
 * the next slice's window into the registers its window has just freed
 * (after the column transform), beside this slice's products. The
 * filters (the A
 * operands: 32 channels x 4 input channels x 36 positions a slice, stored
 * in the operand's lane order) go from L2 straight into registers: a wave
 * holds one slice's 36 operands and reloads the 12 of a transform row for
 * the next slice as soon as that row's products are issued. The halves'
 * partial outputs A^T M A meet in LDS at the end, each half storing two of
 * the four output rows. */

#include <hip/hip_runtime.h>

#include <type_traits>

#include "act.h"
#include "conv.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));

#define W4_CS 4           /* input channels per slice (one MFMA k-step) */
#define W4_OOB 0x80000000u
#define W4_RSRC_FLAGS 0x00020000
#define W4_WAIT_VM0 0x0F70

static __device__ __forceinline__ __amdgpu_buffer_rsrc_t w4_rsrc(const float *p,
                                                               unsigned long long bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, (int)(unsigned)bytes,
                                             W4_RSRC_FLAGS);
}

/* x := B^T x for a 6-vector. */
static __device__ __forceinline__ void w4_bt(float (&x)[6])
{
    const float a = __builtin_fmaf(-4.0f, x[2], x[4]), b = __builtin_fmaf(-4.0f, x[1], x[3]);
    const float c = x[4] - x[2], e = 2.0f * (x[3] - x[1]);
    const float y0 = __builtin_fmaf(4.0f, x[0], __builtin_fmaf(-5.0f, x[2], x[4]));
    const float y5 = __builtin_fmaf(4.0f, x[1], __builtin_fmaf(-5.0f, x[3], x[5]));

    x[0] = y0;
    x[1] = a + b;
    x[2] = a - b;
    x[3] = c + e;
    x[4] = c - e;
    x[5] = y5;
}

/* y := A^T m for a 6-vector m (4 outputs). */
static __device__ __forceinline__ void w4_at(const float (&m)[6], float (&y)[4])
{
    const float p = m[1] + m[2], q = m[1] - m[2], r = m[3] + m[4], s = m[3] - m[4];

    y[0] = m[0] + p + r;
    y[1] = __builtin_fmaf(2.0f, s, q);
    y[2] = __builtin_fmaf(4.0f, r, p);
    y[3] = __builtin_fmaf(8.0f, s, q) + m[5];
}

/* Block L of T to a unit: the 8 XCDs (blocks L, L + 8, ... run on XCD
 * L % 8) each get a contiguous band of units. */
static __device__ __forceinline__ int w4_band(int L, int T)
{
    const int q = T >> 3, rem = T & 7, x = L & 7, idx = L >> 3;

    return (x < rem ? x * (q + 1) : rem * (q + 1) + (x - rem) * q) + idx;
}

#define W4_BK 32
#define W4_PSLOTS 768    /* patch slots: 3 a thread (720 used) */
#define W4_PBUF (W4_PSLOTS * 4) /* floats a patch buffer: 12 KB */
#define W4_LDS (2 * 128 * 64) /* 64 KB: the exchange; the 3 patch buffers */
#define W4_WAIT_VM12_LGKM0 0x007C
#define W4_WAIT_VM9 0x0F79

/* Filter fragments of the half-position form: U(xi nu)(k, c) at
 * Uf[((kb nsl + sl) 18 + q) 256 + lane 4 + i], 4 q + i = 36 hf + 12
 * (xi % 3) + 6 h + nu with hf = xi / 3, h = (k / 16) % 2, lane = (c % 4)
 * 16 + k % 16, kb = k / 32, sl = c / 4; zero for k >= K. */
__global__ void __launch_bounds__(256)
    wino4_frag_kernel(const float *__restrict__ w, int K, int C, int Kp, float *__restrict__ Uf)
{
    const long long id = (long long)blockIdx.x * 256 + threadIdx.x;
    const int nsl = C / W4_CS;

    if (id >= (long long)Kp * C)
        return;
    const int k = (int)(id % Kp), c = (int)(id / Kp);
    double u[36];

    if (k < K) {
        const float *src = w + ((long long)k * C + c) * 9;
        const double G[6][3] = {{0.25, 0.0, 0.0},
                                {-1.0 / 6, -1.0 / 6, -1.0 / 6},
                                {-1.0 / 6, 1.0 / 6, -1.0 / 6},
                                {1.0 / 24, 1.0 / 12, 1.0 / 6},
                                {1.0 / 24, -1.0 / 12, 1.0 / 6},
                                {0.0, 0.0, 1.0}};
        double t[6][3];

        for (int x = 0; x < 6; x++)
            for (int j = 0; j < 3; j++)
                t[x][j] = G[x][0] * src[j] + G[x][1] * src[3 + j] + G[x][2] * src[6 + j];
        for (int x = 0; x < 6; x++)
            for (int y = 0; y < 6; y++)
                u[x * 6 + y] = t[x][0] * G[y][0] + t[x][1] * G[y][1] + t[x][2] * G[y][2];
    }
    else
        for (int i = 0; i < 36; i++)
            u[i] = 0.0;
    {
        const int kb = k / W4_BK, h = (k / 16) & 1, sl = c / W4_CS;
        const int lane = (c % W4_CS) * 16 + k % 16;
        float *dst = Uf + ((long long)kb * nsl + sl) * (72 * 64) + lane * 4;

        for (int xi = 0; xi < 6; xi++)
            for (int nu = 0; nu < 6; nu++) {
                const int g = (xi / 3) * 36 + (xi % 3) * 12 + h * 6 + nu;

                dst[(g >> 2) * 256 + (g & 3)] = (float)u[xi * 6 + nu];
            }
    }
}

template <int BTC>
__global__ void __launch_bounds__(256, 2)
    conv_wino4_kernel(const conv_args a, const float *__restrict__ Uf, int nkb, int tbx,
                       int ntb, int units)
{
    constexpr int BTR = 32 / BTC;
    constexpr int PR = 4 * BTR + 2;
    constexpr int PCH = BTC + 2;
    constexpr int PP = 4 * PCH;
    constexpr int PSZ = PR * PP;
    constexpr int NPC = W4_CS * PR * PCH;
    static_assert(NPC <= W4_PSLOTS, "patch past its DMA slots");
    static_assert(4 * W4_PBUF <= W4_LDS, "patch ring past the LDS");
    __shared__ __align__(16) float lds[W4_LDS];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tg = wave & 1, hf = wave >> 1;
    const int kq = lane >> 4, n = lane & 15;
    const int C = a.C, H = a.H, W = a.W, Ho = a.Ho, Wo = a.Wo;
    const int nsl = C / W4_CS;
    const int u = w4_band(blockIdx.x, units);
    const int bx = u % nkb, t0 = u / nkb, by = t0 % ntb, bz = t0 / ntb;
    const int ty0 = (by / tbx) * BTR, tx0 = (by % tbx) * BTC;
    const long long HW = (long long)H * W;
    const float *in = a.in + (long long)bz * a.in_stride;
    const unsigned long long ibytes = (unsigned long long)C * HW * 4;
    const int t = tg * 16 + n, tr = t / BTC, tc = t % BTC;
    unsigned poff[3];
    floatx4 acc[2][18];

#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int g = 0; g < 18; g++)
            acc[h][g] = (floatx4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < 3; q++) {
        const int s = tid + 256 * q, c = s / (PR * PCH), rem = s - c * (PR * PCH);
        const int r = rem / PCH, ch = rem - r * PCH;
        const int iy = 4 * ty0 - 1 + r, ix = 4 * tx0 - 4 + 4 * ch;

        poff[q] = s < NPC && iy >= 0 && iy < H && ix >= 0 && ix < W
                      ? (unsigned)((c * HW + (long long)iy * W + ix) * 4)
                      : W4_OOB;
    }
    /* 3 DMA instructions a thread for a patch, 5 for filters. */
    /* Past the last slice the window is empty (zeros into a buffer no
     * later slice reads), so that every slice issues the same loads. */
    auto load_patch = [&](int sl, float *buf) {
        const bool in_range = sl < nsl;
        const __amdgpu_buffer_rsrc_t rp = w4_rsrc(
            in + (long long)(in_range ? sl : 0) * W4_CS * HW,
            in_range ? ibytes - (unsigned long long)sl * W4_CS * HW * 4 : 0ull);

#pragma unroll
        for (int q = 0; q < 3; q++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rp, (__attribute__((address_space(3))) void *)(buf + 1024 * q + 256 * wave), 16,
                (int)poff[q], 0, 0, 0);
    };
    /* This wave's operands of slice sl: ug + sl 4608 + 256 j, j < 9 (row
     * xl of the half: j = 3 xl .. 3 xl + 2). */
    const float *ug = Uf + (long long)bx * nsl * (72 * 64) + 9 * 256 * hf + lane * 4;
    floatx4 ur[9];

    /* Window rows hf .. hf + 4 (of 0 .. 5), columns 4 tc + 3 .. + 8, of
     * channel kq, from a patch buffer. */
    auto read_window = [&](const float *buf, float (&d)[5][6]) {
        const float *p = buf + kq * PSZ + (4 * tr + hf) * PP + 4 * tc + 3;

#pragma unroll
        for (int i = 0; i < 5; i++) {
            const float *row = p + i * PP;
            const floatx4 v = *(const floatx4 *)(row + 1);

            d[i][0] = row[0];
            d[i][1] = v[0];
            d[i][2] = v[1];
            d[i][3] = v[2];
            d[i][4] = v[3];
            d[i][5] = row[5];
        }
    };
    /* Slice sl from its window d; once d is spent (the column transform),
     * d takes the next slice's window from nbuf, so that those LDS reads
     * run beside this slice's products. */
    auto compute = [&](int sl, float (&d)[5][6], const float *nbuf) {
        /* The next slice's operands (the last slice reloads its own). */
        const float *un = ug + (long long)(sl + 1 < nsl ? sl + 1 : sl) * (72 * 64);
        float r[3][6];

        /* Rows 3 hf .. 3 hf + 2 of B^T d, from window rows hf .. hf + 4. */
        if (hf == 0) {
#pragma unroll
            for (int j = 0; j < 6; j++) {
                const float e = __builtin_fmaf(-4.0f, d[2][j], d[4][j]);
                const float f = __builtin_fmaf(-4.0f, d[1][j], d[3][j]);

                r[0][j] = __builtin_fmaf(4.0f, d[0][j], __builtin_fmaf(-5.0f, d[2][j], d[4][j]));
                r[1][j] = e + f;
                r[2][j] = e - f;
            }
        }
        else {
            /* Window rows 1 .. 5 as d[0 .. 4]. */
#pragma unroll
            for (int j = 0; j < 6; j++) {
                const float e = d[3][j] - d[1][j], f = d[2][j] - d[0][j];

                r[0][j] = __builtin_fmaf(2.0f, f, e);
                r[1][j] = __builtin_fmaf(-2.0f, f, e);
                r[2][j] = __builtin_fmaf(4.0f, d[0][j], __builtin_fmaf(-5.0f, d[2][j], d[4][j]));
            }
        }
        read_window(nbuf, d);
#pragma unroll
        for (int xl = 0; xl < 3; xl++) {
            w4_bt(r[xl]);
            /* Row xl's operands (loaded during the last slice) have
             * landed once at most 9 loads are outstanding: after them came
             * the later rows' 6 loads of this slice's operands, this
             * slice's patch DMA (3) and the next slice's reloads of rows <
             * xl (3 xl): 9 + 3 xl, of which the wait lets 9 be pending. */
            __builtin_amdgcn_s_waitcnt(W4_WAIT_VM9);
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int nu = 0; nu < 6; nu++) {
                    const int g = 12 * xl + 6 * h + nu;

                    acc[h][xl * 6 + nu] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        ur[g >> 2][g & 3], r[xl][nu], acc[h][xl * 6 + nu], 0, 0, 0);
                }
            /* The row's operands are issued: reload them for the next
             * slice (they land during the rest of this slice and the next
             * one's transform). */
#pragma unroll
            for (int j = 3 * xl; j < 3 * xl + 3; j++)
                ur[j] = *(const floatx4 *)(un + 256 * j);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    /* Patch of slice s in patch buffer s % 4. In slice s the patch of s +
     * 3 (3 loads a thread) is issued first, then the 9 operand loads of s
     * + 1; vector-memory loads complete in order, so a wait down to those
     * 12 at the slice's end has the patch of s + 2 (issued a slice
     * earlier) in LDS for the next slice to read the window after. Every
     * slice issues these 12 (empty or repeated ones at the end), so the
     * counts hold throughout. */
    float *const pb = lds;
    float d[5][6];

#pragma unroll
    for (int j = 0; j < 9; j++)
        ur[j] = *(const floatx4 *)(ug + 256 * j);
#pragma unroll
    for (int i = 0; i < 3; i++)
        load_patch(i, pb + i * W4_PBUF);
    __builtin_amdgcn_s_waitcnt(W4_WAIT_VM0);
    __syncthreads();
    read_window(pb, d);
    {
        int p4 = 0;

        for (int sl = 0; sl < nsl; sl++) {
            const int p4n = (p4 + 1) & 3, p4f = (p4 + 3) & 3;

            load_patch(sl + 3, pb + p4f * W4_PBUF);
            compute(sl, d, pb + p4n * W4_PBUF);
            /* A bare barrier (an asm statement that also keeps the compiler
             * from moving memory accesses across it): __syncthreads' fence
             * would wait for every outstanding load, the patch DMA ahead
             * included. This slice's LDS reads are consumed by now
             * (lgkmcnt 0). */
            __builtin_amdgcn_s_waitcnt(W4_WAIT_VM12_LGKM0);
            asm volatile("s_barrier" ::: "memory");
            p4 = p4n;
        }
    }
    __builtin_amdgcn_s_waitcnt(W4_WAIT_VM0);
    __syncthreads();

    /* Output: Z = M A over nu in registers, then each half's share of
     * Y = A^T Z over its rows xi. Half hf stores output rows ii = 2 hf,
     * 2 hf + 1 of its tiles and passes its share of the other two rows
     * to the partner wave through LDS (the buffers are free: all DMA has
     * landed). Exchange layout: [tg][destination half][h][v][ii % 2][jj]
     * [lane]. */
    float y[2][4][4][4];

#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            float z[3][4];

#pragma unroll
            for (int xl = 0; xl < 3; xl++) {
                const float m[6] = {acc[h][xl * 6 + 0][v], acc[h][xl * 6 + 1][v],
                                    acc[h][xl * 6 + 2][v], acc[h][xl * 6 + 3][v],
                                    acc[h][xl * 6 + 4][v], acc[h][xl * 6 + 5][v]};

                w4_at(m, z[xl]);
            }
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                if (hf == 0) {
                    const float p = z[1][jj] + z[2][jj], q = z[1][jj] - z[2][jj];

                    y[h][v][0][jj] = z[0][jj] + p;
                    y[h][v][1][jj] = q;
                    y[h][v][2][jj] = p;
                    y[h][v][3][jj] = q;
                }
                else {
                    /* Rows 3, 4, 5 of M as z[0 .. 2]. */
                    const float p = z[0][jj] + z[1][jj], q = z[0][jj] - z[1][jj];

                    y[h][v][0][jj] = p;
                    y[h][v][1][jj] = 2.0f * q;
                    y[h][v][2][jj] = 4.0f * p;
                    y[h][v][3][jj] = __builtin_fmaf(8.0f, q, z[2][jj]);
                }
            }
        }
    /* Slot of (h, v, row pair member r, jj) for destination half dh. */
    float *const xs = lds + tg * (128 * 64) + lane;
    auto slot = [&](int dh, int h, int v, int r, int jj) {
        return xs + ((((dh * 2 + h) * 4 + v) * 2 + r) * 4 + jj) * 64;
    };

#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int v = 0; v < 4; v++)
#pragma unroll
            for (int r = 0; r < 2; r++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++)
                    *slot(1 - hf, h, v, r, jj) = hf ? y[h][v][r][jj] : y[h][v][2 + r][jj];
    __syncthreads();

    float *out = a.out + (long long)bz * a.out_stride;
    const int oy = 4 * (ty0 + tr), ox = 4 * (tx0 + tc);
    const bool vec = Wo % 4 == 0 && ox + 4 <= Wo && (a.out_stride & 3) == 0 &&
                     ((unsigned long long)(size_t)a.out & 15) == 0;
    /* Partner sums, bias, activation and stores, with the activation
     * chosen once (a switch per value costs more branches and code than
     * the stores themselves). */
    auto store = [&](auto actc) {
        constexpr int ACT = decltype(actc)::value;

#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int kg = bx * W4_BK + h * 16 + 4 * kq + v;

                if (kg >= a.K)
                    continue;
                const float bias = a.bias ? a.bias[kg] : 0.0f;

#pragma unroll
                for (int r = 0; r < 2; r++) {
                    const int ii = 2 * hf + r;
                    float *row = out + ((long long)kg * Ho + oy + ii) * Wo + ox;
                    float o[4];

                    if (oy + ii >= Ho)
                        continue;
#pragma unroll
                    for (int jj = 0; jj < 4; jj++)
                        o[jj] = icoreg_act((hf ? y[h][v][2 + r][jj] : y[h][v][r][jj]) +
                                               *slot(hf, h, v, r, jj) + bias,
                                           ACT, a.slope);
                    if (vec)
                        *(floatx4 *)row = (floatx4){o[0], o[1], o[2], o[3]};
                    else
#pragma unroll
                        for (int jj = 0; jj < 4; jj++)
                            if (ox + jj < Wo)
                                row[jj] = o[jj];
                }
            }
    };

    switch (a.act) {
    case ACT_GELU:
        store(std::integral_constant<int, ACT_GELU>{});
        break;
    case ACT_RELU:
        store(std::integral_constant<int, ACT_RELU>{});
        break;
    case ACT_LEAKY:
        store(std::integral_constant<int, ACT_LEAKY>{});
        break;
    case ACT_GELU_TANH:
        store(std::integral_constant<int, ACT_GELU_TANH>{});
        break;
    default:
        store(std::integral_constant<int, ACT_NONE>{});
        break;
    }
}

/* Tile-block columns: 16 tiles across (2 x 16 tiles a block) where the
 * map is wide enough to use them, else 8 (4 x 8). */
static int w4_btc(int Wo) { return (Wo + 3) / 4 >= 48 ? 16 : 8; }

bool conv_wino4_ok(int C, int K, bool norm) { return C % W4_CS == 0 && K >= 16 && !norm; }

size_t conv_wino4_weight_floats(int K, int C)
{
    return (size_t)((K + W4_BK - 1) / W4_BK * W4_BK) * C * 36;
}

void conv_wino4_weights(const float *w, int K, int C, float *U, hipStream_t s)
{
    const int Kp = (K + W4_BK - 1) / W4_BK * W4_BK;
    const long long n = (long long)Kp * C;

    hipLaunchKernelGGL(wino4_frag_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       w, K, C, Kp, U);
}

long long conv_wino4_units(int K, int Ho, int Wo, int nb)
{
    const int btc = w4_btc(Wo), btr = 32 / btc;
    const long long tb = (long long)(((Ho + 3) / 4 + btr - 1) / btr) *
                         (((Wo + 3) / 4 + btc - 1) / btc);

    return (long long)((K + W4_BK - 1) / W4_BK) * tb * nb;
}

void conv_wino4_launch(const conv_args &a, const float *U, int nb, hipStream_t s)
{
    const int nkb = (a.K + W4_BK - 1) / W4_BK, btc = w4_btc(a.Wo);
    const int tbx = ((a.Wo + 3) / 4 + btc - 1) / btc;
    const long long units = conv_wino4_units(a.K, a.Ho, a.Wo, nb);
    const int ntb = (int)(units / nkb / nb);

    if (btc == 16)
        hipLaunchKernelGGL(conv_wino4_kernel<16>, dim3((unsigned)units), dim3(256), 0, s, a, U,
                           nkb, tbx, ntb, (int)units);
    else
        hipLaunchKernelGGL(conv_wino4_kernel<8>, dim3((unsigned)units), dim3(256), 0, s, a, U,
                           nkb, tbx, ntb, (int)units);
}

/* SPDX-License-Identifier: Unlicense */

/* 3 x 3, stride 1, padding 1 convolution by Winograd's minimal filtering
 * F(2 x 2, 3 x 3) on the CDNA4 matrix cores: the same result as the
 * reference's direct and im2col + GEMM paths of ops_conv2d (ops.cl:319-387,
 * ops.c:236-336 of i.coregistration.opencl), with 16 multiplications per
 * 2 x 2 output tile and input channel instead of 36.
 *
 * For a tile d (4 x 4 input values, padding zeros included) and a filter g
 * (3 x 3):
 *   V = B^T d B,  U = G g G^T,  Y = A^T (sum over channels of U . V) A,
 * with B^T = [1 0 -1 0; 0 1 1 0; 0 -1 1 0; 0 1 0 -1],
 *      G   = [1 0 0; 1/2 1/2 1/2; 1/2 -1/2 1/2; 0 0 1],
 *      A^T = [1 1 1 0; 0 1 -1 -1]
 * (Lavin and Gray, "Fast Algorithms for Convolutional Neural Networks",
 * 2016). The channel sums are 16 GEMMs, one per position (xi, nu) of the
 * 4 x 4 transform: M[xi nu](k, t) = sum_c U[xi nu](k, c) V[xi nu](c, t).
 *
 * Two kernels. conv_wino_rows_kernel (further down) takes convolutions
 * without input normalisation over whole 8-channel slices: each wave forms
 * its own row of the transform in registers. conv_wino_kernel, the staged
 * form, takes the rest:
 *
 * wino_weights_kernel writes U as [16][C][K]. conv_wino_kernel: a block
 * takes 32 tiles (a 4 x 8 grid of 2 x 2 output tiles, 8 x 16 pixels; the
 * template also allows 8 x 8 tiles) of one image and 32 output channels,
 * and walks the input channels WG_CC at a time:
 *  - the input patch under the tiles (WG_CC x (2 WG_TR + 2) x 18, zero
 *    outside the image, normalised and gated when asked) and the U slice
 *    go to LDS; the next slice is fetched into registers while the
 *    matrix cores work on the current one;
 *  - each thread transforms WG_CC NT / 256 (channel, tile) patches into V
 *    in LDS;
 *  - wave w runs the 4 GEMMs of row xi = w of the transform
 *    (v_mfma_f32_32x32x2f32, 32 channels x 32 tiles per MFMA column);
 *  - at the end each wave applies A over nu in registers, the rows over
 *    xi are combined through LDS, and bias and activation are applied on
 *    the 2 x 2 outputs. */

#include <algorithm>
#include <hip/hip_runtime.h>

#include "act.h"
#include "conv.h"

typedef float floatx16 __attribute__((ext_vector_type(16)));

#define WG_TC 8  /* tile columns per block */
#define WG_BK 32 /* output channels per block */

/* Offset past the end of every buffer read (each below 2 GiB): 0. */
#define WG_OOB 0x80000000u
#define WG_RSRC_FLAGS 0x00020000

static __device__ __forceinline__ __amdgpu_buffer_rsrc_t
wg_rsrc(const float *p, unsigned long long bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0,
                                             (int)(unsigned)bytes,
                                             WG_RSRC_FLAGS);
}

/* U[xi nu][c][k] = (G g G^T)[xi][nu] of filter g = w[k][c]. */
__global__ void __launch_bounds__(256)
    wino_weights_kernel(const float *__restrict__ w, int K, int C,
                        float *__restrict__ U)
{
    const long long id = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long kc = (long long)K * C;
    float g[9], t[4][3];

    if (id >= kc)
        return;
    {
        const int k = (int)(id % K), c = (int)(id / K);
        const float *src = w + ((long long)k * C + c) * 9;

#pragma unroll
        for (int i = 0; i < 9; i++)
            g[i] = src[i];
        /* t = G g (4 x 3). */
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const float g0 = g[j], g1 = g[3 + j], g2 = g[6 + j];

            t[0][j] = g0;
            t[1][j] = 0.5f * (g0 + g1 + g2);
            t[2][j] = 0.5f * (g0 - g1 + g2);
            t[3][j] = g2;
        }
        /* U = t G^T (4 x 4). */
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float a0 = t[i][0], a1 = t[i][1], a2 = t[i][2];
            const float u[4] = {a0, 0.5f * (a0 + a1 + a2),
                                0.5f * (a0 - a1 + a2), a2};

#pragma unroll
            for (int j = 0; j < 4; j++)
                U[(long long)(i * 4 + j) * kc + (long long)c * K + k] = u[j];
        }
    }
}

/* WG_TR tile rows (4 or 8: 32 or 64 tiles per block), WG_CC input
 * channels per K slice, at least MINW waves per SIMD (registers capped to
 * fit them). */
template <bool NORM, int WG_TR, int WG_CC, int MINW>
__global__ void __launch_bounds__(256, MINW)
    conv_wino_kernel(const conv_args a, const float *__restrict__ U)
{
    constexpr int PH = 2 * WG_TR + 2, PW = 2 * WG_TC + 2;
    constexpr int PWP = PW + 1;
    constexpr int PCH = PH * PWP;
    constexpr int PN = WG_CC * PH * PW;      /* patch values per slice */
    constexpr int NP = (PN + 255) / 256;     /* per thread */
    constexpr int NU = 16 * WG_CC * WG_BK / 4 / 256; /* float4 of U */
    constexpr int NT = WG_TR * WG_TC;        /* tiles per block */
    constexpr int NH = NT / 32;              /* 32-tile MFMA columns */
    constexpr int NV = WG_CC * NT / 256;     /* (c, t) transforms each */
    static_assert(16 * WG_CC * (NT + WG_BK) >= 8 * WG_BK * 32,
                  "the output transform reuses the V and U buffers");
    /* [Vs | Us | Ps]: V [pos][c][t], U [pos][c][k], the patch (+ one slot
     * for idle lanes); the output transform reuses Vs and Us. */
    __shared__ __align__(16) float lds[16 * WG_CC * (NT + WG_BK) +
                                        WG_CC * PCH + 1];
    float *const Vs = lds, *const Us = lds + 16 * WG_CC * NT;
    float *const Ps = Us + 16 * WG_CC * WG_BK;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int half = lane >> 5, col = lane & 31;
    const int C = a.C, H = a.H, W = a.W, K = a.K;
    const int tiles_w = (W + 1) / 2, bw = (tiles_w + WG_TC - 1) / WG_TC;
    /* Output-channel blocks on grid x: consecutive blocks go to
     * consecutive XCDs, so each XCD's L2 holds the filter slices of
     * its own channel blocks across all tiles. */
    const int ty0 = (blockIdx.y / bw) * WG_TR, tx0 = (blockIdx.y % bw) * WG_TC;
    const int k0 = blockIdx.x * WG_BK;
    const int iy0 = 2 * ty0 - 1, ix0 = 2 * tx0 - 1;
    const long long HW = (long long)H * W;
    const float *in = a.in + (long long)blockIdx.z * a.in_stride;
    const unsigned long long ibytes = (unsigned long long)C * HW * 4;
    const unsigned long long ubytes = 16ULL * C * K * 4;
    unsigned poff[NP], uoff[NU];
    int ldp[NP];
    float rp[NP];
    float4 ru[NU];
    floatx16 acc[4][NH];

#pragma unroll
    for (int v = 0; v < 4; v++)
#pragma unroll
        for (int h = 0; h < NH; h++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                acc[v][h][r] = 0.0f;

    /* Per-thread offsets, the same for every slice. Patch value
     * (c, py, px); U float4 (position, c, k quad). */
#pragma unroll
    for (int q = 0; q < NP; q++) {
        const int e = tid + 256 * q, c = e / (PH * PW);
        const int rem = e - c * (PH * PW), py = rem / PW, px = rem - py * PW;
        const int iy = iy0 + py, ix = ix0 + px;

        poff[q] = e < PN && iy >= 0 && iy < H && ix >= 0 && ix < W
                      ? (unsigned)((c * HW + (long long)iy * W + ix) * 4)
                      : WG_OOB;
        ldp[q] = e < PN ? c * PCH + py * PWP + px : WG_CC * PCH;
    }
#pragma unroll
    for (int q = 0; q < NU; q++) {
        const int e = tid + 256 * q, kq = e % (WG_BK / 4);
        const int pc = e / (WG_BK / 4), pos = pc / WG_CC, c = pc % WG_CC;

        uoff[q] = k0 + 4 * kq < K
                      ? (unsigned)((((long long)pos * C + c) * K + k0 + 4 * kq) *
                                   4)
                      : WG_OOB;
    }

    auto fetch = [&](int c0) {
        const __amdgpu_buffer_rsrc_t ri =
            wg_rsrc(in + c0 * HW, ibytes - (unsigned long long)c0 * HW * 4);
        /* U rows of this slice start c0 rows on; rows past C (and past
         * the last position's end) read 0 or are multiplied by V = 0. */
        const __amdgpu_buffer_rsrc_t ru_ =
            wg_rsrc(U + (long long)c0 * K, ubytes - (unsigned long long)c0 * K * 4);

#pragma unroll
        for (int q = 0; q < NP; q++)
            rp[q] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(ri, (int)poff[q],
                                                            0, 0));
#pragma unroll
        for (int q = 0; q < NU; q++)
            ru[q] = __builtin_bit_cast(
                float4, __builtin_amdgcn_raw_buffer_load_b128(
                            ru_, (int)uoff[q], 0, 0));
        if (NORM) {
#pragma unroll
            for (int q = 0; q < NP; q++) {
                const int cg = c0 + (tid + 256 * q) / (PH * PW);
                const int cc = cg < C ? cg : C - 1;
                float v = (rp[q] - a.mean[cc]) * a.rstd[cc];

                if (a.gate)
                    v = v >= 0.0f ? v : a.gate[cc] * v;
                rp[q] = poff[q] != WG_OOB && cg < C ? v : 0.0f;
            }
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int q = 0; q < NP; q++)
            Ps[ldp[q]] = rp[q];
#pragma unroll
        for (int q = 0; q < NU; q++)
            *(float4 *)&Us[(tid + 256 * q) * 4] = ru[q];
    };
    /* V of (channel c, tile t) for the two pairs of this thread. */
    auto transform = [&]() {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int pr = tid + 256 * i, c = pr / NT, t = pr % NT;
            const int tr = t / WG_TC, tc = t % WG_TC;
            const float *p = Ps + c * PCH + 2 * tr * PWP + 2 * tc;
            float d[4][4], u[4][4];

#pragma unroll
            for (int y = 0; y < 4; y++)
#pragma unroll
                for (int x = 0; x < 4; x++)
                    d[y][x] = p[y * PWP + x];
            /* Rows: u = B^T d. */
#pragma unroll
            for (int x = 0; x < 4; x++) {
                u[0][x] = d[0][x] - d[2][x];
                u[1][x] = d[1][x] + d[2][x];
                u[2][x] = d[2][x] - d[1][x];
                u[3][x] = d[1][x] - d[3][x];
            }
            /* Columns: V = u B. */
#pragma unroll
            for (int y = 0; y < 4; y++) {
                const float v0 = u[y][0] - u[y][2], v1 = u[y][1] + u[y][2];
                const float v2 = u[y][2] - u[y][1], v3 = u[y][1] - u[y][3];
                float *o = Vs + (y * 4) * WG_CC * NT + c * NT + t;

                o[0] = v0;
                o[WG_CC * NT] = v1;
                o[2 * WG_CC * NT] = v2;
                o[3 * WG_CC * NT] = v3;
            }
        }
    };

    const int nk = (C + WG_CC - 1) / WG_CC;

    fetch(0);
    for (int kt = 0; kt < nk; kt++) {
        stash();
        __syncthreads();
        if (kt + 1 < nk)
            fetch((kt + 1) * WG_CC);
        transform();
        __syncthreads();
        {
            /* Wave w: positions (w, nu), nu = 0..3; A = U (channels k on
             * lanes), B = V (tiles on lanes), K = input channels. */
#pragma unroll
            for (int s = 0; s < WG_CC / 2; s++) {
                const int c = 2 * s + half;
                float av[4], bv[4][NH];

#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int pos = wave * 4 + v;

                    av[v] = Us[(pos * WG_CC + c) * WG_BK + col];
#pragma unroll
                    for (int h = 0; h < NH; h++)
                        bv[v][h] = Vs[(pos * WG_CC + c) * NT + h * 32 + col];
                }
#pragma unroll
                for (int v = 0; v < 4; v++)
#pragma unroll
                    for (int h = 0; h < NH; h++)
                        acc[v][h] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            av[v], bv[v][h], acc[v][h], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    /* Z[xi][j] = (M A)[xi][j] for xi = wave, in registers; then
     * Y[i][j] = (A^T Z)[i][j] through LDS, one 32-tile column at a time.
     * Register r of a 32 x 32 accumulator holds channel
     * (r / 4) * 8 + half * 4 + r % 4, tile col. */
    {
        float *Zs = lds; /* [xi][j][k][t32], 4 * 2 * 32 * 32 floats */
        float *out = a.out + (long long)blockIdx.z * a.out_stride;

#pragma unroll
        for (int h = 0; h < NH; h++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int k = (r >> 2) * 8 + half * 4 + (r & 3);
                const float z0 = acc[0][h][r] + acc[1][h][r] + acc[2][h][r];
                const float z1 = acc[1][h][r] - acc[2][h][r] - acc[3][h][r];

                Zs[((wave * 2 + 0) * WG_BK + k) * 32 + col] = z0;
                Zs[((wave * 2 + 1) * WG_BK + k) * 32 + col] = z1;
            }
            __syncthreads();
            {
                const int ts = tid & 31, t = h * 32 + ts, tr = t / WG_TC;
                const int tc = t % WG_TC;
                const int oy = 2 * (ty0 + tr), ox = 2 * (tx0 + tc);

#pragma unroll
                for (int i = 0; i < WG_BK / 8; i++) {
                    const int k = (tid >> 5) + 8 * i, kg = k0 + k;
                    const float bias = a.bias && kg < K ? a.bias[kg] : 0.0f;

                    if (kg >= K)
                        continue;
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const float z0 = Zs[((0 * 2 + j) * WG_BK + k) * 32 + ts];
                        const float z1 = Zs[((1 * 2 + j) * WG_BK + k) * 32 + ts];
                        const float z2 = Zs[((2 * 2 + j) * WG_BK + k) * 32 + ts];
                        const float z3 = Zs[((3 * 2 + j) * WG_BK + k) * 32 + ts];
                        const float y0 = z0 + z1 + z2, y1 = z1 - z2 - z3;

                        if (ox + j >= a.Wo)
                            continue;
                        if (oy < a.Ho)
                            out[((long long)kg * a.Ho + oy) * a.Wo + ox + j] =
                                icoreg_act(y0 + bias, a.act, a.slope);
                        if (oy + 1 < a.Ho)
                            out[((long long)kg * a.Ho + oy + 1) * a.Wo + ox +
                                j] = icoreg_act(y1 + bias, a.act, a.slope);
                    }
                }
            }
            if (h + 1 < NH)
                __syncthreads();
        }
    }
}

/* ---- Row-split form -------------------------------------------------
 *
 * Row xi of V = B^T d B needs only two rows of the tile (B^T row xi has two
 * non-zeros), so wave xi of a block forms the transform values of its own
 * four GEMMs (positions (xi, nu)) directly from the input patch in LDS, in
 * the lane order of the MFMA B operand, and never writes V back: no V
 * round trip through LDS and no barrier between transform and product. The
 * transformed filters come from global memory (L2) straight into the A
 * operand registers, stored in that operand's lane order (wino_frag_kernel);
 * the input patch goes to LDS by LDS DMA (buffer_load ... lds), two slices
 * in flight (double buffer), one barrier per slice of 8 input channels.
 *
 * Patch layouts in LDS (per slice: 8 channels x 10 rows x 18 columns used):
 *  - 16-byte DMA (W % 4 == 0, 16-byte aligned input): columns fetched in
 *    aligned groups of 4 from 2 tx0 - 4 (a group lies wholly inside or
 *    wholly outside the image row, so zero padding is exact), 24 floats a
 *    row, 240 a channel; the patch column -1 is at offset 3;
 *  - 4-byte DMA (other widths): one load per row pair (lanes 0-31 row 2i,
 *    32-63 row 2i + 1), pairs 80 floats apart so the four tile rows of a
 *    wave read from different banks, 400 floats a channel.
 *
 * Filter fragments Uf[kb][sl][xi][nu][lane][s]: lane = (c & 1) * 32 + k % 32,
 * s = (c % 8) / 2, output channel block kb = k / 32, slice sl = c / 8; zero
 * for k >= K. Row xi = 2 is stored negated, which lets every wave form its
 * row as u = d[ra] + be * d[rb] with one FMA. */

#define WR_CC 8

static __device__ __forceinline__ int wr_nslices(int C) { return (C + WR_CC - 1) / WR_CC; }

__global__ void __launch_bounds__(256)
    wino_frag_kernel(const float *__restrict__ w, int K, int C, int Kp,
                     float *__restrict__ Uf)
{
    const long long id = (long long)blockIdx.x * 256 + threadIdx.x;
    const int nsl = wr_nslices(C);

    if (id >= (long long)Kp * nsl * WR_CC)
        return;
    {
        const int k = (int)(id % Kp), c = (int)(id / Kp);
        float u[16];

        if (k < K && c < C) {
            const float *src = w + ((long long)k * C + c) * 9;
            float g[9], t[4][3];

#pragma unroll
            for (int i = 0; i < 9; i++)
                g[i] = src[i];
#pragma unroll
            for (int j = 0; j < 3; j++) {
                const float g0 = g[j], g1 = g[3 + j], g2 = g[6 + j];

                t[0][j] = g0;
                t[1][j] = 0.5f * (g0 + g1 + g2);
                t[2][j] = 0.5f * (g0 - g1 + g2);
                t[3][j] = g2;
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float a0 = t[i][0], a1 = t[i][1], a2 = t[i][2];
                const float sg = i == 2 ? -1.0f : 1.0f;

                u[i * 4 + 0] = sg * a0;
                u[i * 4 + 1] = sg * 0.5f * (a0 + a1 + a2);
                u[i * 4 + 2] = sg * 0.5f * (a0 - a1 + a2);
                u[i * 4 + 3] = sg * a2;
            }
        }
        else {
#pragma unroll
            for (int i = 0; i < 16; i++)
                u[i] = 0.0f;
        }
        {
            const int kb = k / 32, col = k % 32, sl = c / WR_CC, cc = c % WR_CC;
            const int s = cc / 2, lane = (cc & 1) * 32 + col;
            float *dst = Uf + ((long long)kb * nsl + sl) * 16 * 256 + lane * 4 + s;

#pragma unroll
            for (int p = 0; p < 16; p++)
                dst[p * 256] = u[p];
        }
    }
}

/* gfx9 s_waitcnt immediates: vmcnt(0) alone; vmcnt(0) and lgkmcnt(0). */
/* Block L of T to a position in the unit order: the 8 XCDs (blocks L,
 * L + 8, ... run on XCD L % 8) each get a contiguous band. */
__device__ __forceinline__ int wino_xcd_band(int L, int T)
{
    const int q = T >> 3, rem = T & 7, x = L & 7, idx = L >> 3;

    return (x < rem ? x * (q + 1) : rem * (q + 1) + (x - rem) * q) + idx;
}

/* Unit v of the order (channel group, image, tile block, channel block of
 * the group). */
__device__ __forceinline__ void wino_unit(const wino_split &sp, int v, int &bx, int &by,
                                          int &bz)
{
    const int cbg = sp.nkb / sp.kgroups, per = sp.ntb * sp.nb * cbg;
    const int g = v / per, r = v - g * per, t = r / cbg;

    bx = g * cbg + (r - t * cbg);
    by = t % sp.ntb;
    bz = t / sp.ntb;
}

/* Most pieces per split unit. */
#define WR_MAX_SPLIT 8

/* Output channel kg of a 2 x 2 output tile at (oy, ox): y = (y(oy, ox),
 * y(oy + 1, ox), y(oy, ox + 1), y(oy + 1, ox + 1)) plus bias, activated,
 * clipped to the output. */
static __device__ __forceinline__ void wr_store(const conv_args &a, float *out, int kg, int oy,
                                                int ox, float4 y)
{
    const float yy[2][2] = {{y.x, y.y}, {y.z, y.w}};
    float bias;

    if (kg >= a.K)
        return;
    bias = a.bias ? a.bias[kg] : 0.0f;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        if (ox + j >= a.Wo)
            continue;
        if (oy < a.Ho)
            out[((long long)kg * a.Ho + oy) * a.Wo + ox + j] =
                icoreg_act(yy[j][0] + bias, a.act, a.slope);
        if (oy + 1 < a.Ho)
            out[((long long)kg * a.Ho + oy + 1) * a.Wo + ox + j] =
                icoreg_act(yy[j][1] + bias, a.act, a.slope);
    }
}

#define WR_WAIT_VM0 0x0F70
#define WR_WAIT_VM0_LGKM0 0x0070

template <bool X4>
__global__ void __launch_bounds__(256, 4)
    conv_wino_rows_kernel(const conv_args a, const float *__restrict__ Uf, const wino_split sp)
{
    constexpr int TR = 4, TC = 8, BK = 32;
    /* Per-slice patch buffer (floats) and pitches of the two layouts. */
    constexpr int PSZ = X4 ? 2048 : WR_CC * 400;
    constexpr int CPITCH = X4 ? 240 : 400;
    /* Two patch buffers; the output transform reuses the first 8192. */
    __shared__ __align__(16) float lds[2 * PSZ > 8192 ? 2 * PSZ : 8192];
    float *const P0 = lds, *const P1 = lds + PSZ;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int half = lane >> 5, col = lane & 31;
    const int tr = col >> 3, tc = col & 7;
    const int C = a.C, H = a.H, W = a.W;
    const int nk = (C + WR_CC - 1) / WR_CC;
    /* Unit (image bz, tile block by, channel block bx) in wino_unit's
     * order, channel blocks of a group fastest (they share the input
     * tiles in L2); whole units in XCD bands, units from nfull on cut into
     * split pieces over the input-channel slices. */
    int u = blockIdx.x, piece = -1, kt0 = 0, kt1 = nk, bx, by, bz;

    if (u >= sp.nfull) {
        const int p = u - sp.nfull;

        piece = p % sp.split;
        u = sp.nfull + p / sp.split;
        kt0 = piece * nk / sp.split;
        kt1 = (piece + 1) * nk / sp.split;
    }
    else
        u = wino_xcd_band(u, sp.nfull);
    wino_unit(sp, u, bx, by, bz);
    const int tiles_w = (W + 1) / 2, bw = (tiles_w + TC - 1) / TC;
    const int ty0 = (by / bw) * TR, tx0 = (by % bw) * TC;
    const int k0 = bx * BK;
    const int iy0 = 2 * ty0 - 1, ix0 = 2 * tx0 - 1;
    const long long HW = (long long)H * W;
    const float *in = a.in + (long long)bz * a.in_stride;
    const unsigned long long ibytes = (unsigned long long)C * HW * 4;
    /* This wave's filter fragments: 16 floats a lane, 4096 a slice. */
    const float *uf = Uf + ((long long)bx * nk * 16 + wave * 4) * 256 + lane * 4;
    /* Rows of the tile that row xi of B^T combines: u = d[ra] + be d[rb]
     * (row 2 negated in the filters). */
    const int ra = wave == 0 ? 0 : 1, rb = wave == 3 ? 3 : 2;
    const float be = wave == 1 ? 1.0f : -1.0f;
    floatx16 acc[4];
    float ruA[16], ruB[16];
    unsigned doff[2], rmask = 0;

#pragma unroll
    for (int v = 0; v < 4; v++)
#pragma unroll
        for (int r = 0; r < 16; r++)
            acc[v][r] = 0.0f;

    if (X4) {
        /* 16-byte chunk e of the slice: channel e / 60, row (e % 60) / 6,
         * group e % 6 of 4 columns from 2 tx0 - 4; to floats 4e. */
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int e = tid + 256 * q, c = e / 60, rem = e - c * 60;
            const int r = rem / 6, g = rem - r * 6;
            const int iy = iy0 + r, ix = 2 * tx0 - 4 + 4 * g;

            doff[q] = c < WR_CC && iy >= 0 && iy < H && ix >= 0 && ix < W
                          ? (unsigned)((c * HW + (long long)iy * W + ix) * 4)
                          : WG_OOB;
        }
    }
    else {
        /* Lane: row 2 i + half of pair i, patch column col; the offset is
         * taken from a window W + 1 floats before the slice (never
         * negative), the channel and pair terms go in soffset. */
        const bool col_ok = col < 2 * TC + 2 && ix0 + col >= 0 && ix0 + col < W;

#pragma unroll
        for (int i = 0; i < 5; i++) {
            const int iy = iy0 + 2 * i + half;

            rmask |= col_ok && iy >= 0 && iy < H ? 1u << i : 0u;
        }
        doff[0] = (unsigned)(((iy0 + half) * W + ix0 + col + W + 1) * 4);
        doff[1] = 0;
    }

    auto load_patch = [&](int c0, float *P) {
        if (X4) {
            const __amdgpu_buffer_rsrc_t ri =
                wg_rsrc(in + (long long)c0 * HW, ibytes - (unsigned long long)c0 * HW * 4);

#pragma unroll
            for (int q = 0; q < 2; q++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ri, (__attribute__((address_space(3))) void *)(P + 1024 * q + 256 * wave),
                    16, (int)doff[q], 0, 0, 0);
        }
        else {
            const __amdgpu_buffer_rsrc_t ri =
                wg_rsrc(in + (long long)c0 * HW - (W + 1),
                        ibytes - (unsigned long long)c0 * HW * 4 + (unsigned long long)(W + 1) * 4);

#pragma unroll
            for (int cc = 0; cc < 2; cc++)
#pragma unroll
                for (int i = 0; i < 5; i++) {
                    const int c = 2 * wave + cc;

                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        ri, (__attribute__((address_space(3))) void *)(P + c * 400 + i * 80), 4,
                        (int)((rmask >> i) & 1u ? doff[0] : WG_OOB),
                        (int)((c * HW + 2 * i * W) * 4), 0, 0);
                }
        }
    };
    auto load_u = [&](int kt, float *ru) {
        const float *p = uf + (long long)kt * 16 * 256;

#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float4 t = *(const float4 *)(p + v * 256);

            ru[v * 4 + 0] = t.x;
            ru[v * 4 + 1] = t.y;
            ru[v * 4 + 2] = t.z;
            ru[v * 4 + 3] = t.w;
        }
    };
    /* Slice kt from patch buffer Pc, filters ru; the next slice's patch
     * (to Pn) and filters (to rn) are loaded meanwhile. */
    auto step = [&](int kt, const float *__restrict__ Pc, float *__restrict__ Pn, float *ru,
                    float *rn) {
        const bool more = kt + 1 < kt1;
        float bv[4][4];

        /* ru arrived before the last barrier. Redefining it here (an empty
         * asm) keeps the compiler from placing a wait for the loads issued
         * below in front of the products. */
        asm volatile(""
                     : "+v"(ru[0]), "+v"(ru[1]), "+v"(ru[2]), "+v"(ru[3]), "+v"(ru[4]),
                       "+v"(ru[5]), "+v"(ru[6]), "+v"(ru[7]), "+v"(ru[8]), "+v"(ru[9]),
                       "+v"(ru[10]), "+v"(ru[11]), "+v"(ru[12]), "+v"(ru[13]), "+v"(ru[14]),
                       "+v"(ru[15]));
        if (more) {
            load_patch((kt + 1) * WR_CC, Pn);
            load_u(kt + 1, rn);
        }
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int c = 2 * s + half;
            float da[4], db[4], u[4];

            if (X4) {
                const float *p = Pc + c * CPITCH + 2 * tr * 24 + 3 + 2 * tc;

#pragma unroll
                for (int x = 0; x < 4; x++) {
                    da[x] = p[ra * 24 + x];
                    db[x] = p[rb * 24 + x];
                }
            }
            else {
                const float *p = Pc + c * CPITCH + tr * 80 + 2 * tc;
                const float *pa = p + (ra >> 1) * 80 + (ra & 1) * 32;
                const float *pb = p + (rb >> 1) * 80 + (rb & 1) * 32;
                const float2 a0 = *(const float2 *)pa, a1 = *(const float2 *)(pa + 2);
                const float2 b0 = *(const float2 *)pb, b1 = *(const float2 *)(pb + 2);

                da[0] = a0.x, da[1] = a0.y, da[2] = a1.x, da[3] = a1.y;
                db[0] = b0.x, db[1] = b0.y, db[2] = b1.x, db[3] = b1.y;
            }
#pragma unroll
            for (int x = 0; x < 4; x++)
                u[x] = __builtin_fmaf(be, db[x], da[x]);
            bv[s][0] = u[0] - u[2];
            bv[s][1] = u[1] + u[2];
            bv[s][2] = u[2] - u[1];
            bv[s][3] = u[1] - u[3];
        }
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int v = 0; v < 4; v++)
                acc[v] = __builtin_amdgcn_mfma_f32_32x32x2f32(ru[v * 4 + s], bv[s][v], acc[v], 0,
                                                              0, 0);
        /* The next slice's patch and filters have landed (LDS DMA is
         * counted in vmcnt), then everyone's reads of Pc are done. */
        __builtin_amdgcn_s_waitcnt(WR_WAIT_VM0);
        __syncthreads();
    };

    load_patch(kt0 * WR_CC, P0);
    load_u(kt0, ruA);
    __builtin_amdgcn_s_waitcnt(WR_WAIT_VM0);
    __syncthreads();
    for (int kt = kt0; kt < kt1; kt += 2) {
        step(kt, P0, P1, ruA, ruB);
        if (kt + 1 < kt1)
            step(kt + 1, P1, P0, ruB, ruA);
    }

    /* Output transform as in conv_wino_kernel: Z = M A over nu in
     * registers, Y = A^T Z over xi through LDS. */
    {
        float *Zs = lds; /* [xi][j][k][t32] */
        float *out = a.out + (long long)bz * a.out_stride;
        const int ts = tid & 31, otr = ts / TC, otc = ts % TC;
        const int oy = 2 * (ty0 + otr), ox = 2 * (tx0 + otc);
        /* (y0, y1) of output columns ox, ox + 1 (rows oy, oy + 1) for
         * channel (tid / 32) + 8 i of the block, before bias and
         * activation. */
        float4 yv[BK / 8];

#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int k = (r >> 2) * 8 + half * 4 + (r & 3);
            const float z0 = acc[0][r] + acc[1][r] + acc[2][r];
            const float z1 = acc[1][r] - acc[2][r] - acc[3][r];

            Zs[((wave * 2 + 0) * BK + k) * 32 + col] = z0;
            Zs[((wave * 2 + 1) * BK + k) * 32 + col] = z1;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < BK / 8; i++) {
            const int k = (tid >> 5) + 8 * i;
            float y[2][2];

#pragma unroll
            for (int j = 0; j < 2; j++) {
                const float z0 = Zs[((0 * 2 + j) * BK + k) * 32 + ts];
                const float z1 = Zs[((1 * 2 + j) * BK + k) * 32 + ts];
                const float z2 = Zs[((2 * 2 + j) * BK + k) * 32 + ts];
                const float z3 = Zs[((3 * 2 + j) * BK + k) * 32 + ts];

                y[j][0] = z0 + z1 + z2;
                y[j][1] = z1 - z2 - z3;
            }
            yv[i] = make_float4(y[0][0], y[0][1], y[1][0], y[1][1]);
        }
        if (piece >= 0) {
            /* A piece of a split unit: partial sums to the unit's slot,
             * added up by wino_pieces_kernel. */
            float4 *pp = (float4 *)sp.part +
                         ((long long)(u - sp.nfull) * sp.split + piece) * (BK * 32);

#pragma unroll
            for (int i = 0; i < BK / 8; i++)
                pp[((tid >> 5) + 8 * i) * 32 + ts] = yv[i];
            return;
        }
#pragma unroll
        for (int i = 0; i < BK / 8; i++)
            wr_store(a, out, k0 + (tid >> 5) + 8 * i, oy, ox, yv[i]);
    }
}

/* The split units: one thread per (unit, channel, 2 x 2 tile) adds the
 * pieces' partial sums in piece order (all loads issued first) and
 * stores the output as conv_wino_rows_kernel does. */
__global__ void __launch_bounds__(256)
    wino_pieces_kernel(const conv_args a, const wino_split sp, int tail)
{
    constexpr int TR = 4, TC = 8, BK = 32;
    const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
    const int t = (int)(e / (BK * 32)), w = (int)(e % (BK * 32));
    const int k = w / 32, ts = w % 32;

    if (t >= tail)
        return;
    int bx, by, bz;

    wino_unit(sp, sp.nfull + t, bx, by, bz);
    const int bw = ((a.W + 1) / 2 + TC - 1) / TC;
    const int oy = 2 * ((by / bw) * TR + ts / TC), ox = 2 * ((by % bw) * TC + ts % TC);
    const float4 *q = (const float4 *)sp.part + (long long)t * sp.split * (BK * 32) + w;
    float4 p[WR_MAX_SPLIT], v;

#pragma unroll
    for (int pc = 0; pc < WR_MAX_SPLIT; pc++)
        if (pc < sp.split)
            p[pc] = q[(long long)pc * (BK * 32)];
    v = p[0];
#pragma unroll
    for (int pc = 1; pc < WR_MAX_SPLIT; pc++)
        if (pc < sp.split) {
            v.x += p[pc].x;
            v.y += p[pc].y;
            v.z += p[pc].z;
            v.w += p[pc].w;
        }
    wr_store(a, a.out + (long long)bz * a.out_stride, bx * BK + k, oy, ox, v);
}

/* Blocks of 8 x 16 output pixels (the larger block's 16 x 16 on a
 * different grid, always fewer). */
static long long wino_blocks(int Ho, int Wo, int tr)
{
    return (long long)(((Ho + 1) / 2 + tr - 1) / tr) *
           (((Wo + 1) / 2 + WG_TC - 1) / WG_TC);
}

bool conv_wino_supported(int kh, int kw, int sy, int sx, int py, int px,
                         int dy, int dx, int groups, int C, int K, int Ho,
                         int Wo)
{
    return kh == 3 && kw == 3 && sy == 1 && sx == 1 && py == 1 && px == 1 &&
           dy == 1 && dx == 1 && groups == 1 && K % 4 == 0 && C >= 32 &&
           K >= 32 && wino_blocks(Ho, Wo, 4) <= 65535;
}

/* The row-split kernel takes whole 8-channel slices and no input
 * normalisation; the staged kernel takes the rest. */
static bool wino_rows(int C, bool norm) { return C % WR_CC == 0 && !norm; }

size_t conv_wino_weight_floats(int K, int C, bool norm)
{
    return wino_rows(C, norm) ? (size_t)((K + 31) / 32 * 32) * C * 16 : 16ULL * K * C;
}

void conv_wino_weights(const float *w, int K, int C, bool norm, float *U, hipStream_t s)
{
    if (wino_rows(C, norm)) {
        const int Kp = (K + 31) / 32 * 32;
        const long long n = (long long)Kp * C;

        hipLaunchKernelGGL(wino_frag_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                           w, K, C, Kp, U);
    }
    else {
        const long long n = (long long)K * C;

        hipLaunchKernelGGL(wino_weights_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                           s, w, K, C, U);
    }
}

template <int TR, int CC, int MINW>
static void wino_launch(const conv_args &a, const float *U, int nb,
                        hipStream_t s)
{
    const dim3 grid((a.K + WG_BK - 1) / WG_BK,
                    (unsigned)wino_blocks(a.Ho, a.Wo, TR), nb);

    if (a.mean)
        hipLaunchKernelGGL((conv_wino_kernel<true, TR, CC, MINW>), grid,
                           dim3(256), 0, s, a, U);
    else
        hipLaunchKernelGGL((conv_wino_kernel<false, TR, CC, MINW>), grid,
                           dim3(256), 0, s, a, U);
}

wino_split conv_wino_plan(const conv_args &a, int nb, int cus)
{
    wino_split sp;
    const int nk = (a.C + WR_CC - 1) / WR_CC;
    long long units, rem;

    sp.nkb = (a.K + 31) / 32;
    sp.ntb = (int)wino_blocks(a.Ho, a.Wo, 4);
    sp.part = nullptr;
    sp.nb = nb;
    /* Two channel groups from 8 channel blocks (256 channels) up: an XCD
     * then reads half the filters (2 MB of U at C = K = 256) and a
     * quarter of the inputs, instead of every input tile. */
    sp.kgroups = sp.nkb >= 8 && sp.nkb % 2 == 0 ? 2 : 1;
    units = (long long)sp.nkb * sp.ntb * nb;
    sp.nfull = (int)units;
    sp.split = 1;
    if (!wino_rows(a.C, a.mean != nullptr) || cus < 1 || nk < 4)
        return sp;
    rem = units % cus;
    /* Only when the leftover is a large share of the work: a CU holds
     * up to 4 blocks, and with fewer than 4 units per CU the CUs that get
     * one more unit than the others set the time. */
    if (rem == 0 || units >= 4LL * cus)
        return sp;
    /* rem leftover units over cus CUs: about one piece per CU, at least
     * two slices per piece. */
    sp.split = (int)std::min<long long>(std::min<long long>(cus / rem, nk / 2), WR_MAX_SPLIT);
    if (sp.split < 2) {
        sp.split = 1;
        return sp;
    }
    sp.nfull = (int)(units - rem);
    return sp;
}

size_t conv_wino_part_floats(const conv_args &a, int nb, const wino_split &sp)
{
    const long long units = (long long)sp.nkb * sp.ntb * nb;

    (void)a;
    return sp.split > 1 ? (size_t)(units - sp.nfull) * sp.split * 4096 : 0;
}

void conv_wino_launch(const conv_args &a, const float *U, int nb, const wino_split &sp,
                      hipStream_t s)
{
    if (wino_rows(a.C, a.mean != nullptr)) {
        /* Row-split kernel; 16-byte patch loads when every image row
         * starts 16-byte aligned. */
        const long long units = (long long)sp.nkb * sp.ntb * nb;
        const dim3 grid((unsigned)(sp.nfull + (units - sp.nfull) * sp.split));
        const bool x4 = a.W % 4 == 0 && a.in_stride % 4 == 0 &&
                        ((unsigned long long)(size_t)a.in) % 16 == 0;

        if (x4)
            hipLaunchKernelGGL(conv_wino_rows_kernel<true>, grid, dim3(256), 0, s, a, U, sp);
        else
            hipLaunchKernelGGL(conv_wino_rows_kernel<false>, grid, dim3(256), 0, s, a, U, sp);
        if (sp.split > 1) {
            const long long tail = units - sp.nfull;

            hipLaunchKernelGGL(wino_pieces_kernel, dim3((unsigned)((tail * 1024 + 255) / 256)),
                               dim3(256), 0, s, a, sp, (int)tail);
        }
        return;
    }
    /* 32 tiles x 32 channels per block, 8 input channels per slice,
     * registers capped for 4 waves per SIMD: the 38 KB of LDS and the
     * extra waves in flight beat the larger blocks (64 tiles, or 16
     * channels per slice) on every ELoFTR layer measured. */
    wino_launch<4, 8, 4>(a, U, nb, s);
}

/* SPDX-License-Identifier: Unlicense */

/* The brute-force nearest-neighbour search in front of AdaLAM
 * (adalam.c:38-116 of i.coregistration.opencl) on gfx950: squared
 * distances |a|^2 + |b|^2 - 2 a.b between two descriptor sets, per row
 * the first index of the smallest distance and Lowe's ratio of the two
 * smallest, per column the first index of the smallest.
 *
 *  - nn_tile_kernel: one block per 64 x 64 tile of the distance matrix.
 *    The two 64-row descriptor panels go through LDS in 64-wide k
 *    chunks; each wave forms a 32 x 32 quadrant with
 *    v_mfma_f32_16x16x4f32 (a lane reads four consecutive k of its row
 *    with one 16-byte LDS read and feeds them to four products). The
 *    norms are summed in k order with separate multiply and add, as the
 *    host loop does. The tile is then reduced in LDS: per row (best,
 *    second, first argmin) over its 64 columns, per column (best, first
 *    argmin) over its 64 rows, written as partials; the distance matrix
 *    never reaches HBM.
 *  - nn_merge_kernel: per row the column tiles' partials in column
 *    order, per column the row tiles' in row order.
 *
 * The sequential rule of the host loop (if d < best: second = best,
 * best = d; else if d < second: second = d) leaves best = the smallest
 * value, its first index, and second = the second smallest of the
 * multiset (a tie gives second = best). Partials of consecutive ranges
 * A then B combine exactly: best = B.best < A.best ? B : A, second =
 * min(max(A.best, B.best), A.second, B.second). */

#include <hip/hip_runtime.h>

#include <float.h>

#include "adalam_nn.h"
#include "common.h"

using namespace icoreg;

typedef float floatx4 __attribute__((ext_vector_type(4)));

#define NN_T 64  /* tile side */
#define NN_KC 64 /* k chunk staged per step */
#define NN_P (NN_KC + 4)

struct nn_row {
    float best, second;
    int arg, pad;
};

struct nn_col {
    float best;
    int arg;
};

__device__ inline void row_step(float d, int j, float &best, float &second, int &arg)
{
    if (d < best) {
        second = best;
        best = d;
        arg = j;
    }
    else if (d < second)
        second = d;
}

/* A (earlier indices) followed by B. */
__device__ inline void row_merge(float &bA, float &sA, int &aA, float bB, float sB, int aB)
{
    const float s = fminf(fmaxf(bA, bB), fminf(sA, sB));

    if (bB < bA) {
        bA = bB;
        aA = aB;
    }
    sA = s;
}

__global__ void __launch_bounds__(256)
    nn_tile_kernel(const float *__restrict__ d1, int n1, const float *__restrict__ d2, int n2,
                   int dim, int ntc, nn_row *__restrict__ rowpart,
                   nn_col *__restrict__ colpart)
{
    __shared__ __attribute__((aligned(16))) float P[2][NN_T * NN_P];
    __shared__ float qa[NN_T], qb[NN_T];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int tr = blockIdx.x / ntc, tc = blockIdx.x % ntc;
    const int i0 = tr * NN_T, j0 = tc * NN_T;
    const int qr = 32 * (wv >> 1), qc = 32 * (wv & 1);
    const int lr = lane & 15, g = lane >> 4;
    floatx4 acc[2][2];
    float q = 0.0f;

#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
            acc[a][b] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int k0 = 0; k0 < dim; k0 += NN_KC) {
        const int kn = min(NN_KC, dim - k0);

        __syncthreads();
        /* Rows past n1 / n2 and k past dim are zero: they add nothing. */
#pragma unroll 4
        for (int e = t; e < NN_T * NN_KC; e += 256) {
            const int r = e / NN_KC, c = e % NN_KC;
            const bool kin = c < kn;

            P[0][r * NN_P + c] =
                kin && i0 + r < n1 ? d1[(long long)(i0 + r) * dim + k0 + c] : 0.0f;
            P[1][r * NN_P + c] =
                kin && j0 + r < n2 ? d2[(long long)(j0 + r) * dim + k0 + c] : 0.0f;
        }
        __syncthreads();
        if (t < 2 * NN_T) {
            const float *row = &P[t >> 6][(t & 63) * NN_P];

            for (int k = 0; k < kn; k++)
                q = __fadd_rn(q, __fmul_rn(row[k], row[k]));
        }
#pragma unroll
        for (int ks = 0; ks < NN_KC; ks += 16) {
            floatx4 av[2], bv[2];

#pragma unroll
            for (int a = 0; a < 2; a++)
                av[a] = *(const floatx4 *)&P[0][(qr + 16 * a + lr) * NN_P + ks + 4 * g];
#pragma unroll
            for (int b = 0; b < 2; b++)
                bv[b] = *(const floatx4 *)&P[1][(qc + 16 * b + lr) * NN_P + ks + 4 * g];
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int a = 0; a < 2; a++)
#pragma unroll
                    for (int b = 0; b < 2; b++)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a][s], bv[b][s],
                                                                        acc[a][b], 0, 0, 0);
        }
    }
    if (t < NN_T)
        qa[t] = q;
    else if (t < 2 * NN_T)
        qb[t - NN_T] = q;
    __syncthreads();
    {
        float *T = P[0]; /* 64 x 65 distances */

#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int b = 0; b < 2; b++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int r = qr + 16 * a + 4 * g + v, c = qc + 16 * b + lr;

                    T[r * (NN_T + 1) + c] =
                        __fsub_rn(__fadd_rn(qa[r], qb[c]), 2.0f * acc[a][b][v]);
                }
        __syncthreads();
        /* Rows: four lanes per row, 16 columns each, merged in column
         * order. */
        {
            const int r = t >> 2, part = t & 3;
            const int cn = min(NN_T, n2 - j0);
            float best = FLT_MAX, second = FLT_MAX;
            int arg = 0;

            for (int c = 16 * part; c < min(16 * part + 16, cn); c++)
                row_step(T[r * (NN_T + 1) + c], j0 + c, best, second, arg);
#pragma unroll
            for (int w = 1; w <= 2; w <<= 1) {
                const float bB = __shfl_down(best, w), sB = __shfl_down(second, w);
                const int aB = __shfl_down(arg, w);

                if ((part & (2 * w - 1)) == 0)
                    row_merge(best, second, arg, bB, sB, aB);
            }
            if (part == 0 && i0 + r < n1) {
                nn_row o;

                o.best = best;
                o.second = second;
                o.arg = arg;
                o.pad = 0;
                rowpart[(long long)tc * n1 + i0 + r] = o;
            }
        }
        if (colpart) {
            const int c = t >> 2, part = t & 3;
            const int rn = min(NN_T, n1 - i0);
            float best = FLT_MAX;
            int arg = 0;

            for (int r = 16 * part; r < min(16 * part + 16, rn); r++) {
                const float d = T[r * (NN_T + 1) + c];

                if (d < best) {
                    best = d;
                    arg = i0 + r;
                }
            }
#pragma unroll
            for (int w = 1; w <= 2; w <<= 1) {
                const float bB = __shfl_down(best, w);
                const int aB = __shfl_down(arg, w);

                if ((part & (2 * w - 1)) == 0 && bB < best) {
                    best = bB;
                    arg = aB;
                }
            }
            if (part == 0 && j0 + c < n2) {
                nn_col o;

                o.best = best;
                o.arg = arg;
                colpart[(long long)tr * n2 + j0 + c] = o;
            }
        }
    }
}

/* blockIdx.y 0: rows of d1 (nn12, score); 1: rows of d2 (nn21). */
__global__ void __launch_bounds__(256)
    nn_merge_kernel(const nn_row *__restrict__ rowpart, const nn_col *__restrict__ colpart,
                    int n1, int n2, int ntr, int ntc, int *__restrict__ nn12,
                    float *__restrict__ score, int *__restrict__ nn21)
{
    const int i = blockIdx.x * 256 + threadIdx.x;

    if (blockIdx.y == 0) {
        float best = FLT_MAX, second = FLT_MAX;
        int arg = 0;

        if (i >= n1)
            return;
        for (int tc = 0; tc < ntc; tc++) {
            const nn_row p = rowpart[(long long)tc * n1 + i];

            row_merge(best, second, arg, p.best, p.second, p.arg);
        }
        nn12[i] = arg;
        score[i] = best / (second > 1e-3f ? second : 1e-3f);
    }
    else {
        float best = FLT_MAX;
        int arg = 0;

        if (i >= n2)
            return;
        for (int tr = 0; tr < ntr; tr++) {
            const nn_col p = colpart[(long long)tr * n2 + i];

            if (p.best < best) {
                best = p.best;
                arg = p.arg;
            }
        }
        nn21[i] = arg;
    }
}

static size_t round256(size_t b) { return (b + 255) / 256 * 256; }

extern "C" size_t adalam_nearest_work_bytes(int n1, int n2)
{
    const size_t a = n1 > 0 ? (size_t)n1 : 0, b = n2 > 0 ? (size_t)n2 : 0;
    const size_t ntr = (a + NN_T - 1) / NN_T, ntc = (b + NN_T - 1) / NN_T;

    return round256(ntc * a * sizeof(nn_row)) + round256(ntr * b * sizeof(nn_col));
}

extern "C" void adalam_nearest(struct ops *o, cl_mem d1, int n1, cl_mem d2, int n2, int dim,
                               cl_mem nn12, cl_mem score, cl_mem nn21, cl_mem work)
{
    ICOREG_API_BEGIN
    const char *op = "adalam_nearest";
    hipStream_t st = stream_of(o->ocl);
    const int ntr = (n1 + NN_T - 1) / NN_T, ntc = (n2 + NN_T - 1) / NN_T;

    if (n1 < 0 || n2 < 0 || dim < 0)
        icoreg_fatal("%s: invalid sizes n1=%d n2=%d dim=%d", op, n1, n2, dim);
    count32((long long)n1 * dim, op);
    count32((long long)n2 * dim, op);
    count32((long long)ntr * ntc, op);
    if (n1 == 0 && (n2 == 0 || !nn21))
        return;
    need_floats(d1, 0, (long long)n1 * dim, op, "d1");
    need_floats(d2, 0, (long long)n2 * dim, op, "d2");
    need_bytes(nn12, 0, 4LL * n1, op, "nn12");
    need_floats(score, 0, n1, op, "score");
    if (nn21)
        need_bytes(nn21, 0, 4LL * n2, op, "nn21");
    need_bytes(work, 0, (long long)adalam_nearest_work_bytes(n1, n2), op, "work");
    {
        nn_row *rowpart = (nn_row *)work->ptr;
        nn_col *colpart =
            (nn_col *)((char *)work->ptr + round256((size_t)ntc * n1 * sizeof(nn_row)));
        const int nmax = n1 > n2 ? n1 : n2;
        prof_scope ps(o->ocl, op);

        if (ntr > 0 && ntc > 0)
            hipLaunchKernelGGL(nn_tile_kernel, dim3((unsigned)(ntr * ntc)), dim3(256), 0, st,
                               cfptr(d1), n1, cfptr(d2), n2, dim, ntc, rowpart,
                               nn21 ? colpart : nullptr);
        hipLaunchKernelGGL(nn_merge_kernel, dim3((unsigned)((nmax + 255) / 256), nn21 ? 2 : 1),
                           dim3(256), 0, st, (const nn_row *)rowpart,
                           (const nn_col *)colpart, n1, n2, ntr, ntc,
                           (int *)(nn12 ? nn12->ptr : nullptr), fptr(score),
                           (int *)(nn21 ? nn21->ptr : nullptr));
    }
    launch_check(op);
    ICOREG_API_END
}

extern "C" void adalam_nearest_host(struct ops *o, const float *d1, int n1, const float *d2,
                                    int n2, int dim, int *nn12, float *score, int *nn21)
{
    ICOREG_API_BEGIN
    const char *op = "adalam_nearest_host";
    cl_mem b1 = nullptr, b2 = nullptr, bi = nullptr, bs = nullptr, bj = nullptr, bw = nullptr;

    if (n1 < 0 || n2 < 0 || dim < 0)
        icoreg_fatal("%s: invalid sizes n1=%d n2=%d dim=%d", op, n1, n2, dim);
    try {
        const size_t s1 = (size_t)n1 * dim * 4, s2 = (size_t)n2 * dim * 4;

        b1 = ocl_alloc(o->ocl, s1 ? s1 : 4, "adalam d1");
        b2 = ocl_alloc(o->ocl, s2 ? s2 : 4, "adalam d2");
        bi = ocl_alloc(o->ocl, n1 ? 4 * (size_t)n1 : 4, "adalam nn12");
        bs = ocl_alloc(o->ocl, n1 ? 4 * (size_t)n1 : 4, "adalam score");
        if (nn21)
            bj = ocl_alloc(o->ocl, n2 ? 4 * (size_t)n2 : 4, "adalam nn21");
        bw = ocl_alloc(o->ocl, adalam_nearest_work_bytes(n1, n2) + 256, "adalam work");
        if (s1)
            ocl_write(o->ocl, b1, 0, d1, s1);
        if (s2)
            ocl_write(o->ocl, b2, 0, d2, s2);
        adalam_nearest(o, b1, n1, b2, n2, dim, bi, bs, bj, bw);
        if (n1) {
            ocl_read(o->ocl, bi, 0, nn12, 4 * (size_t)n1);
            ocl_read(o->ocl, bs, 0, score, 4 * (size_t)n1);
        }
        if (nn21 && n2)
            ocl_read(o->ocl, bj, 0, nn21, 4 * (size_t)n2);
    }
    catch (...) {
        ocl_release(&b1);
        ocl_release(&b2);
        ocl_release(&bi);
        ocl_release(&bs);
        ocl_release(&bj);
        ocl_release(&bw);
        throw;
    }
    ocl_release(&b1);
    ocl_release(&b2);
    ocl_release(&bi);
    ocl_release(&bs);
    ocl_release(&bj);
    ocl_release(&bw);
    ICOREG_API_END
}

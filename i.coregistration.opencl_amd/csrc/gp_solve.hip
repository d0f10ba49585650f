/* SPDX-License-Identifier: Unlicense */

/* RoMa's Gaussian-process solve on the device, in double precision:
 * F = (K + noise I)^-1 F for the n x n cosine kernel K (float) and the
 * n x d position basis F (float). The reference factors and solves on
 * the host (roma.c:770-836 of i.coregistration.opencl: Cholesky, then
 * L Z = F and L^T X = Z, all in double), which costs a 10 MB read-back,
 * a host Cholesky of n = 1600 and a write per tile pair; here the same
 * arithmetic stays on the GPU.
 *
 * Blocked right-looking Cholesky with 64-column panels:
 *  - chol_diag: the 64 x 64 diagonal block factored in LDS by one
 *    work-group, and its triangular inverse Linv formed there too;
 *  - the panel below it, L21 = A21 Linv^T, and the trailing update
 *    A22 -= L21 L21^T (lower tiles only) are both fp64 GEMMs;
 *  - the two triangular solves run block by block the same way: a block
 *    of rows times Linv (or Linv^T), then a GEMM update of the rows still
 *    to solve.
 * Working matrices: A (n x n, the trailing updates), L (n x n, the
 * factor), Linv per panel, Z and Y (n x d). Every GEMM reads one matrix
 * and writes another, so no launch reads what it writes. */

#include <hip/hip_runtime.h>

#include <math.h>

#include "common.h"
#include "icoreg_kernels.h"

using namespace icoreg;

#define GP_NB 64 /* panel width */
#define DG_T 64  /* GEMM output tile */
#define DG_K 32  /* GEMM reduction chunk */

/* C = alpha A B + beta C with A(i, q) = A[i a_ri + q a_rk], B(q, j) =
 * B[q b_rk + j b_rj], C(i, j) = C[i c_ri + j]; lower: skip output tiles
 * strictly above the diagonal. */
struct dg_args {
    int M, N, K;
    const double *A;
    long long a_ri, a_rk;
    const double *B;
    long long b_rk, b_rj;
    double *C;
    long long c_ri;
    double alpha;
    int beta, lower;
};

__global__ void __launch_bounds__(256) dgemm_kernel(dg_args a)
{
    __shared__ double As[DG_K][DG_T + 1], Bs[DG_K][DG_T + 1];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int i0 = blockIdx.y * DG_T, j0 = blockIdx.x * DG_T;
    double acc[4][4];

    if (a.lower && j0 > i0 + DG_T - 1)
        return;
#pragma unroll
    for (int p = 0; p < 4; p++)
#pragma unroll
        for (int q = 0; q < 4; q++)
            acc[p][q] = 0.0;
    for (int k0 = 0; k0 < a.K; k0 += DG_K) {
        /* 32 x 64 of A and of B, 8 values per thread, the unit-stride
         * index fastest across threads. Every load reads a valid address
         * (indices clamped to the last row / column) and the value is
         * selected afterwards, so that the 16 loads are all in flight
         * together instead of one per guarded branch. */
        double va[8], vb[8];
        bool oka[8], okb[8];

#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int e = tid + 256 * t;
            const int i = a.a_rk == 1 ? e / DG_K : (e & (DG_T - 1));
            const int q = a.a_rk == 1 ? (e & (DG_K - 1)) : e / DG_T;
            const int j = a.b_rj == 1 ? (e & (DG_T - 1)) : e / DG_K;
            const int qb = a.b_rj == 1 ? e / DG_T : (e & (DG_K - 1));

            oka[t] = i0 + i < a.M && k0 + q < a.K;
            okb[t] = j0 + j < a.N && k0 + qb < a.K;
            va[t] = a.A[(long long)min(i0 + i, a.M - 1) * a.a_ri +
                        (long long)min(k0 + q, a.K - 1) * a.a_rk];
            vb[t] = a.B[(long long)min(k0 + qb, a.K - 1) * a.b_rk +
                        (long long)min(j0 + j, a.N - 1) * a.b_rj];
        }
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int e = tid + 256 * t;
            const int i = a.a_rk == 1 ? e / DG_K : (e & (DG_T - 1));
            const int q = a.a_rk == 1 ? (e & (DG_K - 1)) : e / DG_T;
            const int j = a.b_rj == 1 ? (e & (DG_T - 1)) : e / DG_K;
            const int qb = a.b_rj == 1 ? e / DG_T : (e & (DG_K - 1));

            As[q][i] = oka[t] ? va[t] : 0.0;
            Bs[qb][j] = okb[t] ? vb[t] : 0.0;
        }
        __syncthreads();
#pragma unroll 8
        for (int q = 0; q < DG_K; q++) {
            double av[4], bv[4];

#pragma unroll
            for (int p = 0; p < 4; p++) {
                av[p] = As[q][ty + 16 * p];
                bv[p] = Bs[q][tx + 16 * p];
            }
#pragma unroll
            for (int p = 0; p < 4; p++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc[p][r] = fma(av[p], bv[r], acc[p][r]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const int i = i0 + ty + 16 * p;

        if (i >= a.M)
            continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int j = j0 + tx + 16 * r;

            if (j < a.N) {
                double *c = a.C + (long long)i * a.c_ri + j;

                *c = a.alpha * acc[p][r] + (a.beta ? *c : 0.0);
            }
        }
    }
}

/* Cholesky factor of the nb x nb diagonal block at (k, k) of A (n x n)
 * into L, and the inverse of that factor into Linv (nb x nb, row-major,
 * GP_NB apart), both in one pass over the columns. info gets 1 + the
 * first column whose pivot is not positive (the factor then holds NaN
 * from there on).
 *
 * LDS holds the block: its lower triangle becomes L, its strictly upper
 * triangle holds the inverse transposed (Linv[r][c] at s[c][r], c < r,
 * starting as the identity's zeros), the inverse's diagonal is dinv.
 * Column j: one wave takes the pivot's square root and divides column j
 * below it (L) and above it (row j of the inverse, in transposed
 * storage) by it; then every thread updates the cells it owns (rows
 * ty + 16 a, columns tx + 16 b): the trailing lower triangle of A
 * (A[r][c] -= L[r][j] L[c][j], c > j) and the inverse's rows below j
 * (B[r][c] -= L[r][j] Linv[j][c], c <= j), branch-free so that all its
 * LDS reads issue together. */
__global__ void __launch_bounds__(256)
    chol_diag_kernel(const double *__restrict__ A, double *__restrict__ L,
                     double *__restrict__ Linv, int n, int k, int nb,
                     int *__restrict__ info)
{
    __shared__ double s[GP_NB][GP_NB + 1];
    __shared__ double dinv[GP_NB];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;

    {
        double v[16];

#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int e = tid + 256 * i, r = e >> 6, c = e & 63;

            v[i] = A[(long long)(k + min(r, nb - 1)) * n + k + min(c, nb - 1)];
        }
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int e = tid + 256 * i, r = e >> 6, c = e & 63;

            s[r][c] = r < nb && c <= r ? v[i] : 0.0;
        }
    }
    __syncthreads();
    for (int j = 0; j < nb; j++) {
        if (tid < 64) {
            const double d = s[j][j];
            /* 1 / sqrt(d) from the hardware estimate and two Newton
             * steps (each doubles the correct bits), then sqrt(d) = d r:
             * no division or square-root sequence on the column chain. */
            double r = __builtin_amdgcn_rsq(d);

            r = r * fma(-0.5 * d * r, r, 1.5);
            r = r * fma(-0.5 * d * r, r, 1.5);
            if (tid == 0 && !(d > 0.0) && *info == 0)
                *info = k + j + 1;
            if (tid == j) {
                s[j][j] = d * r;
                dinv[j] = r;
            }
            else if (tid < nb)
                s[tid][j] *= r;
        }
        __syncthreads();
        {
            const double dj = dinv[j];
            double lr[4], lc[4], v[4][4];

#pragma unroll
            for (int a4 = 0; a4 < 4; a4++) {
                lr[a4] = s[ty + 16 * a4][j];
                lc[a4] = s[tx + 16 * a4][j];
            }
#pragma unroll
            for (int a4 = 0; a4 < 4; a4++)
#pragma unroll
                for (int b4 = 0; b4 < 4; b4++)
                    v[a4][b4] = s[ty + 16 * a4][tx + 16 * b4];
#pragma unroll
            for (int a4 = 0; a4 < 4; a4++)
#pragma unroll
                for (int b4 = 0; b4 < 4; b4++) {
                    const int r = ty + 16 * a4, c = tx + 16 * b4;
                    /* lower: factor update; upper (r < c): inverse cell
                     * (c, r), updated for r <= j < c. */
                    const bool low = r < nb && c > j && c <= r;
                    const bool inv = c < nb && r <= j && j < c;
                    const double f = r == j ? dj : lr[a4];

                    s[r][c] = low ? fma(-lr[a4], lc[b4], v[a4][b4])
                              : inv ? fma(-lc[b4], f, v[a4][b4])
                                    : v[a4][b4];
                }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int e = tid + 256 * i, r = e >> 6, c = e & 63;

        if (r < nb && c < nb) {
            L[(long long)(k + r) * n + k + c] = c <= r ? s[r][c] : 0.0;
            Linv[r * GP_NB + c] = r == c ? dinv[c] : r > c ? s[c][r] : 0.0;
        }
    }
}

/* A = K + noise I (double), Z = F (double), info cleared. */
__global__ void __launch_bounds__(256)
    gp_init_kernel(const float *__restrict__ K, int n, double noise,
                   double *__restrict__ A, const float *__restrict__ F,
                   long long nf, double *__restrict__ Z, int *__restrict__ info)
{
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long nn = (long long)n * n;

    if (idx == 0)
        *info = 0;
    if (idx < nn) {
        const int r = (int)(idx / n), c = (int)(idx % n);

        A[idx] = (double)K[idx] + (r == c ? noise : 0.0);
    }
    if (idx < nf)
        Z[idx] = (double)F[idx];
}

__global__ void __launch_bounds__(256)
    gp_store_kernel(const double *__restrict__ X, long long nf,
                    float *__restrict__ F)
{
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;

    if (idx < nf)
        F[idx] = (float)X[idx];
}

static void dgemm(const dg_args &a, hipStream_t s)
{
    if (a.M <= 0 || a.N <= 0)
        return;
    hipLaunchKernelGGL(dgemm_kernel,
                       dim3((unsigned)((a.N + DG_T - 1) / DG_T),
                            (unsigned)((a.M + DG_T - 1) / DG_T)),
                       dim3(256), 0, s, a);
}

extern "C" size_t roma_gp_work_bytes(int n, int d)
{
    const size_t nblk = (size_t)(n + GP_NB - 1) / GP_NB;

    return sizeof(double) * (2 * (size_t)n * n + nblk * GP_NB * GP_NB +
                             2 * (size_t)n * d);
}

extern "C" void roma_gp_solve(struct ops *o, cl_mem K, int n, float noise,
                              cl_mem F, int d, cl_mem work, cl_mem info)
{
    ICOREG_API_BEGIN
    const char *op = "roma_gp_solve";
    hipStream_t s;
    double *A, *L, *Li, *Z, *Y;
    const int nblk = (n + GP_NB - 1) / GP_NB;
    const long long nd = (long long)n * d;

    if (n < 1 || d < 1 || n > 46340)
        icoreg_fatal("%s: invalid sizes n=%d d=%d", op, n, d);
    count32((long long)n * n, op);
    count32(nd, op);
    need_floats(K, 0, (long long)n * n, op, "K");
    need_floats(F, 0, nd, op, "F");
    need_bytes(work, 0, (long long)roma_gp_work_bytes(n, d), op, "work");
    need_bytes(info, 0, (long long)sizeof(int), op, "info");
    s = stream_of(o->ocl);
    A = (double *)work->ptr;
    L = A + (long long)n * n;
    Li = L + (long long)n * n;
    Z = Li + (long long)nblk * GP_NB * GP_NB;
    Y = Z + nd;
    {
        prof_scope ps(o->ocl, op);
        const long long nn = (long long)n * n;
        const long long tot = nn > nd ? nn : nd;

        hipLaunchKernelGGL(gp_init_kernel, dim3((unsigned)((tot + 255) / 256)),
                           dim3(256), 0, s, cfptr(K), n, (double)noise, A,
                           cfptr(F), nd, Z, (int *)info->ptr);
        for (int b = 0; b < nblk; b++) {
            const int k = b * GP_NB, nb = n - k < GP_NB ? n - k : GP_NB;
            const int rest = n - k - nb;
            double *Lk = Li + (long long)b * GP_NB * GP_NB;
            dg_args g;

            hipLaunchKernelGGL(chol_diag_kernel, dim3(1), dim3(256), 0, s, A,
                               L, Lk, n, k, nb, (int *)info->ptr);
            if (rest == 0)
                continue;
            /* L21 = A21 Linv^T. */
            g = dg_args{rest, nb, nb, A + (long long)(k + nb) * n + k, n, 1,
                        Lk, 1, GP_NB, L + (long long)(k + nb) * n + k, n,
                        1.0, 0, 0};
            dgemm(g, s);
            /* A22 -= L21 L21^T, lower tiles. */
            g = dg_args{rest, rest, nb, L + (long long)(k + nb) * n + k, n, 1,
                        L + (long long)(k + nb) * n + k, 1, n,
                        A + (long long)(k + nb) * n + k + nb, n, -1.0, 1, 1};
            dgemm(g, s);
        }
        /* L Y = Z, block by block. */
        for (int b = 0; b < nblk; b++) {
            const int k = b * GP_NB, nb = n - k < GP_NB ? n - k : GP_NB;
            const int rest = n - k - nb;
            dg_args g;

            g = dg_args{nb, d, nb, Li + (long long)b * GP_NB * GP_NB, GP_NB,
                        1, Z + (long long)k * d, d, 1, Y + (long long)k * d,
                        d, 1.0, 0, 0};
            dgemm(g, s);
            if (rest == 0)
                continue;
            g = dg_args{rest, d, nb, L + (long long)(k + nb) * n + k, n, 1,
                        Y + (long long)k * d, d, 1,
                        Z + (long long)(k + nb) * d, d, -1.0, 1, 0};
            dgemm(g, s);
        }
        /* L^T X = Y, from the last block; X goes to Z (consumed). */
        for (int b = nblk - 1; b >= 0; b--) {
            const int k = b * GP_NB, nb = n - k < GP_NB ? n - k : GP_NB;
            dg_args g;

            /* X_k = Linv^T Y_k: A(i, q) = Linv[q][i]. */
            g = dg_args{nb, d, nb, Li + (long long)b * GP_NB * GP_NB, 1,
                        GP_NB, Y + (long long)k * d, d, 1,
                        Z + (long long)k * d, d, 1.0, 0, 0};
            dgemm(g, s);
            if (k == 0)
                continue;
            /* Y[0:k] -= L[k:k+nb, 0:k]^T X_k: A(i, q) = L[k + q][i]. */
            g = dg_args{k, d, nb, L + (long long)k * n, 1, n,
                        Z + (long long)k * d, d, 1, Y, d, -1.0, 1, 0};
            dgemm(g, s);
        }
        hipLaunchKernelGGL(gp_store_kernel, dim3((unsigned)((nd + 255) / 256)),
                           dim3(256), 0, s, Z, nd, fptr(F));
    }
    launch_check(op);
    ICOREG_API_END
}

/* SPDX-License-Identifier: Unlicense */

/* RoMa's Gaussian-process solve on the device, in double precision:
 * F = (K + noise I)^-1 F for the n x n cosine kernel K (float) and the
 * n x d position basis F (float). The reference factors and solves on
 * the host (roma.c:770-836 of i.coregistration.opencl: Cholesky, then
 * L Z = F and L^T X = Z, all in double), which costs a 10 MB read-back,
 * a host Cholesky of n = 1600 and a write per tile pair; here the same
 * arithmetic stays on the GPU.
 *
 * Blocked right-looking Cholesky with 64-column panels, the forward solve
 * carried along as extra columns of the right-hand side [F | I]: the
 * identity block makes the forward solve produce Minv = L^-1 beside
 * Y = L^-1 F, so that the backward solve X = Minv^T Y is a sum over the
 * panels of their block rows' products, added as each becomes final,
 * instead of a chain of one launch per panel after the factorisation.
 *  - chol_diag: the 64 x 64 diagonal block factored and its factor
 *    inverted by one work-group (one wave each, in registers), after
 *    applying the previous panel's update to the block itself
 *    (look-ahead); these run back to back on the main stream while
 *    everything else runs on a second stream, joined back at the end;
 *  - on the second stream, one launch per panel for both L21 = A21
 *    Linv^T and Y_b = Linv_b Z_b (Z_b over the right-hand-side columns
 *    that are not yet zero: F and the identity blocks of this panel and
 *    the ones before), one for the trailing update A22 -= L21 L21^T
 *    (lower tiles but the next diagonal block), Z_rest -= L21 Y_b and
 *    X[0 : k + nb] += Minv_b^T Y_F,b (fp64 GEMM tiles, up to three
 *    problems per launch).
 * Synchronisation, inside the kernels: the diagonal kernel of block b
 * sets a flag once its factor and inverse are stored, which panel b's
 * first products on the second stream poll before reading them; and it
 * waits itself for a flag that a one-wave kernel sets on the second
 * stream after panel b - 2's trailing update. Neither stream then holds
 * a stream wait or an event record between its kernels (each costs 5-7
 * us of command-processor time, on the solve's critical path). Every
 * wait is bounded; one that gives up sets info = -1 and its kernel ends
 * (the caller then runs the solve again with event waits). Under stream
 * capture (a graph has no order between branches that an in-kernel wait
 * could rely on), the two streams wait through stream events instead.
 * Working matrices: A (n x n, the trailing updates), L (n x n, the
 * factor), Linv per panel, Z and Y (n x (d + n)), X (n x d), two flags
 * per panel. No launch reads what another running beside it writes. */

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <math.h>

#include <initializer_list>

#include "common.h"
#include "icoreg_kernels.h"

using namespace icoreg;

#define GP_NB 64 /* panel width */
#define DG_T 64  /* GEMM output tile */
#define DG_K 32  /* GEMM reduction chunk */

/* C = alpha A B + beta C with A(i, q) = A[i a_ri + q a_rk], B(q, j) =
 * B[q b_rk + j b_rj], C(i, j) = C[i c_ri + j]; lower: skip output tiles
 * strictly above the diagonal; skip00: leave output tile (0, 0) alone. */
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
    int skip00;
};

/* Up to three independent problems per launch: blockIdx.z picks one.
 * wait (when given): a flag the launch's blocks poll (one thread each,
 * device-coherent loads, at most spin_max polls, then an acquire) before
 * they read their operands; a wait that gives up sets *info = -1 and
 * goes on, so that the launch still ends. */
#define DG_MAXP 3
struct dg_set {
    dg_args p[DG_MAXP];
    const int *wait;
    int spin_max;
    int *info;
};

__global__ void __launch_bounds__(256) dgemm_kernel(dg_set pr)
{
    __shared__ double As[DG_K][DG_T + 1], Bs[DG_K][DG_T + 1];
    const dg_args &a = pr.p[blockIdx.z];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int i0 = blockIdx.y * DG_T, j0 = blockIdx.x * DG_T;
    double acc[4][4], cprev[4][4];

    if (i0 >= a.M || j0 >= a.N || (a.lower && j0 > i0 + DG_T - 1) ||
        (a.skip00 && i0 == 0 && j0 == 0))
        return;
    if (pr.wait) {
        if (tid == 0) {
            int it = 0;

            while (__hip_atomic_load(pr.wait, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0 &&
                   ++it < pr.spin_max)
                __builtin_amdgcn_s_sleep(1);
            if (it >= pr.spin_max)
                __hip_atomic_store(pr.info, -1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    /* The accumulated C is read at the start, so that its latency
     * overlaps the products. */
#pragma unroll
    for (int p = 0; p < 4; p++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int i = min(i0 + ty + 16 * p, a.M - 1), j = min(j0 + tx + 16 * r, a.N - 1);

            cprev[p][r] = a.beta ? a.C[(long long)i * a.c_ri + j] : 0.0;
        }
#pragma unroll
    for (int p = 0; p < 4; p++)
#pragma unroll
        for (int q = 0; q < 4; q++)
            acc[p][q] = 0.0;
    /* 32 x 64 of A and of B per chunk, 8 values per thread, the
     * unit-stride index fastest across threads. Every load reads a valid
     * address (indices clamped to the last row / column) and the value is
     * selected afterwards, so that the 16 loads are all in flight together;
     * the next chunk's loads are issued before the current chunk's
     * products. */
    double va[8], vb[8];
    bool oka[8], okb[8];

    auto fetch = [&](int k0) {
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
    };
    fetch(0);
    for (int k0 = 0; k0 < a.K; k0 += DG_K) {
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
        if (k0 + DG_K < a.K)
            fetch(k0 + DG_K);
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

            if (j < a.N)
                a.C[(long long)i * a.c_ri + j] = a.alpha * acc[p][r] + cprev[p][r];
        }
    }
}

/* ---- the diagonal block ------------------------------------------------------------ */

/* 1 / sqrt(x) from the hardware estimate (within 2^29 ulp: about 2^-23
 * relative) and one Newton step, which squares that error (about 2^-46:
 * some 100 ulp of a double, far below what the float result can show).
 * -0.5 x does not depend on the estimate, so the step adds three
 * dependent operations to the pivot's chain. */
__device__ __forceinline__ double rsqrt_nr(double x)
{
    const double h = -0.5 * x;
    const double r = __builtin_amdgcn_rsq(x);

    return r * fma(h * r, r, 1.5);
}

/* Lane l's value of v, in every lane. */
__device__ __forceinline__ double readlane_d(double v, int l)
{
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);

    return __builtin_bit_cast(
        double, ((unsigned long long)(unsigned)__builtin_amdgcn_readlane((int)(b >> 32), l) << 32) |
                    (unsigned)__builtin_amdgcn_readlane((int)b, l));
}

typedef double gp_d4 __attribute__((ext_vector_type(4)));

/* Polls of a panel flag before the diagonal kernel gives up (with a
 * 64-clock sleep each: about 0.1 s, far beyond any trailing update): the wait
 * then ends with info = -1 instead of hanging. */
#define GP_SPIN_MAX (1 << 22)

/* Cholesky factor of the nb x nb diagonal block at (k, k) of A (n x n)
 * into L, and the inverse of that factor into Linv (nb x nb, row-major,
 * GP_NB apart). info gets 1 + the first column whose pivot is not
 * positive (the factor then holds NaN from there on), or -1 if the wait
 * for ready gave up. 256 threads.
 *  - ready (when given): set once the trailing update this block needs
 *    has finished on the other stream; polled with device-coherent loads,
 *    then an acquire, so the block's reads see that update.
 *  - done (when given): set to 1 after every store of the block, behind
 *    a release, for the panel's products on the other stream.
 *  - Look-ahead (lprev: the previous panel's Linv; its trailing update of
 *    this block is left to this kernel): P = A[k.., k - 64..] lprev^T,
 *    the block's row of that panel's L21, then s -= P P^T on the lower
 *    triangle, in 16 x 16 tiles on v_mfma_f64_16x16x4f64 (lane l gives
 *    A(l % 16, l / 16) and B(l / 16, l % 16) and holds D(l / 16 + 4 v,
 *    l % 16); the fp32 16 x 16 x 4 form holds rows 4 (l / 16) + v
 *    instead). Its operands (the block row of A, lprev) arrive in LDS in
 *    the same round trip as the block itself; the 16 P tiles (4 a wave,
 *    held in registers until every wave has read lprev) and the 10
 *    lower P P^T tiles are dealt to the 4 waves in turn; P goes through
 *    f.
 *  - Wave 0 then sweeps the columns two at a time: lane r holds row r
 *    of the block (a[c], c <= r; its upper part is never read). At step
 *    j every lane reads the 2 x 2 pivot block [p q; q s] of columns j,
 *    j + 1 from lanes j and j + 1 (cross-lane reads), forms 1 / sqrt(p),
 *    l21 = q / sqrt(p) and 1 / sqrt(s - l21^2), then
 *        L[r][j] = a[j] / sqrt(p),
 *        L[r][j + 1] = (a[j + 1] - L[r][j] l21) / sqrt(s - l21^2)
 *    on and below the pivots (0 above); both columns go to LDS (lc)
 *    and each lane applies the rank-2 update
 *        a[c] -= L[r][j] L[c][j] + L[r][j + 1] L[c][j + 1]   (c > j + 1).
 *    The step's dependent chain (cross-lane reads, two roots, one LDS
 *    round trip, the update of the next pivots) thus serves two
 *    columns.
 *  - Wave 1, beside it and a step behind, runs the forward substitution
 *    of L X = I column by column: lane k holds column k of T (the
 *    identity at first),
 *        T[j][k] /= L[j][j],  T[c][k] -= L[c][j] T[j][k]   (c > j),
 *    taking column j from lc once wave 0 has counted it (an LDS counter,
 *    released at the start of wave 0's next step). Each wave holds 64
 *    values a lane, so a step's column reads (16-byte loads, every lane
 *    the same address) are issued together before its updates.
 *  - All threads store the factor from lc in rows; the inverse is stored
 *    from wave 1's registers (lane k: column k, so each store
 *    instruction writes one row of it).
 * Against the earlier form (1024 threads holding the block in LDS, one
 * barrier per two columns): 59.7 -> 41 us a block at n = 1600 with one
 * column a step. */
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
    chol_diag_kernel(const double *__restrict__ A, double *__restrict__ L,
                      double *__restrict__ Linv, int n, int k, int nb,
                      const double *__restrict__ lprev, const int *ready, int spin_max,
                      int *__restrict__ info, int *done)
{
    __shared__ double s[GP_NB][GP_NB + 1], f[GP_NB][GP_NB + 1];
    /* lc[j][r] = L[r][j]: each column contiguous, read with wide LDS
     * loads (every lane the same address). Before the column sweep the
     * same memory holds ar, the look-ahead's block row of A. */
    __shared__ __align__(16) union {
        double lc[GP_NB][GP_NB];
        double ar[GP_NB][GP_NB + 1];
    } u;
    double (*const lc)[GP_NB] = u.lc;
    __shared__ double dinv[GP_NB];
    __shared__ int prog;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    int bad = 0;

    if (ready) {
        if (tid == 0) {
            int it = 0;

            while (__hip_atomic_load(ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0 &&
                   ++it < spin_max)
                __builtin_amdgcn_s_sleep(1);
            if (it >= spin_max)
                bad = -1;
        }
        __syncthreads();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    /* The block's lower triangle; rows and columns past nb are zero with
     * a unit diagonal (their pivots stay 1 and they touch no real row).
     * With a look-ahead, its operands come in the same round trip: the
     * block row A[k.., k - 64..] (rows past nb zero) into ar and the
     * previous panel's inverse factor into f. */
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int e = tid + 256 * i, r = e >> 6, c = e & 63;
        const long long row = (long long)(k + min(r, nb - 1)) * n;
        const double v = A[row + k + min(c, nb - 1)];

        if (lprev) {
            const double va = A[row + k - GP_NB + c], vl = lprev[e];

            u.ar[r][c] = r < nb ? va : 0.0;
            f[r][c] = vl;
        }
        s[r][c] = r < nb && c <= r ? v : r == c ? 1.0 : 0.0;
    }
    if (tid == 0)
        prog = 0;
    __syncthreads();
    if (lprev) {
        const int kq = lane >> 4;
        gp_d4 pacc[4];

        /* P tiles (i, (wave + i) % 4) of this wave, from LDS; lprev is
         * lower triangular, so tile column tc needs k < 16 (tc + 1). */
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tc = (wave + i) & 3;
            const int ri = 16 * i + (lane & 15), ci = 16 * tc + (lane & 15);

            pacc[i] = (gp_d4){0.0, 0.0, 0.0, 0.0};
#pragma unroll
            for (int kk = 0; kk < 16; kk++)
                if (kk < 4 * (tc + 1))
                    pacc[i] = __builtin_amdgcn_mfma_f64_16x16x4f64(
                        u.ar[ri][4 * kk + kq], f[ci][4 * kk + kq], pacc[i], 0, 0, 0);
        }
        __syncthreads(); /* every wave is done reading f */
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tc = (wave + i) & 3;

#pragma unroll
            for (int v = 0; v < 4; v++)
                f[16 * i + kq + 4 * v][16 * tc + (lane & 15)] = pacc[i][v];
        }
        __syncthreads();
        for (int w = wave; w < 10; w += 4) {
            const int tr2 = w >= 6 ? 3 : w >= 3 ? 2 : w >= 1 ? 1 : 0;
            const int tc2 = w - tr2 * (tr2 + 1) / 2;
            const int r2 = 16 * tr2 + (lane & 15), c2 = 16 * tc2 + (lane & 15);
            gp_d4 acc = {0.0, 0.0, 0.0, 0.0};

#pragma unroll
            for (int kk = 0; kk < 16; kk++)
                acc = __builtin_amdgcn_mfma_f64_16x16x4f64(f[r2][4 * kk + kq], f[c2][4 * kk + kq],
                                                          acc, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int r = 16 * tr2 + kq + 4 * v, c = 16 * tc2 + (lane & 15);

                if (r < nb && c <= r)
                    s[r][c] -= acc[v];
            }
        }
        __syncthreads();
    }
    if (wave == 0) {
        /* The factor: lane r holds row r (a[c], c <= r; its upper part
         * is never read). Column j of L goes to lc[j], the pivot's
         * reciprocal root to dinv, then the step count to prog. Above
         * the pivot L[r][j] = 0 is written too, so lc holds the factor
         * transposed with zeros above its diagonal. */
        double a[GP_NB];

#pragma unroll
        for (int c = 0; c < GP_NB; c++)
            a[c] = s[lane][c];
#pragma unroll
        for (int j = 0; j < GP_NB; j += 2) {
            if (j >= nb)
                continue;
            /* Columns below j and their roots were written a step ago:
             * counted now, the release's wait for them costs nothing. */
            if (j > 0 && lane == 0)
                __hip_atomic_store(&prog, j, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            /* Pair j, j + 1: the 2 x 2 pivot block [p q; q s] from lanes j
             * and j + 1, p's root, then the second pivot s - l21^2 and its
             * root. Column j + 1 of a lane is its entry less its column-j
             * value times l21, so one LDS round trip and one rank-2 update
             * serve both columns. When nb is odd the last step's second
             * column is a padding column (unit pivot, zero elsewhere),
             * which leaves the real ones unchanged. */
            const double p = readlane_d(a[j], j), q = readlane_d(a[j], j + 1);
            const double sq = readlane_d(a[j + 1], j + 1);
            const double rp = rsqrt_nr(p);
            const double l21 = q * rp;
            const double s2 = fma(-l21, l21, sq);
            const double rs = rsqrt_nr(s2);
            const double l0 = lane > j ? a[j] * rp : lane == j ? p * rp : 0.0;
            const double l1 = lane > j + 1   ? fma(-l0, l21, a[j + 1]) * rs
                              : lane == j + 1 ? s2 * rs
                                              : 0.0;

            if (lane == 0 && bad == 0) {
                if (!(p > 0.0))
                    bad = k + j + 1;
                else if (!(s2 > 0.0))
                    bad = k + j + 2;
            }
            lc[j][lane] = l0;
            lc[j + 1][lane] = l1;
            if (lane == 0) {
                dinv[j] = rp;
                dinv[j + 1] = rs;
            }
            /* LDS operations of one wave complete in issue order: these
             * reads see the columns just written. Both columns are read in
             * full before the updates, so that the loads overlap. */
            double c0[GP_NB], c1[GP_NB];

#pragma unroll
            for (int c = j + 2; c < GP_NB; c++) {
                c0[c] = lc[j][c];
                c1[c] = lc[j + 1][c];
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 64, 0); /* LDS reads first */
#pragma unroll
            for (int c = j + 2; c < GP_NB; c++)
                a[c] = fma(-l1, c1[c], fma(-l0, c0[c], a[c]));
        }
        if (lane == 0)
            __hip_atomic_store(&prog, nb, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    else if (wave == 1) {
        /* The inverse, a step behind, two columns at a time as wave 0
         * makes them: lane k holds column k of T (the identity at first),
         *     T[j][k] /= L[j][j],
         *     T[j + 1][k] = (T[j + 1][k] - L[j + 1][j] T[j][k]) / L[j + 1][j + 1],
         * then T[c][k] -= L[c][j] T[j][k] + L[c][j + 1] T[j + 1][k] below,
         * with columns j, j + 1 of L from lc once wave 0 has counted them
         * (or all nb columns, when j + 1 is a padding column). The wait is
         * on wave 0 of the same block, which always counts every column;
         * it is capped all the same. */
        double t[GP_NB];

#pragma unroll
        for (int c = 0; c < GP_NB; c++)
            t[c] = c == lane ? 1.0 : 0.0;
#pragma unroll
        for (int j = 0; j < GP_NB; j += 2) {
            if (j >= nb)
                continue;
            const int need = j + 2 < nb ? j + 2 : nb;
            int it = 0;

            while (__hip_atomic_load(&prog, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <
                       need &&
                   ++it < (1 << 24))
                __builtin_amdgcn_s_sleep(1);
            double c0[GP_NB], c1[GP_NB];

#pragma unroll
            for (int c = j + 1; c < GP_NB; c++)
                c0[c] = lc[j][c];
#pragma unroll
            for (int c = j + 2; c < GP_NB; c++)
                c1[c] = lc[j + 1][c];
            __builtin_amdgcn_sched_group_barrier(0x100, 64, 0);
            const double tj = t[j] * dinv[j];
            const double tj1 = fma(-c0[j + 1], tj, t[j + 1]) * dinv[j + 1];

            t[j] = tj;
            t[j + 1] = tj1;
#pragma unroll
            for (int c = j + 2; c < GP_NB; c++)
                t[c] = fma(-c1[c], tj1, fma(-c0[c], tj, t[c]));
        }
        /* Lane k writes column k, one row of the inverse per store. */
        if (lane < nb)
#pragma unroll
            for (int m = 0; m < GP_NB; m++)
                if (m < nb)
                    Linv[m * GP_NB + lane] = m >= lane ? t[m] : 0.0;
    }
    __syncthreads();
    if (tid == 0 && bad && *info == 0)
        *info = bad;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int e = tid + 256 * i, r = e >> 6, c = e & 63;

        if (r < nb && c < nb)
            L[(long long)(k + r) * n + k + c] = lc[c][r];
    }
    if (done) {
        /* Every store of the block has reached L2 (the barrier waits for
         * them); the release writes them back for the other XCDs, then
         * the flag. */
        __syncthreads();
        if (tid == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            __hip_atomic_store(done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

/* A = K + noise I (double), Z = [F | I] (double, rows d + n wide), X = 0
 * (n x d), info and the nflags panel flags cleared. */
__global__ void __launch_bounds__(256)
    gp_init_kernel(const float *__restrict__ K, int n, double noise,
                   double *__restrict__ A, const float *__restrict__ F, int d,
                   double *__restrict__ Z, double *__restrict__ X, int *__restrict__ info,
                   int *__restrict__ flags, int nflags)
{
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long nn = (long long)n * n, w = (long long)d + n, nz = n * w;

    if (idx == 0)
        *info = 0;
    if (idx < nflags)
        flags[idx] = 0;
    if (idx < nn) {
        const int r = (int)(idx / n), c = (int)(idx % n);

        A[idx] = (double)K[idx] + (r == c ? noise : 0.0);
    }
    if (idx < nz) {
        const long long r = idx / w, c = idx % w;

        Z[idx] = c < d ? (double)F[r * d + c] : c - d == r ? 1.0 : 0.0;
    }
    if (idx < (long long)n * d)
        X[idx] = 0.0;
}

/* Panel flag: set by one lane after the launches before it on its stream
 * (the panel's trailing update) have finished; device-coherent store. */
__global__ void __launch_bounds__(64) gp_mark_kernel(int *flag)
{
    if (threadIdx.x == 0)
        __hip_atomic_store(flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void __launch_bounds__(256)
    gp_store_kernel(const double *__restrict__ X, long long nf, float *__restrict__ F)
{
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;

    if (idx < nf)
        F[idx] = (float)X[idx];
}

static dg_args dg(int M, int N, int K, const double *A, long long a_ri, long long a_rk,
                  const double *B, long long b_rk, long long b_rj, double *C,
                  long long c_ri, double alpha, int beta, int lower)
{
    dg_args a = {M, N, K, A, a_ri, a_rk, B, b_rk, b_rj, C, c_ri, alpha, beta, lower, 0};

    return a;
}

/* One launch for the problems given (those with no output are skipped);
 * wait, spin_max, info as in dg_set. */
static void dgemm(hipStream_t s, std::initializer_list<const dg_args *> ps,
                  const int *wait = nullptr, int spin_max = 0, int *info = nullptr)
{
    dg_set pr;
    int np = 0, tx = 0, ty = 0;

    pr.wait = wait;
    pr.spin_max = spin_max;
    pr.info = info;

    for (const dg_args *a : ps)
        if (a && a->M > 0 && a->N > 0) {
            if (np == DG_MAXP)
                icoreg_fatal("roma_gp_solve: more than %d products in one launch", DG_MAXP);
            pr.p[np++] = *a;
            tx = max(tx, (a->N + DG_T - 1) / DG_T);
            ty = max(ty, (a->M + DG_T - 1) / DG_T);
        }
    if (np == 0)
        return;
    hipLaunchKernelGGL(dgemm_kernel, dim3((unsigned)tx, (unsigned)ty, (unsigned)np),
                       dim3(256), 0, s, pr);
}

extern "C" size_t roma_gp_work_bytes(int n, int d)
{
    const size_t nblk = (size_t)(n + GP_NB - 1) / GP_NB, w = (size_t)d + n;

    return sizeof(double) * (2 * (size_t)n * n + nblk * GP_NB * GP_NB + 2 * (size_t)n * w +
                             (size_t)n * d) +
           sizeof(int) * 2 * nblk;
}

/* Test hooks (icoreg_gp_test_wait): the in-kernel waits' poll limit and
 * whether the panel flags are set at all (by the second stream's flag
 * kernel and by the diagonal kernels). With the flags never set and a
 * short limit, every waiting kernel gives up at once (info = -1) and
 * still exits, so the give-up path and the caller's recovery can be
 * exercised without a stalled stream. */
static int g_spin_max = GP_SPIN_MAX;
static int g_set_flags = 1;

extern "C" void icoreg_gp_test_wait(int spin_max, int set_flags)
{
    g_spin_max = spin_max > 0 ? spin_max : GP_SPIN_MAX;
    g_set_flags = set_flags != 0;
}

/* events: the diagonal kernels wait through stream events (the form a
 * capture needs, and the fallback when the in-kernel wait gave up). */
static void gp_solve_run(struct ops *o, cl_mem K, int n, float noise, cl_mem F, int d,
                         cl_mem work, cl_mem info, bool events, const char *op)
{
    hipStream_t s;
    double *A, *L, *Li, *Z, *Y, *X;
    int *flags;
    const int nblk = (n + GP_NB - 1) / GP_NB;
    const long long nd = (long long)n * d, w = (long long)d + n;

    if (n < 1 || d < 1 || n > 46340)
        icoreg_fatal("%s: invalid sizes n=%d d=%d", op, n, d);
    count32((long long)n * n, op);
    count32((long long)n * w, op);
    need_floats(K, 0, (long long)n * n, op, "K");
    need_floats(F, 0, nd, op, "F");
    need_bytes(work, 0, (long long)roma_gp_work_bytes(n, d), op, "work");
    need_bytes(info, 0, (long long)sizeof(int), op, "info");
    s = stream_of(o->ocl);
    A = (double *)work->ptr;
    L = A + (long long)n * n;
    Li = L + (long long)n * n;
    Z = Li + (long long)nblk * GP_NB * GP_NB;
    Y = Z + n * w;
    X = Y + n * w;
    flags = (int *)(X + nd);
    {
        prof_scope ps(o->ocl, op);
        const long long nn = (long long)n * n, nz = n * w;
        const long long tot = nn > nz ? nn : nz;
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;

        hip_check(hipStreamIsCapturing(s, &cs), "hipStreamIsCapturing");
        const bool capture = events || cs != hipStreamCaptureStatusNone;
        const int spin_max = g_spin_max;

        hipLaunchKernelGGL(gp_init_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s,
                           cfptr(K), n, (double)noise, A, cfptr(F), d, Z, X, (int *)info->ptr,
                           flags, 2 * nblk);
        /* The diagonal blocks on the main stream s, everything else of a
         * panel on the second stream s2: diagonal block b waits for the
         * trailing update of panel b - 2 (which has the whole of block
         * b - 1's factorisation to finish) and applies panel b - 1's
         * update to its own block itself; panel b's products wait for
         * block b. Y = L^-1 [F | I] alongside, over the columns that are
         * not yet zero (F and the identity blocks up to this panel's).
         * flags[b]: panel b's trailing update done (set on s2);
         * dflags[b]: block b factored (set by its diagonal kernel). */
        hipStream_t s2 = aux_stream_of(o->ocl);
        int *const dflags = flags + nblk;

        hip_check(hipEventRecord(aux_event(o->ocl, 2 * nblk), s), "hipEventRecord");
        hip_check(hipStreamWaitEvent(s2, aux_event(o->ocl, 2 * nblk), 0), "hipStreamWaitEvent");
        for (int b = 0; b < nblk; b++) {
            const int k = b * GP_NB, nb = n - k < GP_NB ? n - k : GP_NB;
            const int rest = n - k - nb, wb = d + k + nb;
            double *Lk = Li + (long long)b * GP_NB * GP_NB;
            double *L21 = L + (long long)(k + nb) * n + k;
            const double *lprev = b ? (const double *)(Lk - GP_NB * GP_NB) : nullptr;
            int *info_p = (int *)info->ptr;
            const hipEvent_t done_b = aux_event(o->ocl, 2 * b);

            if (capture) {
                if (b >= 2)
                    hip_check(hipStreamWaitEvent(s, aux_event(o->ocl, 2 * (b - 2) + 1), 0),
                              "hipStreamWaitEvent");
                hipLaunchKernelGGL(chol_diag_kernel, dim3(1), dim3(256), 0, s, A,
                                   L, Lk, n, k, nb, lprev, (const int *)nullptr, spin_max,
                                   info_p, (int *)nullptr);
                hip_check(hipEventRecord(done_b, s), "hipEventRecord");
                hip_check(hipStreamWaitEvent(s2, done_b, 0), "hipStreamWaitEvent");
            }
            else
                /* Panel b's first products wait for dflags[b] inside their
                 * kernel: no stream wait (5-6 us of command-processor
                 * time a panel on s2) and no completion event. */
                hipLaunchKernelGGL(chol_diag_kernel, dim3(1), dim3(256), 0, s, A, L, Lk, n, k,
                                   nb, lprev, b >= 2 ? (const int *)flags + b - 2 : nullptr,
                                   spin_max, info_p, g_set_flags ? dflags + b : nullptr);
            /* L21 = A21 Linv^T and Y_b = Linv_b Z_b. */
            const dg_args panel = dg(rest, nb, nb, A + (long long)(k + nb) * n + k, n, 1,
                                     Lk, 1, GP_NB, L21, n, 1.0, 0, 0);
            const dg_args yb = dg(nb, wb, nb, Lk, GP_NB, 1, Z + k * w, w, 1, Y + k * w, w,
                                  1.0, 0, 0);
            if (capture)
                dgemm(s2, {&yb, &panel});
            else
                dgemm(s2, {&yb, &panel}, dflags + b, spin_max, info_p);
            /* X[0 : k + nb] += Minv_b^T Y_F,b: this panel's block row of
             * Minv = L^-1 (Y[k.., d..], zero right of its own identity
             * block) is final once Y_b is. */
            dg_args xacc = dg(k + nb, d, nb, Y + k * w + d, 1, w, Y + k * w, w, 1, X, d, 1.0, 1,
                              0);
            if (rest > 0) {
                /* A22 -= L21 L21^T (lower tiles but the next diagonal block,
                 * which its own kernel updates) and Z_rest -= L21 Y_b. */
                dg_args trail = dg(rest, rest, nb, L21, n, 1, L21, 1, n,
                                   A + (long long)(k + nb) * n + k + nb, n, -1.0, 1, 1);
                const dg_args zr = dg(rest, wb, nb, L21, n, 1, Y + k * w, w, 1,
                                      Z + (k + nb) * w, w, -1.0, 1, 0);

                trail.skip00 = 1;
                dgemm(s2, {&trail, &zr, &xacc});
            }
            else
                dgemm(s2, {&xacc});
            if (!capture && g_set_flags)
                hipLaunchKernelGGL(gp_mark_kernel, dim3(1), dim3(64), 0, s2, flags + b);
            if (capture || b == nblk - 1)
                hip_check(hipEventRecord(aux_event(o->ocl, 2 * b + 1), s2), "hipEventRecord");
        }
        hip_check(hipStreamWaitEvent(s, aux_event(o->ocl, 2 * (nblk - 1) + 1), 0),
                  "hipStreamWaitEvent");
        hipLaunchKernelGGL(gp_store_kernel, dim3((unsigned)((nd + 255) / 256)), dim3(256), 0, s,
                           (const double *)X, nd, fptr(F));
    }
    launch_check(op);
}

extern "C" void roma_gp_solve(struct ops *o, cl_mem K, int n, float noise,
                              cl_mem F, int d, cl_mem work, cl_mem info)
{
    ICOREG_API_BEGIN
    gp_solve_run(o, K, n, noise, F, d, work, info, false, "roma_gp_solve");
    ICOREG_API_END
}

extern "C" void roma_gp_solve_events(struct ops *o, cl_mem K, int n, float noise,
                                     cl_mem F, int d, cl_mem work, cl_mem info)
{
    ICOREG_API_BEGIN
    gp_solve_run(o, K, n, noise, F, d, work, info, true, "roma_gp_solve_events");
    ICOREG_API_END
}

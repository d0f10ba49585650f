/* SPDX-License-Identifier: Unlicense */

/* Blockwise scaled dot-product attention on the fp32 matrix cores:
 * O = softmax(scale Q K^T) V per head, never storing the scores. The
 * contract is the reference's attention kernel (ops.cl:604-687,
 * ops.c:444-474 of i.coregistration.opencl): token-major operands with
 * head h at columns h * d, d <= 128, optional key mask, a query with no
 * key left gets zeros.
 *
 * A block holds 4 waves of 32 queries each (128 queries of one head)
 * and streams its range of keys in tiles of 32 through double-buffered
 * LDS, shared by the 4 waves, one barrier per tile; with 16-byte
 * aligned rows the next tile is read into registers a tile ahead:
 *  - the scores are computed transposed, S^T = K Q^T, with
 *    v_mfma_f32_32x32x2f32 (A = K from LDS, B = the wave's queries,
 *    pre-scaled and held in registers for the whole kernel), so that
 *    each lane holds 16 keys of one query (its column);
 *  - the online softmax runs per lane on those registers, the two lane
 *    halves of a query combined with one cross-lane exchange; scores are
 *    kept in base 2 (log2 e folded into the query scale, one v_exp_f32
 *    per probability) and the running maximum is raised lazily, only
 *    when a tile exceeds it by 2^8, so the accumulator rescale is rare;
 *  - the output is accumulated transposed, O^T += V^T P^T, with the
 *    probabilities fed to the MFMA straight from the score registers:
 *    MFMA step r pairs, for lane half h, key (r / 4) * 8 + h * 4 + r % 4,
 *    which is where the score MFMA left it, and reads the matching V
 *    rows from LDS. No transpose of P through LDS.
 * When queries x heads give too few waves to fill the chip (ELoFTR's 400
 * tokens, the ViT's 1601 tokens per head), the keys are split into
 * ranges over grid z and a second kernel merges the partial results by
 * their running maxima and sums, as flash-decoding does. */

#include <hip/hip_runtime.h>

#include <mutex>

#include <math.h>

#include "common.h"
#include "ops.h"

using namespace icoreg;

typedef float floatx16 __attribute__((ext_vector_type(16)));

#define ATT_KT 32 /* keys per tile */
#define ATT_NW 4  /* waves per block, 32 queries each */
#define ATT_TAU 8.0f /* lazy rescaling threshold, base-2 units */
#define ATT_PF 2     /* LDS operand reads ahead of their MFMA */

/* Registers <- the key tile from key k0 (zeros past Nk and d), 16-byte
 * loads, consecutive threads along a key row. */
template <int NL, int DP>
__device__ __forceinline__ void att_fetch(float4 (&kr)[NL], float4 (&vr)[NL],
                                          const float *K, int ldk,
                                          const float *V, int ldv, int k0,
                                          int Nk, int d, int tid)
{
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int e = tid + 64 * ATT_NW * i, key = e / (DP / 4);
        const int dd = (e - key * (DP / 4)) * 4, kk = k0 + key;
        const bool ok = kk < Nk && dd < d;
        /* Always load from a valid address (the last key / last four
         * columns) and select per component: a select between whole
         * vectors or pointers is lowered through scratch memory. Nk >= 1
         * and d >= 4 here. */
        const long long kc = min(kk, Nk - 1), dc = min(dd, d - 4);
        const float4 a = *(const float4 *)(K + kc * ldk + dc);
        const float4 b = *(const float4 *)(V + kc * ldv + dc);

        kr[i].x = ok ? a.x : 0.0f;
        kr[i].y = ok ? a.y : 0.0f;
        kr[i].z = ok ? a.z : 0.0f;
        kr[i].w = ok ? a.w : 0.0f;
        vr[i].x = ok ? b.x : 0.0f;
        vr[i].y = ok ? b.y : 0.0f;
        vr[i].z = ok ? b.z : 0.0f;
        vr[i].w = ok ? b.w : 0.0f;
    }
}

/* Tile t of keys into LDS buffers ks / vs from the registers of a VEC
 * fetch (K stored with an odd row pitch, V with 16-byte rows). */
template <int NL, int DP, int KP, int VP>
__device__ __forceinline__ void att_stash(const float4 (&kr)[NL],
                                          const float4 (&vr)[NL], float *ks,
                                          float *vs, int tid)
{
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int e = tid + 64 * ATT_NW * i, key = e / (DP / 4);
        const int dd = (e - key * (DP / 4)) * 4;
        float *kd = ks + key * KP + dd;

        kd[0] = kr[i].x;
        kd[1] = kr[i].y;
        kd[2] = kr[i].z;
        kd[3] = kr[i].w;
        *(float4 *)(vs + key * VP + dd) = vr[i];
    }
}

/* The same straight from global memory, one float per thread and load
 * (rows not 16-byte aligned). */
template <int NL, int DP, int KP, int VP>
__device__ __forceinline__ void att_stash_direct(const float *K, int ldk,
                                                 const float *V, int ldv,
                                                 int k0, int Nk, int d,
                                                 float *ks, float *vs, int tid)
{
    for (int i = 0; i < NL; i++) {
        const int e = tid + 64 * ATT_NW * i, key = e / DP;
        const int dd = e - key * DP, kk = k0 + key;
        const bool ok = kk < Nk && dd < d;

        ks[key * KP + dd] = ok ? K[(long long)kk * ldk + dd] : 0.0f;
        vs[key * VP + dd] = ok ? V[(long long)kk * ldv + dd] : 0.0f;
    }
}

/* One block: 128 queries (4 waves x 32) of one head against the key
 * tiles [t0, t1) of 32 keys. K and V tiles are double-buffered in LDS
 * and shared by the 4 waves: the next tile (fetched into registers one
 * tile earlier) is written to the other buffer between the score and
 * the output MFMAs, so one barrier per tile suffices. With nsplit > 1
 * (blockIdx.z picks the key range) the unnormalised output and the
 * running (max, sum) go to part_o / part_ml for attn_merge_kernel; with
 * one split the normalised output goes to O directly. MASK: a key mask
 * is given. */
template <int ND, bool VEC, bool MASK>
__global__ void __launch_bounds__(64 * ATT_NW)
    attention_kernel(const float *__restrict__ Q, int ldq,
                     const float *__restrict__ K, int ldk,
                     const float *__restrict__ V, int ldv,
                     float *__restrict__ O, int ldo, int Nq, int Nk, int d,
                     float scale, const unsigned char *__restrict__ kmask,
                     int tiles_per_split, float *__restrict__ part_o,
                     float2 *__restrict__ part_ml, int nh, long long bq,
                     long long bk, long long bv, long long bo)
{
    constexpr int DP = 32 * ND;     /* padded head dimension */
    constexpr int KP = DP + 1;      /* K tile row pitch (odd: no conflicts) */
    constexpr int VP = DP + 4;      /* V tile row pitch */
    constexpr int NS = DP / 2;      /* score MFMA steps */
    constexpr int NL = VEC ? ATT_KT * DP / 4 / (64 * ATT_NW)
                           : ATT_KT * DP / (64 * ATT_NW); /* loads / thread */
    __shared__ __align__(16) float Ks[2][ATT_KT * KP];
    __shared__ __align__(16) float Vs[2][ATT_KT * VP];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.y % nh, bi = blockIdx.y / nh;
    const int half = lane >> 5, col = lane & 31;
    const int qi = (blockIdx.x * ATT_NW + wave) * 32 + col;
    const int ntiles = (Nk + ATT_KT - 1) / ATT_KT;
    const int t0 = blockIdx.z * tiles_per_split;
    const int t1 = min(ntiles, t0 + tiles_per_split);
    float q[NS];
    floatx16 o[ND];
    float m = -INFINITY, l = 0.0f;
    float4 kr4[VEC ? NL : 1], vr4[VEC ? NL : 1];

    /* Scores in the base-2 domain: softmax(x) = 2^(x log2 e - max) / sum,
     * so log2 e is folded into the query scale and every exponential is
     * one v_exp_f32. */
    const float qscale = scale * 1.4426950408889634f;

    Q += bi * bq + (long long)h * d;
    K += bi * bk + (long long)h * d;
    V += bi * bv + (long long)h * d;
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int dd = 2 * s + half;

        q[s] = (qi < Nq && dd < d) ? Q[(long long)qi * ldq + dd] * qscale
                                   : 0.0f;
    }
#pragma unroll
    for (int t = 0; t < ND; t++)
#pragma unroll
        for (int r = 0; r < 16; r++)
            o[t][r] = 0.0f;

    if (t0 < t1) {
        if constexpr (VEC) {
            att_fetch<NL, DP>(kr4, vr4, K, ldk, V, ldv, t0 * ATT_KT, Nk, d,
                              tid);
            att_stash<NL, DP, KP, VP>(kr4, vr4, Ks[0], Vs[0], tid);
            if (t0 + 1 < t1)
                att_fetch<NL, DP>(kr4, vr4, K, ldk, V, ldv,
                                  (t0 + 1) * ATT_KT, Nk, d, tid);
        }
        else {
            att_stash_direct<NL, DP, KP, VP>(K, ldk, V, ldv, t0 * ATT_KT, Nk,
                                             d, Ks[0], Vs[0], tid);
        }
    }
    __syncthreads();
    for (int t = t0; t < t1; t++) {
        const int k0 = t * ATT_KT, cur = (t - t0) & 1;
        const float *ks = Ks[cur], *vs = Vs[cur];
        floatx16 s;

#pragma unroll
        for (int r = 0; r < 16; r++)
            s[r] = 0.0f;
        {
            /* K operands read ATT_PF steps ahead of their MFMA; the
             * scheduling barriers keep the reads there. */
            const float *kb = ks + col * KP + half;
            float kv[ATT_PF + 1];

#pragma unroll
            for (int st = 0; st < ATT_PF; st++)
                kv[st] = kb[2 * st];
#pragma unroll
            for (int st = 0; st < NS; st++) {
                if (st + ATT_PF < NS)
                    kv[(st + ATT_PF) % (ATT_PF + 1)] = kb[2 * (st + ATT_PF)];
                __builtin_amdgcn_sched_barrier(0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(
                    kv[st % (ATT_PF + 1)], q[st], s, 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }

        /* Scores out of the accumulator into plain registers; keys past
         * Nk (last tile only) or masked out become -inf by a select on a
         * flag computed first (no conditional writes into the accumulator
         * vector). */
        float p[16];
        float mx = -INFINITY;

        if (MASK || k0 + ATT_KT > Nk) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int kk = k0 + (r >> 2) * 8 + half * 4 + (r & 3);
                bool keep = kk < Nk;

                if (MASK)
                    keep = keep && kmask[min(kk, Nk - 1)] != 0;
                p[r] = keep ? s[r] : -INFINITY;
                mx = fmaxf(mx, p[r]);
            }
        }
        else {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                p[r] = s[r];
                mx = fmaxf(mx, p[r]);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        {
            /* Lazy rescaling: the reference maximum m moves only when a
             * tile's maximum exceeds it by more than ATT_TAU (so the
             * probabilities stay below 2^ATT_TAU), and the accumulated
             * output and sum are rescaled only then, by a wave-uniform
             * branch. Output and sum always share the same m, so the
             * normalised result is the same. */
            const bool need = mx > m + ATT_TAU;
            float sum = 0.0f;

            if (__any(need)) {
                const float mn = need ? mx : m;
                const float corr =
                    need ? (m == -INFINITY ? 0.0f
                                           : __builtin_amdgcn_exp2f(m - mn))
                         : 1.0f;

                m = mn;
                l *= corr;
#pragma unroll
                for (int tt = 0; tt < ND; tt++)
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        o[tt][r] *= corr;
            }
            if (m == -INFINITY) {
#pragma unroll
                for (int r = 0; r < 16; r++)
                    p[r] = 0.0f;
            }
            else {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    p[r] = __builtin_amdgcn_exp2f(p[r] - m);
                    sum += p[r];
                }
            }
            sum += __shfl_xor(sum, 32, 64);
            l += sum;
        }

        /* The next tile into the other buffer (last read one tile ago,
         * before the previous barrier), then its successor's loads. */
        if (t + 1 < t1) {
            if constexpr (VEC) {
                att_stash<NL, DP, KP, VP>(kr4, vr4, Ks[cur ^ 1], Vs[cur ^ 1],
                                          tid);
                if (t + 2 < t1)
                    att_fetch<NL, DP>(kr4, vr4, K, ldk, V, ldv,
                                      (t + 2) * ATT_KT, Nk, d, tid);
            }
            else {
                att_stash_direct<NL, DP, KP, VP>(K, ldk, V, ldv,
                                                 (t + 1) * ATT_KT, Nk, d,
                                                 Ks[cur ^ 1], Vs[cur ^ 1],
                                                 tid);
            }
        }

        {
            /* V operands of step r (key (r / 4) * 8 + half * 4 + r % 4)
             * read ATT_PF steps ahead, as for K. */
            const float *vb = vs + half * 4 * VP + col;
            float vv[ATT_PF + 1][ND];
            auto vread = [&](int r, float *v) {
#pragma unroll
                for (int tt = 0; tt < ND; tt++)
                    v[tt] = vb[((r >> 2) * 8 + (r & 3)) * VP + tt * 32];
            };

#pragma unroll
            for (int r = 0; r < ATT_PF; r++)
                vread(r, vv[r]);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                if (r + ATT_PF < 16)
                    vread(r + ATT_PF, vv[(r + ATT_PF) % (ATT_PF + 1)]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int tt = 0; tt < ND; tt++)
                    o[tt] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                        vv[r % (ATT_PF + 1)][tt], p[r], o[tt], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __syncthreads();
    }

    if (qi >= Nq)
        return;
    if (!part_o) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float *out = O + bi * bo + (long long)qi * ldo + (long long)h * d;

#pragma unroll
        for (int tt = 0; tt < ND; tt++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int dd = tt * 32 + (r >> 2) * 8 + half * 4 + (r & 3);

                if (dd < d)
                    out[dd] = l > 0.0f ? o[tt][r] * inv : 0.0f;
            }
    }
    else {
        const long long row =
            ((long long)blockIdx.z * gridDim.y + blockIdx.y) * Nq + qi;
        float *out = part_o + row * DP;

#pragma unroll
        for (int tt = 0; tt < ND; tt++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                out[tt * 32 + (r >> 2) * 8 + half * 4 + (r & 3)] = o[tt][r];
        if (half == 0)
            part_ml[row] = make_float2(m, l);
    }
}

/* Combine nsplit partial results per (image, query, head): weights
 * 2^(m_s - max m) (the maxima are in the base-2 domain), O = sum_s w_s O_s
 * / sum_s w_s l_s (zeros when no key was kept). One thread per output
 * value. */
__global__ void __launch_bounds__(256)
    attn_merge_kernel(const float *__restrict__ part_o,
                      const float2 *__restrict__ part_ml, int nsplit, int nb,
                      int nh, int Nq, int d, int DP, float *__restrict__ O,
                      int ldo, long long bo)
{
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long total = (long long)nb * Nq * nh * d;

    if (idx >= total)
        return;
    const int dd = (int)(idx % d);
    const int h = (int)((idx / d) % nh);
    const long long bq = idx / ((long long)d * nh);
    const int qi = (int)(bq % Nq), bi = (int)(bq / Nq);
    const int y = bi * nh + h, ny = nb * nh;
    float mx = -INFINITY, L = 0.0f, acc = 0.0f;

    for (int s = 0; s < nsplit; s++)
        mx = fmaxf(mx, part_ml[((long long)s * ny + y) * Nq + qi].x);
    if (mx != -INFINITY)
        for (int s = 0; s < nsplit; s++) {
            const long long row = ((long long)s * ny + y) * Nq + qi;
            const float2 ml = part_ml[row];
            const float w =
                ml.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml.x - mx);

            L += w * ml.y;
            acc += w * part_o[row * DP + dd];
        }
    O[bi * bo + (long long)qi * ldo + (long long)h * d + dd] =
        L > 0.0f ? acc / L : 0.0f;
}

/* attn_merge_kernel with four consecutive values of a row per thread
 * (d % 4 == 0, 16-byte aligned output rows): 16-byte loads and stores,
 * the (max, sum) pairs read once per four values. */
__global__ void __launch_bounds__(256)
    attn_merge4_kernel(const float4 *__restrict__ part_o,
                       const float2 *__restrict__ part_ml, int nsplit, int nb,
                       int nh, int Nq, int d, int DP, float *__restrict__ O,
                       int ldo, long long bo)
{
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    const int d4 = d / 4;
    const long long total = (long long)nb * Nq * nh * d4;

    if (idx >= total)
        return;
    const int dq = (int)(idx % d4);
    const int h = (int)((idx / d4) % nh);
    const long long bq = idx / ((long long)d4 * nh);
    const int qi = (int)(bq % Nq), bi = (int)(bq / Nq);
    const int y = bi * nh + h, ny = nb * nh;
    float mx = -INFINITY, L = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);

    for (int s = 0; s < nsplit; s++)
        mx = fmaxf(mx, part_ml[((long long)s * ny + y) * Nq + qi].x);
    if (mx != -INFINITY)
        for (int s = 0; s < nsplit; s++) {
            const long long row = ((long long)s * ny + y) * Nq + qi;
            const float2 ml = part_ml[row];
            const float w =
                ml.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml.x - mx);
            const float4 p = part_o[row * (DP / 4) + dq];

            L += w * ml.y;
            acc.x += w * p.x;
            acc.y += w * p.y;
            acc.z += w * p.z;
            acc.w += w * p.w;
        }
    *(float4 *)(O + bi * bo + (long long)qi * ldo + (long long)h * d + 4 * dq) =
        L > 0.0f ? make_float4(acc.x / L, acc.y / L, acc.z / L, acc.w / L)
                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

/* Partials of the key splits: the ops work buffer (grown on demand), or,
 * for ops_attention_noalloc, the fixed device array `fixed` of
 * fixed_bytes bytes (too small a one is a fatal error). */
template <int ND, bool VEC, bool MASK>
static void launch_nd(struct ops *ops, hipStream_t st, int nb, int nh,
                      const float *Q, int ldq, long long bq, const float *K,
                      int ldk, long long bk, const float *V, int ldv,
                      long long bv, float *O, int ldo, long long bo, int Nq,
                      int Nk, int d, float scale, const unsigned char *kmask,
                      float *fixed, size_t fixed_bytes)
{
    const int qb = (Nq + 32 * ATT_NW - 1) / (32 * ATT_NW);
    const int ntiles = (Nk + ATT_KT - 1) / ATT_KT;
    /* Key splits so that about 8 waves per CU are resident, each split at
     * least 2 key tiles (measured: more splits cost more in the merge
     * than they gain in occupancy). */
    const long long want = 8LL * (ops->ocl->cu_count > 0 ? ops->ocl->cu_count : 256);
    const long long base = (long long)qb * ATT_NW * nh * nb;
    int nsplit = (int)((want + base - 1) / base);
    int tps;

    nsplit = max(1, min(nsplit, min(ntiles / 2, 64)));
    /* With a block or more per CU, the CUs that get one block more than
     * the others set the time: raise the split (at most two steps) until
     * the blocks spread within 10 % of evenly (the ViT's 1601 tokens: 2
     * -> 3 splits, 4.875 blocks per CU instead of 3.25 on 4-block CUs). */
    {
        const long long cus = ops->ocl->cu_count > 0 ? ops->ocl->cu_count : 256;
        const long long qbh = (long long)qb * nh * nb;

        if (qbh * nsplit >= cus)
            for (int s = nsplit; s <= nsplit + 2 && s <= ntiles / 2; s++) {
                const long long blocks = qbh * s;

                if ((blocks + cus - 1) / cus * cus * 10 <= blocks * 11) {
                    nsplit = s;
                    break;
                }
            }
    }
    tps = ntiles > 0 ? (ntiles + nsplit - 1) / nsplit : 0;
    nsplit = tps > 0 ? (ntiles + tps - 1) / tps : 1;
    if (nsplit == 1) {
        hipLaunchKernelGGL((attention_kernel<ND, VEC, MASK>),
                           dim3((unsigned)qb, (unsigned)(nh * nb), 1),
                           dim3(64 * ATT_NW), 0, st, Q, ldq, K, ldk, V, ldv,
                           O, ldo, Nq, Nk, d, scale, kmask, tps, nullptr,
                           nullptr, nh, bq, bk, bv, bo);
        return;
    }
    {
        const size_t rows = (size_t)nsplit * nb * nh * Nq;
        const size_t ob = rows * 32 * ND * sizeof(float);
        float *po;

        if (fixed) {
            if (ob + rows * sizeof(float2) > fixed_bytes)
                icoreg_fatal("ops_attention_noalloc: the key-split partials (%zu bytes) "
                             "exceed the %zu-byte scratch array",
                             ob + rows * sizeof(float2), fixed_bytes);
            po = fixed;
        }
        else
            po = (float *)scratch_get(ops, ob + rows * sizeof(float2))->ptr;
        float2 *pml = (float2 *)((char *)po + ob);
        const long long total = (long long)nb * Nq * nh * d;

        hipLaunchKernelGGL((attention_kernel<ND, VEC, MASK>),
                           dim3((unsigned)qb, (unsigned)(nh * nb),
                                (unsigned)nsplit),
                           dim3(64 * ATT_NW), 0, st, Q, ldq, K, ldk, V, ldv,
                           O, ldo, Nq, Nk, d, scale, kmask, tps, po, pml, nh,
                           bq, bk, bv, bo);
        if (d % 4 == 0 && ldo % 4 == 0 && bo % 4 == 0 && ((uintptr_t)O & 15) == 0)
            hipLaunchKernelGGL(attn_merge4_kernel,
                               dim3((unsigned)((total / 4 + 255) / 256)), dim3(256), 0,
                               st, (const float4 *)po, pml, nsplit, nb, nh, Nq, d, 32 * ND,
                               O, ldo, bo);
        else
            hipLaunchKernelGGL(attn_merge_kernel,
                               dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                               st, po, pml, nsplit, nb, nh, Nq, d, 32 * ND, O, ldo,
                               bo);
    }
}

static void need_rows(const struct opnd &x, int nb, long long bs, int rows,
                      int cols, const char *op, const char *operand)
{
    if (x.off < 0 || x.ld < 0 || bs < 0)
        icoreg_fatal("%s: %s has a negative offset, ld or batch stride", op,
                     operand);
    need_floats(x.buf, x.off + (nb - 1) * bs,
                (long long)(rows - 1) * x.ld + cols, op, operand);
}

/* nb independent problems at batch strides bq .. bo floats (the key mask,
 * when given, is shared by all of them). */
static void attention_impl(struct ops *o, const char *op, int nb,
                           struct opnd Q, long long bq, struct opnd K,
                           long long bk, struct opnd V, long long bv,
                           struct opnd O, long long bo, int Nq, int Nk, int nh,
                           int d, float scale, cl_mem kmask, float *fixed = nullptr,
                           size_t fixed_bytes = 0)
{
    hipStream_t st = stream_of(o->ocl);

    if (d < 1 || d > OPS_MAX_HEAD_DIM)
        icoreg_fatal("HIP: attention head dimension %d not in 1..%d", d,
                     OPS_MAX_HEAD_DIM);
    if (Nq < 0 || Nk < 0 || nh < 1 || nb < 1 || (long long)nh * nb > 65535)
        icoreg_fatal("%s: invalid sizes Nq=%d Nk=%d nh=%d nb=%d", op, Nq, Nk,
                     nh, nb);
    if (Nq == 0)
        return;
    need_rows(Q, nb, bq, Nq, nh * d, op, "Q");
    need_rows(O, nb, bo, Nq, nh * d, op, "O");
    if (Nk > 0) {
        need_rows(K, nb, bk, Nk, nh * d, op, "K");
        need_rows(V, nb, bv, Nk, nh * d, op, "V");
    }
    if (kmask)
        need_bytes(kmask, 0, Nk, op, "kmask");
    prof_scope ps(o->ocl, "attention");
#define ARGS                                                                   \
    o, st, nb, nh, cfptr(Q.buf) + Q.off, Q.ld, bq, cfptr(K.buf) + K.off, K.ld, \
        bk, cfptr(V.buf) + V.off, V.ld, bv, fptr(O.buf) + O.off, O.ld, bo, Nq, \
        Nk, d, scale, kmask ? (const unsigned char *)kmask->ptr : nullptr, fixed,   \
        fixed_bytes
    {
        /* 16-byte K / V loads when every row and head start is aligned. */
        const bool vec = d % 4 == 0 && K.ld % 4 == 0 && V.ld % 4 == 0 &&
                         K.off % 4 == 0 && V.off % 4 == 0 && bk % 4 == 0 &&
                         bv % 4 == 0 && ((uintptr_t)K.buf->ptr & 15) == 0 &&
                         ((uintptr_t)V.buf->ptr & 15) == 0;

#define DISPATCH(ND)                                                           \
    if (kmask)                                                                 \
        vec ? launch_nd<ND, true, true>(ARGS)                                  \
            : launch_nd<ND, false, true>(ARGS);                                \
    else                                                                       \
        vec ? launch_nd<ND, true, false>(ARGS)                                 \
            : launch_nd<ND, false, false>(ARGS)
        if (d <= 32) {
            DISPATCH(1);
        }
        else if (d <= 64) {
            DISPATCH(2);
        }
        else if (d <= 96) {
            DISPATCH(3);
        }
        else {
            DISPATCH(4);
        }
#undef DISPATCH
    }
#undef ARGS
    launch_check("attention");
}

extern "C" void ops_attention(struct ops *o, struct opnd Q, struct opnd K,
                              struct opnd V, struct opnd O, int Nq, int Nk,
                              int nh, int d, float scale, cl_mem kmask)
{
    ICOREG_API_BEGIN
    attention_impl(o, "ops_attention", 1, Q, 0, K, 0, V, 0, O, 0, Nq, Nk, nh,
                   d, scale, kmask);
    ICOREG_API_END
}

/* ---- ops_attention without allocation ------------------------------------------ */

/* The key-split partials of ops_attention_noalloc: a fixed array per
 * GPU, held until the process ends, shared by every call on that GPU.
 * Its device memory is reserved wherever the library's code object is
 * loaded, whether or not the entry point is called, so it is sized to
 * the largest caller on the path: RoMa's ViT attention (1601 tokens, 16
 * heads of 64, 3 key splits) needs 20.3 MB. */
#define ATT_NOALLOC_BYTES ((size_t)24 << 20)
static __device__ __align__(256) float scratch[ATT_NOALLOC_BYTES / sizeof(float)];

/* scratch's device address on each GPU (hipGetSymbolAddress once per
 * device, with that device current); the host symbol is only a
 * stand-in and is never handed to a kernel or a copy. */
static float *scratch_dev[64];
static std::mutex scratch_mu;

static float *noalloc_scratch(void)
{
    int dev = -1;
    float *p;

    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= 64)
        icoreg_fatal("ops_attention_noalloc: device %d out of range", dev);
    std::lock_guard<std::mutex> lk(scratch_mu);
    if (!scratch_dev[dev]) {
        p = nullptr;
        hip_check(hipGetSymbolAddress((void **)&p, HIP_SYMBOL(scratch)),
                  "hipGetSymbolAddress(scratch)");
        if (!p)
            icoreg_fatal("ops_attention_noalloc: no device address for the scratch array");
        scratch_dev[dev] = p;
    }
    return scratch_dev[dev];
}

extern "C" void ops_attention_noalloc(struct ops *o, struct opnd Q, struct opnd K,
                                      struct opnd V, struct opnd O, int Nq, int Nk,
                                      int nh, int d, float scale, cl_mem kmask)
{
    ICOREG_API_BEGIN
    float *p = noalloc_scratch();

    attention_impl(o, "ops_attention_noalloc", 1, Q, 0, K, 0, V, 0, O, 0, Nq, Nk, nh,
                   d, scale, kmask, p, ATT_NOALLOC_BYTES);
    ICOREG_API_END
}

extern "C" void ops_attention_batch(struct ops *o, int nb, struct opnd Q,
                                    long bq, struct opnd K, long bk,
                                    struct opnd V, long bv, struct opnd O,
                                    long bo, int Nq, int Nk, int nh, int d,
                                    float scale, cl_mem kmask)
{
    ICOREG_API_BEGIN
    attention_impl(o, "ops_attention_batch", nb, Q, bq, K, bk, V, bv, O, bo,
                   Nq, Nk, nh, d, scale, kmask);
    ICOREG_API_END
}

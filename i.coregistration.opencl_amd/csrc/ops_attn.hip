/* SPDX-License-Identifier: Unlicense */

/* Blockwise scaled dot-product attention on the fp32 matrix cores:
 * O = softmax(scale Q K^T) V per head, never storing the scores. The
 * contract is the reference's attention kernel (ops.cl:604-687,
 * ops.c:444-474 of i.coregistration.opencl): token-major operands with
 * head h at columns h * d, d <= 128, optional key mask, a query with no
 * key left gets zeros.
 *
 * A block holds 4 waves of 32 queries each (128 queries of one head)
 * and streams its range of keys in tiles of 32 through LDS, shared by
 * the 4 waves; with 16-byte aligned rows the next tile is read into
 * registers while the current one is used:
 *  - the scores are computed transposed, S^T = K Q^T, with
 *    v_mfma_f32_32x32x2f32 (A = K from LDS, B = the wave's queries,
 *    pre-scaled and held in registers for the whole kernel), so that
 *    each lane holds 16 keys of one query (its column);
 *  - the online softmax runs per lane on those registers, the two lane
 *    halves of a query combined with one cross-lane exchange;
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

#include <math.h>

#include "common.h"
#include "ops.h"

using namespace icoreg;

typedef float floatx16 __attribute__((ext_vector_type(16)));

#define ATT_KT 32 /* keys per tile */
#define ATT_NW 4  /* waves per block, 32 queries each */

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

/* One block: 128 queries (4 waves x 32) of one head against the key
 * tiles [t0, t1) of 32 keys; the block's K and V tiles are shared through
 * LDS, the next tile is loaded into registers while the current one is
 * used. With nsplit > 1 (blockIdx.z picks the key range) the
 * unnormalised output and the running (max, sum) go to part_o / part_ml
 * for attn_merge_kernel; with one split the normalised output goes to O
 * directly. */
template <int ND, bool VEC>
__global__ void __launch_bounds__(64 * ATT_NW)
    attention_kernel(const float *__restrict__ Q, int ldq,
                     const float *__restrict__ K, int ldk,
                     const float *__restrict__ V, int ldv,
                     float *__restrict__ O, int ldo, int Nq, int Nk, int d,
                     float scale, const unsigned char *__restrict__ kmask,
                     int tiles_per_split, float *__restrict__ part_o,
                     float2 *__restrict__ part_ml)
{
    constexpr int DP = 32 * ND;     /* padded head dimension */
    constexpr int KP = DP + 1;      /* K tile row pitch (odd: no conflicts) */
    constexpr int VP = DP + 4;      /* V tile row pitch */
    constexpr int NS = DP / 2;      /* score MFMA steps */
    constexpr int NL = VEC ? ATT_KT * DP / 4 / (64 * ATT_NW)
                           : ATT_KT * DP / (64 * ATT_NW); /* loads / thread */
    __shared__ __align__(16) float Ks[ATT_KT * KP];
    __shared__ __align__(16) float Vs[ATT_KT * VP];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.y, half = lane >> 5, col = lane & 31;
    const int qi = (blockIdx.x * ATT_NW + wave) * 32 + col;
    const int ntiles = (Nk + ATT_KT - 1) / ATT_KT;
    const int t0 = blockIdx.z * tiles_per_split;
    const int t1 = min(ntiles, t0 + tiles_per_split);
    float q[NS];
    floatx16 o[ND];
    float m = -INFINITY, l = 0.0f;
    float4 kr4[VEC ? NL : 1], vr4[VEC ? NL : 1];

    Q += (long long)h * d;
    K += (long long)h * d;
    V += (long long)h * d;
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int dd = 2 * s + half;

        q[s] = (qi < Nq && dd < d) ? Q[(long long)qi * ldq + dd] * scale : 0.0f;
    }
#pragma unroll
    for (int t = 0; t < ND; t++)
#pragma unroll
        for (int r = 0; r < 16; r++)
            o[t][r] = 0.0f;

    if constexpr (VEC) {
        if (t0 < t1) {
            att_fetch<NL, DP>(kr4, vr4, K, ldk, V, ldv, t0 * ATT_KT, Nk, d, tid);
        }
    }
    for (int t = t0; t < t1; t++) {
        const int k0 = t * ATT_KT;
        floatx16 s;

        __syncthreads();
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < NL; i++) {
                const int e = tid + 64 * ATT_NW * i, key = e / (DP / 4);
                const int dd = (e - key * (DP / 4)) * 4;
                float *kd = Ks + key * KP + dd;

                kd[0] = kr4[i].x;
                kd[1] = kr4[i].y;
                kd[2] = kr4[i].z;
                kd[3] = kr4[i].w;
                *(float4 *)(Vs + key * VP + dd) = vr4[i];
            }
        }
        else {
            for (int i = 0; i < NL; i++) {
                const int e = tid + 64 * ATT_NW * i, key = e / DP;
                const int dd = e - key * DP, kk = k0 + key;
                const bool ok = kk < Nk && dd < d;

                Ks[key * KP + dd] = ok ? K[(long long)kk * ldk + dd] : 0.0f;
                Vs[key * VP + dd] = ok ? V[(long long)kk * ldv + dd] : 0.0f;
            }
        }
        __syncthreads();
        if constexpr (VEC) {
            if (t + 1 < t1) {
                att_fetch<NL, DP>(kr4, vr4, K, ldk, V, ldv, (t + 1) * ATT_KT, Nk,
                                  d, tid);
            }
        }

#pragma unroll
        for (int r = 0; r < 16; r++)
            s[r] = 0.0f;
#pragma unroll
        for (int st = 0; st < NS; st++)
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(
                Ks[col * KP + 2 * st + half], q[st], s, 0, 0, 0);

        /* Scores out of the accumulator into plain registers; keys past
         * Nk or masked out become -inf by a select on a flag computed
         * first (no conditional writes into the accumulator vector). */
        float p[16];
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int kk = k0 + (r >> 2) * 8 + half * 4 + (r & 3);
            bool keep = kk < Nk;

            if (kmask && keep)
                keep = kmask[kk] != 0;
            p[r] = keep ? s[r] : -INFINITY;
            mx = fmaxf(mx, p[r]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        {
            const float mn = fmaxf(m, mx);
            float corr, sum = 0.0f;

            if (mn == -INFINITY) {
                corr = 1.0f;
#pragma unroll
                for (int r = 0; r < 16; r++)
                    p[r] = 0.0f;
            }
            else {
                corr = m == -INFINITY ? 0.0f : expf(m - mn);
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    p[r] = expf(p[r] - mn);
                    sum += p[r];
                }
                m = mn;
            }
            sum += __shfl_xor(sum, 32, 64);
            l = l * corr + sum;
#pragma unroll
            for (int tt = 0; tt < ND; tt++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    o[tt][r] *= corr;
        }
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = (r >> 2) * 8 + half * 4 + (r & 3);

#pragma unroll
            for (int tt = 0; tt < ND; tt++)
                o[tt] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                    Vs[key * VP + tt * 32 + col], p[r], o[tt], 0, 0, 0);
        }
    }

    if (qi >= Nq)
        return;
    if (!part_o) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float *out = O + (long long)qi * ldo + (long long)h * d;

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
            ((long long)blockIdx.z * gridDim.y + h) * Nq + qi;
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

/* Combine nsplit partial results per (query, head): weights
 * exp(m_s - max m), O = sum_s w_s O_s / sum_s w_s l_s (zeros when no key
 * was kept). One thread per output value. */
__global__ void __launch_bounds__(256)
    attn_merge_kernel(const float *__restrict__ part_o,
                      const float2 *__restrict__ part_ml, int nsplit, int nh,
                      int Nq, int d, int DP, float *__restrict__ O, int ldo)
{
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long total = (long long)Nq * nh * d;

    if (idx >= total)
        return;
    const int dd = (int)(idx % d);
    const int h = (int)((idx / d) % nh);
    const int qi = (int)(idx / ((long long)d * nh));
    float mx = -INFINITY, L = 0.0f, acc = 0.0f;

    for (int s = 0; s < nsplit; s++)
        mx = fmaxf(mx, part_ml[((long long)s * nh + h) * Nq + qi].x);
    if (mx != -INFINITY)
        for (int s = 0; s < nsplit; s++) {
            const long long row = ((long long)s * nh + h) * Nq + qi;
            const float2 ml = part_ml[row];
            const float w = ml.x == -INFINITY ? 0.0f : expf(ml.x - mx);

            L += w * ml.y;
            acc += w * part_o[row * DP + dd];
        }
    O[(long long)qi * ldo + (long long)h * d + dd] = L > 0.0f ? acc / L : 0.0f;
}

template <int ND, bool VEC>
static void launch_nd(struct ops *ops, hipStream_t st, int nh, const float *Q,
                      int ldq, const float *K, int ldk, const float *V, int ldv,
                      float *O, int ldo, int Nq, int Nk, int d, float scale,
                      const unsigned char *kmask)
{
    const int qb = (Nq + 32 * ATT_NW - 1) / (32 * ATT_NW);
    const int ntiles = (Nk + ATT_KT - 1) / ATT_KT;
    /* Key splits so that about 16 waves per CU are resident. */
    const long long want = 16LL * (ops->ocl->cu_count > 0 ? ops->ocl->cu_count : 256);
    const long long base = (long long)qb * ATT_NW * nh;
    int nsplit = (int)((want + base - 1) / base);
    int tps;

    nsplit = max(1, min(nsplit, min(ntiles, 64)));
    tps = ntiles > 0 ? (ntiles + nsplit - 1) / nsplit : 0;
    nsplit = tps > 0 ? (ntiles + tps - 1) / tps : 1;
    if (nsplit == 1) {
        hipLaunchKernelGGL((attention_kernel<ND, VEC>),
                           dim3((unsigned)qb, (unsigned)nh, 1),
                           dim3(64 * ATT_NW), 0, st, Q, ldq, K, ldk, V, ldv,
                           O, ldo, Nq, Nk, d, scale, kmask, tps, nullptr,
                           nullptr);
        return;
    }
    {
        const size_t rows = (size_t)nsplit * nh * Nq;
        const size_t ob = rows * 32 * ND * sizeof(float);
        cl_mem sc = scratch_get(ops, ob + rows * sizeof(float2));
        float *po = (float *)sc->ptr;
        float2 *pml = (float2 *)((char *)sc->ptr + ob);
        const long long total = (long long)Nq * nh * d;

        hipLaunchKernelGGL((attention_kernel<ND, VEC>),
                           dim3((unsigned)qb, (unsigned)nh, (unsigned)nsplit),
                           dim3(64 * ATT_NW), 0, st, Q, ldq, K, ldk, V, ldv,
                           O, ldo, Nq, Nk, d, scale, kmask, tps, po, pml);
        hipLaunchKernelGGL(attn_merge_kernel,
                           dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                           st, po, pml, nsplit, nh, Nq, d, 32 * ND, O, ldo);
    }
}

static void need_rows(const struct opnd &x, int rows, int cols,
                      const char *operand)
{
    if (x.off < 0 || x.ld < 0)
        icoreg_fatal("ops_attention: %s has a negative offset or ld", operand);
    need_floats(x.buf, x.off, (long long)(rows - 1) * x.ld + cols,
                "ops_attention", operand);
}

extern "C" void ops_attention(struct ops *o, struct opnd Q, struct opnd K,
                              struct opnd V, struct opnd O, int Nq, int Nk,
                              int nh, int d, float scale, cl_mem kmask)
{
    ICOREG_API_BEGIN
    hipStream_t st = stream_of(o->ocl);

    if (d < 1 || d > OPS_MAX_HEAD_DIM)
        icoreg_fatal("HIP: attention head dimension %d not in 1..%d", d,
                     OPS_MAX_HEAD_DIM);
    if (Nq < 0 || Nk < 0 || nh < 1 || nh > 65535)
        icoreg_fatal("ops_attention: invalid sizes Nq=%d Nk=%d nh=%d", Nq, Nk,
                     nh);
    if (Nq == 0)
        return;
    need_rows(Q, Nq, nh * d, "Q");
    need_rows(O, Nq, nh * d, "O");
    if (Nk > 0) {
        need_rows(K, Nk, nh * d, "K");
        need_rows(V, Nk, nh * d, "V");
    }
    if (kmask)
        need_bytes(kmask, 0, Nk, "ops_attention", "kmask");
    prof_scope ps(o->ocl, "attention");
#define ARGS                                                                   \
    o, st, nh, cfptr(Q.buf) + Q.off, Q.ld, cfptr(K.buf) + K.off, K.ld,         \
        cfptr(V.buf) + V.off, V.ld, fptr(O.buf) + O.off, O.ld, Nq, Nk, d,     \
        scale, kmask ? (const unsigned char *)kmask->ptr : nullptr
    {
        /* 16-byte K / V loads when every row and head start is aligned. */
        const bool vec = d % 4 == 0 && K.ld % 4 == 0 && V.ld % 4 == 0 &&
                         K.off % 4 == 0 && V.off % 4 == 0 &&
                         ((uintptr_t)K.buf->ptr & 15) == 0 &&
                         ((uintptr_t)V.buf->ptr & 15) == 0;

        if (d <= 32)
            vec ? launch_nd<1, true>(ARGS) : launch_nd<1, false>(ARGS);
        else if (d <= 64)
            vec ? launch_nd<2, true>(ARGS) : launch_nd<2, false>(ARGS);
        else if (d <= 96)
            vec ? launch_nd<3, true>(ARGS) : launch_nd<3, false>(ARGS);
        else
            vec ? launch_nd<4, true>(ARGS) : launch_nd<4, false>(ARGS);
    }
#undef ARGS
    launch_check("attention");
    ICOREG_API_END
}

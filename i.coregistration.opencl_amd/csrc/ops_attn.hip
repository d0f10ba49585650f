/* SPDX-License-Identifier: Unlicense */

/* Blockwise scaled dot-product attention on the fp32 matrix cores:
 * O = softmax(scale Q K^T) V per head, never storing the scores. The
 * contract is the reference's attention kernel (ops.cl:604-687,
 * ops.c:444-474 of i.coregistration.opencl): token-major operands with
 * head h at columns h * d, d <= 128, optional key mask, a query with no
 * key left gets zeros.
 *
 * Each wave owns 32 queries of one head and streams the keys in tiles
 * of 32 through LDS:
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
 *    rows from LDS. No transpose of P through LDS. */

#include <hip/hip_runtime.h>

#include <math.h>

#include "common.h"
#include "ops.h"

using namespace icoreg;

typedef float floatx16 __attribute__((ext_vector_type(16)));

#define ATT_KT 32 /* keys per tile */

template <int ND, int NW>
__global__ void __launch_bounds__(64 * NW)
    attention_kernel(const float *__restrict__ Q, int ldq,
                     const float *__restrict__ K, int ldk,
                     const float *__restrict__ V, int ldv,
                     float *__restrict__ O, int ldo, int Nq, int Nk, int d,
                     float scale, const unsigned char *__restrict__ kmask)
{
    constexpr int DP = 32 * ND;     /* padded head dimension */
    constexpr int KP = DP + 1;      /* K tile row pitch (odd: no conflicts) */
    constexpr int VP = DP + 4;      /* V tile row pitch */
    constexpr int NS = DP / 2;      /* score MFMA steps */
    __shared__ float Ks[ATT_KT * KP];
    __shared__ float Vs[ATT_KT * VP];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.y, half = lane >> 5, col = lane & 31;
    const int q0 = (blockIdx.x * NW + wave) * 32;
    const int qi = q0 + col;
    float q[NS];
    floatx16 o[ND];
    float m = -INFINITY, l = 0.0f;

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

    for (int k0 = 0; k0 < Nk; k0 += ATT_KT) {
        floatx16 s;

        __syncthreads();
        for (int e = tid; e < ATT_KT * DP; e += 64 * NW) {
            const int key = e / DP, dd = e - key * DP, kk = k0 + key;
            const bool ok = kk < Nk && dd < d;

            Ks[key * KP + dd] = ok ? K[(long long)kk * ldk + dd] : 0.0f;
            Vs[key * VP + dd] = ok ? V[(long long)kk * ldv + dd] : 0.0f;
        }
        __syncthreads();

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
            for (int t = 0; t < ND; t++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    o[t][r] *= corr;
        }
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = (r >> 2) * 8 + half * 4 + (r & 3);

#pragma unroll
            for (int t = 0; t < ND; t++)
                o[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                    Vs[key * VP + t * 32 + col], p[r], o[t], 0, 0, 0);
        }
    }

    if (qi < Nq) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float *out = O + (long long)qi * ldo + (long long)h * d;

#pragma unroll
        for (int t = 0; t < ND; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int dd = t * 32 + (r >> 2) * 8 + half * 4 + (r & 3);

                if (dd < d)
                    out[dd] = l > 0.0f ? o[t][r] * inv : 0.0f;
            }
    }
}

template <int ND>
static void launch_nd(hipStream_t st, int nh, const float *Q, int ldq,
                      const float *K, int ldk, const float *V, int ldv,
                      float *O, int ldo, int Nq, int Nk, int d, float scale,
                      const unsigned char *kmask)
{
    dim3 grid((unsigned)((Nq + 31) / 32), (unsigned)nh);

    hipLaunchKernelGGL((attention_kernel<ND, 1>), grid, dim3(64), 0, st, Q, ldq,
                       K, ldk, V, ldv, O, ldo, Nq, Nk, d, scale, kmask);
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
    st, nh, cfptr(Q.buf) + Q.off, Q.ld, cfptr(K.buf) + K.off, K.ld,            \
        cfptr(V.buf) + V.off, V.ld, fptr(O.buf) + O.off, O.ld, Nq, Nk, d,     \
        scale, kmask ? (const unsigned char *)kmask->ptr : nullptr
    if (d <= 32)
        launch_nd<1>(ARGS);
    else if (d <= 64)
        launch_nd<2>(ARGS);
    else if (d <= 96)
        launch_nd<3>(ARGS);
    else
        launch_nd<4>(ARGS);
#undef ARGS
    launch_check("attention");
    ICOREG_API_END
}

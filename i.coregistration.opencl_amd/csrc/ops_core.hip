/* SPDX-License-Identifier: Unlicense */

/* ops_init/free, the GEMM entry points (ops_gemm, ops_linear,
 * ops_conv1x1), the convolution dispatch (ops_conv2d: implicit-GEMM MFMA
 * for one group, a direct kernel for grouped convolutions) and the
 * host-side BatchNorm fold. Host layer of the reference's ops.c:86-336,
 * 612-626 (i.coregistration.opencl): same arguments and errors, HIP
 * launches, and every access checked against its buffer before launch. */

#include <hip/hip_runtime.h>

#include <math.h>
#include <string.h>

#include "act.h"
#include "common.h"
#include "conv.h"
#include "gemm.h"
#include "ops.h"

using namespace icoreg;

extern "C" void ops_init(struct ops *o, struct ocl_backend *ocl)
{
    memset(o, 0, sizeof(*o));
    o->ocl = ocl;
    o->im2col_bytes = (size_t)256 << 20;
}

namespace icoreg {

cl_mem scratch_get(struct ops *o, size_t bytes)
{
    if (bytes <= o->scratch_bytes && o->scratch)
        return o->scratch;
    hip_check(hipStreamSynchronize(stream_of(o->ocl)), "hipStreamSynchronize");
    ocl_release(&o->scratch);
    bytes = (bytes + 0xfffff) & ~(size_t)0xfffff;
    o->scratch = ocl_alloc(o->ocl, bytes, "ops scratch");
    o->scratch_bytes = bytes;
    return o->scratch;
}

} // namespace icoreg

extern "C" void ops_free(struct ops *o)
{
    if (!o->ocl)
        return;
    ocl_release(&o->scratch);
    memset(o, 0, sizeof(*o));
}

extern "C" struct opnd ops_mat(cl_mem buf, long off, int ld)
{
    struct opnd m = {buf, off, ld, 0, 0};

    return m;
}

extern "C" struct opnd ops_bmat(cl_mem buf, long off, int ld, long s0, long s1)
{
    struct opnd m = {buf, off, ld, s0, s1};

    return m;
}

extern "C" struct conv_geom ops_geom(int k, int s, int p)
{
    struct conv_geom g = {k, k, s, s, p, p, 1, 1, 1};

    return g;
}

extern "C" int ops_conv_out(int n, int k, int s, int p, int d)
{
    return (n + 2 * p - d * (k - 1) - 1) / s + 1;
}

/* Largest b0 * s0 + b1 * s1 over batches b < nb (b0 = b / nb1, b1 =
 * b % nb1), strides non-negative. */
static long long max_batch_off(int nb, int nb1, long long s0, long long s1)
{
    long long b0max = (nb - 1) / nb1, v;

    v = b0max * s0 + (long long)((nb - 1) % nb1) * s1;
    if (b0max >= 1) {
        long long w = (b0max - 1) * s0 + (long long)(nb1 - 1) * s1;

        if (w > v)
            v = w;
    }
    return v;
}

/* Check a rows x cols operand with leading dimension ld from element
 * off, over the batches. */
static void need_matrix(cl_mem b, long long off, long long ld, long long s0,
                        long long s1, int rows, int cols, int nb, int nb1,
                        const char *op, const char *operand)
{
    long long span;

    if (rows <= 0 || cols <= 0)
        return;
    if (ld < 0 || s0 < 0 || s1 < 0 || off < 0)
        icoreg_fatal("%s: %s has a negative offset, stride or leading "
                     "dimension",
                     op, operand);
    span = (long long)(rows - 1) * ld + cols;
    need_floats(b, off, max_batch_off(nb, nb1, s0, s1) + span, op, operand);
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

static bool vec_ok(const struct opnd &x)
{
    return x.buf && aligned16(x.buf->ptr) && x.ld % 4 == 0 && x.off % 4 == 0 &&
           x.s0 % 4 == 0 && x.s1 % 4 == 0;
}

/* ops_gemm's checks and kernel arguments (M, N > 0). */
static gemm_args gemm_make(const char *op, int M, int N, int K, struct opnd A, struct opnd B,
                           int transb, struct opnd C, int nb, int nb1, cl_mem bias,
                           int biasrow, cl_mem R, long roff, float alpha, int act, float slope)
{
    gemm_args g;

    need_matrix(A.buf, A.off, A.ld, A.s0, A.s1, M, K, nb, nb1, op, "A");
    if (transb)
        need_matrix(B.buf, B.off, B.ld, B.s0, B.s1, N, K, nb, nb1, op, "B");
    else
        need_matrix(B.buf, B.off, B.ld, B.s0, B.s1, K, N, nb, nb1, op, "B");
    need_matrix(C.buf, C.off, C.ld, C.s0, C.s1, M, N, nb, nb1, op, "C");
    if (R)
        need_matrix(R, roff, C.ld, C.s0, C.s1, M, N, nb, nb1, op, "R");
    if (bias)
        need_floats(bias, 0, biasrow ? M : N, op, "bias");
    count32((long long)M * N, "gemm output");

    memset(&g, 0, sizeof(g));
    g.M = M;
    g.N = N;
    g.K = K;
    g.A = cfptr(A.buf) + A.off;
    g.lda = A.ld;
    g.sa0 = A.s0;
    g.sa1 = A.s1;
    g.B = cfptr(B.buf) + B.off;
    g.ldb = B.ld;
    g.sb0 = B.s0;
    g.sb1 = B.s1;
    g.C = fptr(C.buf) + C.off;
    g.ldc = C.ld;
    g.sc0 = C.s0;
    g.sc1 = C.s1;
    g.R = R ? cfptr(R) + roff : nullptr;
    g.nb1 = nb1;
    g.bias = cfptr(bias);
    g.biasrow = biasrow;
    g.alpha = alpha;
    g.act = act;
    g.slope = slope;
    if (!gemm_shape_ok(g, transb ? GEMM_B_NK : GEMM_B_KN))
        icoreg_fatal("%s: leading dimensions lda=%d ldb=%d not supported "
                     "(each at least its row length, below 4 Mi floats)",
                     op, A.ld, B.ld);
    return g;
}

extern "C" void ops_gemm(struct ops *o, int M, int N, int K, struct opnd A,
                         struct opnd B, int transb, struct opnd C, int nb,
                         int nb1, cl_mem bias, int biasrow, cl_mem R, long roff,
                         float alpha, int act, float slope)
{
    ICOREG_API_BEGIN
    const char *op = "ops_gemm";

    if (M < 0 || N < 0 || K < 0 || nb < 1 || nb1 < 1 || nb > 65535)
        icoreg_fatal("%s: invalid sizes M=%d N=%d K=%d nb=%d nb1=%d", op, M, N,
                     K, nb, nb1);
    if (act < ACT_NONE || act > ACT_GELU_TANH)
        icoreg_fatal("%s: unknown activation %d", op, act);
    if (M == 0 || N == 0)
        return;
    {
        const int bmode = transb ? GEMM_B_NK : GEMM_B_KN;
        gemm_args g = gemm_make(op, M, N, K, A, B, transb, C, nb, nb1, bias, biasrow, R, roff,
                                alpha, act, slope);
        /* Partial sums of cut tiles, when the grid leaves CUs uneven. */
        const size_t pf = gemm_split_floats(g, bmode, nb, vec_ok(A), vec_ok(B), o->ocl->cu_count);

        if (pf)
            g.part = fptr(scratch_get(o, pf * sizeof(float)));
        prof_scope ps(o->ocl, "gemm");
        gemm_launch(g, bmode, nb, vec_ok(A), vec_ok(B), o->ocl->cu_count, stream_of(o->ocl));
        launch_check("gemm");
    }
    ICOREG_API_END
}

void ops_linear2_rope(struct ops *o, int rows, int in, cl_mem X1, cl_mem W1, cl_mem Y1, int n1,
                      int rc1, cl_mem X2, cl_mem W2, cl_mem Y2, int n2, int rc2, cl_mem cs,
                      int rd, int npos)
{
    const char *op = "ops_linear2_rope";
    const int cus = o->ocl->cu_count;

    if (rows < 1 || in < 1 || n1 < 1 || n2 < 1 || rd < 2 || rd % 2 || npos < 1 || rc1 < 0 ||
        rc2 < 0 || rc1 % rd || rc2 % rd || rc1 > n1 || rc2 > n2)
        icoreg_fatal("%s: invalid sizes rows=%d in=%d n1=%d n2=%d rc1=%d rc2=%d rd=%d", op, rows,
                     in, n1, n2, rc1, rc2, rd);
    if (rc1 || rc2)
        need_floats(cs, 0, (long long)(rows < npos ? rows : npos) * rd, op, "cs");
    {
        const struct opnd x1 = ops_mat(X1, 0, in), w1 = ops_mat(W1, 0, in);
        const struct opnd x2 = ops_mat(X2, 0, in), w2 = ops_mat(W2, 0, in);
        gemm_args g1 = gemm_make(op, rows, n1, in, x1, w1, 1, ops_mat(Y1, 0, n1), 1, 1, NULL, 0,
                                 NULL, 0, 1.0f, ACT_NONE, 0.0f);
        gemm_args g2 = gemm_make(op, rows, n2, in, x2, w2, 1, ops_mat(Y2, 0, n2), 1, 1, NULL, 0,
                                 NULL, 0, 1.0f, ACT_NONE, 0.0f);

        if (gemm_smallk_ok(g1, GEMM_B_NK, 1, vec_ok(x1), vec_ok(w1), cus) &&
            gemm_smallk_ok(g2, GEMM_B_NK, 1, vec_ok(x2), vec_ok(w2), cus)) {
            g1.rope = rc1 ? (const float2 *)cfptr(cs) : nullptr;
            g1.rcols = rc1;
            g2.rope = rc2 ? (const float2 *)cfptr(cs) : nullptr;
            g2.rcols = rc2;
            g1.rd = g2.rd = rd;
            g1.rnpos = g2.rnpos = npos;
            prof_scope ps(o->ocl, "gemm");
            gemm_launch_smallk2(g1, g2, stream_of(o->ocl));
            launch_check("gemm");
            return;
        }
    }
    ops_linear(o, rows, in, n1, X1, 0, W1, NULL, Y1, 0, ACT_NONE, 0.0f, 0);
    ops_linear(o, rows, in, n2, X2, 0, W2, NULL, Y2, 0, ACT_NONE, 0.0f, 0);
    if (rc1)
        ops_rope(o, Y1, 0, n1, rows, rc1 / rd, rd, npos, cs, 1);
    if (rc2)
        ops_rope(o, Y2, 0, n2, rows, rc2 / rd, rd, npos, cs, 1);
}

void ops_gemm_upres(struct ops *o, int M, int N, int K, struct opnd A,
                    struct opnd B, struct opnd C, int nb, cl_mem R,
                    long rstride, int rh, int rw, int H, int W, int up, int pre,
                    int act, float slope)
{
    const char *op = "ops_gemm_upres";
    gemm_args g;

    if (M < 1 || N < 1 || K < 1 || nb < 1 || nb > 65535 || rh < 1 || rw < 1 ||
        H < 1 || W < 1 || (up != 2 && up != 4) || (long long)H * W != N ||
        rstride < (long long)M * rh * rw)
        icoreg_fatal("%s: invalid sizes M=%d N=%d K=%d rh=%d rw=%d H=%d W=%d up=%d nb=%d",
                     op, M, N, K, rh, rw, H, W, up, nb);
    need_matrix(A.buf, A.off, A.ld, A.s0, A.s1, M, K, nb, 1, op, "A");
    need_matrix(B.buf, B.off, B.ld, B.s0, B.s1, K, N, nb, 1, op, "B");
    need_matrix(C.buf, C.off, C.ld, C.s0, C.s1, M, N, nb, 1, op, "C");
    need_floats(R, 0, (long long)(nb - 1) * rstride + (long long)M * rh * rw, op, "R");
    if (C.ld != N)
        icoreg_fatal("%s: C rows must be whole planes (ld %lld, N %d)", op, (long long)C.ld, N);
    count32((long long)M * N, "gemm output");

    memset(&g, 0, sizeof(g));
    g.M = M;
    g.N = N;
    g.K = K;
    g.A = cfptr(A.buf) + A.off;
    g.lda = A.ld;
    g.sa0 = A.s0;
    g.B = cfptr(B.buf) + B.off;
    g.ldb = B.ld;
    g.sb0 = B.s0;
    g.C = fptr(C.buf) + C.off;
    g.ldc = C.ld;
    g.sc0 = C.s0;
    g.nb1 = 1;
    g.alpha = 1.0f;
    g.act = act;
    g.slope = slope;
    g.R = cfptr(R);
    g.rup = up;
    g.rpre = pre != 0;
    g.rsc = 1.0f / (float)up;
    g.rh = rh;
    g.rw = rw;
    g.rwo = W;
    g.rs0 = rstride;
    if (!gemm_shape_ok(g, GEMM_B_KN))
        icoreg_fatal("%s: leading dimensions not supported", op);
    {
        prof_scope ps(o->ocl, "gemm");

        gemm_launch(g, GEMM_B_KN, nb, vec_ok(A), vec_ok(B), o->ocl->cu_count,
                    stream_of(o->ocl));
        launch_check("gemm");
    }
}

extern "C" void ops_linear(struct ops *o, int rows, int in, int out, cl_mem X,
                           long xoff, cl_mem W, cl_mem b, cl_mem Y, long yoff,
                           int act, float slope, int residual)
{
    ICOREG_API_BEGIN
    ops_gemm(o, rows, out, in, ops_mat(X, xoff, in), ops_mat(W, 0, in), 1,
             ops_mat(Y, yoff, out), 1, 1, b, 0, residual ? Y : NULL, yoff, 1.0f,
             act, slope);
    ICOREG_API_END
}

extern "C" void ops_conv1x1(struct ops *o, cl_mem X, long xoff, int C, int HW,
                            cl_mem W, cl_mem b, int K, cl_mem Y, long yoff,
                            int act, float slope)
{
    ICOREG_API_BEGIN
    ops_gemm(o, K, HW, C, ops_mat(W, 0, C), ops_mat(X, xoff, HW), 0,
             ops_mat(Y, yoff, HW), 1, 1, b, 1, NULL, 0, 1.0f, act, slope);
    ICOREG_API_END
}

/* Grouped (or general) convolution, one thread per output value: the
 * contract of the reference's conv2d (ops.cl:389-448), used here for
 * groups > 1 only (ELoFTR's depthwise 4 x 4 / stride 4 aggregation). */
__global__ void __launch_bounds__(256)
    conv2d_direct(const float *__restrict__ in, int C, int H, int W,
                  const float *__restrict__ wt, const float *__restrict__ bias,
                  int K, int Ho, int Wo, int kh, int kw, int sy, int sx, int py,
                  int px, int dy, int dx, int groups,
                  const float *__restrict__ mean, const float *__restrict__ rstd,
                  const float *__restrict__ alpha, int act, float slope,
                  float *__restrict__ out)
{
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long total = (long long)K * Ho * Wo;
    int x, y, k, cg, kg, c0;
    const float *w;
    float acc = 0.0f;

    if (idx >= total)
        return;
    x = (int)(idx % Wo);
    y = (int)((idx / Wo) % Ho);
    k = (int)(idx / ((long long)Wo * Ho));
    cg = C / groups;
    kg = K / groups;
    c0 = (k / kg) * cg;
    w = wt + (long long)k * cg * kh * kw;
    for (int c = 0; c < cg; c++) {
        const float *src = in + (long long)(c0 + c) * H * W;
        float m = 0.0f, r = 1.0f, a = 1.0f;

        if (mean) {
            m = mean[c0 + c];
            r = rstd[c0 + c];
            if (alpha)
                a = alpha[c0 + c];
        }
        for (int i = 0; i < kh; i++) {
            const int iy = y * sy - py + i * dy;

            if (iy < 0 || iy >= H)
                continue;
            for (int j = 0; j < kw; j++) {
                const int ix = x * sx - px + j * dx;
                float v;

                if (ix < 0 || ix >= W)
                    continue;
                v = src[(long long)iy * W + ix];
                if (mean) {
                    v = (v - m) * r;
                    v = v >= 0.0f ? v : a * v;
                }
                acc = fmaf(v, w[(c * kh + i) * kw + j], acc);
            }
        }
    }
    if (bias)
        acc += bias[k];
    out[idx] = icoreg_act(acc, act, slope);
}

/* Which Winograd form a convolution takes (icoreg_conv_wino_form): 0 the
 * shape's choice, 2 or 4 the F(2 x 2) or F(4 x 4) form wherever it
 * applies. Process-wide; for tests and measurements. */
static int g_wino_form = 0;

extern "C" void icoreg_conv_wino_form(int form)
{
    g_wino_form = form == 2 || form == 4 ? form : 0;
}

/* F(4 x 4) where its kernel applies: channels in slices of 4, rows of
 * 16-byte aligned 4-float chunks (the input patch arrives by 16-byte LDS
 * DMA), byte offsets within an image below 2^31. */
static bool wino4_applies(const conv_args &a)
{
    return conv_wino4_ok(a.C, a.K, a.mean != nullptr) && a.W % 4 == 0 &&
           a.in_stride % 4 == 0 && ((unsigned long long)(size_t)a.in & 15) == 0 &&
           (long long)a.C * a.H * a.W * 4 < (1LL << 31);
}

/* The shape's choice: F(4 x 4) where its launch gives every CU a block
 * (32 output channels x 32 tiles of 4 x 4); with fewer blocks than CUs
 * (ELoFTR's 80 x 80 layers: 240 blocks) a CU runs one wave a SIMD and
 * F(2 x 2), whose smaller blocks fill the GPU, was faster. */
static bool wino4_chosen(const conv_args &a, int nb, int cus)
{
    if (g_wino_form == 2 || !wino4_applies(a))
        return false;
    if (g_wino_form == 4)
        return true;
    return conv_wino4_units(a.K, a.Ho, a.Wo, nb) >= cus;
}

/* The Winograd form conv_impl gives a 3 x 3, stride 1, padding 1
 * convolution of nb images of C x H x W (contiguous, 16-byte aligned) to
 * K channels without input normalisation on this device: 4, 2, or 0 (not
 * a Winograd shape). */
extern "C" int icoreg_conv_wino_choice(struct ops *o, int nb, int C, int H, int W, int K)
{
    conv_args a = {};

    if (!o || nb < 1 || !conv_wino_supported(3, 3, 1, 1, 1, 1, 1, 1, 1, C, K, H, W))
        return 0;
    a.in = reinterpret_cast<const float *>(static_cast<uintptr_t>(256));
    a.in_stride = (long long)C * H * W;
    a.C = C;
    a.H = a.Ho = H;
    a.W = a.Wo = W;
    a.K = K;
    return wino4_chosen(a, nb, o->ocl->cu_count) ? 4 : 2;
}

/* ops_conv2d over nb images (in_stride / out_stride floats apart). */
/* U: the filters already in Winograd form (conv_wino_prepare) or NULL. */
static void conv_impl(struct ops *o, int nb, cl_mem in, long long in_stride,
                      int C, int H, int W, cl_mem w, cl_mem b, int K,
                      const struct conv_geom *g, cl_mem mean, cl_mem rstd,
                      cl_mem alpha, int act, float slope, cl_mem out,
                      long long out_stride, cl_mem U = nullptr)
{
    const char *op = "ops_conv2d";
    int Ho, Wo, cg;

    if (g->groups < 1 || C % g->groups || K % g->groups)
        icoreg_fatal("HIP: %d -> %d channels in %d groups", C, K, g->groups);
    if (g->kh < 1 || g->kw < 1 || g->sy < 1 || g->sx < 1 || g->dy < 1 ||
        g->dx < 1 || g->py < 0 || g->px < 0)
        icoreg_fatal("%s: invalid window geometry", op);
    if (act < ACT_NONE || act > ACT_GELU_TANH)
        icoreg_fatal("%s: unknown activation %d", op, act);
    if (mean && !rstd)
        icoreg_fatal("%s: mean given without rstd", op);
    if (nb < 1 || nb > 65535 || in_stride < 0 || out_stride < 0)
        icoreg_fatal("%s: invalid batch (%d images)", op, nb);
    Ho = ops_conv_out(H, g->kh, g->sy, g->py, g->dy);
    Wo = ops_conv_out(W, g->kw, g->sx, g->px, g->dx);
    if (Ho < 1 || Wo < 1 || C < 1 || K < 1)
        icoreg_fatal("%s: empty convolution (%d x %d output)", op, Ho, Wo);
    count32((long long)C * H * W, "convolution input");
    count32((long long)K * Ho * Wo, "convolution output");
    cg = C / g->groups;
    need_floats(in, 0, (long long)(nb - 1) * in_stride + (long long)C * H * W,
                op, "input");
    need_floats(w, 0, (long long)K * cg * g->kh * g->kw, op, "weights");
    need_floats(out, 0,
                (long long)(nb - 1) * out_stride + (long long)K * Ho * Wo, op,
                "output");
    if (b)
        need_floats(b, 0, K, op, "bias");
    if (mean) {
        need_floats(mean, 0, C, op, "mean");
        need_floats(rstd, 0, C, op, "rstd");
        if (alpha)
            need_floats(alpha, 0, C, op, "alpha");
    }
    if (conv_wino_supported(g->kh, g->kw, g->sy, g->sx, g->py, g->px, g->dy,
                            g->dx, g->groups, C, K, Ho, Wo) &&
        conv_direct_fits((long long)C * H * W,
                         (long long)conv_wino_weight_floats(K, C, mean != nullptr))) {
        /* 3 x 3, stride 1, same size: Winograd F(2 x 2, 3 x 3). */
        conv_args a;

        a.in = cfptr(in);
        a.w = nullptr;
        a.bias = cfptr(b);
        a.out = fptr(out);
        a.in_stride = in_stride;
        a.out_stride = out_stride;
        a.C = C;
        a.H = H;
        a.W = W;
        a.K = K;
        a.Ho = Ho;
        a.Wo = Wo;
        a.pad = 1;
        a.mean = cfptr(mean);
        a.rstd = cfptr(rstd);
        a.gate = mean ? cfptr(alpha) : nullptr;
        a.act = act;
        a.slope = slope;
        a.split = 1;
        a.part = nullptr;
        if (wino4_chosen(a, nb, o->ocl->cu_count) &&
            (!U || U->bytes >= (conv_wino4_offset(K, C) + conv_wino4_weight_floats(K, C)) *
                                   sizeof(float))) {
            /* F(4 x 4, 3 x 3): the prepared filters' second form, or the
             * filters transformed into scratch. */
            const float *U4;

            if (U)
                U4 = cfptr(U) + conv_wino4_offset(K, C);
            else {
                cl_mem sc = scratch_get(o, conv_wino4_weight_floats(K, C) * sizeof(float));

                prof_scope ps(o->ocl, "conv_wino_weights");
                conv_wino4_weights(cfptr(w), K, C, fptr(sc), stream_of(o->ocl));
                launch_check("conv_wino_weights");
                U4 = cfptr(sc);
            }
            prof_scope ps(o->ocl, "conv_wino4");
            conv_wino4_launch(a, U4, nb, stream_of(o->ocl));
            launch_check("conv_wino4");
            return;
        }
        wino_split sp = conv_wino_plan(a, nb, o->ocl->cu_count);
        const size_t pb = conv_wino_part_floats(a, nb, sp) * sizeof(float);
        const float *Uf;

        if (!U) {
            /* Filters, then the split pieces' partial sums, in scratch. */
            const size_t ub = (conv_wino_weight_floats(K, C, mean != nullptr) *
                                   sizeof(float) + 255) & ~(size_t)255;
            cl_mem sc = scratch_get(o, ub + pb);

            Uf = cfptr(sc);
            sp.part = pb ? (float *)((char *)sc->ptr + ub) : nullptr;
            prof_scope ps(o->ocl, "conv_wino_weights");
            conv_wino_weights(cfptr(w), K, C, mean != nullptr, fptr(sc),
                              stream_of(o->ocl));
            launch_check("conv_wino_weights");
        }
        else {
            Uf = cfptr(U);
            sp.part = pb ? fptr(scratch_get(o, pb)) : nullptr;
            /* Prepared filters are in the order of a convolution without
             * input normalisation. */
            if (mean)
                icoreg_fatal("%s: prepared Winograd filters with input "
                             "normalisation", op);
            need_floats(U, 0, (long long)conv_wino_weight_floats(K, C, false),
                        op, "Winograd filters");
        }
        prof_scope ps(o->ocl, "conv_wino");
        conv_wino_launch(a, Uf, nb, sp, stream_of(o->ocl));
        launch_check("conv_wino");
        return;
    }
    if (conv_direct_supported(g->kh, g->kw, g->sy, g->sx, g->dy, g->dx,
                              g->groups) &&
        g->py == g->px &&
        conv_direct_fits((long long)C * H * W,
                         (long long)K * C * g->kh * g->kw)) {
        conv_args a;

        a.in = cfptr(in);
        a.w = cfptr(w);
        a.bias = cfptr(b);
        a.out = fptr(out);
        a.in_stride = in_stride;
        a.out_stride = out_stride;
        a.C = C;
        a.H = H;
        a.W = W;
        a.K = K;
        a.Ho = Ho;
        a.Wo = Wo;
        a.pad = g->py;
        a.mean = cfptr(mean);
        a.rstd = cfptr(rstd);
        a.gate = mean ? cfptr(alpha) : nullptr;
        a.act = act;
        a.slope = slope;
        a.split = 1;
        a.part = nullptr;
        {
            const size_t pb = conv_direct_part_bytes(a, g->kh, g->sy, nb, o->ocl->cu_count);

            if (pb)
                a.part = fptr(scratch_get(o, pb));
        }
        prof_scope ps(o->ocl, "conv_direct");
        conv_direct_launch(a, g->kh, g->sy, nb, o->ocl->cu_count,
                           stream_of(o->ocl));
        launch_check("conv_direct");
        return;
    }
    if (g->groups == 1) {
        gemm_args a;
        int kred = C * g->kh * g->kw;

        count32((long long)kred * 128, "convolution reduction");
        memset(&a, 0, sizeof(a));
        a.M = K;
        a.N = Ho * Wo;
        a.K = kred;
        a.A = cfptr(w);
        a.lda = kred;
        a.B = cfptr(in);
        a.sb0 = in_stride;
        a.C = fptr(out);
        a.ldc = (long long)Ho * Wo;
        a.sc0 = out_stride;
        a.nb1 = 1;
        a.bias = cfptr(b);
        a.biasrow = 1;
        a.alpha = 1.0f;
        a.act = act;
        a.slope = slope;
        a.cc = C;
        a.ch = H;
        a.cw = W;
        a.kh = g->kh;
        a.kw = g->kw;
        a.sy = g->sy;
        a.sx = g->sx;
        a.py = g->py;
        a.px = g->px;
        a.dy = g->dy;
        a.dx = g->dx;
        a.wo = Wo;
        a.mean = cfptr(mean);
        a.rstd = cfptr(rstd);
        a.gate = mean ? cfptr(alpha) : nullptr;
        if (!gemm_shape_ok(a, GEMM_B_CONV))
            icoreg_fatal("%s: reduction of %d too long", op, kred);
        prof_scope ps(o->ocl, "conv_igemm");
        gemm_launch(a, GEMM_B_CONV, nb,
                    kred % 4 == 0 && aligned16(w->ptr), false,
                    o->ocl->cu_count, stream_of(o->ocl));
        launch_check("conv_igemm");
        return;
    }
    for (int i = 0; i < nb; i++) {
        long long total = (long long)K * Ho * Wo;
        prof_scope ps(o->ocl, "conv2d_direct");

        hipLaunchKernelGGL(conv2d_direct, dim3((unsigned)((total + 255) / 256)),
                           dim3(256), 0, stream_of(o->ocl),
                           cfptr(in) + i * in_stride, C, H, W, cfptr(w),
                           cfptr(b), K, Ho, Wo, g->kh, g->kw, g->sy, g->sx,
                           g->py, g->px, g->dy, g->dx, g->groups, cfptr(mean),
                           cfptr(rstd), cfptr(alpha), act, slope,
                           fptr(out) + i * out_stride);
        launch_check("conv2d_direct");
    }
}

extern "C" void ops_conv2d(struct ops *o, cl_mem in, int C, int H, int W,
                           cl_mem w, cl_mem b, int K,
                           const struct conv_geom *g, cl_mem mean, cl_mem rstd,
                           cl_mem alpha, int act, float slope, cl_mem out)
{
    ICOREG_API_BEGIN
    conv_impl(o, 1, in, 0, C, H, W, w, b, K, g, mean, rstd, alpha, act, slope,
              out, 0);
    ICOREG_API_END
}

extern "C" void ops_conv2d_batch(struct ops *o, int nb, cl_mem in,
                                 long in_stride, int C, int H, int W,
                                 cl_mem w, cl_mem b, int K,
                                 const struct conv_geom *g, cl_mem mean,
                                 cl_mem rstd, cl_mem alpha, int act,
                                 float slope, cl_mem out, long out_stride)
{
    ICOREG_API_BEGIN
    conv_impl(o, nb, in, in_stride, C, H, W, w, b, K, g, mean, rstd, alpha, act,
              slope, out, out_stride);
    ICOREG_API_END
}

size_t conv_wino4_offset(int K, int C)
{
    return (conv_wino_weight_floats(K, C, false) + 63) & ~(size_t)63;
}

cl_mem conv_wino_prepare(struct ops *o, cl_mem w, int K, int C)
{
    const bool f4 = conv_wino4_ok(C, K, false);
    size_t n = conv_wino_weight_floats(K, C, false);
    cl_mem U;

    need_floats(w, 0, (long long)K * C * 9, "conv_wino_prepare", "weights");
    if (f4)
        n = conv_wino4_offset(K, C) + conv_wino4_weight_floats(K, C);
    U = ocl_alloc(o->ocl, n * sizeof(float), "Winograd filters");
    conv_wino_weights(cfptr(w), K, C, false, fptr(U), stream_of(o->ocl));
    if (f4)
        conv_wino4_weights(cfptr(w), K, C, fptr(U) + conv_wino4_offset(K, C),
                           stream_of(o->ocl));
    launch_check("conv_wino_weights");
    return U;
}

void conv3x3_wino_batch(struct ops *o, int nb, cl_mem in, long in_stride,
                        int C, int H, int W, cl_mem w, cl_mem U, cl_mem b,
                        int K, int act, float slope, cl_mem out,
                        long out_stride)
{
    const struct conv_geom g = {3, 3, 1, 1, 1, 1, 1, 1, 1};

    conv_impl(o, nb, in, in_stride, C, H, W, w, b, K, &g, nullptr, nullptr,
              nullptr, act, slope, out, out_stride, U);
}

extern "C" void ops_fold_bn(float *w, float *b, int K, long per,
                            const float *gamma, const float *beta,
                            const float *mean, const float *var, float eps)
{
    for (int k = 0; k < K; k++) {
        const double s = gamma[k] / sqrt((double)var[k] + eps);

        for (long i = 0; i < per; i++)
            w[(size_t)k * per + i] = (float)(w[(size_t)k * per + i] * s);
        b[k] = (float)((b[k] - mean[k]) * s + beta[k]);
    }
}

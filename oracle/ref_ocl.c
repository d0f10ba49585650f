/* SPDX-License-Identifier: Unlicense */

/* ORACLE — test and measurement infrastructure only (bench.py's
 * baseline leg, tests/test_reference_kernels_gpu.py): the reference's own
 * OpenCL kernels on the MI355X. oracle/Makefile compiles ops.cl,
 * roma_kernels.cl, eloftr_kernels.cl and disk_kernels.cl of
 * i.coregistration.opencl, where they lie, to gfx950 code objects in
 * oracle/_ref/ (clang, the options of ocl_backend.c:166-187); this
 * program loads them through the ROCm OpenCL runtime and launches
 * kernels with the argument conventions and work sizes of the
 * reference's host dispatch (ops.c, roma.c, eloftr.c, disk.c). Timing
 * cases time each case with OpenCL profiling events, check a sample of
 * outputs against a double-precision recomputation (so that a mis-set
 * argument cannot pass as a timing), and print one JSON line per case.
 *
 *   ref_ocl DIR CASE...
 *   CASE: gemm:M:N:K:transb      ops_gemm (ops.c:148-188), one product
 *         vitblock:N             roma.c:675-713: DINOv2's block schedule
 *                                (1024 wide, 16 heads) on one image
 *         attention:Nq:Nk:nh:d   ops_attention (ops.c:443-474)
 *         localcorr:C:h:w:r      roma_local_corr as roma.c:956-968
 *         warpsample:C:h:w       roma_warp_sample as roma.c:936-945
 *         gridsample:C:H:W:n     ops_grid_sample (ops.c:520-534); with
 *                                n = H W the points of a smooth warp
 *
 * Parity cases: the reference's kernels on inputs given as raw files
 * (written by a test, which runs this library's kernels on the same
 * inputs), outputs written as raw files:
 *         coarse:n:blk:S:OUT     eloftr_row_lse / col_lse / conf_row /
 *                                conf_col over row blocks of blk rows of
 *                                the n x n scores S, the schedule of
 *                                eloftr.c:485-548; OUT: row_max (n
 *                                floats), row_arg, col_arg (n ints each),
 *                                col_max (n floats)
 *         nms:h:w:W:off:thresh:HEAT:OUT   nms5x5 as disk.c:209-222 on
 *                                HEAT (off + h W floats); OUT: h w bytes
 *         gather:H:W:D:n:FEAT:XY:OUT      gather_desc as disk.c:255-268;
 *                                FEAT (D + 1) H W floats, XY 2 n ints;
 *                                OUT: n D floats
 *         cls:n:ld:C:res:L:OUT   roma_cls_to_flow as roma.c:898-919 on
 *                                L (n ld floats); OUT: flow (2 n floats),
 *                                cert (n floats)
 *         gemmx:M:N:K:transb:act:A:B:BIAS:OUT   ops_gemm, C = act(A B +
 *                                bias), A M x K, B K x N (N x K when
 *                                transb); OUT: M N floats
 *         lnx:rows:C:eps:X:G:BETA:OUT           ops_layernorm
 *         smx:rows:L:scale:S:OUT                ops_softmax_rows
 *         attnx:Nq:Nk:nh:d:scale:Q:K:V:OUT      ops_attention, rows of
 *                                nh d floats, no key mask
 *         lcx:C:h:w:r:F1:F2:FLOW:OUT            roma_local_corr
 *         warpx:C:h:w:IN:FLOW:OUT               roma_warp_sample
 *         gridx:C:H:W:n:align:IN:GRID:OUT       ops_grid_sample
 *         dwx:C:H:W:IN:WT:BIAS:OUT              roma_dwconv5
 *         c5x:C:H:W:K:norm:IN:WT:BIAS:MEAN:RSTD:ALPHA:OUT   conv5x5
 *         convx:C:H:W:K:kh:kw:sy:sx:py:px:groups:act:IN:WT:BIAS:OUT conv2d
 *         statx:C:HW:eps:X:OUT                  chan_stats (mean, rstd)
 *         resx:C:h:w:H:W:align:scale:IN:OUT     resize_bilinear
 *         poolx:C:H:W:ks:s:p:max:IN:OUT         pool2d
 *         ropex:rows:ld:nh:d:npos:interleaved:X:CS:OUT   rope
 *         finex:H:W:M:T:F0:F1:CELLS:OUT          eloftr_fine
 *         smallx:KIND:a:b:c:x:y:F1:F2:F3:F4:F5:OUT   the small
 *                                element-wise kernels (exec_small) */

#define CL_TARGET_OPENCL_VERSION 120
#include <CL/cl.h>

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static cl_context ctx;
static cl_command_queue q;
static cl_device_id devid;
static cl_program prog_ops, prog_roma, prog_eloftr, prog_disk;

static void die(const char *what, cl_int e)
{
    fprintf(stderr, "ref_ocl: %s failed (%d)\n", what, (int)e);
    exit(2);
}

#define CK(call)                                                               \
    do {                                                                       \
        cl_int e_ = (call);                                                    \
        if (e_ != CL_SUCCESS)                                                  \
            die(#call, e_);                                                    \
    } while (0)

static cl_program load_program(const char *path)
{
    FILE *fp = fopen(path, "rb");
    unsigned char *bin;
    size_t n;
    cl_int e, st;
    cl_program p;

    if (!fp) {
        fprintf(stderr, "ref_ocl: cannot open %s\n", path);
        exit(2);
    }
    fseek(fp, 0, SEEK_END);
    n = (size_t)ftell(fp);
    fseek(fp, 0, SEEK_SET);
    bin = malloc(n);
    if (fread(bin, 1, n, fp) != n)
        die("fread", -1);
    fclose(fp);
    p = clCreateProgramWithBinary(ctx, 1, &devid, &n, (const unsigned char **)&bin, &st, &e);
    if (e != CL_SUCCESS || st != CL_SUCCESS) {
        fprintf(stderr, "ref_ocl: clCreateProgramWithBinary(%s): %d / %d\n", path, (int)e,
                (int)st);
        exit(2);
    }
    e = clBuildProgram(p, 1, &devid, "", NULL, NULL);
    if (e != CL_SUCCESS) {
        char log[8192] = "";

        clGetProgramBuildInfo(p, devid, CL_PROGRAM_BUILD_LOG, sizeof(log) - 1, log, NULL);
        fprintf(stderr, "ref_ocl: clBuildProgram(%s): %d\n%s\n", path, (int)e, log);
        exit(2);
    }
    free(bin);
    return p;
}

static cl_kernel kern(cl_program p, const char *name)
{
    cl_int e;
    cl_kernel k = clCreateKernel(p, name, &e);

    if (e != CL_SUCCESS)
        die(name, e);
    return k;
}

static cl_mem buf(size_t bytes, const void *host)
{
    cl_int e;
    cl_mem m = clCreateBuffer(ctx, CL_MEM_READ_WRITE, bytes ? bytes : 4, NULL, &e);

    if (e != CL_SUCCESS)
        die("clCreateBuffer", e);
    if (host)
        CK(clEnqueueWriteBuffer(q, m, CL_TRUE, 0, bytes, host, 0, NULL, NULL));
    return m;
}

static void readb(cl_mem m, size_t bytes, void *host)
{
    CK(clEnqueueReadBuffer(q, m, CL_TRUE, 0, bytes, host, 0, NULL, NULL));
}

/* Deterministic uniform values in [-s, s). */
static unsigned long long rng_state = 88172645463325252ULL;

static float urand(float s)
{
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return s * (2.0f * (float)((rng_state >> 40) * (1.0 / 16777216.0)) - 1.0f);
}

static float *rand_host(size_t n, float s)
{
    float *h = malloc(n * sizeof(float) + 4);

    for (size_t i = 0; i < n; i++)
        h[i] = urand(s);
    return h;
}

#define SET(k, i, v)                                                           \
    do {                                                                       \
        __typeof__(v) v_ = (v);                                                \
        CK(clSetKernelArg(k, i, sizeof(v_), &v_));                             \
    } while (0)

/* Launch and return the kernel's duration in ms (profiling event). */
static double launch(cl_kernel k, cl_uint dims, const size_t *g, const size_t *l)
{
    cl_event ev;
    cl_ulong t0, t1;

    CK(clEnqueueNDRangeKernel(q, k, dims, NULL, g, l, 0, NULL, &ev));
    CK(clWaitForEvents(1, &ev));
    CK(clGetEventProfilingInfo(ev, CL_PROFILING_COMMAND_START, sizeof(t0), &t0, NULL));
    CK(clGetEventProfilingInfo(ev, CL_PROFILING_COMMAND_END, sizeof(t1), &t1, NULL));
    clReleaseEvent(ev);
    return (t1 - t0) * 1e-6;
}

/* ---- ops_gemm, ops.c:148-188 ------------------------------------------- */

struct opnd {
    cl_mem buf;
    cl_long off;
    cl_int ld;
    cl_long s0, s1;
};

static cl_kernel k_gemm, k_gemm_big, k_softmax, k_layernorm, k_attention, k_grid;
static cl_kernel k_corr, k_warp;
static const char *last_gemm = "gemm";

static double gemm(int M, int N, int K, struct opnd A, struct opnd B, int transb,
                   struct opnd C, int nb, int nb1, cl_mem bias, int biasrow, cl_mem R,
                   long roff, float alpha, int act)
{
    const int big = M >= 128 && N >= 64 && K % 4 == 0 && A.ld % 4 == 0 && A.off % 4 == 0 &&
                    A.s0 % 4 == 0 && A.s1 % 4 == 0 && B.ld % 4 == 0 && B.off % 4 == 0 &&
                    B.s0 % 4 == 0 && B.s1 % 4 == 0;
    const int tile = big ? 128 : 64;
    cl_kernel k = big ? k_gemm_big : k_gemm;
    size_t g[3], l[3] = {16, 16, 1};

    last_gemm = big ? "gemm_big" : "gemm";

    SET(k, 0, (cl_int)M);
    SET(k, 1, (cl_int)N);
    SET(k, 2, (cl_int)K);
    SET(k, 3, A.buf);
    SET(k, 4, A.off);
    SET(k, 5, A.ld);
    SET(k, 6, A.s0);
    SET(k, 7, A.s1);
    SET(k, 8, B.buf);
    SET(k, 9, B.off);
    SET(k, 10, B.ld);
    SET(k, 11, B.s0);
    SET(k, 12, B.s1);
    SET(k, 13, (cl_int)transb);
    SET(k, 14, C.buf);
    SET(k, 15, C.off);
    SET(k, 16, C.ld);
    SET(k, 17, C.s0);
    SET(k, 18, C.s1);
    SET(k, 19, (cl_int)nb1);
    SET(k, 20, bias);
    SET(k, 21, (cl_int)biasrow);
    SET(k, 22, R);
    SET(k, 23, (cl_long)roff);
    SET(k, 24, (cl_float)alpha);
    SET(k, 25, (cl_int)act);
    SET(k, 26, (cl_float)0.0f);
    g[0] = (size_t)((N + tile - 1) / tile) * 16;
    g[1] = (size_t)((M + tile - 1) / tile) * 16;
    g[2] = (size_t)nb;
    return launch(k, 3, g, l);
}

static struct opnd mat(cl_mem b, long off, int ld, long s0)
{
    struct opnd o = {b, off, ld, s0, 0};

    return o;
}

/* ops.c:397-410: a power of two from 32 up to 256, at least L. */
static size_t row_group(int L)
{
    size_t l = 32;

    while (l < 256 && (int)l < L)
        l *= 2;
    return l;
}

static double layernorm(long rows, int C, cl_mem X, cl_mem Y, cl_mem g, cl_mem b)
{
    size_t ls = row_group(C), gs = rows * ls;

    SET(k_layernorm, 0, X);
    SET(k_layernorm, 1, Y);
    SET(k_layernorm, 2, g);
    SET(k_layernorm, 3, b);
    SET(k_layernorm, 4, (cl_int)C);
    SET(k_layernorm, 5, (cl_float)1e-6f);
    SET(k_layernorm, 6, (cl_int)0);
    SET(k_layernorm, 7, (cl_float)0.0f);
    return launch(k_layernorm, 1, &gs, &ls);
}

static double softmax(cl_mem S, long rows, int L)
{
    size_t ls = row_group(L), gs = rows * ls;

    SET(k_softmax, 0, S);
    SET(k_softmax, 1, (cl_int)L);
    SET(k_softmax, 2, (cl_float)1.0f);
    return launch(k_softmax, 1, &gs, &ls);
}

static int reps = 10;

static void case_gemm(const char *spec, int M, int N, int K, int transb)
{
    const size_t na = (size_t)M * K, nbb = (size_t)K * N, nc = (size_t)M * N;
    float *A = rand_host(na, 1.0f), *B = rand_host(nbb, 1.0f), *Ch = malloc(nc * 4);
    cl_mem a = buf(na * 4, A), b = buf(nbb * 4, B), c = buf(nc * 4, NULL);
    double ms = 0, err = 0, ref = 0;

    gemm(M, N, K, mat(a, 0, K, 0), mat(b, 0, transb ? K : N, 0), transb, mat(c, 0, N, 0), 1,
         1, NULL, 0, NULL, 0, 1.0f, 0);
    for (int r = 0; r < reps; r++)
        ms += gemm(M, N, K, mat(a, 0, K, 0), mat(b, 0, transb ? K : N, 0), transb,
                   mat(c, 0, N, 0), 1, 1, NULL, 0, NULL, 0, 1.0f, 0);
    readb(c, nc * 4, Ch);
    for (int s = 0; s < 64; s++) {
        const size_t i = (size_t)(s * 7919) % M, j = (size_t)(s * 104729) % N;
        double d = 0;

        for (int kk = 0; kk < K; kk++)
            d += (double)A[i * K + kk] * (transb ? B[j * K + kk] : B[(size_t)kk * N + j]);
        err = fmax(err, fabs(d - Ch[i * N + j]));
        ref = fmax(ref, fabs(d));
    }
    printf("{\"case\": \"%s\", \"kernel\": \"%s\", \"ms\": %.5f, \"gflop\": %.3f, "
           "\"check_rel\": %.3g}\n",
           spec, last_gemm, ms / reps, 2.0 * M * N * K / 1e9, err / fmax(ref, 1e-30));
    clReleaseMemObject(a);
    clReleaseMemObject(b);
    clReleaseMemObject(c);
    free(A);
    free(B);
    free(Ch);
}

/* roma.c:675-713 on one image of N tokens: LayerNorm, qkv, scores,
 * softmax, values, proj + residual, LayerNorm, fc1 + GELU, fc2 +
 * residual; ops_linear maps to ops_gemm with B the [out, in] weight. */
static void case_vitblock(const char *spec, int N)
{
    const int D = 1024, H = 16, hd = 64;
    const long nn = (long)N * N;
    float *hx = rand_host((size_t)N * D, 1.0f), *w = rand_host((size_t)4 * D * D, 0.03f);
    float *bvec = rand_host((size_t)4 * D, 0.1f), *g = rand_host(D, 1.0f);
    cl_mem x = buf((size_t)N * D * 4, hx), t = buf((size_t)N * D * 4, NULL);
    cl_mem qkv = buf((size_t)N * 3 * D * 4, NULL), s = buf((size_t)H * nn * 4, NULL);
    cl_mem o = buf((size_t)N * D * 4, NULL), h = buf((size_t)N * 4 * D * 4, NULL);
    cl_mem wq = buf((size_t)3 * D * D * 4, w), wp = buf((size_t)D * D * 4, w);
    cl_mem w1 = buf((size_t)4 * D * D * 4, w), w2 = buf((size_t)4 * D * D * 4, w);
    cl_mem bb = buf((size_t)4 * D * 4, bvec), gg = buf((size_t)D * 4, g);
    double tot[9] = {0};
    const char *names[9] = {"layernorm", "qkv", "scores", "softmax", "values", "proj",
                            "layernorm2", "fc1", "fc2"};
    float *hs = malloc((size_t)N * 4);

    for (int r = -1; r < reps; r++) {
        double e[9];

        clEnqueueWriteBuffer(q, x, CL_TRUE, 0, (size_t)N * D * 4, hx, 0, NULL, NULL);
        e[0] = layernorm(N, D, x, t, gg, bb);
        e[1] = gemm(N, 3 * D, D, mat(t, 0, D, 0), mat(wq, 0, D, 0), 1, mat(qkv, 0, 3 * D, 0),
                    1, 1, bb, 0, NULL, 0, 1.0f, 0);
        e[2] = gemm(N, N, hd, mat(qkv, 0, 3 * D, hd), mat(qkv, D, 3 * D, hd), 1,
                    mat(s, 0, N, nn), H, 1, NULL, 0, NULL, 0, 1.0f / sqrtf((float)hd), 0);
        e[3] = softmax(s, (long)H * N, N);
        e[4] = gemm(N, hd, N, mat(s, 0, N, nn), mat(qkv, 2 * D, 3 * D, hd), 0,
                    mat(o, 0, D, hd), H, 1, NULL, 0, NULL, 0, 1.0f, 0);
        e[5] = gemm(N, D, D, mat(o, 0, D, 0), mat(wp, 0, D, 0), 1, mat(x, 0, D, 0), 1, 1, bb,
                    0, x, 0, 1.0f, 0);
        e[6] = layernorm(N, D, x, t, gg, bb);
        e[7] = gemm(N, 4 * D, D, mat(t, 0, D, 0), mat(w1, 0, D, 0), 1, mat(h, 0, 4 * D, 0), 1,
                    1, bb, 0, NULL, 0, 1.0f, 1);
        e[8] = gemm(N, D, 4 * D, mat(h, 0, 4 * D, 0), mat(w2, 0, 4 * D, 0), 1,
                    mat(x, 0, D, 0), 1, 1, bb, 0, x, 0, 1.0f, 0);
        if (r >= 0)
            for (int i = 0; i < 9; i++)
                tot[i] += e[i];
    }
    /* Check: the softmax rows of head 0, query 0 sum to one. */
    readb(s, (size_t)N * 4, hs);
    {
        double sum = 0, all = 0;

        for (int j = 0; j < N; j++)
            sum += hs[j];
        printf("{\"case\": \"%s\", \"kernel\": \"vit_block\", \"ms\": ", spec);
        for (int i = 0; i < 9; i++)
            all += tot[i] / reps;
        printf("%.5f, \"parts_ms\": {", all);
        for (int i = 0; i < 9; i++)
            printf("%s\"%s\": %.5f", i ? ", " : "", names[i], tot[i] / reps);
        printf("}, \"gflop\": %.3f, \"check_rel\": %.3g}\n",
               (2.0 * N * D * 12 * D + 4.0 * H * (double)N * N * hd) / 1e9, fabs(sum - 1));
    }
    clReleaseMemObject(x);
    clReleaseMemObject(t);
    clReleaseMemObject(qkv);
    clReleaseMemObject(s);
    clReleaseMemObject(o);
    clReleaseMemObject(h);
    clReleaseMemObject(wq);
    clReleaseMemObject(wp);
    clReleaseMemObject(w1);
    clReleaseMemObject(w2);
    clReleaseMemObject(bb);
    clReleaseMemObject(gg);
    free(hx);
    free(w);
    free(bvec);
    free(g);
    free(hs);
}

static void case_attention(const char *spec, int Nq, int Nk, int nh, int d)
{
    const int ld = nh * d;
    float *Q = rand_host((size_t)Nq * ld, 1.0f), *K = rand_host((size_t)Nk * ld, 1.0f);
    float *V = rand_host((size_t)Nk * ld, 1.0f), *O = malloc((size_t)Nq * ld * 4);
    cl_mem bq = buf((size_t)Nq * ld * 4, Q), bk = buf((size_t)Nk * ld * 4, K);
    cl_mem bv = buf((size_t)Nk * ld * 4, V), bo = buf((size_t)Nq * ld * 4, NULL);
    const float scale = 1.0f / sqrtf((float)d);
    size_t gs[3] = {16, (size_t)(Nq + 15) / 16 * 16, (size_t)nh}, ls[3] = {16, 16, 1};
    double ms = 0, err = 0, ref = 0;
    const cl_long zero = 0;
    const cl_mem none = NULL;

    SET(k_attention, 0, bq);
    SET(k_attention, 1, zero);
    SET(k_attention, 2, (cl_int)ld);
    SET(k_attention, 3, bk);
    SET(k_attention, 4, zero);
    SET(k_attention, 5, (cl_int)ld);
    SET(k_attention, 6, bv);
    SET(k_attention, 7, zero);
    SET(k_attention, 8, (cl_int)ld);
    SET(k_attention, 9, bo);
    SET(k_attention, 10, zero);
    SET(k_attention, 11, (cl_int)ld);
    SET(k_attention, 12, (cl_int)Nq);
    SET(k_attention, 13, (cl_int)Nk);
    SET(k_attention, 14, (cl_int)d);
    SET(k_attention, 15, (cl_float)scale);
    SET(k_attention, 16, none);
    launch(k_attention, 3, gs, ls);
    for (int r = 0; r < reps; r++)
        ms += launch(k_attention, 3, gs, ls);
    readb(bo, (size_t)Nq * ld * 4, O);
    for (int s = 0; s < 8; s++) {
        const int i = (s * 7919) % Nq, h = s % nh;
        double m = -1e300, sum = 0, *p = malloc((size_t)Nk * sizeof(double));

        for (int j = 0; j < Nk; j++) {
            double dot = 0;

            for (int c = 0; c < d; c++)
                dot += (double)Q[(size_t)i * ld + h * d + c] * K[(size_t)j * ld + h * d + c];
            p[j] = dot * scale;
            m = fmax(m, p[j]);
        }
        for (int j = 0; j < Nk; j++)
            sum += p[j] = exp(p[j] - m);
        for (int c = 0; c < d; c++) {
            double v = 0;

            for (int j = 0; j < Nk; j++)
                v += p[j] * V[(size_t)j * ld + h * d + c];
            v /= sum;
            err = fmax(err, fabs(v - O[(size_t)i * ld + h * d + c]));
            ref = fmax(ref, fabs(v));
        }
        free(p);
    }
    printf("{\"case\": \"%s\", \"kernel\": \"attention\", \"ms\": %.5f, \"gflop\": %.3f, "
           "\"check_rel\": %.3g}\n",
           spec, ms / reps, 4.0 * nh * (double)Nq * Nk * d / 1e9, err / fmax(ref, 1e-30));
    clReleaseMemObject(bq);
    clReleaseMemObject(bk);
    clReleaseMemObject(bv);
    clReleaseMemObject(bo);
    free(Q);
    free(K);
    free(V);
    free(O);
}

/* A smooth warp on the h x w grid (normalised coordinates). */
static float *smooth_flow(int h, int w)
{
    float *f = malloc((size_t)2 * h * w * 4);

    for (int y = 0; y < h; y++)
        for (int x = 0; x < w; x++) {
            const float gx = 2 * (x + 0.5f) / w - 1, gy = 2 * (y + 0.5f) / h - 1;

            f[(size_t)y * w + x] = gx + 0.03f * sinf(gy * 3);
            f[(size_t)h * w + (size_t)y * w + x] = gy + 0.03f * cosf(gx * 2);
        }
    return f;
}

static double bilin(const float *p, int H, int W, double x, double y)
{
    const double ix = ((x + 1) * W - 1) * 0.5, iy = ((y + 1) * H - 1) * 0.5;
    const int x0 = (int)floor(ix), y0 = (int)floor(iy);
    const double fx = ix - x0, fy = iy - y0;
#define AT(yy, xx) ((xx) >= 0 && (xx) < W && (yy) >= 0 && (yy) < H ? p[(size_t)(yy) * W + (xx)] : 0.0)
    return (1 - fy) * ((1 - fx) * AT(y0, x0) + fx * AT(y0, x0 + 1)) +
           fy * ((1 - fx) * AT(y0 + 1, x0) + fx * AT(y0 + 1, x0 + 1));
#undef AT
}

static void case_localcorr(const char *spec, int C, int h, int w, int r)
{
    const size_t n = (size_t)h * w;
    const int side = 2 * r + 1;
    float *f1 = rand_host(C * n, 1.0f), *f2 = rand_host(C * n, 1.0f), *fl = smooth_flow(h, w);
    float *out = malloc((size_t)side * side * n * 4);
    cl_mem b1 = buf(C * n * 4, f1), b2 = buf(C * n * 4, f2), bf = buf(2 * n * 4, fl);
    cl_mem bo = buf((size_t)side * side * n * 4, NULL);
    size_t gc = n * 64, lc = 64;
    double ms = 0, err = 0, ref = 0;

    if (C > 512 || r > 7) {
        fprintf(stderr, "ref_ocl: localcorr needs C <= 512, r <= 7\n");
        exit(2);
    }
    SET(k_corr, 0, b1);
    SET(k_corr, 1, b2);
    SET(k_corr, 2, (cl_int)C);
    SET(k_corr, 3, (cl_int)h);
    SET(k_corr, 4, (cl_int)w);
    SET(k_corr, 5, (cl_int)r);
    SET(k_corr, 6, bf);
    SET(k_corr, 7, bo);
    SET(k_corr, 8, (cl_int)0);
    launch(k_corr, 1, &gc, &lc);
    for (int t = 0; t < reps; t++)
        ms += launch(k_corr, 1, &gc, &lc);
    readb(bo, (size_t)side * side * n * 4, out);
    for (int s = 0; s < 32; s++) {
        const size_t i = (size_t)(s * 7919) % n;
        /* Window offset k = (a, b), a the row: the warp moved by (b - r,
         * a - r) cells, a cell being 2 / w by 2 / h in normalised units. */
        for (int k = 0; k < side * side; k++) {
            const double x = fl[i] + (k % side - r) * (2.0 / w);
            const double y = fl[n + i] + (k / side - r) * (2.0 / h);
            double v = 0;

            for (int c = 0; c < C; c++)
                v += (double)f1[c * n + i] * bilin(f2 + c * n, h, w, x, y);
            v /= sqrt((double)C);
            err = fmax(err, fabs(v - out[(size_t)k * n + i]));
            ref = fmax(ref, fabs(v));
        }
    }
    printf("{\"case\": \"%s\", \"kernel\": \"roma_local_corr\", \"ms\": %.5f, "
           "\"bytes\": %.0f, \"check_rel\": %.3g}\n",
           spec, ms / reps, 8.0 * C * n + 8.0 * n + 4.0 * side * side * n,
           err / fmax(ref, 1e-30));
    clReleaseMemObject(b1);
    clReleaseMemObject(b2);
    clReleaseMemObject(bf);
    clReleaseMemObject(bo);
    free(f1);
    free(f2);
    free(fl);
    free(out);
}

static void case_warpsample(const char *spec, int C, int h, int w)
{
    const size_t n = (size_t)h * w;
    float *in = rand_host(C * n, 1.0f), *fl = smooth_flow(h, w), *out = malloc(C * n * 4);
    cl_mem bi = buf(C * n * 4, in), bf = buf(2 * n * 4, fl), bo = buf(C * n * 4, NULL);
    size_t g2[2] = {n, (size_t)C};
    double ms = 0, err = 0, ref = 0;

    SET(k_warp, 0, bi);
    SET(k_warp, 1, (cl_int)C);
    SET(k_warp, 2, (cl_int)h);
    SET(k_warp, 3, (cl_int)w);
    SET(k_warp, 4, bf);
    SET(k_warp, 5, bo);
    SET(k_warp, 6, (cl_int)0);
    launch(k_warp, 2, g2, NULL);
    for (int t = 0; t < reps; t++)
        ms += launch(k_warp, 2, g2, NULL);
    readb(bo, C * n * 4, out);
    for (int s = 0; s < 256; s++) {
        const size_t i = (size_t)(s * 7919) % n, c = (size_t)(s * 31) % C;
        const double v = bilin(in + c * n, h, w, fl[i], fl[n + i]);

        err = fmax(err, fabs(v - out[c * n + i]));
        ref = fmax(ref, fabs(v));
    }
    printf("{\"case\": \"%s\", \"kernel\": \"roma_warp_sample\", \"ms\": %.5f, "
           "\"bytes\": %.0f, \"check_rel\": %.3g}\n",
           spec, ms / reps, 8.0 * C * n + 8.0 * n, err / fmax(ref, 1e-30));
    clReleaseMemObject(bi);
    clReleaseMemObject(bf);
    clReleaseMemObject(bo);
    free(in);
    free(fl);
    free(out);
}

static void case_gridsample(const char *spec, int C, int H, int W, int n)
{
    float *in = rand_host((size_t)C * H * W, 1.0f), *grid = rand_host(2 * (size_t)n, 1.05f);

    /* n = H W: the points of a smooth warp of the same grid (the
     * refiners' access pattern), else uniform points. */
    if ((size_t)n == (size_t)H * W) {
        float *f = smooth_flow(H, W);

        for (int i = 0; i < n; i++) {
            grid[2 * i] = f[i];
            grid[2 * i + 1] = f[(size_t)n + i];
        }
        free(f);
    }
    float *out = malloc((size_t)C * n * 4);
    cl_mem bi = buf((size_t)C * H * W * 4, in), bg = buf(2 * (size_t)n * 4, grid);
    cl_mem bo = buf((size_t)C * n * 4, NULL);
    size_t g[2] = {(size_t)(n + 63) / 64 * 64, (size_t)C}, l[2] = {64, 1};
    double ms = 0, err = 0, ref = 0;

    SET(k_grid, 0, bi);
    SET(k_grid, 1, (cl_int)C);
    SET(k_grid, 2, (cl_int)H);
    SET(k_grid, 3, (cl_int)W);
    SET(k_grid, 4, bg);
    SET(k_grid, 5, (cl_int)n);
    SET(k_grid, 6, (cl_int)0);
    SET(k_grid, 7, bo);
    launch(k_grid, 2, g, l);
    for (int t = 0; t < reps; t++)
        ms += launch(k_grid, 2, g, l);
    readb(bo, (size_t)C * n * 4, out);
    for (int s = 0; s < 256; s++) {
        const size_t i = (size_t)(s * 7919) % n, c = (size_t)(s * 31) % C;
        const double v = bilin(in + c * H * W, H, W, grid[2 * i], grid[2 * i + 1]);

        err = fmax(err, fabs(v - out[c * n + i]));
        ref = fmax(ref, fabs(v));
    }
    printf("{\"case\": \"%s\", \"kernel\": \"grid_sample\", \"ms\": %.5f, \"bytes\": %.0f, "
           "\"check_rel\": %.3g}\n",
           spec, ms / reps, 4.0 * C * H * W + 8.0 * n + 4.0 * C * n, err / fmax(ref, 1e-30));
    clReleaseMemObject(bi);
    clReleaseMemObject(bg);
    clReleaseMemObject(bo);
    free(in);
    free(grid);
    free(out);
}

/* ---- parity cases: inputs and outputs as raw files ------------------- */

static void *read_file(const char *path, size_t bytes)
{
    FILE *fp = fopen(path, "rb");
    void *p = malloc(bytes ? bytes : 4);

    if (!fp || fread(p, 1, bytes, fp) != bytes) {
        fprintf(stderr, "ref_ocl: cannot read %zu bytes of %s\n", bytes, path);
        exit(2);
    }
    fclose(fp);
    return p;
}

static void write_file(const char *path, const void *p, size_t bytes)
{
    FILE *fp = fopen(path, "wb");

    if (!fp || fwrite(p, 1, bytes, fp) != bytes) {
        fprintf(stderr, "ref_ocl: cannot write %s\n", path);
        exit(2);
    }
    fclose(fp);
}

static cl_program need_program(cl_program p, const char *what)
{
    if (!p) {
        fprintf(stderr, "ref_ocl: %s.co was not built\n", what);
        exit(2);
    }
    return p;
}

static void exec_coarse(const char *spec, int n, int blk, const char *sf, const char *of)
{
    cl_program pe = need_program(prog_eloftr, "eloftr_kernels");
    cl_kernel k_rl = kern(pe, "eloftr_row_lse"), k_cl = kern(pe, "eloftr_col_lse");
    cl_kernel k_cr = kern(pe, "eloftr_conf_row"), k_cc = kern(pe, "eloftr_conf_col");
    const size_t nn = (size_t)n * n;
    float *S = read_file(sf, nn * 4), *f = malloc((size_t)n * 4);
    int *iv = malloc((size_t)n * 4);
    cl_mem sb = buf((size_t)blk * n * 4, NULL), lse = buf((size_t)n * 4, NULL);
    cl_mem cm, cs, cmax, carg, rmax = buf((size_t)n * 4, NULL), rarg = buf((size_t)n * 4, NULL);
    unsigned char *out = malloc((size_t)n * 16);
    double ms = 0.0;
    int i, pass, r0;

    /* Column state as eloftr.c:485-496 writes it. */
    for (i = 0; i < n; i++)
        f[i] = -INFINITY;
    cm = buf((size_t)n * 4, f);
    for (i = 0; i < n; i++)
        f[i] = 0.0f;
    cs = buf((size_t)n * 4, f);
    for (i = 0; i < n; i++)
        f[i] = -1.0f;
    cmax = buf((size_t)n * 4, f);
    for (i = 0; i < n; i++)
        iv[i] = -1;
    carg = buf((size_t)n * 4, iv);
    for (pass = 0; pass < 2; pass++)
        for (r0 = 0; r0 < n; r0 += blk) {
            const int rows = n - r0 < blk ? n - r0 : blk;
            size_t gr = (size_t)rows * 256, lr = 256;
            size_t gc = (size_t)(n + 63) / 64 * 64, lc = 64;

            CK(clEnqueueWriteBuffer(q, sb, CL_TRUE, 0, (size_t)rows * n * 4,
                                    S + (size_t)r0 * n, 0, NULL, NULL));
            if (pass == 0) {
                SET(k_rl, 0, sb);
                SET(k_rl, 1, (cl_int)n);
                SET(k_rl, 2, (cl_int)r0);
                SET(k_rl, 3, lse);
                ms += launch(k_rl, 1, &gr, &lr);
                SET(k_cl, 0, sb);
                SET(k_cl, 1, (cl_int)rows);
                SET(k_cl, 2, (cl_int)n);
                SET(k_cl, 3, cm);
                SET(k_cl, 4, cs);
                ms += launch(k_cl, 1, &gc, &lc);
            }
            else {
                SET(k_cr, 0, sb);
                SET(k_cr, 1, (cl_int)n);
                SET(k_cr, 2, (cl_int)r0);
                SET(k_cr, 3, lse);
                SET(k_cr, 4, cm);
                SET(k_cr, 5, cs);
                SET(k_cr, 6, rmax);
                SET(k_cr, 7, rarg);
                ms += launch(k_cr, 1, &gr, &lr);
                SET(k_cc, 0, sb);
                SET(k_cc, 1, (cl_int)rows);
                SET(k_cc, 2, (cl_int)n);
                SET(k_cc, 3, (cl_int)r0);
                SET(k_cc, 4, lse);
                SET(k_cc, 5, cm);
                SET(k_cc, 6, cs);
                SET(k_cc, 7, cmax);
                SET(k_cc, 8, carg);
                ms += launch(k_cc, 1, &gc, &lc);
            }
        }
    readb(rmax, (size_t)n * 4, out);
    readb(rarg, (size_t)n * 4, out + (size_t)n * 4);
    readb(carg, (size_t)n * 4, out + (size_t)n * 8);
    readb(cmax, (size_t)n * 4, out + (size_t)n * 12);
    write_file(of, out, (size_t)n * 16);
    printf("{\"case\": \"%s\", \"kernel\": \"eloftr coarse dual softmax\", \"ms\": %.5f}\n",
           spec, ms);
    {
        cl_mem all[8] = {sb, lse, cm, cs, cmax, carg, rmax, rarg};

        for (i = 0; i < 8; i++)
            clReleaseMemObject(all[i]);
    }
    clReleaseKernel(k_rl);
    clReleaseKernel(k_cl);
    clReleaseKernel(k_cr);
    clReleaseKernel(k_cc);
    free(S);
    free(f);
    free(iv);
    free(out);
}
static void exec_nms(const char *spec, int h, int w, int W, long off, float thresh,
                     const char *hf, const char *of)
{
    cl_kernel k = kern(need_program(prog_disk, "disk_kernels"), "nms5x5");
    const size_t nh = (size_t)off + (size_t)h * W;
    float *heat = read_file(hf, nh * 4);
    unsigned char *mask = malloc((size_t)h * w + 1);
    cl_mem bh = buf(nh * 4, heat), bm = buf((size_t)h * w, NULL);
    size_t g[2] = {(size_t)w, (size_t)h};
    double ms;

    SET(k, 0, bh);
    SET(k, 1, (cl_ulong)off);
    SET(k, 2, (cl_int)W);
    SET(k, 3, (cl_int)h);
    SET(k, 4, (cl_int)w);
    SET(k, 5, (cl_float)thresh);
    SET(k, 6, bm);
    ms = launch(k, 2, g, NULL);
    readb(bm, (size_t)h * w, mask);
    write_file(of, mask, (size_t)h * w);
    printf("{\"case\": \"%s\", \"kernel\": \"nms5x5\", \"ms\": %.5f}\n", spec, ms);
    clReleaseMemObject(bh);
    clReleaseMemObject(bm);
    clReleaseKernel(k);
    free(heat);
    free(mask);
}

static void exec_gather(const char *spec, int H, int W, int D, int n, const char *ff,
                        const char *xf, const char *of)
{
    cl_kernel k = kern(need_program(prog_disk, "disk_kernels"), "gather_desc");
    const size_t nf = (size_t)(D + 1) * H * W;
    float *feat = read_file(ff, nf * 4), *desc = malloc((size_t)n * D * 4 + 4);
    int *xy = read_file(xf, (size_t)n * 8);
    cl_mem bf = buf(nf * 4, feat), bx = buf((size_t)n * 8, xy), bd = buf((size_t)n * D * 4, NULL);
    size_t g = (size_t)n;
    double ms;

    SET(k, 0, bf);
    SET(k, 1, (cl_int)H);
    SET(k, 2, (cl_int)W);
    SET(k, 3, (cl_int)D);
    SET(k, 4, bx);
    SET(k, 5, (cl_int)n);
    SET(k, 6, bd);
    ms = launch(k, 1, &g, NULL);
    readb(bd, (size_t)n * D * 4, desc);
    write_file(of, desc, (size_t)n * D * 4);
    printf("{\"case\": \"%s\", \"kernel\": \"gather_desc\", \"ms\": %.5f}\n", spec, ms);
    clReleaseMemObject(bf);
    clReleaseMemObject(bx);
    clReleaseMemObject(bd);
    clReleaseKernel(k);
    free(feat);
    free(xy);
    free(desc);
}

static void exec_cls(const char *spec, int n, int ld, int C, int res, const char *lf,
                     const char *of)
{
    cl_kernel k = kern(prog_roma, "roma_cls_to_flow");
    float *L = read_file(lf, (size_t)n * ld * 4), *out = malloc((size_t)n * 12);
    cl_mem bl = buf((size_t)n * ld * 4, L), bf = buf((size_t)n * 8, NULL),
           bc = buf((size_t)n * 4, NULL);
    size_t g = (size_t)n * 256, l = 256;
    double ms;

    SET(k, 0, bl);
    SET(k, 1, (cl_int)ld);
    SET(k, 2, (cl_int)C);
    SET(k, 3, (cl_int)res);
    SET(k, 4, (cl_int)n);
    SET(k, 5, bf);
    SET(k, 6, bc);
    ms = launch(k, 1, &g, &l);
    readb(bf, (size_t)n * 8, out);
    readb(bc, (size_t)n * 4, out + 2 * (size_t)n);
    write_file(of, out, (size_t)n * 12);
    printf("{\"case\": \"%s\", \"kernel\": \"roma_cls_to_flow\", \"ms\": %.5f}\n", spec,
           ms);
    clReleaseMemObject(bl);
    clReleaseMemObject(bf);
    clReleaseMemObject(bc);
    clReleaseKernel(k);
    free(L);
    free(out);
}

/* A file of n floats into a new buffer. */
static cl_mem file_buf(const char *path, size_t n, float **host)
{
    float *h = read_file(path, n * 4);
    cl_mem m = buf(n * 4, h);

    if (host)
        *host = h;
    else
        free(h);
    return m;
}

/* A buffer of n floats to a file. */
static void buf_file(cl_mem m, size_t n, const char *path)
{
    float *h = malloc(n * 4);

    readb(m, n * 4, h);
    write_file(path, h, n * 4);
    free(h);
}

/* gemmx: C = act(A B + bias), ops_gemm's dispatch (ops.c:148-188). */
static void exec_gemm(const char *spec, int M, int N, int K, int transb, int act, const char *fa,
                      const char *fb, const char *fbias, const char *fo)
{
    cl_mem ba = file_buf(fa, (size_t)M * K, NULL), bb = file_buf(fb, (size_t)K * N, NULL);
    cl_mem bi = file_buf(fbias, (size_t)N, NULL), bc = buf((size_t)M * N * 4, NULL);
    const double ms = gemm(M, N, K, mat(ba, 0, K, 0), mat(bb, 0, transb ? K : N, 0), transb,
                           mat(bc, 0, N, 0), 1, 1, bi, 0, NULL, 0, 1.0f, act);

    buf_file(bc, (size_t)M * N, fo);
    printf("{\"case\": \"%s\", \"kernel\": \"%s\", \"ms\": %.5f}\n", spec, last_gemm, ms);
    clReleaseMemObject(ba);
    clReleaseMemObject(bb);
    clReleaseMemObject(bi);
    clReleaseMemObject(bc);
}

/* lnx: layernorm over rows of C, ops_layernorm's dispatch (ops.c:412-429). */
static void exec_layernorm(const char *spec, int rows, int C, float eps, const char *fx,
                           const char *fg, const char *fbeta, const char *fo)
{
    cl_mem bx = file_buf(fx, (size_t)rows * C, NULL), bg = file_buf(fg, (size_t)C, NULL);
    cl_mem bb = file_buf(fbeta, (size_t)C, NULL), by = buf((size_t)rows * C * 4, NULL);
    size_t ls = row_group(C), gs = (size_t)rows * ls;

    SET(k_layernorm, 0, bx);
    SET(k_layernorm, 1, by);
    SET(k_layernorm, 2, bg);
    SET(k_layernorm, 3, bb);
    SET(k_layernorm, 4, (cl_int)C);
    SET(k_layernorm, 5, (cl_float)eps);
    SET(k_layernorm, 6, (cl_int)0);
    SET(k_layernorm, 7, (cl_float)0.0f);
    launch(k_layernorm, 1, &gs, &ls);
    buf_file(by, (size_t)rows * C, fo);
    printf("{\"case\": \"%s\", \"kernel\": \"layernorm\"}\n", spec);
    clReleaseMemObject(bx);
    clReleaseMemObject(bg);
    clReleaseMemObject(bb);
    clReleaseMemObject(by);
}

/* smx: softmax over rows of L in place, ops_softmax_rows' dispatch
 * (ops.c:432-442). */
static void exec_softmax(const char *spec, int rows, int L, float scale, const char *fs,
                         const char *fo)
{
    cl_mem bs = file_buf(fs, (size_t)rows * L, NULL);
    size_t ls = row_group(L), gs = (size_t)rows * ls;

    SET(k_softmax, 0, bs);
    SET(k_softmax, 1, (cl_int)L);
    SET(k_softmax, 2, (cl_float)scale);
    launch(k_softmax, 1, &gs, &ls);
    buf_file(bs, (size_t)rows * L, fo);
    printf("{\"case\": \"%s\", \"kernel\": \"softmax_rows\"}\n", spec);
    clReleaseMemObject(bs);
}

/* attnx: heads of d columns in rows of nh d floats, no key mask,
 * ops_attention's dispatch (ops.c:443-474). */
static void exec_attention(const char *spec, int Nq, int Nk, int nh, int d, float scale,
                           const char *fq, const char *fk, const char *fv, const char *fo)
{
    const int ld = nh * d;
    const cl_long zero = 0;
    const cl_mem none = NULL;
    cl_mem bq = file_buf(fq, (size_t)Nq * ld, NULL), bk = file_buf(fk, (size_t)Nk * ld, NULL);
    cl_mem bv = file_buf(fv, (size_t)Nk * ld, NULL), bo = buf((size_t)Nq * ld * 4, NULL);
    size_t gs[3] = {16, (size_t)(Nq + 15) / 16 * 16, (size_t)nh}, ls[3] = {16, 16, 1};

    SET(k_attention, 0, bq);
    SET(k_attention, 1, zero);
    SET(k_attention, 2, (cl_int)ld);
    SET(k_attention, 3, bk);
    SET(k_attention, 4, zero);
    SET(k_attention, 5, (cl_int)ld);
    SET(k_attention, 6, bv);
    SET(k_attention, 7, zero);
    SET(k_attention, 8, (cl_int)ld);
    SET(k_attention, 9, bo);
    SET(k_attention, 10, zero);
    SET(k_attention, 11, (cl_int)ld);
    SET(k_attention, 12, (cl_int)Nq);
    SET(k_attention, 13, (cl_int)Nk);
    SET(k_attention, 14, (cl_int)d);
    SET(k_attention, 15, (cl_float)scale);
    SET(k_attention, 16, none);
    launch(k_attention, 3, gs, ls);
    buf_file(bo, (size_t)Nq * ld, fo);
    printf("{\"case\": \"%s\", \"kernel\": \"attention\"}\n", spec);
    clReleaseMemObject(bq);
    clReleaseMemObject(bk);
    clReleaseMemObject(bv);
    clReleaseMemObject(bo);
}

/* lcx: roma_local_corr as roma.c:956-968 (output channels from 0). */
static void exec_localcorr(const char *spec, int C, int h, int w, int r, const char *f1,
                           const char *f2, const char *ffl, const char *fo)
{
    const size_t n = (size_t)h * w, side = 2 * (size_t)r + 1;
    cl_mem b1 = file_buf(f1, (size_t)C * n, NULL), b2 = file_buf(f2, (size_t)C * n, NULL);
    cl_mem bf = file_buf(ffl, 2 * n, NULL), bo = buf(side * side * n * 4, NULL);
    size_t gc = n * 64, lc = 64;

    SET(k_corr, 0, b1);
    SET(k_corr, 1, b2);
    SET(k_corr, 2, (cl_int)C);
    SET(k_corr, 3, (cl_int)h);
    SET(k_corr, 4, (cl_int)w);
    SET(k_corr, 5, (cl_int)r);
    SET(k_corr, 6, bf);
    SET(k_corr, 7, bo);
    SET(k_corr, 8, (cl_int)0);
    launch(k_corr, 1, &gc, &lc);
    buf_file(bo, side * side * n, fo);
    printf("{\"case\": \"%s\", \"kernel\": \"roma_local_corr\"}\n", spec);
    clReleaseMemObject(b1);
    clReleaseMemObject(b2);
    clReleaseMemObject(bf);
    clReleaseMemObject(bo);
}

/* warpx: roma_warp_sample as roma.c:936-945 (output channels from 0). */
static void exec_warpsample(const char *spec, int C, int h, int w, const char *fi,
                            const char *ffl, const char *fo)
{
    const size_t n = (size_t)h * w;
    cl_mem bi = file_buf(fi, (size_t)C * n, NULL), bf = file_buf(ffl, 2 * n, NULL);
    cl_mem bo = buf((size_t)C * n * 4, NULL);
    size_t g2[2] = {n, (size_t)C};

    SET(k_warp, 0, bi);
    SET(k_warp, 1, (cl_int)C);
    SET(k_warp, 2, (cl_int)h);
    SET(k_warp, 3, (cl_int)w);
    SET(k_warp, 4, bf);
    SET(k_warp, 5, bo);
    SET(k_warp, 6, (cl_int)0);
    launch(k_warp, 2, g2, NULL);
    buf_file(bo, (size_t)C * n, fo);
    printf("{\"case\": \"%s\", \"kernel\": \"roma_warp_sample\"}\n", spec);
    clReleaseMemObject(bi);
    clReleaseMemObject(bf);
    clReleaseMemObject(bo);
}

/* gridx: grid_sample, ops_grid_sample's dispatch (ops.c:520-534). */
static void exec_gridsample(const char *spec, int C, int H, int W, int n, int align,
                            const char *fi, const char *fg, const char *fo)
{
    cl_mem bi = file_buf(fi, (size_t)C * H * W, NULL), bg = file_buf(fg, 2 * (size_t)n, NULL);
    cl_mem bo = buf((size_t)C * n * 4, NULL);
    size_t g[2] = {(size_t)(n + 63) / 64 * 64, (size_t)C}, l[2] = {64, 1};

    SET(k_grid, 0, bi);
    SET(k_grid, 1, (cl_int)C);
    SET(k_grid, 2, (cl_int)H);
    SET(k_grid, 3, (cl_int)W);
    SET(k_grid, 4, bg);
    SET(k_grid, 5, (cl_int)n);
    SET(k_grid, 6, (cl_int)align);
    SET(k_grid, 7, bo);
    launch(k_grid, 2, g, l);
    buf_file(bo, (size_t)C * n, fo);
    printf("{\"case\": \"%s\", \"kernel\": \"grid_sample\"}\n", spec);
    clReleaseMemObject(bi);
    clReleaseMemObject(bg);
    clReleaseMemObject(bo);
}

/* dwx: roma_dwconv5 (depthwise 5 x 5, bias, ReLU) as roma.c:970-981. */
static void exec_dwconv(const char *spec, int C, int H, int W, const char *fi, const char *fw,
                        const char *fb, const char *fo)
{
    cl_kernel k = kern(prog_roma, "roma_dwconv5");
    const size_t n = (size_t)H * W;
    cl_mem bi = file_buf(fi, (size_t)C * n, NULL), bw = file_buf(fw, (size_t)C * 25, NULL);
    cl_mem bb = file_buf(fb, (size_t)C, NULL), bo = buf((size_t)C * n * 4, NULL);
    size_t g[3] = {(size_t)(W + 15) / 16 * 16, (size_t)(H + 15) / 16 * 16, (size_t)C},
           l[3] = {16, 16, 1};

    SET(k, 0, bi);
    SET(k, 1, (cl_int)H);
    SET(k, 2, (cl_int)W);
    SET(k, 3, bw);
    SET(k, 4, bb);
    SET(k, 5, bo);
    launch(k, 3, g, l);
    buf_file(bo, (size_t)C * n, fo);
    printf("{\"case\": \"%s\", \"kernel\": \"roma_dwconv5\"}\n", spec);
    clReleaseMemObject(bi);
    clReleaseMemObject(bw);
    clReleaseMemObject(bb);
    clReleaseMemObject(bo);
    clReleaseKernel(k);
}

/* c5x: conv5x5 (stride 1, padding 2, bias, no activation), with the
 * input normalised and gated (instance norm + PReLU) when norm is set,
 * ops_conv2d's first branch (ops.c:285-305). MEAN, RSTD, ALPHA: C floats
 * each (read only with norm). */
static void exec_conv5(const char *spec, int C, int H, int W, int K, int norm, const char *fi,
                       const char *fw, const char *fb, const char *fm, const char *fr,
                       const char *fa, const char *fo)
{
    cl_kernel k = kern(prog_ops, "conv5x5");
    cl_mem bi = file_buf(fi, (size_t)C * H * W, NULL), bw = file_buf(fw, (size_t)K * C * 25, NULL);
    cl_mem bb = file_buf(fb, (size_t)K, NULL), bm = file_buf(fm, (size_t)C, NULL);
    cl_mem br = file_buf(fr, (size_t)C, NULL), ba = file_buf(fa, (size_t)C, NULL);
    cl_mem bo = buf((size_t)K * H * W * 4, NULL);
    size_t gs[3] = {(size_t)(W + 15) / 16 * 16, (size_t)(H + 15) / 16 * 16, (size_t)(K + 7) / 8};
    size_t ls[3] = {16, 16, 1};

    SET(k, 0, bi);
    SET(k, 1, (cl_int)C);
    SET(k, 2, (cl_int)H);
    SET(k, 3, (cl_int)W);
    SET(k, 4, bw);
    SET(k, 5, bb);
    SET(k, 6, (cl_int)K);
    SET(k, 7, norm ? bm : bw);
    SET(k, 8, norm ? br : bw);
    SET(k, 9, norm ? ba : bw);
    SET(k, 10, (cl_int)norm);
    SET(k, 11, bo);
    launch(k, 3, gs, ls);
    buf_file(bo, (size_t)K * H * W, fo);
    printf("{\"case\": \"%s\", \"kernel\": \"conv5x5\"}\n", spec);
    clReleaseMemObject(bi);
    clReleaseMemObject(bw);
    clReleaseMemObject(bb);
    clReleaseMemObject(bm);
    clReleaseMemObject(br);
    clReleaseMemObject(ba);
    clReleaseMemObject(bo);
    clReleaseKernel(k);
}

/* convx: the general conv2d kernel (ops.c:307-334) with geometry kh kw
 * sy sx py px (dilation 1), groups, bias and activation, no input
 * normalisation. */
static void exec_conv(const char *spec, const int *gm, int act, const char *fi, const char *fw,
                      const char *fb, const char *fo)
{
    const int C = gm[0], H = gm[1], W = gm[2], K = gm[3], kh = gm[4], kw = gm[5], sy = gm[6],
              sx = gm[7], py = gm[8], px = gm[9], groups = gm[10];
    const int Ho = (H + 2 * py - kh) / sy + 1, Wo = (W + 2 * px - kw) / sx + 1;
    cl_kernel k = kern(prog_ops, "conv2d");
    const cl_mem none = NULL;
    cl_mem bi = file_buf(fi, (size_t)C * H * W, NULL);
    cl_mem bw = file_buf(fw, (size_t)K * (C / groups) * kh * kw, NULL);
    cl_mem bb = file_buf(fb, (size_t)K, NULL), bo = buf((size_t)K * Ho * Wo * 4, NULL);
    const cl_int v[11] = {Ho, Wo, kh, kw, sy, sx, py, px, 1, 1, groups};
    size_t gs[3] = {(size_t)(Wo + 15) / 16 * 16, (size_t)(Ho + 3) / 4 * 4, (size_t)K};
    size_t ls[3] = {16, 4, 1};

    SET(k, 0, bi);
    SET(k, 1, (cl_int)C);
    SET(k, 2, (cl_int)H);
    SET(k, 3, (cl_int)W);
    SET(k, 4, bw);
    SET(k, 5, bb);
    SET(k, 6, (cl_int)K);
    for (int i = 0; i < 11; i++)
        SET(k, 7 + i, v[i]);
    SET(k, 18, none);
    SET(k, 19, none);
    SET(k, 20, none);
    SET(k, 21, (cl_int)act);
    SET(k, 22, (cl_float)0.1f);
    SET(k, 23, bo);
    launch(k, 3, gs, ls);
    buf_file(bo, (size_t)K * Ho * Wo, fo);
    printf("{\"case\": \"%s\", \"kernel\": \"conv2d\"}\n", spec);
    clReleaseMemObject(bi);
    clReleaseMemObject(bw);
    clReleaseMemObject(bb);
    clReleaseMemObject(bo);
    clReleaseKernel(k);
}

/* statx: chan_stats (ops.c:338-352); OUT: mean then rstd, C floats each. */
static void exec_stats(const char *spec, int C, int HW, float eps, const char *fx,
                       const char *fo)
{
    cl_kernel k = kern(prog_ops, "chan_stats");
    cl_mem bx = file_buf(fx, (size_t)C * HW, NULL), bo = buf((size_t)2 * C * 4, NULL);
    cl_mem bm = buf((size_t)C * 4, NULL), br = buf((size_t)C * 4, NULL);
    size_t g = (size_t)C * 256, l = 256;
    float *h = malloc((size_t)2 * C * 4);

    SET(k, 0, bx);
    SET(k, 1, (cl_int)HW);
    SET(k, 2, (cl_float)eps);
    SET(k, 3, bm);
    SET(k, 4, br);
    launch(k, 1, &g, &l);
    readb(bm, (size_t)C * 4, h);
    readb(br, (size_t)C * 4, h + C);
    write_file(fo, h, (size_t)2 * C * 4);
    printf("{\"case\": \"%s\", \"kernel\": \"chan_stats\"}\n", spec);
    free(h);
    clReleaseMemObject(bx);
    clReleaseMemObject(bo);
    clReleaseMemObject(bm);
    clReleaseMemObject(br);
    clReleaseKernel(k);
}

/* resx: resize_bilinear (ops.c:496-516), output channels from 0. */
static void exec_resize(const char *spec, int C, int h, int w, int H, int W, int align,
                        float scale, const char *fi, const char *fo)
{
    cl_kernel k = kern(prog_ops, "resize_bilinear");
    cl_mem bi = file_buf(fi, (size_t)C * h * w, NULL), bo = buf((size_t)C * H * W * 4, NULL);
    const cl_float sy = scale > 0 ? 1.0f / scale : (float)h / H;
    const cl_float sx = scale > 0 ? 1.0f / scale : (float)w / W;
    size_t g[3] = {(size_t)W, (size_t)H, (size_t)C};

    SET(k, 0, bi);
    SET(k, 1, (cl_int)h);
    SET(k, 2, (cl_int)w);
    SET(k, 3, bo);
    SET(k, 4, (cl_int)H);
    SET(k, 5, (cl_int)W);
    SET(k, 6, (cl_int)0);
    SET(k, 7, (cl_int)align);
    SET(k, 8, sy);
    SET(k, 9, sx);
    launch(k, 3, g, NULL);
    buf_file(bo, (size_t)C * H * W, fo);
    printf("{\"case\": \"%s\", \"kernel\": \"resize_bilinear\"}\n", spec);
    clReleaseMemObject(bi);
    clReleaseMemObject(bo);
    clReleaseKernel(k);
}

/* poolx: pool2d (ops.c:559-578), max or average. */
static void exec_pool(const char *spec, int C, int H, int W, int ks, int s, int p, int max,
                      const char *fi, const char *fo)
{
    cl_kernel k = kern(prog_ops, "pool2d");
    const int Ho = (H + 2 * p - ks) / s + 1, Wo = (W + 2 * p - ks) / s + 1;
    cl_mem bi = file_buf(fi, (size_t)C * H * W, NULL), bo = buf((size_t)C * Ho * Wo * 4, NULL);
    size_t g[3] = {(size_t)Wo, (size_t)Ho, (size_t)C};

    SET(k, 0, bi);
    SET(k, 1, (cl_int)H);
    SET(k, 2, (cl_int)W);
    SET(k, 3, (cl_int)Ho);
    SET(k, 4, (cl_int)Wo);
    SET(k, 5, (cl_int)ks);
    SET(k, 6, (cl_int)s);
    SET(k, 7, (cl_int)p);
    SET(k, 8, (cl_int)max);
    SET(k, 9, bo);
    launch(k, 3, g, NULL);
    buf_file(bo, (size_t)C * Ho * Wo, fo);
    printf("{\"case\": \"%s\", \"kernel\": \"pool2d\"}\n", spec);
    clReleaseMemObject(bi);
    clReleaseMemObject(bo);
    clReleaseKernel(k);
}

/* ropex: rope in place on rows of ld floats from offset 0 (ops.c:476-494);
 * CS: npos x d / 2 (cos, sin) pairs. */
static void exec_rope(const char *spec, int rows, int ld, int nh, int d, int npos,
                      int interleaved, const char *fx, const char *fcs, const char *fo)
{
    cl_kernel k = kern(prog_ops, "rope");
    cl_mem bx = file_buf(fx, (size_t)rows * ld, NULL), bc = file_buf(fcs, (size_t)npos * d, NULL);
    const cl_int n = rows * nh * (d / 2);
    size_t l = 256, g = ((size_t)n + l - 1) / l * l;

    SET(k, 0, bx);
    SET(k, 1, (cl_long)0);
    SET(k, 2, (cl_int)ld);
    SET(k, 3, (cl_int)nh);
    SET(k, 4, (cl_int)d);
    SET(k, 5, (cl_int)npos);
    SET(k, 6, bc);
    SET(k, 7, (cl_int)interleaved);
    SET(k, 8, n);
    launch(k, 1, &g, &l);
    buf_file(bx, (size_t)rows * ld, fo);
    printf("{\"case\": \"%s\", \"kernel\": \"rope\"}\n", spec);
    clReleaseMemObject(bx);
    clReleaseMemObject(bc);
    clReleaseKernel(k);
}

/* finex: eloftr_fine for M coarse matches, eloftr.c:606-634; CELLS: M
 * int4 (x0, y0, x1, y1); OUT: M float4 keypoints. */
static void exec_fine(const char *spec, int H, int W, int M, float T, const char *ff0,
                      const char *ff1, const char *fc, const char *fo)
{
    cl_program pe = need_program(prog_eloftr, "eloftr_kernels");
    cl_kernel k = kern(pe, "eloftr_fine");
    const size_t n = (size_t)64 * H * W;
    int *cells = read_file(fc, (size_t)M * 16);
    cl_mem b0 = file_buf(ff0, n, NULL), b1 = file_buf(ff1, n, NULL);
    cl_mem bc = buf((size_t)M * 16, cells), bo = buf((size_t)M * 16, NULL);
    size_t g = (size_t)M * 256, l = 256;

    SET(k, 0, b0);
    SET(k, 1, b1);
    SET(k, 2, (cl_int)H);
    SET(k, 3, (cl_int)W);
    SET(k, 4, bc);
    SET(k, 5, (cl_int)M);
    SET(k, 6, (cl_float)T);
    SET(k, 7, bo);
    launch(k, 1, &g, &l);
    buf_file(bo, (size_t)M * 4, fo);
    printf("{\"case\": \"%s\", \"kernel\": \"eloftr_fine\"}\n", spec);
    free(cells);
    clReleaseMemObject(b0);
    clReleaseMemObject(b1);
    clReleaseMemObject(bc);
    clReleaseMemObject(bo);
    clReleaseKernel(k);
}

/* Launch kernel name on a 1-D range of n items (local size 256, as
 * ops.c's run1d, or the runtime's choice when l0 is 0, as roma.c's run). */
static void launch1d(cl_kernel k, size_t n, int l0)
{
    size_t l = 256, g = (n + l - 1) / l * l;

    if (l0)
        launch(k, 1, &g, &l);
    else
        launch(k, 1, &n, NULL);
}

/* smallx:KIND:a:b:c:x:y:F1:F2:F3:F4:F5:OUT — the small element-wise
 * kernels with their reference dispatch; a, b, c integers, x, y floats,
 * F1..F5 input files ("-" unused), OUT the output buffer(s) in order:
 *   affine   chan_affine (ops.c:354-373): C=a HW=b act=c slope=x;
 *            X MEAN RSTD G B; OUT Y
 *   prelu    prelu (ops.c:375-386): C=a HW=b; X ALPHA; OUT Y
 *   act      act_map (ops.c:388-400): n=a act=c slope=x; X; OUT Y
 *   unfold   unfold (ops.c:218-234), 3 x 3 stride b padding c over
 *            C=a channels of an 16 x 20 map; IN; OUT
 *   avgpool2 avgpool2 (ops.c:546-557): C=a H=b W=c; IN; OUT
 *   transpose transpose2d (ops.c:580-593): B=a R=b C=c; IN; OUT
 *   axpby    axpby (ops.c:595-610): n=a bmod=b alpha=x beta=y; A B; OUT
 *   rownorm  roma_row_norm (roma.c:858-868): rows=a C=b; X; OUT
 *   cosexp   roma_cos_exp (roma.c:838-856): N=a M=b T=x eps=y; S NX NY;
 *            OUT S
 *   disp     roma_disp (roma.c:940-952): H=a W=b fx=x fy=y; FLOW; OUT
 *   update   roma_update (roma.c:987-995): n=a scale=x Wf=y Hf=c;
 *            FLOW CERT D; OUT FLOW then CERT
 *   update2  roma2_update (roma.c:1095-1103): n=a W=x H=y; FLOW CONF D;
 *            OUT FLOW then CONF */
static void exec_small(const char *spec, const char *kind, int a, int b, int c, float x,
                       float y, char f[5][1024], const char *fo)
{
    cl_mem in[5] = {NULL, NULL, NULL, NULL, NULL}, o1 = NULL, o2 = NULL;
    size_t no1 = 0, no2 = 0, sz[5] = {0, 0, 0, 0, 0};
    cl_kernel k;
    int i;

    if (!strcmp(kind, "affine")) {
        const size_t n = (size_t)a * b;

        sz[0] = n, sz[1] = sz[2] = sz[3] = sz[4] = (size_t)a;
        for (i = 0; i < 5; i++)
            in[i] = file_buf(f[i], sz[i], NULL);
        o1 = buf(n * 4, NULL), no1 = n;
        k = kern(prog_ops, "chan_affine");
        SET(k, 0, in[0]);
        SET(k, 1, o1);
        SET(k, 2, (cl_int)b);
        SET(k, 3, (cl_int)n);
        SET(k, 4, in[1]);
        SET(k, 5, in[2]);
        SET(k, 6, in[3]);
        SET(k, 7, in[4]);
        SET(k, 8, (cl_int)c);
        SET(k, 9, (cl_float)x);
        launch1d(k, n, 1);
    }
    else if (!strcmp(kind, "prelu")) {
        const size_t n = (size_t)a * b;

        in[0] = file_buf(f[0], n, NULL), in[1] = file_buf(f[1], (size_t)a, NULL);
        o1 = buf(n * 4, NULL), no1 = n;
        k = kern(prog_ops, "prelu");
        SET(k, 0, in[0]);
        SET(k, 1, o1);
        SET(k, 2, (cl_int)b);
        SET(k, 3, (cl_int)n);
        SET(k, 4, in[1]);
        launch1d(k, n, 1);
    }
    else if (!strcmp(kind, "act")) {
        in[0] = file_buf(f[0], (size_t)a, NULL);
        o1 = buf((size_t)a * 4, NULL), no1 = (size_t)a;
        k = kern(prog_ops, "act_map");
        SET(k, 0, in[0]);
        SET(k, 1, o1);
        SET(k, 2, (cl_int)a);
        SET(k, 3, (cl_int)c);
        SET(k, 4, (cl_float)x);
        launch1d(k, (size_t)a, 1);
    }
    else if (!strcmp(kind, "unfold")) {
        const int H = 16, W = 20, Ho = (H + 2 * c - 3) / b + 1, Wo = (W + 2 * c - 3) / b + 1;
        const cl_int v[13] = {a, H, W, 3, 3, b, b, c, c, Ho, Wo, 0, Ho * Wo};
        size_t gs[2] = {(size_t)(Ho * Wo + 63) / 64 * 64, (size_t)a * 9}, ls[2] = {64, 1};

        in[0] = file_buf(f[0], (size_t)a * H * W, NULL);
        no1 = (size_t)a * 9 * Ho * Wo, o1 = buf(no1 * 4, NULL);
        k = kern(prog_ops, "unfold");
        SET(k, 0, in[0]);
        for (i = 0; i < 13; i++)
            SET(k, 1 + i, v[i]);
        SET(k, 14, o1);
        launch(k, 2, gs, ls);
    }
    else if (!strcmp(kind, "avgpool2")) {
        size_t g[3] = {(size_t)c / 2, (size_t)b / 2, (size_t)a};

        in[0] = file_buf(f[0], (size_t)a * b * c, NULL);
        no1 = (size_t)a * (b / 2) * (c / 2), o1 = buf(no1 * 4, NULL);
        k = kern(prog_ops, "avgpool2");
        SET(k, 0, in[0]);
        SET(k, 1, (cl_int)b);
        SET(k, 2, (cl_int)c);
        SET(k, 3, o1);
        launch(k, 3, g, NULL);
    }
    else if (!strcmp(kind, "transpose")) {
        size_t g[3] = {(size_t)(c + 15) / 16 * 16, (size_t)(b + 15) / 16 * 16, (size_t)a};
        size_t l[3] = {16, 16, 1};

        in[0] = file_buf(f[0], (size_t)a * b * c, NULL);
        no1 = (size_t)a * b * c, o1 = buf(no1 * 4, NULL);
        k = kern(prog_ops, "transpose2d");
        SET(k, 0, in[0]);
        SET(k, 1, o1);
        SET(k, 2, (cl_int)b);
        SET(k, 3, (cl_int)c);
        launch(k, 3, g, l);
    }
    else if (!strcmp(kind, "axpby")) {
        in[0] = file_buf(f[0], (size_t)a, NULL), in[1] = file_buf(f[1], (size_t)b, NULL);
        o1 = buf((size_t)a * 4, NULL), no1 = (size_t)a;
        k = kern(prog_ops, "axpby");
        SET(k, 0, o1);
        SET(k, 1, in[0]);
        SET(k, 2, (cl_float)x);
        SET(k, 3, in[1]);
        SET(k, 4, (cl_float)y);
        SET(k, 5, (cl_int)a);
        SET(k, 6, (cl_int)b);
        launch1d(k, (size_t)a, 1);
    }
    else if (!strcmp(kind, "rownorm")) {
        in[0] = file_buf(f[0], (size_t)a * b, NULL);
        o1 = buf((size_t)a * 4, NULL), no1 = (size_t)a;
        k = kern(prog_roma, "roma_row_norm");
        SET(k, 0, in[0]);
        SET(k, 1, (cl_int)a);
        SET(k, 2, (cl_int)b);
        SET(k, 3, o1);
        launch1d(k, (size_t)a, 0);
    }
    else if (!strcmp(kind, "cosexp")) {
        size_t g[2] = {(size_t)b, (size_t)a};

        o1 = file_buf(f[0], (size_t)a * b, NULL), no1 = (size_t)a * b;
        in[1] = file_buf(f[1], (size_t)a, NULL), in[2] = file_buf(f[2], (size_t)b, NULL);
        k = kern(prog_roma, "roma_cos_exp");
        SET(k, 0, o1);
        SET(k, 1, in[1]);
        SET(k, 2, in[2]);
        SET(k, 3, (cl_int)a);
        SET(k, 4, (cl_int)b);
        SET(k, 5, (cl_float)x);
        SET(k, 6, (cl_float)y);
        launch(k, 2, g, NULL);
    }
    else if (!strcmp(kind, "disp")) {
        const size_t n = (size_t)a * b;

        in[0] = file_buf(f[0], 2 * n, NULL);
        o1 = buf(2 * n * 4, NULL), no1 = 2 * n;
        k = kern(prog_roma, "roma_disp");
        SET(k, 0, in[0]);
        SET(k, 1, (cl_int)a);
        SET(k, 2, (cl_int)b);
        SET(k, 3, (cl_float)x);
        SET(k, 4, (cl_float)y);
        SET(k, 5, o1);
        launch1d(k, n, 0);
    }
    else if (!strcmp(kind, "update")) {
        o1 = file_buf(f[0], 2 * (size_t)a, NULL), no1 = 2 * (size_t)a;
        o2 = file_buf(f[1], (size_t)a, NULL), no2 = (size_t)a;
        in[2] = file_buf(f[2], 3 * (size_t)a, NULL);
        k = kern(prog_roma, "roma_update");
        SET(k, 0, o1);
        SET(k, 1, o2);
        SET(k, 2, in[2]);
        SET(k, 3, (cl_int)a);
        SET(k, 4, (cl_float)x);
        SET(k, 5, (cl_float)y);
        SET(k, 6, (cl_float)c);
        launch1d(k, (size_t)a, 0);
    }
    else if (!strcmp(kind, "update2")) {
        o1 = file_buf(f[0], 2 * (size_t)a, NULL), no1 = 2 * (size_t)a;
        o2 = file_buf(f[1], 4 * (size_t)a, NULL), no2 = 4 * (size_t)a;
        in[2] = file_buf(f[2], 6 * (size_t)a, NULL);
        k = kern(prog_roma, "roma2_update");
        SET(k, 0, o1);
        SET(k, 1, o2);
        SET(k, 2, in[2]);
        SET(k, 3, (cl_int)a);
        SET(k, 4, (cl_float)x);
        SET(k, 5, (cl_float)y);
        launch1d(k, (size_t)a, 0);
    }
    else {
        fprintf(stderr, "ref_ocl: unknown small kernel %s\n", kind);
        exit(2);
    }
    {
        float *h = malloc((no1 + no2) * 4);

        readb(o1, no1 * 4, h);
        if (o2)
            readb(o2, no2 * 4, h + no1);
        write_file(fo, h, (no1 + no2) * 4);
        free(h);
    }
    printf("{\"case\": \"%s\", \"kernel\": \"%s\"}\n", spec, kind);
    for (i = 0; i < 5; i++)
        if (in[i] && in[i] != o1)
            clReleaseMemObject(in[i]);
    clReleaseMemObject(o1);
    if (o2)
        clReleaseMemObject(o2);
    clReleaseKernel(k);
}

/* A code object of DIR when it was built, else NULL. */
static cl_program load_optional(const char *dir, const char *name)
{
    char path[4096];
    FILE *fp;

    snprintf(path, sizeof(path), "%s/%s.co", dir, name);
    fp = fopen(path, "rb");
    if (!fp)
        return NULL;
    fclose(fp);
    return load_program(path);
}

int main(int argc, char **argv)
{
    cl_platform_id plat;
    cl_uint np = 0;
    cl_int e;
    char path[4096], name[256] = "";

    if (argc < 3) {
        fprintf(stderr, "usage: ref_ocl DIR CASE...\n");
        return 2;
    }
    CK(clGetPlatformIDs(1, &plat, &np));
    CK(clGetDeviceIDs(plat, CL_DEVICE_TYPE_GPU, 1, &devid, NULL));
    clGetDeviceInfo(devid, CL_DEVICE_NAME, sizeof(name), name, NULL);
    ctx = clCreateContext(NULL, 1, &devid, NULL, NULL, &e);
    if (e != CL_SUCCESS)
        die("clCreateContext", e);
    q = clCreateCommandQueue(ctx, devid, CL_QUEUE_PROFILING_ENABLE, &e);
    if (e != CL_SUCCESS)
        die("clCreateCommandQueue", e);
    snprintf(path, sizeof(path), "%s/ops.co", argv[1]);
    prog_ops = load_program(path);
    snprintf(path, sizeof(path), "%s/roma_kernels.co", argv[1]);
    prog_roma = load_program(path);
    k_gemm = kern(prog_ops, "gemm");
    k_gemm_big = kern(prog_ops, "gemm_big");
    k_softmax = kern(prog_ops, "softmax_rows");
    k_layernorm = kern(prog_ops, "layernorm");
    k_attention = kern(prog_ops, "attention");
    k_grid = kern(prog_ops, "grid_sample");
    k_corr = kern(prog_roma, "roma_local_corr");
    k_warp = kern(prog_roma, "roma_warp_sample");
    prog_eloftr = load_optional(argv[1], "eloftr_kernels");
    prog_disk = load_optional(argv[1], "disk_kernels");
    fprintf(stderr, "ref_ocl: device %s\n", name);
    for (int i = 2; i < argc; i++) {
        int a = 0, b = 0, c = 0, d = 0, e5 = 0;
        long lo = 0;
        float fl = 0.0f;
        int gm[11] = {0};
        float fl2 = 0.0f;
        char kind[32], ff[5][1024];
        char f1[1024], f2[1024], f3[1024], f4[1024], f5[1024], f6[1024], f7[1024];

        if (sscanf(argv[i], "coarse:%d:%d:%1023[^:]:%1023s", &a, &b, f1, f2) == 4)
            exec_coarse(argv[i], a, b, f1, f2);
        else if (sscanf(argv[i], "nms:%d:%d:%d:%ld:%f:%1023[^:]:%1023s", &a, &b, &c, &lo, &fl,
                        f1, f2) == 7)
            exec_nms(argv[i], a, b, c, lo, fl, f1, f2);
        else if (sscanf(argv[i], "gather:%d:%d:%d:%d:%1023[^:]:%1023[^:]:%1023s", &a, &b, &c,
                        &d, f1, f2, f3) == 7)
            exec_gather(argv[i], a, b, c, d, f1, f2, f3);
        else if (sscanf(argv[i], "cls:%d:%d:%d:%d:%1023[^:]:%1023s", &a, &b, &c, &d, f1, f2) == 6)
            exec_cls(argv[i], a, b, c, d, f1, f2);
        else if (sscanf(argv[i], "gemmx:%d:%d:%d:%d:%d:%1023[^:]:%1023[^:]:%1023[^:]:%1023s",
                        &a, &b, &c, &d, &e5, f1, f2, f3, f4) == 9)
            exec_gemm(argv[i], a, b, c, d, e5, f1, f2, f3, f4);
        else if (sscanf(argv[i], "lnx:%d:%d:%f:%1023[^:]:%1023[^:]:%1023[^:]:%1023s", &a, &b,
                        &fl, f1, f2, f3, f4) == 7)
            exec_layernorm(argv[i], a, b, fl, f1, f2, f3, f4);
        else if (sscanf(argv[i], "smx:%d:%d:%f:%1023[^:]:%1023s", &a, &b, &fl, f1, f2) == 5)
            exec_softmax(argv[i], a, b, fl, f1, f2);
        else if (sscanf(argv[i], "attnx:%d:%d:%d:%d:%f:%1023[^:]:%1023[^:]:%1023[^:]:%1023s",
                        &a, &b, &c, &d, &fl, f1, f2, f3, f4) == 9)
            exec_attention(argv[i], a, b, c, d, fl, f1, f2, f3, f4);
        else if (sscanf(argv[i], "lcx:%d:%d:%d:%d:%1023[^:]:%1023[^:]:%1023[^:]:%1023s", &a,
                        &b, &c, &d, f1, f2, f3, f4) == 8)
            exec_localcorr(argv[i], a, b, c, d, f1, f2, f3, f4);
        else if (sscanf(argv[i], "warpx:%d:%d:%d:%1023[^:]:%1023[^:]:%1023s", &a, &b, &c, f1,
                        f2, f3) == 6)
            exec_warpsample(argv[i], a, b, c, f1, f2, f3);
        else if (sscanf(argv[i], "gridx:%d:%d:%d:%d:%d:%1023[^:]:%1023[^:]:%1023s", &a, &b, &c,
                        &d, &e5, f1, f2, f3) == 8)
            exec_gridsample(argv[i], a, b, c, d, e5, f1, f2, f3);
        else if (sscanf(argv[i], "dwx:%d:%d:%d:%1023[^:]:%1023[^:]:%1023[^:]:%1023s", &a, &b,
                        &c, f1, f2, f3, f4) == 7)
            exec_dwconv(argv[i], a, b, c, f1, f2, f3, f4);
        else if (sscanf(argv[i], "c5x:%d:%d:%d:%d:%d:%1023[^:]:%1023[^:]:%1023[^:]:%1023[^:]:"
                        "%1023[^:]:%1023[^:]:%1023s", &a, &b, &c, &d, &e5, f1, f2, f3, f4, f5,
                        f6, f7) == 12)
            exec_conv5(argv[i], a, b, c, d, e5, f1, f2, f3, f4, f5, f6, f7);
        else if (sscanf(argv[i], "convx:%d:%d:%d:%d:%d:%d:%d:%d:%d:%d:%d:%d:%1023[^:]:%1023[^:]:"
                        "%1023[^:]:%1023s", &gm[0], &gm[1], &gm[2], &gm[3], &gm[4], &gm[5],
                        &gm[6], &gm[7], &gm[8], &gm[9], &gm[10], &e5, f1, f2, f3, f4) == 16)
            exec_conv(argv[i], gm, e5, f1, f2, f3, f4);
        else if (sscanf(argv[i], "statx:%d:%d:%f:%1023[^:]:%1023s", &a, &b, &fl, f1, f2) == 5)
            exec_stats(argv[i], a, b, fl, f1, f2);
        else if (sscanf(argv[i], "resx:%d:%d:%d:%d:%d:%d:%f:%1023[^:]:%1023s", &a, &b, &c, &d,
                        &gm[0], &e5, &fl, f1, f2) == 9)
            exec_resize(argv[i], a, b, c, d, gm[0], e5, fl, f1, f2);
        else if (sscanf(argv[i], "poolx:%d:%d:%d:%d:%d:%d:%d:%1023[^:]:%1023s", &a, &b, &c,
                        &gm[0], &gm[1], &gm[2], &e5, f1, f2) == 9)
            exec_pool(argv[i], a, b, c, gm[0], gm[1], gm[2], e5, f1, f2);
        else if (sscanf(argv[i], "ropex:%d:%d:%d:%d:%d:%d:%1023[^:]:%1023[^:]:%1023s", &a, &b,
                        &c, &d, &gm[0], &e5, f1, f2, f3) == 9)
            exec_rope(argv[i], a, b, c, d, gm[0], e5, f1, f2, f3);
        else if (sscanf(argv[i], "finex:%d:%d:%d:%f:%1023[^:]:%1023[^:]:%1023[^:]:%1023s", &a,
                        &b, &c, &fl, f1, f2, f3, f4) == 8)
            exec_fine(argv[i], a, b, c, fl, f1, f2, f3, f4);
        else if (sscanf(argv[i], "smallx:%31[^:]:%d:%d:%d:%f:%f:%1023[^:]:%1023[^:]:%1023[^:]:"
                        "%1023[^:]:%1023[^:]:%1023s", kind, &a, &b, &c, &fl, &fl2, ff[0], ff[1],
                        ff[2], ff[3], ff[4], f1) == 12)
            exec_small(argv[i], kind, a, b, c, fl, fl2, ff, f1);
        else if (sscanf(argv[i], "gemm:%d:%d:%d:%d", &a, &b, &c, &d) == 4)
            case_gemm(argv[i], a, b, c, d);
        else if (sscanf(argv[i], "vitblock:%d", &a) == 1)
            case_vitblock(argv[i], a);
        else if (sscanf(argv[i], "attention:%d:%d:%d:%d", &a, &b, &c, &d) == 4)
            case_attention(argv[i], a, b, c, d);
        else if (sscanf(argv[i], "localcorr:%d:%d:%d:%d", &a, &b, &c, &d) == 4)
            case_localcorr(argv[i], a, b, c, d);
        else if (sscanf(argv[i], "warpsample:%d:%d:%d", &a, &b, &c) == 3)
            case_warpsample(argv[i], a, b, c);
        else if (sscanf(argv[i], "gridsample:%d:%d:%d:%d", &a, &b, &c, &d) == 4)
            case_gridsample(argv[i], a, b, c, d);
        else {
            fprintf(stderr, "ref_ocl: unknown case %s\n", argv[i]);
            return 2;
        }
        fflush(stdout);
    }
    clReleaseCommandQueue(q);
    clReleaseContext(ctx);
    return 0;
}

/* SPDX-License-Identifier: Unlicense */

/* ORACLE — test infrastructure only (see oracle.h): CPU restatement of
 * the reference's generic kernels (ops.cl) and ELoFTR kernels
 * (eloftr_kernels.cl) of i.coregistration.opencl, float32 arithmetic in
 * each kernel's own order of summation where it matters (GEMM and
 * convolution sums in k order with fused multiply-adds, as mad). */

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define ACT_NONE 0
#define ACT_GELU 1
#define ACT_RELU 2
#define ACT_LEAKY 3
#define ACT_GELU_TANH 4

/* ---- xorshift64, tests/ops_check.c:33-42 ------------------------------ */

static uint64_t rng = 88172645463325252ULL;

void orc_rng_seed(uint64_t s) { rng = s; }
uint64_t orc_rng_state(void) { return rng; }

float orc_urand(float lo, float hi)
{
    rng ^= rng << 13;
    rng ^= rng >> 7;
    rng ^= rng << 17;
    return lo + (hi - lo) * (float)((rng >> 11) * (1.0 / 9007199254740992.0));
}

void orc_rand_fill(float *v, long n, float lo, float hi)
{
    long i;

    for (i = 0; i < n; i++)
        v[i] = orc_urand(lo, hi);
}

/* ---- activations, ops.cl:23-37 ----------------------------------------- */

float orc_act(float v, int act, float slope)
{
    switch (act) {
    case ACT_GELU:
        return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
    case ACT_RELU:
        return fmaxf(v, 0.0f);
    case ACT_LEAKY:
        return v >= 0.0f ? v : slope * v;
    case ACT_GELU_TANH:
        return 0.5f * v *
               (1.0f + tanhf(0.79788456080286536f * (v + 0.044715f * v * v * v)));
    }
    return v;
}

/* ---- GEMM, ops.cl:39-138 ----------------------------------------------- */

void orc_gemm(int M, int N, int K, const float *A, long aoff, int lda,
              long sa0, long sa1, const float *B, long boff, int ldb,
              long sb0, long sb1, int transb, float *C, long coff, int ldc,
              long sc0, long sc1, int nb, int nb1, const float *bias,
              int biasrow, const float *R, long roff, float alpha, int act,
              float slope)
{
    long bm;

#pragma omp parallel for schedule(static)
    for (bm = 0; bm < (long)nb * M; bm++) {
        const long b = bm / M, m = bm % M, b0 = b / nb1, b1 = b % nb1;
        const float *a = A + aoff + b0 * sa0 + b1 * sa1 + m * lda;
        const float *bb = B + boff + b0 * sb0 + b1 * sb1;
        float *c = C + coff + b0 * sc0 + b1 * sc1 + m * ldc;
        const float *r = R ? R + roff + b0 * sc0 + b1 * sc1 + m * ldc : NULL;
        int n, k;

        /* Without transb the row of C is accumulated k-outer over
         * contiguous rows of B: the same fmaf sequence per output (k
         * ascending) as the dot-product loop, so the same values. */
        float *row = NULL;

        if (!transb) {
            row = calloc(N > 0 ? N : 1, sizeof(float));
            for (k = 0; k < K; k++) {
                const float ak = a[k], *bk = bb + (long)k * ldb;

                for (n = 0; n < N; n++)
                    row[n] = fmaf(ak, bk[n], row[n]);
            }
        }
        for (n = 0; n < N; n++) {
            float acc = 0.0f, v;

            if (transb)
                for (k = 0; k < K; k++)
                    acc = fmaf(a[k], bb[(long)n * ldb + k], acc);
            else
                acc = row[n];
            v = alpha * acc;
            if (bias)
                v += bias[biasrow ? m : n];
            v = orc_act(v, act, slope);
            if (r)
                v += r[n];
            c[n] = v;
        }
        free(row);
    }
}

/* ---- convolution, ops.cl:389-448 ---------------------------------------- */

void orc_conv2d(const float *in, int C, int H, int W, const float *w,
                const float *b, int K, int kh, int kw, int sy, int sx, int py,
                int px, int dy, int dx, int groups, const float *mean,
                const float *rstd, const float *alpha, int act, float slope,
                float *out)
{
    const int Ho = (H + 2 * py - dy * (kh - 1) - 1) / sy + 1;
    const int Wo = (W + 2 * px - dx * (kw - 1) - 1) / sx + 1;
    const int cg = C / groups, kg = K / groups;
    long ky;

#pragma omp parallel for schedule(static)
    for (ky = 0; ky < (long)K * Ho; ky++) {
        const int k = (int)(ky / Ho), y = (int)(ky % Ho), c0 = (k / kg) * cg;
        const float *wk = w + (long)k * cg * kh * kw;
        int x;

        for (x = 0; x < Wo; x++) {
            float acc = 0.0f;
            int c, i, j;

            for (c = 0; c < cg; c++) {
                const float *src = in + (long)(c0 + c) * H * W;
                float m = 0.0f, r = 1.0f, a = 1.0f;

                if (mean) {
                    m = mean[c0 + c];
                    r = rstd[c0 + c];
                    if (alpha)
                        a = alpha[c0 + c];
                }
                for (i = 0; i < kh; i++) {
                    const int iy = y * sy - py + i * dy;

                    if (iy < 0 || iy >= H)
                        continue;
                    for (j = 0; j < kw; j++) {
                        const int ix = x * sx - px + j * dx;
                        float v;

                        if (ix < 0 || ix >= W)
                            continue;
                        v = src[(long)iy * W + ix];
                        if (mean) {
                            v = (v - m) * r;
                            v = v >= 0.0f ? v : a * v;
                        }
                        acc = fmaf(v, wk[(c * kh + i) * kw + j], acc);
                    }
                }
            }
            if (b)
                acc += b[k];
            out[((long)k * Ho + y) * Wo + x] = orc_act(acc, act, slope);
        }
    }
}

/* ---- normalisation and element-wise ------------------------------------ */

void orc_chan_stats(const float *x, int C, int HW, float eps, float *mean,
                    float *rstd)
{
    int c, i;

    for (c = 0; c < C; c++) {
        const float *p = x + (long)c * HW;
        float s = 0.0f, m;

        for (i = 0; i < HW; i++)
            s += p[i];
        m = s / HW;
        s = 0.0f;
        for (i = 0; i < HW; i++) {
            const float d = p[i] - m;

            s += d * d;
        }
        mean[c] = m;
        rstd[c] = 1.0f / sqrtf(s / HW + eps);
    }
}

void orc_chan_affine(const float *X, float *Y, int C, int HW,
                     const float *mean, const float *rstd, const float *g,
                     const float *b, int act, float slope)
{
    long i, n = (long)C * HW;

    for (i = 0; i < n; i++) {
        const int c = (int)(i / HW);
        float v = X[i];

        if (mean)
            v = (v - mean[c]) * rstd[c];
        if (g)
            v *= g[c];
        if (b)
            v += b[c];
        Y[i] = orc_act(v, act, slope);
    }
}

void orc_prelu(const float *X, float *Y, int C, int HW, const float *alpha)
{
    long i, n = (long)C * HW;

    for (i = 0; i < n; i++)
        Y[i] = X[i] >= 0.0f ? X[i] : alpha[i / HW] * X[i];
}

void orc_act_map(const float *X, float *Y, long n, int act, float slope)
{
    long i;

    for (i = 0; i < n; i++)
        Y[i] = orc_act(X[i], act, slope);
}

void orc_layernorm(long rows, int C, const float *X, float *Y, const float *g,
                   const float *b, float eps, int act, float slope)
{
    long r;

#pragma omp parallel for schedule(static)
    for (r = 0; r < rows; r++) {
        const float *x = X + r * C;
        float *y = Y + r * C;
        float s = 0.0f, mean, var, rs;
        int c;

        for (c = 0; c < C; c++)
            s += x[c];
        mean = s / C;
        s = 0.0f;
        for (c = 0; c < C; c++) {
            const float d = x[c] - mean;

            s += d * d;
        }
        var = s / C;
        rs = 1.0f / sqrtf(var + eps);
        for (c = 0; c < C; c++) {
            float v = (x[c] - mean) * rs;

            if (g)
                v *= g[c];
            if (b)
                v += b[c];
            y[c] = orc_act(v, act, slope);
        }
    }
}

void orc_softmax_rows(float *S, long rows, int L, float scale)
{
    long r;

#pragma omp parallel for schedule(static)
    for (r = 0; r < rows; r++) {
        float *s = S + r * L, m = -INFINITY, sum = 0.0f, inv;
        int j;

        for (j = 0; j < L; j++)
            m = fmaxf(m, s[j] * scale);
        for (j = 0; j < L; j++) {
            s[j] = expf(s[j] * scale - m);
            sum += s[j];
        }
        inv = 1.0f / sum;
        for (j = 0; j < L; j++)
            s[j] *= inv;
    }
}

/* ---- attention, ops.cl:604-687 (whole rows instead of key blocks: the
 * same softmax) -------------------------------------------------------------- */

void orc_attention(const float *Q, long qoff, int ldq, const float *K,
                   long koff, int ldk, const float *V, long voff, int ldv,
                   float *O, long ooff, int ldo, int Nq, int Nk, int nh, int d,
                   float scale, const unsigned char *kmask)
{
    long hq;

#pragma omp parallel for schedule(static)
    for (hq = 0; hq < (long)nh * Nq; hq++) {
        const int h = (int)(hq / Nq), qi = (int)(hq % Nq);
        const float *q = Q + qoff + (long)qi * ldq + h * d;
        float *o = O + ooff + (long)qi * ldo + h * d;
        float *p = malloc((Nk > 0 ? Nk : 1) * sizeof(float));
        float m = -INFINITY, l = 0.0f;
        int j, c;

        for (j = 0; j < Nk; j++) {
            const float *k = K + koff + (long)j * ldk + h * d;
            float s = 0.0f;

            if (kmask && !kmask[j]) {
                p[j] = -INFINITY;
                continue;
            }
            for (c = 0; c < d; c++)
                s = fmaf(q[c] * scale, k[c], s);
            p[j] = s;
            m = fmaxf(m, s);
        }
        for (c = 0; c < d; c++)
            o[c] = 0.0f;
        if (m > -INFINITY) {
            for (j = 0; j < Nk; j++) {
                p[j] = p[j] == -INFINITY ? 0.0f : expf(p[j] - m);
                l += p[j];
            }
            for (j = 0; j < Nk; j++) {
                const float *v = V + voff + (long)j * ldv + h * d;

                if (p[j] == 0.0f)
                    continue;
                for (c = 0; c < d; c++)
                    o[c] = fmaf(p[j], v[c], o[c]);
            }
            for (c = 0; c < d; c++)
                o[c] /= l;
        }
        free(p);
    }
}

/* ---- RoPE, ops.cl:689-716 --------------------------------------------------- */

void orc_rope(float *X, long off, int ld, long rows, int nh, int d, int npos,
              const float *cs, int interleaved)
{
    const int nf = d / 2;
    long r;
    int h, f;

    for (r = 0; r < rows; r++)
        for (h = 0; h < nh; h++)
            for (f = 0; f < nf; f++) {
                float *x = X + off + r * ld + h * d;
                const float *rot = cs + ((r % npos) * nf + f) * 2;
                const int i0 = interleaved ? 2 * f : f;
                const int i1 = interleaved ? 2 * f + 1 : f + nf;
                const float a = x[i0], b = x[i1];

                x[i0] = a * rot[0] - b * rot[1];
                x[i1] = a * rot[1] + b * rot[0];
            }
}

/* ---- resampling ---------------------------------------------------------------- */

void orc_resize(const float *in, int C, int h, int w, float *out, int H, int W,
                int coff, int align_corners, float scale)
{
    const float sy = scale > 0 ? 1.0f / scale : (float)h / H;
    const float sx = scale > 0 ? 1.0f / scale : (float)w / W;
    int c, y, x;

    for (c = 0; c < C; c++)
        for (y = 0; y < H; y++)
            for (x = 0; x < W; x++) {
                const float *p = in + (long)c * h * w;
                float ux, uy, fx, fy;
                int x0, y0, x1, y1;

                if (align_corners) {
                    ux = W > 1 ? (float)x * (float)(w - 1) / (float)(W - 1)
                               : 0.0f;
                    uy = H > 1 ? (float)y * (float)(h - 1) / (float)(H - 1)
                               : 0.0f;
                }
                else {
                    ux = fmaxf(((float)x + 0.5f) * sx - 0.5f, 0.0f);
                    uy = fmaxf(((float)y + 0.5f) * sy - 0.5f, 0.0f);
                }
                x0 = (int)ux;
                y0 = (int)uy;
                x1 = x0 + 1 < w - 1 ? x0 + 1 : w - 1;
                y1 = y0 + 1 < h - 1 ? y0 + 1 : h - 1;
                fx = ux - x0;
                fy = uy - y0;
                out[((long)(c + coff) * H + y) * W + x] =
                    (1.0f - fy) *
                        ((1.0f - fx) * p[y0 * w + x0] + fx * p[y0 * w + x1]) +
                    fy * ((1.0f - fx) * p[y1 * w + x0] + fx * p[y1 * w + x1]);
            }
}

static float tap(const float *p, int H, int W, int y, int x)
{
    return x >= 0 && x < W && y >= 0 && y < H ? p[(long)y * W + x] : 0.0f;
}

void orc_grid_sample(const float *in, int C, int H, int W, const float *grid,
                     int n, int align_corners, float *out)
{
    int i, c;

    for (i = 0; i < n; i++) {
        const float gx = grid[2 * i], gy = grid[2 * i + 1];
        float ix, iy, fx, fy;
        int x0, y0;

        if (align_corners) {
            ix = (gx + 1.0f) * 0.5f * (W - 1);
            iy = (gy + 1.0f) * 0.5f * (H - 1);
        }
        else {
            ix = ((gx + 1.0f) * W - 1.0f) * 0.5f;
            iy = ((gy + 1.0f) * H - 1.0f) * 0.5f;
        }
        for (c = 0; c < C; c++) {
            const float *p = in + (long)c * H * W;
            float v = 0.0f;

            if (isfinite(ix) && isfinite(iy) && fabsf(ix) < 1e9f &&
                fabsf(iy) < 1e9f) {
                x0 = (int)floorf(ix);
                y0 = (int)floorf(iy);
                fx = ix - x0;
                fy = iy - y0;
                v = (1.0f - fy) * ((1.0f - fx) * tap(p, H, W, y0, x0) +
                                   fx * tap(p, H, W, y0, x0 + 1)) +
                    fy * ((1.0f - fx) * tap(p, H, W, y0 + 1, x0) +
                          fx * tap(p, H, W, y0 + 1, x0 + 1));
            }
            out[(long)c * n + i] = v;
        }
    }
}

void orc_unfold(const float *in, int C, int H, int W, int kh, int kw, int sy,
                int sx, int py, int px, float *out)
{
    const int Ho = (H + 2 * py - kh) / sy + 1, Wo = (W + 2 * px - kw) / sx + 1;
    const long L = (long)Ho * Wo;
    long row, t;

    for (row = 0; row < (long)C * kh * kw; row++) {
        const int c = (int)(row / (kh * kw)), i = (int)((row / kw) % kh);
        const int j = (int)(row % kw);

        for (t = 0; t < L; t++) {
            const int iy = (int)(t / Wo) * sy - py + i;
            const int ix = (int)(t % Wo) * sx - px + j;

            out[row * L + t] = iy >= 0 && iy < H && ix >= 0 && ix < W
                                   ? in[((long)c * H + iy) * W + ix]
                                   : 0.0f;
        }
    }
}

void orc_avgpool2(const float *in, int C, int H, int W, float *out)
{
    const int h = H / 2, w = W / 2;
    int c, y, x;

    for (c = 0; c < C; c++)
        for (y = 0; y < h; y++)
            for (x = 0; x < w; x++) {
                const float *p = in + ((long)c * H + 2 * y) * W + 2 * x;

                out[((long)c * h + y) * w + x] =
                    0.25f * (p[0] + p[1] + p[W] + p[W + 1]);
            }
}

void orc_pool2d(const float *in, int C, int H, int W, int k, int s, int p,
                int max, float *out)
{
    const int Ho = (H + 2 * p - k) / s + 1, Wo = (W + 2 * p - k) / s + 1;
    int c, y, x, i, j;

    for (c = 0; c < C; c++)
        for (y = 0; y < Ho; y++)
            for (x = 0; x < Wo; x++) {
                const float *src = in + (long)c * H * W;
                float acc = max ? -INFINITY : 0.0f;

                for (i = 0; i < k; i++) {
                    const int iy = y * s - p + i;

                    if (iy < 0 || iy >= H)
                        continue;
                    for (j = 0; j < k; j++) {
                        const int ix = x * s - p + j;

                        if (ix < 0 || ix >= W)
                            continue;
                        acc = max ? fmaxf(acc, src[iy * W + ix])
                                  : acc + src[iy * W + ix];
                    }
                }
                out[((long)c * Ho + y) * Wo + x] = max ? acc : acc / (k * k);
            }
}

void orc_transpose(const float *in, float *out, int B, int R, int C)
{
    int b, r, c;

    for (b = 0; b < B; b++)
        for (r = 0; r < R; r++)
            for (c = 0; c < C; c++)
                out[(long)b * R * C + (long)c * R + r] =
                    in[(long)b * R * C + (long)r * C + c];
}

void orc_axpby(float *out, const float *a, float alpha, const float *b,
               float beta, long n, long bmod)
{
    long i;

    if (bmod < 1)
        bmod = 1;
    for (i = 0; i < n; i++)
        out[i] = alpha * a[i] + (b ? beta * b[i % bmod] : 0.0f);
}

void orc_fold_bn(float *w, float *b, int K, long per, const float *gamma,
                 const float *beta, const float *mean, const float *var,
                 float eps)
{
    int k;
    long i;

    for (k = 0; k < K; k++) {
        const double s = gamma[k] / sqrt((double)var[k] + eps);

        for (i = 0; i < per; i++)
            w[(long)k * per + i] = (float)(w[(long)k * per + i] * s);
        b[k] = (float)((b[k] - mean[k]) * s + beta[k]);
    }
}

/* ---- ELoFTR coarse matching, eloftr_kernels.cl:10-144, eloftr.c:473-571 -- */

void orc_eloftr_coarse(const float *F0, const float *F1, int n, int D,
                       float alpha, int blk, float *row_max, int *row_arg,
                       int *col_arg, float *row_margin, float *col_margin,
                       float *col_max)
{
    float *S = malloc((size_t)n * n * sizeof(float));
    float *lse = malloc((size_t)n * sizeof(float));
    float *cm = malloc((size_t)n * sizeof(float));
    float *cs = malloc((size_t)n * sizeof(float));
    float *cmax = malloc((size_t)n * sizeof(float));
    float *c2 = malloc((size_t)n * sizeof(float));
    long i;
    int j, r0;

    if (blk < 1)
        blk = n;
    orc_gemm(n, n, D, F0, 0, D, 0, 0, F1, 0, D, 0, 0, 1, S, 0, n, 0, 0, 1, 1,
             NULL, 0, NULL, 0, alpha, ACT_NONE, 0.0f);
    /* Pass 0: row log-sum-exp; running column maximum and sum over the
     * row blocks. */
#pragma omp parallel for schedule(static)
    for (i = 0; i < n; i++) {
        const float *s = S + i * (long)n;
        float m = -INFINITY, sum = 0.0f;
        int k;

        for (k = 0; k < n; k++)
            m = fmaxf(m, s[k]);
        for (k = 0; k < n; k++)
            sum += expf(s[k] - m);
        lse[i] = m + logf(sum);
    }
    for (j = 0; j < n; j++) {
        cm[j] = -INFINITY;
        cs[j] = 0.0f;
        cmax[j] = -1.0f;
        c2[j] = -1.0f;
        col_arg[j] = -1;
    }
    for (r0 = 0; r0 < n; r0 += blk) {
        const int rows = n - r0 < blk ? n - r0 : blk;

#pragma omp parallel for schedule(static)
        for (i = 0; i < n; i++) {
            float m = -INFINITY, s = 0.0f, mo, mn;
            int r;

            for (r = 0; r < rows; r++)
                m = fmaxf(m, S[(long)(r0 + r) * n + i]);
            for (r = 0; r < rows; r++)
                s += expf(S[(long)(r0 + r) * n + i] - m);
            mo = cm[i];
            mn = fmaxf(mo, m);
            cs[i] = (mo == -INFINITY ? 0.0f : cs[i] * expf(mo - mn)) +
                    s * expf(m - mn);
            cm[i] = mn;
        }
    }
    /* Pass 1: dual-softmax confidence, row maximum and first argmax,
     * column first argmax over the row blocks in order. */
#pragma omp parallel for schedule(static)
    for (i = 0; i < n; i++) {
        const float *s = S + i * (long)n;
        float best = -1.0f, second = -1.0f;
        int bi = 0, k;

        for (k = 0; k < n; k++) {
            const float c =
                expf(s[k] - lse[i]) * expf(s[k] - (cm[k] + logf(cs[k])));

            if (c > best) {
                second = best;
                best = c;
                bi = k;
            }
            else if (c > second)
                second = c;
        }
        row_max[i] = best;
        row_arg[i] = bi;
        if (row_margin)
            row_margin[i] = best - second;
    }
#pragma omp parallel for schedule(static)
    for (i = 0; i < n; i++) {
        float best = -1.0f, second = -1.0f;
        int bi = -1, r;

        for (r = 0; r < n; r++) {
            const float s = S[(long)r * n + i];
            const float c = expf(s - lse[r]) * expf(s - (cm[i] + logf(cs[i])));

            if (c > best) {
                second = best;
                best = c;
                bi = r;
            }
            else if (c > second)
                second = c;
        }
        cmax[i] = best;
        col_arg[i] = bi;
        c2[i] = second;
        if (col_margin)
            col_margin[i] = best - second;
        if (col_max)
            col_max[i] = best;
    }
    free(S);
    free(lse);
    free(cm);
    free(cs);
    free(cmax);
    free(c2);
}

int orc_eloftr_select(const float *row_max, const int *row_arg,
                      const int *col_arg, int h, int w, float thr, int border,
                      int *mi, int *mj, float *mconf)
{
    const int n = h * w;
    int i, nm = 0;

    for (i = 0; i < n; i++) {
        const int j = row_arg[i];
        const int xi = i % w, yi = i / w, xj = j % w, yj = j / w;

        if (!(row_max[i] > thr) || col_arg[j] != i)
            continue;
        if (xi < border || yi < border || xi >= w - border ||
            yi >= h - border || xj < border || yj < border ||
            xj >= w - border || yj >= h - border)
            continue;
        mi[nm] = i;
        mj[nm] = j;
        mconf[nm++] = row_max[i];
    }
    return nm;
}

/* ---- ELoFTR fine matching, eloftr_kernels.cl:146-295 ---------------------- */

#define FW 8
#define FW1 10
#define FC 64
#define FS 8
#define NP 64
#define NQ 100

static float fine_at(const float *f, int H, int W, int c, int x, int y)
{
    if (x < 0 || y < 0 || x >= W || y >= H)
        return 0.0f;
    return f[((long)c * H + y) * W + x];
}

void orc_eloftr_fine(const float *f0, const float *f1, int H, int W,
                     const int *cells, int M, float T, float *out,
                     float *margin)
{
    int k;

#pragma omp parallel for schedule(dynamic, 16)
    for (k = 0; k < M; k++) {
        const int cx0 = cells[4 * k], cy0 = cells[4 * k + 1];
        const int cx1 = cells[4 * k + 2], cy1 = cells[4 * k + 3];
        float sc[NP * NQ], pm[NQ], ps[NQ], qm[NP], qs[NP], s2[9];
        float best = -1.0f, second = -1.0f, inv = 1.0f / FC;
        int bi = 0, e, p, q, c, bp, bq, qi, qj, t;

        for (e = 0; e < NP * NQ; e++) {
            const int pp = e / NQ, qq = e % NQ;
            const int ax = cx0 * FW + pp % FW, ay = cy0 * FW + pp / FW;
            const int bx = cx1 * FW - 1 + qq % FW1, by = cy1 * FW - 1 + qq / FW1;
            float d = 0.0f;

            for (c = 0; c < FC - FS; c++)
                d = fmaf(fine_at(f0, H, W, c, ax, ay),
                         fine_at(f1, H, W, c, bx, by), d);
            sc[e] = d * inv;
        }
        for (q = 0; q < NQ; q++) {
            float m = -INFINITY, s = 0.0f;

            for (p = 0; p < NP; p++)
                m = fmaxf(m, sc[p * NQ + q]);
            for (p = 0; p < NP; p++)
                s += expf(sc[p * NQ + q] - m);
            pm[q] = m;
            ps[q] = s;
        }
        for (p = 0; p < NP; p++) {
            float m = -INFINITY, s = 0.0f;

            for (q = 0; q < NQ; q++)
                m = fmaxf(m, sc[p * NQ + q]);
            for (q = 0; q < NQ; q++)
                s += expf(sc[p * NQ + q] - m);
            qm[p] = m;
            qs[p] = s;
        }
        for (e = 0; e < NP * FW * FW; e++) {
            const int pp = e / (FW * FW), ii = (e / FW) % FW, jj = e % FW;
            const int qq = (ii + 1) * FW1 + jj + 1;
            const float s = sc[pp * NQ + qq];
            const float v =
                expf(s - pm[qq]) / ps[qq] * (expf(s - qm[pp]) / qs[pp]);

            if (v > best) {
                second = best;
                best = v;
                bi = e;
            }
            else if (v > second)
                second = v;
        }
        if (margin)
            margin[k] = best - second;
        bp = bi / (FW * FW);
        bq = bi % (FW * FW);
        qi = bq / FW;
        qj = bq % FW;
        for (t = 0; t < 9; t++) {
            const int ii = (qi + t / 3 - 1 + FW1) % FW1;
            const int jj = (qj + t % 3 - 1 + FW1) % FW1;
            const int ax = cx0 * FW + bp % FW, ay = cy0 * FW + bp / FW;
            const int bx = cx1 * FW - 1 + jj, by = cy1 * FW - 1 + ii;
            float d = 0.0f;

            for (c = FC - FS; c < FC; c++)
                d = fmaf(fine_at(f0, H, W, c, ax, ay),
                         fine_at(f1, H, W, c, bx, by), d);
            s2[t] = d * (1.0f / sqrtf((float)FS)) / T;
        }
        {
            float m = -INFINITY, s = 0.0f, ex = 0.0f, ey = 0.0f;

            for (t = 0; t < 9; t++)
                m = fmaxf(m, s2[t]);
            for (t = 0; t < 9; t++)
                s += expf(s2[t] - m);
            for (t = 0; t < 9; t++) {
                const float wgt = expf(s2[t] - m) / s;

                ex += wgt * (t % 3 - 1);
                ey += wgt * (t / 3 - 1);
            }
            out[4 * k] = cx0 * FW + bp % FW - (FW / 2 - 0.5f);
            out[4 * k + 1] = cy0 * FW + bp / FW - (FW / 2 - 0.5f);
            out[4 * k + 2] = cx1 * FW + qj - (FW / 2 - 0.5f) + ex;
            out[4 * k + 3] = cy1 * FW + qi - (FW / 2 - 0.5f) + ey;
        }
    }
}

/* OpenMP threads the oracle's parallel loops use, and how to set them
 * (timing of the CPU baseline states and pins the count). */
int orc_threads(void) { return omp_get_max_threads(); }

void orc_set_threads(int n)
{
    if (n > 0)
        omp_set_num_threads(n);
}

/* SPDX-License-Identifier: Unlicense */

/* ORACLE — test infrastructure only (see oracle.h): CPU restatement of
 * roma_kernels.cl (i.coregistration.opencl), float32 in the kernels'
 * order of operations. */

#include <math.h>
#include <stdlib.h>

#include "oracle.h"

void orc_roma_row_norm(const float *X, int rows, int C, float *out)
{
    int r, c;

    for (r = 0; r < rows; r++) {
        float s = 0.0f;

        for (c = 0; c < C; c++)
            s += X[(long)r * C + c] * X[(long)r * C + c];
        out[r] = sqrtf(s);
    }
}

void orc_roma_cos_exp(float *S, const float *nx, const float *ny, int N, int M,
                      float T, float eps)
{
    long i, j;

    for (i = 0; i < N; i++)
        for (j = 0; j < M; j++) {
            const float c = S[i * M + j] / (nx[i] * ny[j] + eps);

            S[i * M + j] = expf((c - 1.0f) / T);
        }
}

void orc_roma_cls_to_flow(const float *L, int ld, int C, int res, int n,
                          float *flow, float *cert)
{
    int t;

    for (t = 0; t < n; t++) {
        const float *p = L + (long)t * ld;
        float m = -INFINITY, s = 0.0f, fx = 0.0f, fy = 0.0f, tot = 0.0f;
        int arg = 0, j, k, nb[5];

        for (j = 0; j < C; j++)
            if (p[j] > m) {
                m = p[j];
                arg = j;
            }
        for (j = 0; j < C; j++)
            s += expf(p[j] - m);
        nb[0] = arg - 1;
        nb[1] = arg;
        nb[2] = arg + 1;
        nb[3] = arg - res;
        nb[4] = arg + res;
        for (k = 0; k < 5; k++) {
            const int c = nb[k] < 0 ? 0 : nb[k] > C - 1 ? C - 1 : nb[k];
            const float pr = expf(p[c] - m) / s;

            fx += pr * (-1.0f + (2 * (c % res) + 1) / (float)res);
            fy += pr * (-1.0f + (2 * (c / res) + 1) / (float)res);
            tot += pr;
        }
        flow[t] = fx / tot;
        flow[n + t] = fy / tot;
        cert[t] = p[C];
    }
}

/* bilinear0, roma_kernels.cl:104-126. */
static float bilinear0(const float *p, int H, int W, float x, float y)
{
    const float ix = ((x + 1.0f) * W - 1.0f) * 0.5f;
    const float iy = ((y + 1.0f) * H - 1.0f) * 0.5f;
    int x0, y0;
    float fx, fy, v00, v01, v10, v11;

    if (!isfinite(ix) || !isfinite(iy) || fabsf(ix) > 1e8f || fabsf(iy) > 1e8f)
        return 0.0f;
    x0 = (int)floorf(ix);
    y0 = (int)floorf(iy);
    fx = ix - x0;
    fy = iy - y0;
#define AT(yy, xx)                                                             \
    ((xx) >= 0 && (xx) < W && (yy) >= 0 && (yy) < H ? p[(long)(yy) * W + (xx)] \
                                                    : 0.0f)
    v00 = AT(y0, x0);
    v01 = AT(y0, x0 + 1);
    v10 = AT(y0 + 1, x0);
    v11 = AT(y0 + 1, x0 + 1);
#undef AT
    return (1.0f - fy) * ((1.0f - fx) * v00 + fx * v01) +
           fy * ((1.0f - fx) * v10 + fx * v11);
}

void orc_roma_warp_sample(const float *in, int C, int H, int W,
                          const float *flow, float *out, int coff)
{
    const long n = (long)H * W;
    long i;
    int c;

    for (c = 0; c < C; c++)
        for (i = 0; i < n; i++)
            out[(long)(coff + c) * n + i] =
                bilinear0(in + (long)c * n, H, W, flow[i], flow[n + i]);
}

void orc_roma_local_corr(const float *f1, const float *f2, int C, int H,
                         int W, int r, const float *flow, float *out, int coff)
{
    const long n = (long)H * W;
    const int side = 2 * r + 1, ps = 2 * r + 2;
    const float rc = 1.0f / sqrtf((float)C);
    long i;

#pragma omp parallel for schedule(static)
    for (i = 0; i < n; i++) {
        const float ix = ((flow[i] + 1.0f) * W - 1.0f) * 0.5f;
        const float iy = ((flow[n + i] + 1.0f) * H - 1.0f) * 0.5f;
        const int ok = isfinite(ix) && isfinite(iy) && fabsf(ix) < 1e8f &&
                       fabsf(iy) < 1e8f;
        const int x0 = ok ? (int)floorf(ix) : 0, y0 = ok ? (int)floorf(iy) : 0;
        const float fx = ok ? ix - x0 : 0.0f, fy = ok ? iy - y0 : 0.0f;
        float S[256];
        int e, k, c;

        for (e = 0; e < ps * ps; e++) {
            const int yy = y0 - r + e / ps, xx = x0 - r + e % ps;
            float s = 0.0f;

            if (ok && xx >= 0 && xx < W && yy >= 0 && yy < H)
                for (c = 0; c < C; c++)
                    s += (f1[(long)c * n + i] * rc) *
                         f2[(long)c * n + (long)yy * W + xx];
            S[e] = s;
        }
        for (k = 0; k < side * side; k++) {
            const int e0 = (k / side) * ps + k % side, e1 = e0 + ps;

            out[(long)(coff + k) * n + i] =
                (1.0f - fy) * ((1.0f - fx) * S[e0] + fx * S[e0 + 1]) +
                fy * ((1.0f - fx) * S[e1] + fx * S[e1 + 1]);
        }
    }
}

void orc_roma_disp(const float *flow, int H, int W, float fx, float fy,
                   float *out)
{
    const long n = (long)H * W;
    long i;

    for (i = 0; i < n; i++) {
        const float gx =
            -1.0f + 1.0f / W + (i % W) * (2.0f - 2.0f / W) / (W - 1);
        const float gy =
            -1.0f + 1.0f / H + (i / W) * (2.0f - 2.0f / H) / (H - 1);

        out[i] = fx * (flow[i] - gx);
        out[n + i] = fy * (flow[n + i] - gy);
    }
}

void orc_roma_update(float *flow, float *cert, const float *d, int n,
                     float scale, float Wf, float Hf)
{
    int i;

    for (i = 0; i < n; i++) {
        flow[i] += scale * (d[i] / (4.0f * Wf));
        flow[n + i] += scale * (d[n + i] / (4.0f * Hf));
        cert[i] += d[2 * n + i];
    }
}

static float softplus20(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

void orc_roma2_update(float *flow, float *conf, const float *d, int n, float W,
                      float H)
{
    int i;

    for (i = 0; i < n; i++) {
        const float l00 = softplus20(d[3 * n + i]) + 1e-6f;
        const float l10 = d[4 * n + i];
        const float l11 = softplus20(d[5 * n + i]) + 1e-6f;

        flow[i] += d[i] / (4.0f * W);
        flow[n + i] += d[n + i] / (4.0f * H);
        conf[i] += d[2 * n + i];
        conf[n + i] += l00 * l00;
        conf[2 * n + i] += l00 * l10;
        conf[3 * n + i] += l10 * l10 + l11 * l11;
    }
}

void orc_roma_dwconv5(const float *in, int C, int H, int W, const float *w,
                      const float *bias, float *out)
{
    long c;

#pragma omp parallel for schedule(static)
    for (c = 0; c < C; c++) {
        const float *p = in + c * (long)H * W, *wk = w + c * 25;
        int x, y, i, j;

        for (y = 0; y < H; y++)
            for (x = 0; x < W; x++) {
                float acc = bias[c];

                for (i = 0; i < 5; i++)
                    for (j = 0; j < 5; j++) {
                        const int yy = y - 2 + i, xx = x - 2 + j;

                        if (yy >= 0 && yy < H && xx >= 0 && xx < W)
                            acc += p[(long)yy * W + xx] * wk[i * 5 + j];
                    }
                out[(c * (long)H + y) * W + x] = acc > 0.0f ? acc : 0.0f;
            }
    }
}

/* SPDX-License-Identifier: Unlicense */

/* ORACLE — test infrastructure only (see oracle.h): DISK's kernels
 * (disk_kernels.cl:8-60 of i.coregistration.opencl) and the U-Net,
 * NMS, host top-n and descriptor schedule of disk.c:23-273, one image at
 * a time, from named weight arrays. */

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define DESC 128
#define LAYERS 9

static const int layer_cin[LAYERS] = {3, 16, 32, 64, 64, 128, 128, 96, 80};
static const int layer_cout[LAYERS] = {16, 32, 64, 64, 64, 64, 64, 64, DESC + 1};

void orc_disk_nms5x5(const float *heat, int W, int h, int w, float thresh,
                     unsigned char *mask)
{
    int x, y, dx, dy;

    for (y = 0; y < h; y++)
        for (x = 0; x < w; x++) {
            float v;
            int keep = 1;

            if (x < 2 || y < 2 || x >= w - 2 || y >= h - 2) {
                mask[(long)y * w + x] = 0;
                continue;
            }
            v = heat[(long)y * W + x];
            for (dy = -2; dy <= 2 && keep; dy++)
                for (dx = -2; dx <= 2; dx++)
                    if ((dx || dy) && !(v > heat[(long)(y + dy) * W + x + dx])) {
                        keep = 0;
                        break;
                    }
            mask[(long)y * w + x] = keep && v > thresh;
        }
}

void orc_disk_gather_desc(const float *feat, int H, int W, int D,
                          const int *xy, int n, float *desc)
{
    const long plane = (long)H * W;
    int k, d;

    for (k = 0; k < n; k++) {
        const long off = (long)xy[2 * k + 1] * W + xy[2 * k];
        float ss = 0.0f, inv;

        for (d = 0; d < D; d++)
            ss += feat[d * plane + off] * feat[d * plane + off];
        inv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
        for (d = 0; d < D; d++)
            desc[(long)k * D + d] = feat[d * plane + off] * inv;
    }
}

static const float *need(const struct orc_named *t, int nt, const char *name,
                         long numel)
{
    int i;

    for (i = 0; i < nt; i++)
        if (strcmp(t[i].name, name) == 0) {
            if (t[i].numel != numel) {
                fprintf(stderr, "oracle: <%s> has %ld values, %ld expected\n",
                        name, t[i].numel, numel);
                abort();
            }
            return t[i].data;
        }
    fprintf(stderr, "oracle: tensor <%s> missing\n", name);
    abort();
}

static int cmp_desc(const void *a, const void *b)
{
    const float x = *(const float *)a, y = *(const float *)b;

    return (x < y) - (x > y);
}

/* disk.c:228-253: cut = the (n+1)-th highest candidate (the lowest with
 * no more than n), keep the candidates above it in raster order. */
int orc_disk_topn(const float *heat, int W, int h, int w,
                  const unsigned char *mask, const unsigned char *valid, int n,
                  int *xy, float *score)
{
    float *cand = malloc(((size_t)h * w + 1) * sizeof(float)), cut = -INFINITY;
    int x, y, ncand = 0, nk = 0;

    for (y = 0; y < h; y++)
        for (x = 0; x < w; x++)
            if (mask[(long)y * w + x] && (!valid || valid[(long)y * w + x]))
                cand[ncand++] = heat[(long)y * W + x];
    if (ncand > 0) {
        qsort(cand, ncand, sizeof(float), cmp_desc);
        cut = cand[ncand > n ? n : ncand - 1];
    }
    free(cand);
    for (y = 0; y < h && nk < n; y++)
        for (x = 0; x < w && nk < n; x++) {
            const long i = (long)y * w + x;
            const float v = heat[(long)y * W + x];

            if (!mask[i] || (valid && !valid[i]) || !(v > cut))
                continue;
            xy[2 * nk] = x;
            xy[2 * nk + 1] = y;
            score[nk++] = v;
        }
    return nk;
}

int orc_disk_detect(const struct orc_named *weights, int nweights,
                    const float *img, int H, int W, int h, int w, int n,
                    float thresh, const unsigned char *valid, int *xy,
                    float *score, float *desc, float *out_full)
{
    const long px = (long)H * W;
    const float *wt[LAYERS], *bs[LAYERS], *al[LAYERS];
    float *f[5], *u[3], *tmp, *cat, *out, mean[128], rstd[128];
    unsigned char *mask;
    int l, k, lev, j, nk = 0;
    char name[128];

    for (l = 0; l < LAYERS; l++) {
        const int down = l < 5, idx = down ? l : l - 5;

#define NAME(sub, what)                                                        \
    (down ? snprintf(name, sizeof(name), "unet.path_down.%d.1.%d.%s", idx,     \
                     sub, what)                                                \
          : snprintf(name, sizeof(name), "unet.path_up.%d.conv.%d.%s", idx,    \
                     sub, what))
        NAME(3, "weight");
        wt[l] = need(weights, nweights, name,
                     (long)layer_cout[l] * layer_cin[l] * 25);
        NAME(3, "bias");
        bs[l] = need(weights, nweights, name, layer_cout[l]);
        al[l] = NULL;
        if (l > 0) {
            NAME(1, "weight");
            al[l] = need(weights, nweights, name, layer_cin[l]);
        }
#undef NAME
    }
    for (k = 0; k < 5; k++)
        f[k] = malloc(layer_cout[k] * (px >> (2 * k)) * sizeof(float));
    for (k = 0; k < 3; k++)
        u[k] = malloc(64 * (px >> (2 * (3 - k))) * sizeof(float));
    tmp = malloc(16 * (px >> 2) * sizeof(float));
    cat = malloc(80 * px * sizeof(float));
    out = out_full ? out_full : malloc((DESC + 1) * px * sizeof(float));
    mask = malloc((size_t)h * w + 1);

    orc_conv2d(img, 3, H, W, wt[0], bs[0], 16, 5, 5, 1, 1, 2, 2, 1, 1, 1, NULL,
               NULL, NULL, 0, 0.0f, f[0]);
    for (lev = 1; lev < 5; lev++) {
        const int c = layer_cout[lev - 1], hh = H >> lev, ww = W >> lev;
        float *t = lev == 1 ? tmp : cat;

        orc_avgpool2(f[lev - 1], c, H >> (lev - 1), W >> (lev - 1), t);
        orc_chan_stats(t, c, hh * ww, 1e-5f, mean, rstd);
        orc_conv2d(t, c, hh, ww, wt[lev], bs[lev], layer_cout[lev], 5, 5, 1, 1,
                   2, 2, 1, 1, 1, mean, rstd, al[lev], 0, 0.0f, f[lev]);
    }
    for (j = 0; j < 4; j++) {
        const int ll = 5 + j, lvl = 3 - j, hh = H >> lvl, ww = W >> lvl;
        const float *bot = j == 0 ? f[4] : u[j - 1];
        const int cb = 64, ch = layer_cout[lvl];
        const long plane = (long)hh * ww;

        orc_resize(bot, cb, hh / 2, ww / 2, cat, hh, ww, 0, 0, 2.0f);
        memcpy(cat + cb * plane, f[lvl], ch * plane * sizeof(float));
        orc_chan_stats(cat, cb + ch, (int)plane, 1e-5f, mean, rstd);
        orc_conv2d(cat, cb + ch, hh, ww, wt[ll], bs[ll], layer_cout[ll], 5, 5, 1,
                   1, 2, 2, 1, 1, 1, mean, rstd, al[ll], 0, 0.0f,
                   j < 3 ? u[j] : out);
    }
    {
        const float *heat = out + (long)DESC * px;

        orc_disk_nms5x5(heat, W, h, w, thresh, mask);
        nk = orc_disk_topn(heat, W, h, w, mask, valid, n, xy, score);
    }
    if (nk > 0)
        orc_disk_gather_desc(out, H, W, DESC, xy, nk, desc);
    for (k = 0; k < 5; k++)
        free(f[k]);
    for (k = 0; k < 3; k++)
        free(u[k]);
    free(tmp);
    free(cat);
    if (!out_full)
        free(out);
    free(mask);
    return nk;
}

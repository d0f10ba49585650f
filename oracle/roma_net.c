/* SPDX-License-Identifier: Unlicense */

/* ORACLE — test infrastructure only (see oracle.h): the RoMa schedule of
 * the reference (roma.c:42-1435 of i.coregistration.opencl) on the CPU
 * kernels of oracle.c and roma_kernels.c, one image at a time as the
 * reference runs it, from named weight arrays (the same safetensors the
 * HIP path loads). Folding (roma.c:103-238, 353-398, 452-532), position
 * embedding interpolation (:241-298), GP basis (:326-350), DINOv2
 * (:675-738), VGG (:740-768, 997-1027), the host double-precision GP
 * solve (:770-896), decoder (:898-919), refiners (:921-995, 1029-1104),
 * host resampling (:1106-1186) and the pass schedule with its epilogue
 * (:1229-1435). */

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define ACT_NONE 0
#define ACT_GELU 1
#define ACT_RELU 2

#define DV 1024 /* ViT and decoder width */
#define VIT_DEPTH 24
#define DEC_DEPTH 5
#define VIT_GRID 37
#define GP_DIM 512
#define NCLS 4096
#define CLS_RES 64
#define SCALES 5
#define SCALES2 3
#define HIDDEN 8

static const int ref_scale[SCALES] = {16, 8, 4, 2, 1};
static const int ref_feat[SCALES] = {512, 512, 256, 64, 9};
static const int ref_emb[SCALES] = {128, 64, 32, 16, 6};
static const int ref_radius[SCALES] = {7, 3, 2, 0, 0};
static const int proj_in[SCALES] = {1024, 512, 256, 128, 64};
static const int ref2_scale[SCALES2] = {4, 2, 1};
static const int ref2_in[SCALES2] = {256, 128, 64};
static const int ref2_feat[SCALES2] = {192, 48, 12};
static const int ref2_emb[SCALES2] = {79, 23, 8};
static const int ref2_radius[SCALES2] = {3, 1, 0};
static const int vgg_blocks[4] = {2, 2, 4, 4};
static const int vgg_width[4] = {64, 128, 256, 512};
static const float im_mean[3] = {0.485f, 0.456f, 0.406f};
static const float im_std[3] = {0.229f, 0.224f, 0.225f};

struct wset {
    const struct orc_named *t;
    int n;
};

static const float *get(const struct wset *w, const char *name, long numel)
{
    int i;

    for (i = 0; i < w->n; i++)
        if (strcmp(w->t[i].name, name) == 0) {
            if (numel >= 0 && w->t[i].numel != numel) {
                fprintf(stderr, "oracle: <%s> has %ld values, %ld expected\n",
                        name, w->t[i].numel, numel);
                abort();
            }
            return w->t[i].data;
        }
    return NULL;
}

static const float *need(const struct wset *w, const char *name, long numel)
{
    const float *p = get(w, name, numel);

    if (!p) {
        fprintf(stderr, "oracle: tensor <%s> missing\n", name);
        abort();
    }
    return p;
}

static float *dup(const float *p, long n)
{
    float *q = malloc(n * sizeof(float));

    memcpy(q, p, n * sizeof(float));
    return q;
}

static float *zalloc(long n) { return calloc(n, sizeof(float)); }

/* Convolution <conv> (bias optional) + BatchNorm <bn>, folded. */
static void conv_bn(const struct wset *ws, const char *conv, const char *bn,
                    int co, long per, float **w, float **b)
{
    char name[300], n1[300], n2[300], n3[300], n4[300];
    const float *bias;

    snprintf(name, sizeof(name), "%s.weight", conv);
    *w = dup(need(ws, name, co * per), co * per);
    snprintf(name, sizeof(name), "%s.bias", conv);
    bias = get(ws, name, co);
    *b = bias ? dup(bias, co) : zalloc(co);
    snprintf(n1, sizeof(n1), "%s.weight", bn);
    snprintf(n2, sizeof(n2), "%s.bias", bn);
    snprintf(n3, sizeof(n3), "%s.running_mean", bn);
    snprintf(n4, sizeof(n4), "%s.running_var", bn);
    orc_fold_bn(*w, *b, co, per, need(ws, n1, co), need(ws, n2, co),
                need(ws, n3, co), need(ws, n4, co), 1e-5f);
}

struct blk {
    const float *n1g, *n1b, *qkv_w, *qkv_b, *n2g, *n2b, *fc1_w, *fc1_b;
    float *proj_w, *proj_b, *fc2_w, *fc2_b;
};

static void load_block(const struct wset *ws, const char *pre, int qkv_bias,
                       int ls, struct blk *b)
{
    char name[300];
    int j, i, c;

#define LD(f, suffix, n)                                                       \
    snprintf(name, sizeof(name), "%s.%s", pre, suffix);                        \
    b->f = need(ws, name, n)
    LD(n1g, "norm1.weight", DV);
    LD(n1b, "norm1.bias", DV);
    LD(qkv_w, "attn.qkv.weight", 3L * DV * DV);
    if (qkv_bias) {
        LD(qkv_b, "attn.qkv.bias", 3 * DV);
    }
    else
        b->qkv_b = NULL;
    LD(n2g, "norm2.weight", DV);
    LD(n2b, "norm2.bias", DV);
    LD(fc1_w, "mlp.fc1.weight", 4L * DV * DV);
    LD(fc1_b, "mlp.fc1.bias", 4 * DV);
#undef LD
    for (j = 0; j < 2; j++) {
        const int in = j ? 4 * DV : DV;
        float *w, *bias;

        snprintf(name, sizeof(name), "%s.%s.weight", pre,
                 j ? "mlp.fc2" : "attn.proj");
        w = dup(need(ws, name, (long)DV * in), (long)DV * in);
        snprintf(name, sizeof(name), "%s.%s.bias", pre,
                 j ? "mlp.fc2" : "attn.proj");
        bias = dup(need(ws, name, DV), DV);
        if (ls) {
            const float *g;

            snprintf(name, sizeof(name), "%s.ls%d.gamma", pre, j + 1);
            g = need(ws, name, DV);
            for (i = 0; i < DV; i++) {
                for (c = 0; c < in; c++)
                    w[(long)i * in + c] *= g[i];
                bias[i] *= g[i];
            }
        }
        if (j) {
            b->fc2_w = w;
            b->fc2_b = bias;
        }
        else {
            b->proj_w = w;
            b->proj_b = bias;
        }
    }
}

static void free_block(struct blk *b)
{
    free(b->proj_w);
    free(b->proj_b);
    free(b->fc2_w);
    free(b->fc2_b);
}

struct refiner {
    int scale, feat, emb, radius, cin, nout;
    float *dw_w[HIDDEN + 1], *dw_b[HIDDEN + 1];
    const float *pw_w[HIDDEN + 1], *pw_b[HIDDEN + 1];
    float *out_w, *out_b;
    const float *emb_w, *emb_b;
};

static void load_ref_blocks(const struct wset *ws, const char *pre,
                            const char *dw, const char *bn, const char *pw,
                            struct refiner *r)
{
    char blk[200], conv[260], norm[260], name[300];
    int b;

    for (b = 0; b <= HIDDEN; b++) {
        if (b == 0)
            snprintf(blk, sizeof(blk), "%s.block1", pre);
        else
            snprintf(blk, sizeof(blk), "%s.hidden_blocks.%d", pre, b - 1);
        snprintf(conv, sizeof(conv), "%s.%s", blk, dw);
        snprintf(norm, sizeof(norm), "%s.%s", blk, bn);
        conv_bn(ws, conv, norm, r->cin, 25, &r->dw_w[b], &r->dw_b[b]);
        snprintf(name, sizeof(name), "%s.%s.weight", blk, pw);
        r->pw_w[b] = need(ws, name, (long)r->cin * r->cin);
        snprintf(name, sizeof(name), "%s.%s.bias", blk, pw);
        r->pw_b[b] = need(ws, name, r->cin);
    }
}

static void free_refiner(struct refiner *r)
{
    int b;

    for (b = 0; b <= HIDDEN; b++) {
        free(r->dw_w[b]);
        free(r->dw_b[b]);
    }
    free(r->out_w);
    free(r->out_b);
}

struct net {
    int coarse, c16, n16, ntok, imagenet, v2;
    float *vgg_w[16], *vgg_b[16];
    int vgg_cin[16], vgg_cout[16];
    float *vgg2_w[8], *vgg2_b[8];
    int vgg2_cin[8], vgg2_cout[8];
    const float *patch_w, *patch_b, *cls, *norm_g, *norm_b;
    float *pos;
    struct blk vit[VIT_DEPTH], dec[DEC_DEPTH];
    float *proj_w[SCALES], *proj_b[SCALES];
    const float *proj2_w[SCALES2], *proj2_b[SCALES2];
    float *basis;
    const float *to_out_w, *to_out_b;
    struct refiner ref[SCALES], ref2[SCALES2];
};

static void load_vgg(const struct wset *ws, const char *pre, int nblk,
                     float **w, float **b, int *cin_out, int *cout_out)
{
    int blk, j, l = 0, idx = 0, cin = 3;

    for (blk = 0; blk < nblk; blk++) {
        for (j = 0; j < vgg_blocks[blk]; j++, l++) {
            char conv[100], bn[100];

            snprintf(conv, sizeof(conv), "%s.%d", pre, idx);
            snprintf(bn, sizeof(bn), "%s.%d", pre, idx + 1);
            conv_bn(ws, conv, bn, vgg_width[blk], (long)cin * 9, &w[l], &b[l]);
            cin_out[l] = cin;
            cout_out[l] = vgg_width[blk];
            cin = vgg_width[blk];
            idx += 3;
        }
        idx++;
    }
}

/* roma.c:241-253 */
static void cubic_w(double t, double w[4])
{
    const double A = -0.75;
    double x = t + 1;

    w[0] = ((A * x - 5 * A) * x + 8 * A) * x - 4 * A;
    x = t;
    w[1] = ((A + 2) * x - (A + 3)) * x * x + 1;
    x = 1 - t;
    w[2] = ((A + 2) * x - (A + 3)) * x * x + 1;
    x = 2 - t;
    w[3] = ((A * x - 5 * A) * x + 8 * A) * x - 4 * A;
}

static int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

static void load(struct net *m, const struct wset *ws, const struct wset *dn,
                 const struct wset *w2)
{
    char pre[100], name[300];
    int s, i, j, c;

    load_vgg(ws, "encoder.cnn.layers", 4, m->vgg_w, m->vgg_b, m->vgg_cin,
             m->vgg_cout);
    /* DINOv2 */
    m->patch_w = need(dn, "patch_embed.proj.weight", (long)DV * 3 * 14 * 14);
    m->patch_b = need(dn, "patch_embed.proj.bias", DV);
    m->cls = need(dn, "cls_token", DV);
    m->norm_g = need(dn, "norm.weight", DV);
    m->norm_b = need(dn, "norm.bias", DV);
    {
        const float *pos = need(dn, "pos_embed", (long)(VIT_GRID * VIT_GRID + 1) * DV);
        const double inv = VIT_GRID / (m->c16 + 0.1);
        int oy, ox;

        m->pos = malloc((size_t)m->ntok * DV * sizeof(float));
        memcpy(m->pos, pos, DV * sizeof(float));
        for (oy = 0; oy < m->c16; oy++)
            for (ox = 0; ox < m->c16; ox++) {
                const double ry = inv * (oy + 0.5) - 0.5, rx = inv * (ox + 0.5) - 0.5;
                const int iy = (int)floor(ry), ix = (int)floor(rx);
                double wy[4], wx[4];
                float *o = m->pos + (size_t)(1 + oy * m->c16 + ox) * DV;

                cubic_w(ry - iy, wy);
                cubic_w(rx - ix, wx);
                for (c = 0; c < DV; c++) {
                    double acc = 0;

                    for (i = 0; i < 4; i++)
                        for (j = 0; j < 4; j++)
                            acc += wy[i] * wx[j] *
                                   pos[(size_t)(1 + clampi(iy - 1 + i, 0, VIT_GRID - 1) *
                                                        VIT_GRID +
                                                clampi(ix - 1 + j, 0, VIT_GRID - 1)) *
                                           DV + c];
                    o[c] = (float)acc;
                }
            }
    }
    for (i = 0; i < VIT_DEPTH; i++) {
        snprintf(pre, sizeof(pre), "blocks.%d", i);
        load_block(dn, pre, 1, 1, &m->vit[i]);
    }
    for (s = 0; s < SCALES; s++) {
        char conv[100], bn[100];

        snprintf(conv, sizeof(conv), "decoder.proj.%d.0", ref_scale[s]);
        snprintf(bn, sizeof(bn), "decoder.proj.%d.1", ref_scale[s]);
        conv_bn(ws, conv, bn, ref_feat[s], proj_in[s], &m->proj_w[s],
                &m->proj_b[s]);
    }
    {
        const float *gw = need(ws, "decoder.gps.16.pos_conv.weight", GP_DIM * 2);
        const float *gb = need(ws, "decoder.gps.16.pos_conv.bias", GP_DIM);
        const int cc = m->c16;

        m->basis = malloc((size_t)m->n16 * GP_DIM * sizeof(float));
        for (i = 0; i < m->n16; i++) {
            const float x = -1.0f + 1.0f / cc + (i % cc) * (2.0f - 2.0f / cc) / (cc - 1);
            const float y = -1.0f + 1.0f / cc + (i / cc) * (2.0f - 2.0f / cc) / (cc - 1);

            for (j = 0; j < GP_DIM; j++) {
                const float v = gw[2 * j] * x + gw[2 * j + 1] * y + gb[j];

                m->basis[(size_t)i * GP_DIM + j] = cosf(8.0f * (float)M_PI * v);
            }
        }
    }
    for (i = 0; i < DEC_DEPTH; i++) {
        snprintf(pre, sizeof(pre), "decoder.embedding_decoder.blocks.%d", i);
        load_block(ws, pre, 0, 0, &m->dec[i]);
    }
    m->to_out_w = need(ws, "decoder.embedding_decoder.to_out.weight",
                       (long)(NCLS + 1) * DV);
    m->to_out_b = need(ws, "decoder.embedding_decoder.to_out.bias", NCLS + 1);
    for (s = 0; s < SCALES; s++) {
        struct refiner *r = &m->ref[s];
        int corr;

        r->scale = ref_scale[s];
        r->feat = ref_feat[s];
        r->emb = ref_emb[s];
        r->radius = ref_radius[s];
        corr = r->radius ? (2 * r->radius + 1) * (2 * r->radius + 1) : 0;
        r->cin = 2 * r->feat + r->emb + corr;
        r->nout = 3;
        snprintf(pre, sizeof(pre), "decoder.conv_refiner.%d", r->scale);
        load_ref_blocks(ws, pre, "0", "1", "3", r);
        snprintf(name, sizeof(name), "%s.out_conv.weight", pre);
        r->out_w = dup(need(ws, name, 3L * r->cin), 3L * r->cin);
        snprintf(name, sizeof(name), "%s.out_conv.bias", pre);
        r->out_b = dup(need(ws, name, 3), 3);
        snprintf(name, sizeof(name), "%s.disp_emb.weight", pre);
        r->emb_w = need(ws, name, 2L * r->emb);
        snprintf(name, sizeof(name), "%s.disp_emb.bias", pre);
        r->emb_b = need(ws, name, r->emb);
    }
    if (!w2)
        return;
    m->v2 = 1;
    load_vgg(w2, "refiner_features.layers", 3, m->vgg2_w, m->vgg2_b,
             m->vgg2_cin, m->vgg2_cout);
    for (s = 0; s < SCALES2; s++) {
        struct refiner *r = &m->ref2[s];
        int corr;

        r->scale = ref2_scale[s];
        r->feat = ref2_feat[s];
        r->emb = ref2_emb[s];
        r->radius = ref2_radius[s];
        corr = r->radius ? (2 * r->radius + 1) * (2 * r->radius + 1) : 0;
        r->cin = 2 * r->feat + r->emb + corr;
        r->nout = 6;
        snprintf(pre, sizeof(pre), "refiners.%d", r->scale);
        snprintf(name, sizeof(name), "%s.proj.weight", pre);
        m->proj2_w[s] = need(w2, name, (long)r->feat * ref2_in[s]);
        snprintf(name, sizeof(name), "%s.proj.bias", pre);
        m->proj2_b[s] = need(w2, name, r->feat);
        load_ref_blocks(w2, pre, "conv_depthwise", "norm", "conv_pointwise", r);
        r->out_w = malloc(6L * r->cin * sizeof(float));
        r->out_b = malloc(6 * sizeof(float));
        snprintf(name, sizeof(name), "%s.warp_head.weight", pre);
        memcpy(r->out_w, need(w2, name, 2L * r->cin), 2L * r->cin * sizeof(float));
        snprintf(name, sizeof(name), "%s.confidence_head.weight", pre);
        memcpy(r->out_w + 2L * r->cin, need(w2, name, 4L * r->cin),
               4L * r->cin * sizeof(float));
        snprintf(name, sizeof(name), "%s.warp_head.bias", pre);
        memcpy(r->out_b, need(w2, name, 2), 2 * sizeof(float));
        snprintf(name, sizeof(name), "%s.confidence_head.bias", pre);
        memcpy(r->out_b + 2, need(w2, name, 4), 4 * sizeof(float));
        snprintf(name, sizeof(name), "%s.disp_emb.weight", pre);
        r->emb_w = need(w2, name, 2L * r->emb);
        snprintf(name, sizeof(name), "%s.disp_emb.bias", pre);
        r->emb_b = need(w2, name, r->emb);
    }
}

static void unload(struct net *m)
{
    int i;

    for (i = 0; i < 16; i++) {
        free(m->vgg_w[i]);
        free(m->vgg_b[i]);
    }
    for (i = 0; i < 8; i++) {
        free(m->vgg2_w[i]);
        free(m->vgg2_b[i]);
    }
    for (i = 0; i < VIT_DEPTH; i++)
        free_block(&m->vit[i]);
    for (i = 0; i < DEC_DEPTH; i++)
        free_block(&m->dec[i]);
    for (i = 0; i < SCALES; i++) {
        free(m->proj_w[i]);
        free(m->proj_b[i]);
        free_refiner(&m->ref[i]);
    }
    if (m->v2)
        for (i = 0; i < SCALES2; i++)
            free_refiner(&m->ref2[i]);
    free(m->pos);
    free(m->basis);
}

/* ---- the network ------------------------------------------------------------ */

/* 1 x 1 convolution W (K, C) X (C, n) + b into Y (K, n), ops_conv1x1. */
static void conv1x1(const float *X, int C, int n, const float *W,
                    const float *b, int K, float *Y)
{
    orc_gemm(K, n, C, W, 0, C, 0, 0, X, 0, n, 0, 0, 0, Y, 0, n, 0, 0, 1, 1, b,
             1, NULL, 0, 1.0f, ACT_NONE, 0.0f);
}

/* linear: Y (rows, out) = X W^T + b (+ Y), ops_linear. */
static void linear(const float *X, int rows, int in, int out, const float *W,
                   const float *b, float *Y, int act, int residual)
{
    orc_gemm(rows, out, in, X, 0, in, 0, 0, W, 0, in, 0, 0, 1, Y, 0, out, 0, 0,
             1, 1, b, 0, residual ? Y : NULL, 0, 1.0f, act, 0.0f);
}

/* Pre-norm block on X (N x DV), roma.c:675-713: full scores per head,
 * softmax, values. */
static void block(const struct blk *b, float *X, int N, int heads, float eps)
{
    const int hd = DV / heads;
    const long nn = (long)N * N;
    float *t_n = malloc((size_t)N * DV * 4), *qkv = malloc((size_t)N * 3 * DV * 4);
    float *S = malloc((size_t)heads * nn * 4), *o = malloc((size_t)N * DV * 4);
    float *h = malloc((size_t)N * 4 * DV * 4);

    orc_layernorm(N, DV, X, t_n, b->n1g, b->n1b, eps, ACT_NONE, 0.0f);
    linear(t_n, N, DV, 3 * DV, b->qkv_w, b->qkv_b, qkv, ACT_NONE, 0);
    orc_gemm(N, N, hd, qkv, 0, 3 * DV, hd, 0, qkv, DV, 3 * DV, hd, 0, 1, S, 0,
             N, nn, 0, heads, 1, NULL, 0, NULL, 0, 1.0f / sqrtf((float)hd),
             ACT_NONE, 0.0f);
    orc_softmax_rows(S, (long)heads * N, N, 1.0f);
    orc_gemm(N, hd, N, S, 0, N, nn, 0, qkv, 2 * DV, 3 * DV, hd, 0, 0, o, 0, DV,
             hd, 0, heads, 1, NULL, 0, NULL, 0, 1.0f, ACT_NONE, 0.0f);
    linear(o, N, DV, DV, b->proj_w, b->proj_b, X, ACT_NONE, 1);
    orc_layernorm(N, DV, X, t_n, b->n2g, b->n2b, eps, ACT_NONE, 0.0f);
    linear(t_n, N, DV, 4 * DV, b->fc1_w, b->fc1_b, h, ACT_GELU, 0);
    linear(h, N, 4 * DV, DV, b->fc2_w, b->fc2_b, X, ACT_NONE, 1);
    free(t_n);
    free(qkv);
    free(S);
    free(o);
    free(h);
}

/* One pre-norm ViT block of width DV on X (N x DV) in place, weights w[12]
 * = norm1 g, b; qkv W, b (b may be NULL); proj W, b; norm2 g, b; fc1 W, b;
 * fc2 W, b, with layer scale already folded into proj and fc2 (the form
 * load_block keeps). The same block() DINOv2 runs (roma.c:675-713). */
void orc_vit_block(const float *const w[12], float *X, int N, int heads,
                   float eps)
{
    float *own[4];
    struct blk b;
    int i;

    for (i = 0; i < 4; i++) {
        const long n = i == 0 ? (long)DV * DV : i == 2 ? 4L * DV * DV : DV;
        own[i] = dup(w[4 + i + (i >= 2 ? 4 : 0)], n);
    }
    b.n1g = w[0];
    b.n1b = w[1];
    b.qkv_w = w[2];
    b.qkv_b = w[3];
    b.proj_w = own[0];
    b.proj_b = own[1];
    b.n2g = w[6];
    b.n2b = w[7];
    b.fc1_w = w[8];
    b.fc1_b = w[9];
    b.fc2_w = own[2];
    b.fc2_b = own[3];
    block(&b, X, N, heads, eps);
    free_block(&b);
}

/* DINOv2 on img (3, c, c): normed patch tokens (DV, n16) into feat and the
 * 1/16 projection (512, n16) into P0. roma.c:715-738. */
static void dino(const struct net *m, const float *img, float *feat, float *P0)
{
    const int c = m->coarse, n16 = m->n16, ntok = m->ntok;
    float *t = malloc((size_t)DV * n16 * 4), *x = malloc((size_t)ntok * DV * 4);
    float *tn = malloc((size_t)ntok * DV * 4);
    int i;

    orc_conv2d(img, 3, c, c, m->patch_w, m->patch_b, DV, 14, 14, 14, 14, 0, 0,
               1, 1, 1, NULL, NULL, NULL, ACT_NONE, 0.0f, t);
    memcpy(x, m->cls, DV * 4);
    orc_transpose(t, x + DV, 1, DV, n16);
    orc_axpby(x, x, 1.0f, m->pos, 1.0f, (long)ntok * DV, (long)ntok * DV);
    for (i = 0; i < VIT_DEPTH; i++)
        block(&m->vit[i], x, ntok, 16, 1e-6f);
    orc_layernorm(ntok, DV, x, tn, m->norm_g, m->norm_b, 1e-6f, ACT_NONE, 0.0f);
    orc_transpose(tn + DV, feat, 1, n16, DV);
    conv1x1(feat, DV, n16, m->proj_w[0], m->proj_b[0], GP_DIM, P0);
    free(t);
    free(x);
    free(tn);
}

/* VGG19-BN of nblk blocks on img (3, H, W); projections into P[r] per
 * block b (r = sob[b]). roma.c:740-768, 997-1027. */
static void vgg(float *const *w, float *const *b, const int *cin,
                const int *cout, int nblk, const int *sob,
                const float *const *pw, const float *const *pb,
                const int *pin, const int *pout,
                const float *img, int H, int W, float **P)
{
    float *va = malloc((size_t)64 * H * W * 4), *vb = malloc((size_t)64 * H * W * 4);
    const float *in = img;
    float *out;
    int blk, j, l = 0, h = H, wd = W;

    for (blk = 0; blk < nblk; blk++) {
        const int r = sob[blk];

        for (j = 0; j < vgg_blocks[blk]; j++, l++) {
            out = in == va ? vb : va;
            orc_conv2d(in, cin[l], h, wd, w[l], b[l], cout[l], 3, 3, 1, 1, 1, 1,
                       1, 1, 1, NULL, NULL, NULL, ACT_RELU, 0.0f, out);
            in = out;
        }
        conv1x1(in, pin[r], h * wd, pw[r], pb[r], pout[r], P[r]);
        if (blk < nblk - 1) {
            out = in == va ? vb : va;
            orc_pool2d(in, vgg_width[blk], h, wd, 2, 2, 0, 1, out);
            in = out;
            h /= 2;
            wd /= 2;
        }
    }
    free(va);
    free(vb);
}

/* Host Cholesky solve of (K + noise I) X = F in place, double precision,
 * roma.c:770-836. Returns 0 or 1 + the failing column. */
static int gp_solve(const float *K, int n, float *F, int d)
{
    double *L = malloc((size_t)n * n * sizeof(double));
    double *Z = malloc((size_t)n * d * sizeof(double));
    int i, j, bad = 0;

    for (j = 0; j < n && !bad; j++) {
        double s = (double)K[(size_t)j * n + j] + 0.1;
        const double *lj = L + (size_t)j * n;
        int k;

        for (k = 0; k < j; k++)
            s -= lj[k] * lj[k];
        if (!(s > 0)) {
            bad = j + 1;
            break;
        }
        L[(size_t)j * n + j] = sqrt(s);
#pragma omp parallel for schedule(static)
        for (i = j + 1; i < n; i++) {
            const double *li = L + (size_t)i * n;
            double t = K[(size_t)i * n + j];
            int q;

            for (q = 0; q < j; q++)
                t -= li[q] * lj[q];
            L[(size_t)i * n + j] = t / lj[j];
        }
    }
    if (!bad) {
        for (i = 0; i < n; i++) {
            double *z = Z + (size_t)i * d;
            const double *li = L + (size_t)i * n;
            int q, c;

            for (c = 0; c < d; c++)
                z[c] = F[(size_t)i * d + c];
            for (q = 0; q < i; q++) {
                const double *zq = Z + (size_t)q * d;
                const double a = li[q];

                for (c = 0; c < d; c++)
                    z[c] -= a * zq[c];
            }
            for (c = 0; c < d; c++)
                z[c] /= li[i];
        }
        for (i = n - 1; i >= 0; i--) {
            double *z = Z + (size_t)i * d;
            int q, c;

            for (q = i + 1; q < n; q++) {
                const double *zq = Z + (size_t)q * d;
                const double a = L[(size_t)q * n + i];

                for (c = 0; c < d; c++)
                    z[c] -= a * zq[c];
            }
            for (c = 0; c < d; c++) {
                z[c] /= L[(size_t)i * n + i];
                F[(size_t)i * d + c] = (float)z[c];
            }
        }
    }
    free(L);
    free(Z);
    return bad;
}

/* Refiner body (roma.c:921-995, 1029-1104): output (nout, n) into dc. */
static void refiner_body(const struct refiner *r, const float *fa,
                         const float *fb, int hs, int ws, float fx, float fy,
                         const float *fl, float *da, float *db, float *dc)
{
    const int n = hs * ws;
    float *disp = malloc(2L * n * 4);
    int b;

    memcpy(da, fa, (size_t)r->feat * n * 4);
    orc_roma_warp_sample(fb, r->feat, hs, ws, fl, da, r->feat);
    orc_roma_disp(fl, hs, ws, fx, fy, disp);
    conv1x1(disp, 2, n, r->emb_w, r->emb_b, r->emb, da + 2L * r->feat * n);
    if (r->radius)
        orc_roma_local_corr(fa, fb, r->feat, hs, ws, r->radius, fl, da,
                            2 * r->feat + r->emb);
    for (b = 0; b <= HIDDEN; b++) {
        orc_roma_dwconv5(da, r->cin, hs, ws, r->dw_w[b], r->dw_b[b], db);
        conv1x1(db, r->cin, n, r->pw_w[b], r->pw_b[b], r->cin, da);
    }
    conv1x1(da, r->cin, n, r->out_w, r->out_b, r->nout, dc);
    free(disp);
}

/* roma.c:1106-1186 */
static double pil_cubic(double x)
{
    const double a = -0.5;

    x = fabs(x);
    if (x < 1)
        return ((a + 2) * x - (a + 3)) * x * x + 1;
    if (x < 2)
        return (((x - 5) * x + 8) * x - 4) * a;
    return 0;
}

static void resize_axis(const float *in, int n_in, long in_stride, float *out,
                        int n_out, long out_stride, int count, long in_step,
                        long out_step)
{
    const double scale = (double)n_in / n_out, fs = scale > 1 ? scale : 1;
    const double support = 2 * fs;
    int o, c, x;

    for (o = 0; o < n_out; o++) {
        const double center = (o + 0.5) * scale;
        double k[64], ww = 0;
        int xmin = (int)(center - support + 0.5), xmax;

        if (xmin < 0)
            xmin = 0;
        xmax = (int)(center + support + 0.5);
        if (xmax > n_in)
            xmax = n_in;
        xmax -= xmin;
        for (x = 0; x < xmax; x++) {
            k[x] = pil_cubic((x + xmin - center + 0.5) / fs);
            ww += k[x];
        }
        for (x = 0; x < xmax; x++)
            k[x] = ww != 0 ? k[x] / ww : 0;
        for (c = 0; c < count; c++) {
            const float *src = in + c * in_step + (long)xmin * in_stride;
            double s = 0;

            for (x = 0; x < xmax; x++)
                s += k[x] * src[x * in_stride];
            out[c * out_step + o * out_stride] = (float)s;
        }
    }
}

void orc_roma_prepare(const float *in, int H, int W, float *out, int h, int w,
                      int imagenet)
{
    const size_t p = (size_t)h * w;
    int c;

    if (H == h && W == w)
        memcpy(out, in, 3 * p * sizeof(float));
    else {
        float *tmp = malloc((size_t)H * w * sizeof(float));

        for (c = 0; c < 3; c++) {
            resize_axis(in + (size_t)c * H * W, W, 1, tmp, w, 1, H, W, w);
            resize_axis(tmp, H, w, out + c * p, h, w, w, 1, 1);
        }
        free(tmp);
    }
    if (imagenet)
        for (c = 0; c < 3; c++) {
            size_t i;

            for (i = 0; i < p; i++)
                out[c * p + i] = (out[c * p + i] - im_mean[c]) / im_std[c];
        }
}

static int side(int n, int s) { return s == 0 ? n / 14 : n / ref_scale[s]; }

/* Scratch of one pass. */
struct pass {
    float *P[SCALES][2], *P2[SCALES2][2];
    float *fl[2], *ce[2], *cf[2], *da, *db, *dc;
};

static void refiners(const struct net *m, struct pass *ps, int p, int s0, int s1,
                     int Hp, int Wp, float sf, int *cur, float *cert16,
                     struct orc_roma_out *out)
{
    int s;

    for (s = s0; s < s1; s++) {
        const struct refiner *r = &m->ref[s];
        const int hs = side(Hp, s), ws = side(Wp, s), n = hs * ws;
        const float fac = 40.0f / 32.0f * sf;

        refiner_body(r, ps->P[s][0], ps->P[s][1], hs, ws, fac, fac,
                     ps->fl[*cur], ps->da, ps->db, ps->dc);
        orc_roma_update(ps->fl[*cur], ps->ce[*cur], ps->dc, n, (float)r->scale,
                        (float)Wp, (float)Hp);
        if (p == 0 && s == 0)
            memcpy(cert16, ps->ce[*cur], (size_t)n * 4);
        if (out->scale_flow[p][s])
            memcpy(out->scale_flow[p][s], ps->fl[*cur], 2L * n * 4);
        if (s < s1 - 1) {
            const int hn = side(Hp, s + 1), wn = side(Wp, s + 1);

            orc_resize(ps->fl[*cur], 2, hs, ws, ps->fl[!*cur], hn, wn, 0, 0,
                       0.0f);
            orc_resize(ps->ce[*cur], 1, hs, ws, ps->ce[!*cur], hn, wn, 0, 0,
                       0.0f);
            *cur = !*cur;
        }
    }
}

static void refiners2(const struct net *m, struct pass *ps, int Hp, int Wp,
                      int *h, int *w, int *cur, int zero_prec)
{
    int j;

    for (j = 0; j < SCALES2; j++) {
        const struct refiner *r = &m->ref2[j];
        const int hs = Hp / ref2_scale[j], ws = Wp / ref2_scale[j];
        const size_t n = (size_t)*h * *w;

        if (zero_prec && j == 0)
            memset(ps->cf[*cur] + n, 0, 3 * n * 4);
        orc_resize(ps->fl[*cur], 2, *h, *w, ps->fl[!*cur], hs, ws, 0, 0, 0.0f);
        orc_resize(ps->cf[*cur], 4, *h, *w, ps->cf[!*cur], hs, ws, 0, 0, 0.0f);
        *cur = !*cur;
        refiner_body(r, ps->P2[j][0], ps->P2[j][1], hs, ws,
                     (float)Wp / 512, (float)Hp / 512, ps->fl[*cur], ps->da,
                     ps->db, ps->dc);
        orc_roma2_update(ps->fl[*cur], ps->cf[*cur], ps->dc, hs * ws, (float)ws,
                         (float)hs);
        *h = hs;
        *w = ws;
    }
}

int orc_roma_forward(const struct orc_named *weights, int nweights,
                     const struct orc_named *dino_w, int ndino,
                     const struct orc_named *v2_w, int nv2, const float *imgA,
                     const float *imgB, int H, int W, int coarse, int imagenet,
                     const float *cls_flow_in, struct orc_roma_out *out)
{
    struct wset ws = {weights, nweights}, dn = {dino_w, ndino}, w2 = {v2_w, nv2};
    struct net m;
    struct pass ps;
    const int hm = H > coarse ? H : coarse, wm = W > coarse ? W : coarse;
    const size_t HM = (size_t)hm * wm, hw = (size_t)H * W;
    const int sob[4] = {4, 3, 2, 1}, sob2[3] = {2, 1, 0};
    float *img[2], *feat, *gy[2], *nx, *ny, *kyy, *kxy, *F, *x, *logits;
    float *cert16;
    int k, s, cur = 0, info, n16, i;
    size_t dmax = 0;

    memset(&m, 0, sizeof(m));
    memset(&ps, 0, sizeof(ps));
    m.coarse = coarse;
    m.c16 = coarse / 14;
    m.n16 = n16 = m.c16 * m.c16;
    m.ntok = n16 + 1;
    m.imagenet = imagenet;
    load(&m, &ws, &dn, nv2 ? &w2 : NULL);
    /* Buffers. */
    for (k = 0; k < 2; k++) {
        img[k] = malloc(3 * HM * 4);
        ps.P[0][k] = malloc((size_t)GP_DIM * n16 * 4);
        for (s = 1; s < SCALES; s++)
            ps.P[s][k] = malloc((size_t)ref_feat[s] * (hm / ref_scale[s]) *
                                (wm / ref_scale[s]) * 4);
        if (m.v2)
            for (s = 0; s < SCALES2; s++)
                ps.P2[s][k] = malloc((size_t)ref2_feat[s] * (hm / ref2_scale[s]) *
                                     (wm / ref2_scale[s]) * 4);
        ps.fl[k] = malloc(2 * HM * 4);
        ps.ce[k] = malloc(HM * 4);
        ps.cf[k] = malloc(4 * HM * 4);
        gy[k] = malloc((size_t)n16 * GP_DIM * 4);
    }
    for (k = 0; k < 2; k++)
        for (s = k; s < SCALES; s++) {
            const size_t n = (size_t)side(k ? H : coarse, s) * side(k ? W : coarse, s);

            if ((size_t)m.ref[s].cin * n > dmax)
                dmax = (size_t)m.ref[s].cin * n;
        }
    if (m.v2)
        for (k = 0; k < 2; k++)
            for (s = 0; s < SCALES2; s++) {
                const int ph = k ? H : coarse, pw = k ? W : coarse;
                const size_t n = (size_t)(ph / ref2_scale[s]) * (pw / ref2_scale[s]);

                if ((size_t)m.ref2[s].cin * n > dmax)
                    dmax = (size_t)m.ref2[s].cin * n;
            }
    ps.da = malloc(dmax * 4);
    ps.db = malloc(dmax * 4);
    ps.dc = malloc(6 * HM * 4);
    feat = malloc((size_t)DV * n16 * 4);
    cert16 = malloc((size_t)n16 * 4);

    /* Coarse pass. */
    for (k = 0; k < 2; k++) {
        float *P[SCALES];

        orc_roma_prepare(k ? imgB : imgA, H, W, img[k], coarse, coarse, imagenet);
        for (s = 0; s < SCALES; s++)
            P[s] = ps.P[s][k];
        vgg(m.vgg_w, m.vgg_b, m.vgg_cin, m.vgg_cout, 4, sob,
            (const float *const *)m.proj_w, (const float *const *)m.proj_b,
            proj_in, ref_feat, img[k], coarse, coarse, P);
        if (m.v2) {
            float *P2[SCALES2];

            for (s = 0; s < SCALES2; s++)
                P2[s] = ps.P2[s][k];
            vgg(m.vgg2_w, m.vgg2_b, m.vgg2_cin, m.vgg2_cout, 3, sob2,
                m.proj2_w, m.proj2_b, ref2_in,
                ref2_feat, img[k], coarse, coarse, P2);
        }
        dino(&m, img[k], feat, ps.P[0][k]);
        if (out->dino[k])
            memcpy(out->dino[k], feat, (size_t)DV * n16 * 4);
    }
    /* GP, roma.c:870-896. */
    nx = malloc(n16 * 4);
    ny = malloc(n16 * 4);
    kyy = malloc((size_t)n16 * n16 * 4);
    kxy = malloc((size_t)n16 * n16 * 4);
    F = malloc((size_t)n16 * GP_DIM * 4);
    x = calloc((size_t)n16 * DV, 4);
    orc_transpose(ps.P[0][0], gy[0], 1, GP_DIM, n16);
    orc_transpose(ps.P[0][1], gy[1], 1, GP_DIM, n16);
    orc_roma_row_norm(gy[0], n16, GP_DIM, nx);
    orc_roma_row_norm(gy[1], n16, GP_DIM, ny);
    orc_gemm(n16, n16, GP_DIM, gy[1], 0, GP_DIM, 0, 0, gy[1], 0, GP_DIM, 0, 0, 1,
             kyy, 0, n16, 0, 0, 1, 1, NULL, 0, NULL, 0, 1.0f, ACT_NONE, 0.0f);
    orc_roma_cos_exp(kyy, ny, ny, n16, n16, 0.2f, 1e-6f);
    orc_gemm(n16, n16, GP_DIM, gy[0], 0, GP_DIM, 0, 0, gy[1], 0, GP_DIM, 0, 0, 1,
             kxy, 0, n16, 0, 0, 1, 1, NULL, 0, NULL, 0, 1.0f, ACT_NONE, 0.0f);
    orc_roma_cos_exp(kxy, nx, ny, n16, n16, 0.2f, 1e-6f);
    memcpy(F, m.basis, (size_t)n16 * GP_DIM * 4);
    info = gp_solve(kyy, n16, F, GP_DIM);
    orc_gemm(n16, GP_DIM, n16, kxy, 0, n16, 0, 0, F, 0, GP_DIM, 0, 0, 0, x, 0,
             DV, 0, 0, 1, 1, NULL, 0, NULL, 0, 1.0f, ACT_NONE, 0.0f);
    for (i = 0; i < n16; i++)
        memcpy(x + (size_t)i * DV + GP_DIM, gy[0] + (size_t)i * GP_DIM,
               GP_DIM * 4);
    if (out->gp)
        for (i = 0; i < n16; i++)
            memcpy(out->gp + (size_t)i * GP_DIM, x + (size_t)i * DV, GP_DIM * 4);
    /* Decoder, roma.c:898-919. */
    for (i = 0; i < DEC_DEPTH; i++)
        block(&m.dec[i], x, n16, 8, 1e-5f);
    logits = malloc((size_t)n16 * (NCLS + 1) * 4);
    linear(x, n16, DV, NCLS + 1, m.to_out_w, m.to_out_b, logits, ACT_NONE, 0);
    if (out->logits)
        memcpy(out->logits, logits, (size_t)n16 * (NCLS + 1) * 4);
    orc_roma_cls_to_flow(logits, NCLS + 1, NCLS, CLS_RES, n16, ps.fl[0], ps.ce[0]);
    if (out->cls_flow)
        memcpy(out->cls_flow, ps.fl[0], 2L * n16 * 4);
    if (out->cls_cert)
        memcpy(out->cls_cert, ps.ce[0], (size_t)n16 * 4);
    if (cls_flow_in)
        memcpy(ps.fl[0], cls_flow_in, 2L * n16 * 4);
    refiners(&m, &ps, 0, 0, m.v2 ? 2 : SCALES, coarse, coarse, 1.0f, &cur,
             cert16, out);
    if (m.v2) {
        int h = coarse / 8, w = coarse / 8;
        const size_t n = (size_t)h * w;

        memset(ps.cf[cur], 0, 4 * n * 4);
        memcpy(ps.cf[cur], ps.ce[cur], n * 4);
        refiners2(&m, &ps, coarse, coarse, &h, &w, &cur, 0);
        for (k = 0; k < 2; k++) {
            float *P2[SCALES2];

            orc_roma_prepare(k ? imgB : imgA, H, W, img[k], H, W, imagenet);
            for (s = 0; s < SCALES2; s++)
                P2[s] = ps.P2[s][k];
            vgg(m.vgg2_w, m.vgg2_b, m.vgg2_cin, m.vgg2_cout, 3, sob2,
                m.proj2_w, m.proj2_b, ref2_in,
                ref2_feat, img[k], H, W, P2);
        }
        refiners2(&m, &ps, H, W, &h, &w, &cur, 1);
        memcpy(out->flow, ps.fl[cur], 2 * hw * 4);
        memcpy(out->cert, ps.cf[cur], hw * 4);
        if (out->sd)
            for (i = 0; i < (int)hw; i++) {
                const float *pr = ps.cf[cur] + hw;
                const double det = (double)pr[i] * pr[2 * hw + i] -
                                   (double)pr[hw + i] * pr[hw + i];

                out->sd[i] = det > 0 ? (float)pow(det, -0.25) : NAN;
            }
        for (i = 0; i < (int)hw; i++) {
            float c = 1.0f / (1.0f + expf(-out->cert[i]));
            float *fx = out->flow + i, *fy = out->flow + hw + i;

            if (fabsf(*fx) > 1 || fabsf(*fy) > 1)
                c = 0;
            *fx = *fx < -1 ? -1 : *fx > 1 ? 1 : *fx;
            *fy = *fy < -1 ? -1 : *fy > 1 ? 1 : *fy;
            out->cert[i] = c;
        }
    }
    else {
        float *low = malloc(hw * 4);
        const float sf = sqrtf((float)H * W) / coarse;

        for (k = 0; k < 2; k++) {
            float *P[SCALES];

            orc_roma_prepare(k ? imgB : imgA, H, W, img[k], H, W, imagenet);
            for (s = 0; s < SCALES; s++)
                P[s] = ps.P[s][k];
            vgg(m.vgg_w, m.vgg_b, m.vgg_cin, m.vgg_cout, 4, sob,
                (const float *const *)m.proj_w, (const float *const *)m.proj_b,
                proj_in, ref_feat, img[k], H, W, P);
        }
        orc_resize(ps.fl[cur], 2, coarse, coarse, ps.fl[!cur], side(H, 1),
                   side(W, 1), 0, 0, 0.0f);
        orc_resize(ps.ce[cur], 1, coarse, coarse, ps.ce[!cur], side(H, 1),
                   side(W, 1), 0, 0, 0.0f);
        cur = !cur;
        refiners(&m, &ps, 1, 1, SCALES, H, W, sf, &cur, cert16, out);
        orc_resize(cert16, 1, m.c16, m.c16, low, H, W, 0, 0, 0.0f);
        memcpy(out->flow, ps.fl[cur], 2 * hw * 4);
        for (i = 0; i < (int)hw; i++) {
            float c = ps.ce[cur][i] - (low[i] < 0 ? 0.5f * low[i] : 0.0f);
            float *fx = out->flow + i, *fy = out->flow + hw + i;

            c = 1.0f / (1.0f + expf(-c));
            if (fabsf(*fx) > 1 || fabsf(*fy) > 1)
                c = 0;
            *fx = *fx < -1 ? -1 : *fx > 1 ? 1 : *fx;
            *fy = *fy < -1 ? -1 : *fy > 1 ? 1 : *fy;
            out->cert[i] = c;
        }
        free(low);
    }
    for (k = 0; k < 2; k++) {
        free(img[k]);
        for (s = 0; s < SCALES; s++)
            free(ps.P[s][k]);
        for (s = 0; s < SCALES2; s++)
            free(ps.P2[s][k]);
        free(ps.fl[k]);
        free(ps.ce[k]);
        free(ps.cf[k]);
        free(gy[k]);
    }
    free(ps.da);
    free(ps.db);
    free(ps.dc);
    free(feat);
    free(cert16);
    free(nx);
    free(ny);
    free(kyy);
    free(kxy);
    free(F);
    free(x);
    free(logits);
    unload(&m);
    return info;
}

/* The fine pass of RoMa's match alone (roma.c:1404-1413 and the refiner
 * loop it runs, :1229-1256): VGG19-BN on both (3, H, W) images already
 * prepared (ImageNet-normalised at the tile's size), then the refiners of
 * scales 8 .. 1 from the given 1/8 warp (2, H/8, W/8) and certainty logit
 * (H/8, W/8), with the displacement scale of a coarse pass of side
 * coarse. out->flow / out->cert get the last refiner's warp and
 * certainty logit (no epilogue); out->scale_flow[1][s] the warp after
 * each scale. Returns 0. */
int orc_roma_refine(const struct orc_named *weights, int nweights,
                    const struct orc_named *dino_w, int ndino, const float *pairA,
                    const float *pairB, int H, int W, int coarse, const float *flow8,
                    const float *cert8, struct orc_roma_out *out)
{
    struct wset ws = {weights, nweights}, dn = {dino_w, ndino};
    struct net m;
    struct pass ps;
    const int sob[4] = {4, 3, 2, 1};
    const size_t hw = (size_t)H * W;
    const size_t n8 = (size_t)side(H, 1) * side(W, 1);
    const float sf = sqrtf((float)H * W) / coarse;
    size_t dmax = 0;
    int k, s, cur = 0;

    memset(&m, 0, sizeof(m));
    memset(&ps, 0, sizeof(ps));
    m.coarse = coarse;
    m.c16 = coarse / 14;
    m.n16 = m.c16 * m.c16;
    m.ntok = m.n16 + 1;
    m.imagenet = 1;
    load(&m, &ws, &dn, NULL);
    for (k = 0; k < 2; k++) {
        float *P[SCALES] = {NULL};

        for (s = 1; s < SCALES; s++)
            ps.P[s][k] = P[s] = malloc((size_t)ref_feat[s] * side(H, s) * side(W, s) * 4);
        ps.fl[k] = malloc(2 * hw * 4);
        ps.ce[k] = malloc(hw * 4);
        vgg(m.vgg_w, m.vgg_b, m.vgg_cin, m.vgg_cout, 4, sob,
            (const float *const *)m.proj_w, (const float *const *)m.proj_b,
            proj_in, ref_feat, k ? pairB : pairA, H, W, P);
    }
    for (s = 1; s < SCALES; s++) {
        const size_t n = (size_t)side(H, s) * side(W, s);

        if ((size_t)m.ref[s].cin * n > dmax)
            dmax = (size_t)m.ref[s].cin * n;
    }
    ps.da = malloc(dmax * 4);
    ps.db = malloc(dmax * 4);
    ps.dc = malloc(6 * hw * 4);
    memcpy(ps.fl[0], flow8, 2 * n8 * 4);
    memcpy(ps.ce[0], cert8, n8 * 4);
    refiners(&m, &ps, 1, 1, SCALES, H, W, sf, &cur, NULL, out);
    memcpy(out->flow, ps.fl[cur], 2 * hw * 4);
    memcpy(out->cert, ps.ce[cur], hw * 4);
    for (k = 0; k < 2; k++) {
        for (s = 0; s < SCALES; s++)
            free(ps.P[s][k]);
        free(ps.fl[k]);
        free(ps.ce[k]);
    }
    free(ps.da);
    free(ps.db);
    free(ps.dc);
    unload(&m);
    return 0;
}

/* RoMa's coarse forward alone (the benchmark's unit, roma.c:715-919): on
 * a pair of (3, coarse, coarse) images already ImageNet-normalised,
 * DINOv2 on each, the GP posterior and the decoder, into the anchor warp
 * cls_flow (2, n16) and certainty logit cls_cert (n16). Returns the GP
 * status (0, or 1 + the failing column). */
int orc_roma_coarse(const struct orc_named *weights, int nweights,
                    const struct orc_named *dino_w, int ndino, const float *pairA,
                    const float *pairB, int coarse, float *cls_flow, float *cls_cert)
{
    struct wset ws = {weights, nweights}, dn = {dino_w, ndino};
    struct net m;
    float *feat, *P0[2], *gy[2], *nx, *ny, *kyy, *kxy, *F, *x, *logits;
    int k, i, info, n16;

    memset(&m, 0, sizeof(m));
    m.coarse = coarse;
    m.c16 = coarse / 14;
    m.n16 = n16 = m.c16 * m.c16;
    m.ntok = n16 + 1;
    m.imagenet = 1;
    load(&m, &ws, &dn, NULL);
    feat = malloc((size_t)DV * n16 * 4);
    for (k = 0; k < 2; k++) {
        P0[k] = malloc((size_t)GP_DIM * n16 * 4);
        gy[k] = malloc((size_t)n16 * GP_DIM * 4);
        dino(&m, k ? pairB : pairA, feat, P0[k]);
        orc_transpose(P0[k], gy[k], 1, GP_DIM, n16);
    }
    nx = malloc(n16 * 4);
    ny = malloc(n16 * 4);
    kyy = malloc((size_t)n16 * n16 * 4);
    kxy = malloc((size_t)n16 * n16 * 4);
    F = malloc((size_t)n16 * GP_DIM * 4);
    x = calloc((size_t)n16 * DV, 4);
    orc_roma_row_norm(gy[0], n16, GP_DIM, nx);
    orc_roma_row_norm(gy[1], n16, GP_DIM, ny);
    orc_gemm(n16, n16, GP_DIM, gy[1], 0, GP_DIM, 0, 0, gy[1], 0, GP_DIM, 0, 0, 1,
             kyy, 0, n16, 0, 0, 1, 1, NULL, 0, NULL, 0, 1.0f, ACT_NONE, 0.0f);
    orc_roma_cos_exp(kyy, ny, ny, n16, n16, 0.2f, 1e-6f);
    orc_gemm(n16, n16, GP_DIM, gy[0], 0, GP_DIM, 0, 0, gy[1], 0, GP_DIM, 0, 0, 1,
             kxy, 0, n16, 0, 0, 1, 1, NULL, 0, NULL, 0, 1.0f, ACT_NONE, 0.0f);
    orc_roma_cos_exp(kxy, nx, ny, n16, n16, 0.2f, 1e-6f);
    memcpy(F, m.basis, (size_t)n16 * GP_DIM * 4);
    info = gp_solve(kyy, n16, F, GP_DIM);
    orc_gemm(n16, GP_DIM, n16, kxy, 0, n16, 0, 0, F, 0, GP_DIM, 0, 0, 0, x, 0,
             DV, 0, 0, 1, 1, NULL, 0, NULL, 0, 1.0f, ACT_NONE, 0.0f);
    for (i = 0; i < n16; i++)
        memcpy(x + (size_t)i * DV + GP_DIM, gy[0] + (size_t)i * GP_DIM, GP_DIM * 4);
    for (i = 0; i < DEC_DEPTH; i++)
        block(&m.dec[i], x, n16, 8, 1e-5f);
    logits = malloc((size_t)n16 * (NCLS + 1) * 4);
    linear(x, n16, DV, NCLS + 1, m.to_out_w, m.to_out_b, logits, ACT_NONE, 0);
    orc_roma_cls_to_flow(logits, NCLS + 1, NCLS, CLS_RES, n16, cls_flow, cls_cert);
    for (k = 0; k < 2; k++) {
        free(P0[k]);
        free(gy[k]);
    }
    free(feat);
    free(nx);
    free(ny);
    free(kyy);
    free(kxy);
    free(F);
    free(x);
    free(logits);
    unload(&m);
    return info;
}

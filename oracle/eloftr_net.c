/* SPDX-License-Identifier: Unlicense */

/* ORACLE — test infrastructure only (see oracle.h): the Efficient LoFTR
 * schedule of the reference (eloftr.c:41-681 of i.coregistration.opencl)
 * on the CPU kernels of oracle.c, from named weight arrays (the same
 * safetensors the HIP path loads). Folding (eloftr.c:86-162, 192-230),
 * backbone (:367-394), aggregated attention (:405-463), coarse matching
 * (:471-571), fusion (:573-604) and fine matching (:606-636). */

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define D 256
#define MLP 512
#define HEADS 8

static const int stage_blocks[4] = {1, 2, 4, 14};
static const int stage_out[4] = {64, 64, 128, 256};
static const int stage_stride[4] = {2, 1, 2, 2};

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

static void fold(const struct wset *ws, const char *prefix, int c, long per,
                 float *w, float *b)
{
    char n1[256], n2[256], n3[256], n4[256];

    snprintf(n1, sizeof(n1), "%s.weight", prefix);
    snprintf(n2, sizeof(n2), "%s.bias", prefix);
    snprintf(n3, sizeof(n3), "%s.running_mean", prefix);
    snprintf(n4, sizeof(n4), "%s.running_var", prefix);
    orc_fold_bn(w, b, c, per, need(ws, n1, c), need(ws, n2, c),
                need(ws, n3, c), need(ws, n4, c), 1e-5f);
}

struct net {
    float *bw[21], *bb[21];
    int cin[21], cout[21], stride[21];
    const float *qa[2][4], *ng[2][4], *nb[2][4], *wq[2][4], *wk[2][4],
        *wv[2][4], *wo[2][4], *fc1[2][4], *fc2[2][4], *mg[2][4], *mb[2][4];
    float *f_out, *f2_w[2], *f2_b[2];
    const float *f1_w[2], *f3_w[2];
};

static void load(struct net *m, const struct wset *ws)
{
    int s, b, l = 0, cin = 1, i, k, c, kind;
    char pre[200], name[260];

    for (s = 0; s < 4; s++)
        for (b = 0; b < stage_blocks[s]; b++, l++) {
            const int co = stage_out[s], st = b == 0 ? stage_stride[s] : 1;
            float *w, *bias, *w1, *b1;

            m->cin[l] = cin;
            m->cout[l] = co;
            m->stride[l] = st;
            snprintf(pre, sizeof(pre),
                     "efficientloftr.backbone.stages.%d.blocks.%d", s, b);
            snprintf(name, sizeof(name), "%s.conv1.conv.weight", pre);
            w = dup(need(ws, name, (long)co * cin * 9), (long)co * cin * 9);
            bias = calloc(co, sizeof(float));
            snprintf(name, sizeof(name), "%s.conv1.norm", pre);
            fold(ws, name, co, (long)cin * 9, w, bias);
            snprintf(name, sizeof(name), "%s.conv2.conv.weight", pre);
            w1 = dup(need(ws, name, (long)co * cin), (long)co * cin);
            b1 = calloc(co, sizeof(float));
            snprintf(name, sizeof(name), "%s.conv2.norm", pre);
            fold(ws, name, co, cin, w1, b1);
            for (k = 0; k < co; k++) {
                for (c = 0; c < cin; c++)
                    w[((long)k * cin + c) * 9 + 4] += w1[(long)k * cin + c];
                bias[k] += b1[k];
            }
            snprintf(name, sizeof(name), "%s.identity.weight", pre);
            if (get(ws, name, -1)) {
                float *wi = calloc((long)co * cin, sizeof(float));
                float *bi = calloc(co, sizeof(float));

                for (k = 0; k < co; k++)
                    wi[(long)k * cin + k] = 1;
                snprintf(name, sizeof(name), "%s.identity", pre);
                fold(ws, name, co, cin, wi, bi);
                for (k = 0; k < co; k++) {
                    for (c = 0; c < cin; c++)
                        w[((long)k * cin + c) * 9 + 4] += wi[(long)k * cin + c];
                    bias[k] += bi[k];
                }
                free(wi);
                free(bi);
            }
            m->bw[l] = w;
            m->bb[l] = bias;
            free(w1);
            free(b1);
            cin = co;
        }
    for (i = 0; i < 4; i++)
        for (kind = 0; kind < 2; kind++) {
            snprintf(pre, sizeof(pre),
                     "efficientloftr.local_feature_transformer.layers.%d.%s", i,
                     kind ? "cross_attention" : "self_attention");
#define LD(f, suffix, n)                                                       \
    snprintf(name, sizeof(name), "%s.%s", pre, suffix);                        \
    m->f[kind][i] = need(ws, name, n)
            LD(qa, "aggregation.q_aggregation.weight", D * 16);
            LD(ng, "aggregation.norm.weight", D);
            LD(nb, "aggregation.norm.bias", D);
            LD(wq, "attention.q_proj.weight", D * D);
            LD(wk, "attention.k_proj.weight", D * D);
            LD(wv, "attention.v_proj.weight", D * D);
            LD(wo, "attention.o_proj.weight", D * D);
            LD(fc1, "mlp.fc1.weight", MLP * 2 * D);
            LD(fc2, "mlp.fc2.weight", D * MLP);
            LD(mg, "mlp.layer_norm.weight", D);
            LD(mb, "mlp.layer_norm.bias", D);
#undef LD
        }
    m->f_out = dup(need(ws, "refinement_layer.out_conv.weight", 256 * 256),
                   256 * 256);
    for (k = 0; k < 256 * 256; k++)
        m->f_out[k] /= 16.0f;
    {
        static const int dims[3] = {256, 128, 64};

        for (i = 0; i < 2; i++) {
            const int hid = dims[i + 1], inter = dims[i];

            snprintf(name, sizeof(name),
                     "refinement_layer.out_conv_layers.%d.out_conv1.weight", i);
            m->f1_w[i] = need(ws, name, (long)inter * hid);
            snprintf(name, sizeof(name),
                     "refinement_layer.out_conv_layers.%d.out_conv2.weight", i);
            m->f2_w[i] = dup(need(ws, name, (long)inter * inter * 9),
                             (long)inter * inter * 9);
            m->f2_b[i] = calloc(inter, sizeof(float));
            snprintf(name, sizeof(name),
                     "refinement_layer.out_conv_layers.%d.batch_norm", i);
            fold(ws, name, inter, (long)inter * 9, m->f2_w[i], m->f2_b[i]);
            snprintf(name, sizeof(name),
                     "refinement_layer.out_conv_layers.%d.out_conv3.weight", i);
            m->f3_w[i] = need(ws, name, (long)hid * inter * 9);
        }
    }
}

static void unload(struct net *m)
{
    int l;

    for (l = 0; l < 21; l++) {
        free(m->bw[l]);
        free(m->bb[l]);
    }
    free(m->f_out);
    free(m->f2_w[0]);
    free(m->f2_w[1]);
    free(m->f2_b[0]);
    free(m->f2_b[1]);
}

/* conv 3 x 3, pad 1, with bias and activation (leaky slope 0.01). */
static void conv3(const float *in, int C, int H, int W, const float *w,
                  const float *b, int K, int s, int act, float *out)
{
    orc_conv2d(in, C, H, W, w, b, K, 3, 3, s, s, 1, 1, 1, 1, 1, NULL, NULL,
               NULL, act, 0.01f, out);
}

/* Y = X W^T (token-major linear, no bias). */
static void linear(const float *X, int rows, int in, const float *Wt, int out,
                   float *Y, int act, float slope)
{
    orc_gemm(rows, out, in, X, 0, in, 0, 0, Wt, 0, in, 0, 0, 1, Y, 0, out, 0,
             0, 1, 1, NULL, 0, NULL, 0, 1.0f, act, slope);
}

static void conv1x1(const float *X, int C, int HW, const float *Wt, int K,
                    float *Y)
{
    orc_gemm(K, HW, C, Wt, 0, C, 0, 0, X, 0, HW, 0, 0, 0, Y, 0, HW, 0, 0, 1,
             1, NULL, 0, NULL, 0, 1.0f, 0, 0.0f);
}

static void agg_attn(const struct net *m, int kind, int li, float *X,
                     const float *Y, int h, int w, const float *rope,
                     int use_rope)
{
    const int n = h * w, ah = h / 4, aw = w / 4, na = ah * aw;
    float *tq = malloc((size_t)D * na * 4), *tkv = malloc((size_t)D * na * 4);
    float *qn = malloc((size_t)D * na * 4), *kvn = malloc((size_t)D * na * 4);
    float *Q = malloc((size_t)D * na * 4), *K = malloc((size_t)D * na * 4);
    float *V = malloc((size_t)D * na * 4), *O = malloc((size_t)D * na * 4);
    float *O2 = malloc((size_t)D * na * 4);
    float *cat = malloc((size_t)2 * D * n * 4), *tok = malloc((size_t)2 * D * n * 4);
    float *h1 = malloc((size_t)MLP * n * 4), *h2 = malloc((size_t)D * n * 4);

    orc_conv2d(X, D, h, w, m->qa[kind][li], NULL, D, 4, 4, 4, 4, 0, 0, 1, 1, D,
               NULL, NULL, NULL, 0, 0.0f, tq);
    orc_pool2d(Y, D, h, w, 4, 4, 0, 1, tkv);
    orc_transpose(tq, qn, 1, D, na);
    orc_transpose(tkv, kvn, 1, D, na);
    orc_layernorm(na, D, qn, qn, m->ng[kind][li], m->nb[kind][li], 1e-5f, 0, 0);
    orc_layernorm(na, D, kvn, kvn, m->ng[kind][li], m->nb[kind][li], 1e-5f, 0,
                  0);
    linear(qn, na, D, m->wq[kind][li], D, Q, 0, 0);
    linear(kvn, na, D, m->wk[kind][li], D, K, 0, 0);
    linear(kvn, na, D, m->wv[kind][li], D, V, 0, 0);
    if (use_rope) {
        orc_rope(Q, 0, D, na, 1, D, na, rope, 1);
        orc_rope(K, 0, D, na, 1, D, na, rope, 1);
    }
    orc_attention(Q, 0, D, K, 0, D, V, 0, D, O, 0, D, na, na, HEADS, D / HEADS,
                  1.0f / sqrtf((float)(D / HEADS)), NULL);
    linear(O, na, D, m->wo[kind][li], D, Q, 0, 0);
    orc_transpose(Q, O2, 1, na, D);
    memcpy(cat, X, (size_t)D * n * 4);
    orc_resize(O2, D, ah, aw, cat, h, w, D, 0, 4.0f);
    orc_transpose(cat, tok, 1, 2 * D, n);
    linear(tok, n, 2 * D, m->fc1[kind][li], MLP, h1, 3, 0.01f);
    linear(h1, n, MLP, m->fc2[kind][li], D, h2, 0, 0);
    orc_layernorm(n, D, h2, h2, m->mg[kind][li], m->mb[kind][li], 1e-5f, 0, 0);
    orc_transpose(h2, cat, 1, n, D);
    orc_axpby(X, X, 1.0f, cat, 1.0f, (long)D * n, (long)D * n);
    free(tq);
    free(tkv);
    free(qn);
    free(kvn);
    free(Q);
    free(K);
    free(V);
    free(O);
    free(O2);
    free(cat);
    free(tok);
    free(h1);
    free(h2);
}

static void fusion(const struct net *m, const float *x, const float *f2,
                   const float *f1, int h, int w, float *fine)
{
    const int H4 = 2 * h, W4 = 2 * w, H2 = 4 * h, W2 = 4 * w;
    const size_t big = (size_t)256 * H2 * W2;
    float *a = malloc(big * 4), *b = malloc(big * 4), *c = malloc(big * 4);

    conv1x1(x, 256, h * w, m->f_out, 256, a);
    orc_resize(a, 256, h, w, b, H4, W4, 0, 0, 2.0f);
    conv1x1(f2, 128, H4 * W4, m->f1_w[0], 256, c);
    orc_axpby(c, c, 1.0f, b, 1.0f, 256L * H4 * W4, 256L * H4 * W4);
    conv3(c, 256, H4, W4, m->f2_w[0], m->f2_b[0], 256, 1, 3, a);
    conv3(a, 256, H4, W4, m->f3_w[0], NULL, 128, 1, 0, b);
    orc_resize(b, 128, H4, W4, c, H2, W2, 0, 0, 2.0f);
    conv1x1(f1, 64, H2 * W2, m->f1_w[1], 128, a);
    orc_axpby(a, a, 1.0f, c, 1.0f, 128L * H2 * W2, 128L * H2 * W2);
    conv3(a, 128, H2, W2, m->f2_w[1], m->f2_b[1], 128, 1, 3, b);
    conv3(b, 128, H2, W2, m->f3_w[1], NULL, 64, 1, 0, c);
    orc_resize(c, 64, H2, W2, fine, 8 * h, 8 * w, 0, 0, 2.0f);
    free(a);
    free(b);
    free(c);
}

int orc_eloftr_forward(const struct orc_named *weights, int nweights,
                       const float *grey0, const float *grey1, int H, int W,
                       float pos_scale, struct orc_eloftr_out *out)
{
    struct wset ws = {weights, nweights};
    struct net m;
    const int h = H / 8, w = W / 8, ah = h / 4, aw = w / 4, n = h * w;
    float *x[2], *f1[2], *f2[2], *fine[2], *rope, *tok0, *tok1;
    int k, nm = 0;

    memset(&m, 0, sizeof(m));
    load(&m, &ws);
    /* Backbone of both images. */
    for (k = 0; k < 2; k++) {
        const float *in = k ? grey1 : grey0;
        float *sa = malloc((size_t)16 * H * W * 4), *sb = malloc((size_t)16 * H * W * 4);
        const float *cur = in;
        int l = 0, s, b, Hc = H, Wc = W;

        f1[k] = malloc((size_t)16 * H * W * 4);
        f2[k] = malloc((size_t)8 * H * W * 4);
        x[k] = malloc((size_t)D * n * 4);
        for (s = 0; s < 4; s++)
            for (b = 0; b < stage_blocks[s]; b++, l++) {
                const int last = b == stage_blocks[s] - 1;
                float *o;

                if (last && s == 1)
                    o = f1[k];
                else if (last && s == 2)
                    o = f2[k];
                else if (last && s == 3)
                    o = x[k];
                else
                    o = cur == sa ? sb : sa;
                conv3(cur, m.cin[l], Hc, Wc, m.bw[l], m.bb[l], m.cout[l],
                      m.stride[l], 2, o);
                Hc /= m.stride[l];
                Wc /= m.stride[l];
                cur = o;
            }
        free(sa);
        free(sb);
        if (out->backbone[k])
            memcpy(out->backbone[k], x[k], (size_t)D * n * 4);
    }
    /* RoPE table (eloftr.c:267-291). */
    rope = malloc((size_t)ah * aw * 128 * 2 * 4);
    {
        int i, j, p;

        for (i = 0; i < ah; i++)
            for (j = 0; j < aw; j++)
                for (p = 0; p < 128; p++) {
                    const float f =
                        (float)(1.0 / pow(10000.0, (double)(2 * (p / 2)) / 128));
                    const float a =
                        (p % 2 ? (float)(j + 1) : (float)(i + 1)) * pos_scale * f;
                    float *q = rope + (((size_t)i * aw + j) * 128 + p) * 2;

                    q[0] = cosf(a);
                    q[1] = sinf(a);
                }
    }
    for (k = 0; k < 4; k++) {
        agg_attn(&m, 0, k, x[0], x[0], h, w, rope, 1);
        agg_attn(&m, 0, k, x[1], x[1], h, w, rope, 1);
        agg_attn(&m, 1, k, x[0], x[1], h, w, rope, 0);
        agg_attn(&m, 1, k, x[1], x[0], h, w, rope, 0);
    }
    free(rope);
    for (k = 0; k < 2; k++)
        if (out->coarse[k])
            memcpy(out->coarse[k], x[k], (size_t)D * n * 4);
    /* Coarse matching, one block of rows per 256 Mi scores. */
    tok0 = malloc((size_t)D * n * 4);
    tok1 = malloc((size_t)D * n * 4);
    orc_transpose(x[0], tok0, 1, D, n);
    orc_transpose(x[1], tok1, 1, D, n);
    orc_eloftr_coarse(tok0, tok1, n, D, 1.0f / (D * 0.1f), n, out->row_max,
                      out->row_arg, out->col_arg, out->row_margin,
                      out->col_margin, out->col_max);
    free(tok0);
    free(tok1);
    nm = orc_eloftr_select(out->row_max, out->row_arg, out->col_arg, h, w,
                           0.2f, 2, out->mi, out->mj, out->mconf);
    out->nm = nm;
    for (k = 0; k < 2; k++) {
        fine[k] = out->fine[k] ? out->fine[k]
                               : malloc((size_t)64 * H * W * 4);
        fusion(&m, x[k], f2[k], f1[k], h, w, fine[k]);
    }
    if (nm > 0) {
        int *cells = malloc((size_t)nm * 4 * sizeof(int)), i;

        for (i = 0; i < nm; i++) {
            cells[4 * i] = out->mi[i] % w;
            cells[4 * i + 1] = out->mi[i] / w;
            cells[4 * i + 2] = out->mj[i] % w;
            cells[4 * i + 3] = out->mj[i] / w;
        }
        orc_eloftr_fine(fine[0], fine[1], H, W, cells, nm, 10.0f, out->kp,
                        out->fine_margin);
        free(cells);
    }
    for (k = 0; k < 2; k++) {
        if (!out->fine[k])
            free(fine[k]);
        free(f1[k]);
        free(f2[k]);
        free(x[k]);
    }
    unload(&m);
    return nm;
}

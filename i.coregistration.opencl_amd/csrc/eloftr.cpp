/* SPDX-License-Identifier: Unlicense */

/* Efficient LoFTR driver on the HIP path: weight folding at load, work
 * buffers, and the stage schedule of one tile pair. The model, its
 * constants and the order of operations are those of the reference
 * (eloftr.c:41-681 of i.coregistration.opencl, itself following
 * EfficientLoFTRForKeypointMatching), because the results must be the
 * same; every stage runs on this build's kernels (ops.h and
 * icoreg_kernels.h). Departures, none of which changes a result:
 *  - both images stay resident; eloftr_match_device takes them from
 *    device memory (the timed path of bench.py);
 *  - the coarse score matrix is processed in blocks of up to 256 Mi
 *    floats (the reference: 64 Mi, sized for a 16 GiB card); with a
 *    single block the second pass reuses the scores instead of
 *    recomputing the identical GEMM;
 *  - statistics buffers are initialised by device fills, not host
 *    writes;
 *  - the two self-attention blocks of a layer run as one batch, and the
 *    MLP of every attention block runs on channel-major maps (products
 *    W * [x; message] instead of token-major linears between
 *    transposes, the MLP LayerNorm fused with the residual add): the
 *    same sums per output value, in another memory layout;
 *  - k_proj and v_proj run as one product with their weights stacked;
 *  - an attention block's aggregation, pooling, transposes to tokens and
 *    both LayerNorms are one kernel;
 *  - fc1 [x; up4(o_proj O^T)] runs as fc1[:, :256] x + up4(Wm O^T) with
 *    Wm = fc1[:, 256:] o_proj multiplied at load: the 4x upsampling is
 *    linear within each channel plane, so it commutes with the channel
 *    products, and the message half of fc1 runs on the 400 aggregated
 *    tokens instead of the 6400 upsampled ones (sampled in the product's
 *    epilogue, with the resize's arithmetic);
 *  - the fusion's "1 x 1 convolution + upsampled coarser level" sums are
 *    the 1 x 1 products' residual inputs instead of separate adds;
 *  - the same-size 3 x 3 convolutions run as Winograd F(2 x 2, 3 x 3)
 *    with the filters transformed once at load: the same sums, regrouped
 *    (16 instead of 36 multiplications per 2 x 2 output tile and input
 *    channel), equal to the direct sums within float rounding. */

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "common.h"
#include "conv.h"
#include "eloftr.h"
#include "eloftr_fused.h"
#include "gemm.h"
#include "icoreg_kernels.h"

using namespace icoreg;

/* config.json of zju-community/efficientloftr (eloftr.c:41-55). */
static const int stage_blocks[4] = {1, 2, 4, 14};
static const int stage_out[4] = {64, 64, 128, 256};
static const int stage_stride[4] = {2, 1, 2, 2};
#define HEADS 8
#define MLP 512
#define EPS_BN 1e-5f
#define EPS_LN 1e-5f
#define LEAKY 0.01f
#define COARSE_T 0.1f
#define COARSE_THR 0.2f
#define BORDER 2
#define FINE_T 10.0f
#define ROPE_BASE 10000.0
#define ROPE_DIM 128 /* head_dim x partial_rotary_factor: 32 x 4. */
/* Largest coarse score block, in floats. */
#define SCORE_BLOCK_FLOATS ((size_t)256 << 20)

static float *read_host(struct pth_file *pf, const char *name, int ndim,
                        const long *shape)
{
    return pth_read_f32(pf, pth_require(pf, name, ndim, shape));
}

static cl_mem upload(struct eloftr_model *m, const float *v, size_t n,
                     const char *what)
{
    return ocl_upload(m->ocl, v, n * sizeof(float), what);
}

static cl_mem load_dev(struct eloftr_model *m, struct pth_file *pf,
                       const char *name, int ndim, const long *shape)
{
    float *v = read_host(pf, name, ndim, shape);
    long n = 1;
    cl_mem b;

    for (int d = 0; d < ndim; d++)
        n *= shape[d];
    b = upload(m, v, (size_t)n, name);
    free(v);
    return b;
}

/* BatchNorm <prefix>.{weight,bias,running_mean,running_var} of c
 * channels folded into w (c x per) and b. */
static void fold(struct pth_file *pf, const char *prefix, int c, long per,
                 float *w, float *b)
{
    char name[256];
    long shape[1] = {c};
    float *g, *bt, *mu, *var;

    snprintf(name, sizeof(name), "%s.weight", prefix);
    g = read_host(pf, name, 1, shape);
    snprintf(name, sizeof(name), "%s.bias", prefix);
    bt = read_host(pf, name, 1, shape);
    snprintf(name, sizeof(name), "%s.running_mean", prefix);
    mu = read_host(pf, name, 1, shape);
    snprintf(name, sizeof(name), "%s.running_var", prefix);
    var = read_host(pf, name, 1, shape);
    ops_fold_bn(w, b, c, per, g, bt, mu, var, EPS_BN);
    free(g);
    free(bt);
    free(mu);
    free(var);
}

/* RepVGG block l (eloftr.c:108-162): conv1 3 x 3 + conv2 1 x 1 +
 * identity, each with its BatchNorm, as one 3 x 3 convolution. */
static void load_block(struct eloftr_model *m, struct pth_file *pf, int l,
                       int stage, int blk)
{
    const int ci = m->bcin[l], co = m->bcout[l];
    long s3[4] = {co, ci, 3, 3}, s1[4] = {co, ci, 1, 1};
    char pre[160], name[200];
    float *w, *b, *w1, *b1;

    snprintf(pre, sizeof(pre), "efficientloftr.backbone.stages.%d.blocks.%d",
             stage, blk);
    snprintf(name, sizeof(name), "%s.conv1.conv.weight", pre);
    w = read_host(pf, name, 4, s3);
    b = (float *)calloc(co, sizeof(float));
    snprintf(name, sizeof(name), "%s.conv1.norm", pre);
    fold(pf, name, co, (long)ci * 9, w, b);
    snprintf(name, sizeof(name), "%s.conv2.conv.weight", pre);
    w1 = read_host(pf, name, 4, s1);
    b1 = (float *)calloc(co, sizeof(float));
    snprintf(name, sizeof(name), "%s.conv2.norm", pre);
    fold(pf, name, co, ci, w1, b1);
    for (int k = 0; k < co; k++) {
        for (int c = 0; c < ci; c++)
            w[((size_t)k * ci + c) * 9 + 4] += w1[(size_t)k * ci + c];
        b[k] += b1[k];
    }
    snprintf(name, sizeof(name), "%s.identity.weight", pre);
    if (pth_find(pf, name)) {
        float *wi, *bi;

        if (ci != co || m->bstride[l] != 1)
            icoreg_fatal("ELoFTR: unexpected identity branch in <%s>", pre);
        wi = (float *)calloc((size_t)co * ci, sizeof(float));
        bi = (float *)calloc(co, sizeof(float));
        for (int k = 0; k < co; k++)
            wi[(size_t)k * ci + k] = 1;
        snprintf(name, sizeof(name), "%s.identity", pre);
        fold(pf, name, co, ci, wi, bi);
        for (int k = 0; k < co; k++) {
            for (int c = 0; c < ci; c++)
                w[((size_t)k * ci + c) * 9 + 4] += wi[(size_t)k * ci + c];
            b[k] += bi[k];
        }
        free(wi);
        free(bi);
    }
    else if (ci == co && m->bstride[l] == 1)
        icoreg_fatal("ELoFTR: identity branch missing in <%s>", pre);
    m->bw[l] = upload(m, w, (size_t)co * ci * 9, "backbone weight");
    m->bb[l] = upload(m, b, co, "backbone bias");
    free(w);
    free(b);
    free(w1);
    free(b1);
}

static void load_attn(struct eloftr_model *m, struct pth_file *pf, int layer,
                      const char *kind, struct eloftr_attn *a)
{
    char pre[160], name[240];
    long qa[4] = {ELOFTR_DIM, 1, 4, 4}, sq[2] = {ELOFTR_DIM, ELOFTR_DIM};
    long s1[2] = {MLP, 2 * ELOFTR_DIM}, s2[2] = {ELOFTR_DIM, MLP};
    long v1[1] = {ELOFTR_DIM};

    snprintf(pre, sizeof(pre),
             "efficientloftr.local_feature_transformer.layers.%d.%s", layer,
             kind);
#define LD(field, suffix, nd, shape)                                           \
    snprintf(name, sizeof(name), "%s.%s", pre, suffix);                        \
    a->field = load_dev(m, pf, name, nd, shape)
    LD(q_agg, "aggregation.q_aggregation.weight", 4, qa);
    LD(norm_g, "aggregation.norm.weight", 1, v1);
    LD(norm_b, "aggregation.norm.bias", 1, v1);
    LD(wq, "attention.q_proj.weight", 2, sq);
    LD(fc1, "mlp.fc1.weight", 2, s1);
    LD(fc2, "mlp.fc2.weight", 2, s2);
    LD(mlp_g, "mlp.layer_norm.weight", 1, v1);
    LD(mlp_b, "mlp.layer_norm.bias", 1, v1);
#undef LD
    {
        /* k_proj and v_proj stacked into one (512, 256) weight, so that
         * keys and values come from one product with the shared input. */
        const size_t dd = (size_t)ELOFTR_DIM * ELOFTR_DIM;
        float *kv = (float *)malloc(2 * dd * sizeof(float)), *w;

        if (!kv)
            icoreg_fatal("ELoFTR: out of host memory");
        snprintf(name, sizeof(name), "%s.attention.k_proj.weight", pre);
        w = read_host(pf, name, 2, sq);
        memcpy(kv, w, dd * sizeof(float));
        free(w);
        snprintf(name, sizeof(name), "%s.attention.v_proj.weight", pre);
        w = read_host(pf, name, 2, sq);
        memcpy(kv + dd, w, dd * sizeof(float));
        free(w);
        a->wkv = upload(m, kv, 2 * dd, "attention.kv_proj");
        free(kv);
    }
    {
        /* The message reaches the MLP only as fc1[:, D:2D] up4(o_proj O^T)
         * (O the attention output, up4 the 4x bilinear upsampling). The
         * upsampling mixes pixels of one channel plane and the products
         * mix channels of one pixel, so this equals
         * up4((fc1[:, D:2D] o_proj) O^T): the two weights are multiplied
         * here once, in double, and fc1's message half then runs on the
         * na aggregated tokens instead of the n upsampled ones. */
        const int D = ELOFTR_DIM;
        float *wo, *f1, *wm = (float *)malloc((size_t)MLP * D * sizeof(float));
        double *acc = (double *)malloc((size_t)D * sizeof(double));

        if (!wm || !acc)
            icoreg_fatal("ELoFTR: out of host memory");
        snprintf(name, sizeof(name), "%s.attention.o_proj.weight", pre);
        wo = read_host(pf, name, 2, sq);
        snprintf(name, sizeof(name), "%s.mlp.fc1.weight", pre);
        f1 = read_host(pf, name, 2, s1);
        for (int i = 0; i < MLP; i++) {
            for (int j = 0; j < D; j++)
                acc[j] = 0.0;
            for (int c = 0; c < D; c++) {
                const double f = f1[(size_t)i * 2 * D + D + c];
                const float *wr = wo + (size_t)c * D;

                for (int j = 0; j < D; j++)
                    acc[j] += f * wr[j];
            }
            for (int j = 0; j < D; j++)
                wm[(size_t)i * D + j] = (float)acc[j];
        }
        a->wmsg = upload(m, wm, (size_t)MLP * D, "attention.message");
        free(wo);
        free(f1);
        free(wm);
        free(acc);
    }
}

static void load_fusion(struct eloftr_model *m, struct pth_file *pf)
{
    static const int dims[3] = {256, 128, 64};
    long so[4] = {256, 256, 1, 1};
    float *w;

    /* The coarse features enter the fusion divided by sqrt(256), folded
     * into out_conv (no bias). eloftr.c:199-205. */
    w = read_host(pf, "refinement_layer.out_conv.weight", 4, so);
    for (int k = 0; k < 256 * 256; k++)
        w[k] /= 16.0f;
    m->f_out = upload(m, w, 256 * 256, "out_conv");
    free(w);
    for (int i = 0; i < 2; i++) {
        const int hid = dims[i + 1], inter = dims[i];
        long s1[4] = {inter, hid, 1, 1}, s2[4] = {inter, inter, 3, 3};
        long s3[4] = {hid, inter, 3, 3};
        char name[160];
        float *b = (float *)calloc(inter, sizeof(float));

        snprintf(name, sizeof(name),
                 "refinement_layer.out_conv_layers.%d.out_conv1.weight", i);
        m->f1_w[i] = load_dev(m, pf, name, 4, s1);
        snprintf(name, sizeof(name),
                 "refinement_layer.out_conv_layers.%d.out_conv2.weight", i);
        w = read_host(pf, name, 4, s2);
        snprintf(name, sizeof(name),
                 "refinement_layer.out_conv_layers.%d.batch_norm", i);
        fold(pf, name, inter, (long)inter * 9, w, b);
        m->f2_w[i] = upload(m, w, (size_t)inter * inter * 9, "out_conv2");
        m->f2_b[i] = upload(m, b, inter, "out_conv2 bias");
        free(w);
        free(b);
        snprintf(name, sizeof(name),
                 "refinement_layer.out_conv_layers.%d.out_conv3.weight", i);
        m->f3_w[i] = load_dev(m, pf, name, 4, s3);
    }
}

extern "C" void eloftr_load(struct eloftr_model *m, struct ops *ops,
                            struct pth_file *pf)
{
    ICOREG_API_BEGIN
    int l = 0, cin = 1;

    memset(m, 0, sizeof(*m));
    m->ops = ops;
    m->ocl = ops->ocl;
    m->pos_scale = 1.0f;
    for (int s = 0; s < 4; s++)
        for (int b = 0; b < stage_blocks[s]; b++, l++) {
            m->bcin[l] = cin;
            m->bcout[l] = stage_out[s];
            m->bstride[l] = b == 0 ? stage_stride[s] : 1;
            load_block(m, pf, l, s, b);
            cin = stage_out[s];
        }
    for (int i = 0; i < ELOFTR_LAYERS; i++) {
        load_attn(m, pf, i, "self_attention", &m->self_attn[i]);
        load_attn(m, pf, i, "cross_attention", &m->cross_attn[i]);
    }
    load_fusion(m, pf);
    /* Same-size 3 x 3 filters in Winograd form, once. */
    for (l = 0; l < ELOFTR_BLOCKS; l++)
        if (m->bstride[l] == 1 &&
            conv_wino_supported(3, 3, 1, 1, 1, 1, 1, 1, 1, m->bcin[l],
                                m->bcout[l], 1, 1))
            m->bU[l] = conv_wino_prepare(ops, m->bw[l], m->bcout[l],
                                         m->bcin[l]);
    for (int i = 0; i < 2; i++) {
        const int d = i ? 128 : 256, d3 = i ? 64 : 128;

        m->f2_U[i] = conv_wino_prepare(ops, m->f2_w[i], d, d);
        m->f3_U[i] = conv_wino_prepare(ops, m->f3_w[i], d3, d);
    }
    ICOREG_API_END
}

static cl_mem walloc(struct eloftr_model *m, size_t floats, const char *what)
{
    return ocl_alloc(m->ocl, floats * sizeof(float), what);
}

/* Image k's part of a pair buffer of 2 x floats. */
static cl_mem view(cl_mem pair, int k, size_t floats)
{
    return ocl_wrap((float *)pair->ptr + (size_t)k * floats,
                    floats * sizeof(float));
}

/* RoPE (cos, sin) table of the aggregated grid (eloftr.c:267-291):
 * position (i, j), 1-based, times pos_scale; pair p of the 256 channels
 * turns by i f(p / 2) for even p, j f(p / 2) for odd p, f(k) =
 * 10000^(-2k / 128). */
static void rope_table(struct eloftr_model *m)
{
    const int np = ELOFTR_DIM / 2;
    float *t = (float *)malloc((size_t)m->ah * m->aw * np * 2 * sizeof(float));

    for (int i = 0; i < m->ah; i++)
        for (int j = 0; j < m->aw; j++)
            for (int p = 0; p < np; p++) {
                const float f = (float)(1.0 / pow(ROPE_BASE, (double)(2 * (p / 2)) /
                                                               ROPE_DIM));
                const float a = (p % 2 ? (float)(j + 1) : (float)(i + 1)) *
                                m->pos_scale * f;
                float *q = t + (((size_t)i * m->aw + j) * np + p) * 2;

                q[0] = cosf(a);
                q[1] = sinf(a);
            }
    m->rope = upload(m, t, (size_t)m->ah * m->aw * np * 2, "rope");
    free(t);
}

extern "C" void eloftr_alloc(struct eloftr_model *m, int H, int W)
{
    ICOREG_API_BEGIN
    size_t hw = (size_t)H * W, n, na;

    if (H <= 0 || W <= 0 || H % ELOFTR_MULTIPLE || W % ELOFTR_MULTIPLE)
        icoreg_fatal("ELoFTR tile %d x %d is not a multiple of %d", H, W,
                     ELOFTR_MULTIPLE);
    m->H = H;
    m->W = W;
    m->h = H / 8;
    m->w = W / 8;
    m->ah = m->h / 4;
    m->aw = m->w / 4;
    n = (size_t)m->h * m->w;
    na = (size_t)m->ah * m->aw;
    m->img = walloc(m, 2 * hw, "images");
    m->s_a = walloc(m, 2 * 16 * hw, "backbone");
    m->s_b = walloc(m, 2 * 16 * hw, "backbone");
    m->f1p = walloc(m, 2 * 16 * hw, "1/2 features");
    m->f2p = walloc(m, 2 * 8 * hw, "1/4 features");
    m->xp = walloc(m, 2 * ELOFTR_DIM * n, "1/8 features");
    m->finep = walloc(m, 2 * ELOFTR_FINE_DIM * hw, "fine features");
    for (int k = 0; k < 2; k++) {
        m->f1[k] = view(m->f1p, k, 16 * hw);
        m->f2[k] = view(m->f2p, k, 8 * hw);
        m->x[k] = view(m->xp, k, ELOFTR_DIM * n);
        m->fine[k] = view(m->finep, k, ELOFTR_FINE_DIM * hw);
    }
    /* Transformer work buffers hold both images (self-attention runs the
     * pair as one batch). */
    m->t_qn = walloc(m, 2 * ELOFTR_DIM * na, "tokens");
    m->t_kvn = walloc(m, 2 * ELOFTR_DIM * na, "tokens");
    m->t_Q = walloc(m, 2 * ELOFTR_DIM * na, "queries");
    m->t_KV = walloc(m, 4 * ELOFTR_DIM * na, "keys and values");
    m->t_O = walloc(m, 2 * ELOFTR_DIM * na, "attention");
    m->t_O2 = walloc(m, 2 * MLP * na, "attention");
    m->t_tok = walloc(m, ELOFTR_DIM * n, "tokens");
    m->t_h1 = walloc(m, 2 * MLP * n, "mlp");
    m->t_h2 = walloc(m, 2 * ELOFTR_DIM * n, "mlp");
    rope_table(m);
    m->blk_rows = (int)(SCORE_BLOCK_FLOATS / n);
    if (m->blk_rows > (int)n)
        m->blk_rows = (int)n;
    if (m->blk_rows < 1)
        m->blk_rows = 1;
    m->s_blk = walloc(m, (size_t)m->blk_rows * n, "scores");
    m->row_lse = walloc(m, n, "row lse");
    m->col_m = walloc(m, n, "column max");
    m->col_s = walloc(m, n, "column sum");
    m->row_max = walloc(m, n, "row max");
    m->col_max = walloc(m, n, "column max");
    m->row_arg = ocl_alloc(m->ocl, n * sizeof(int), "row argmax");
    m->col_arg = ocl_alloc(m->ocl, n * sizeof(int), "column argmax");
    m->fu_a = walloc(m, 2 * 32 * hw, "fusion");
    m->fu_b = walloc(m, 2 * 32 * hw, "fusion");
    m->fu_c = walloc(m, 2 * 32 * hw, "fusion");
    for (int k = 0; k < 2; k++)
        m->fine_h[k] = view(m->fu_c, k, (size_t)ELOFTR_FINE_DIM * (m->H / 2) * (m->W / 2));
    m->nmax = (int)n;
    m->m_idx = ocl_alloc(m->ocl, n * 4 * sizeof(int), "match cells");
    m->m_out = walloc(m, n * 4, "fine matches");
    m->d_mi = ocl_alloc(m->ocl, n * sizeof(int), "matches");
    m->d_mj = ocl_alloc(m->ocl, n * sizeof(int), "matches");
    m->d_mconf = walloc(m, n, "match confidences");
    m->m_count = ocl_alloc(m->ocl, 2 * sizeof(int), "match count");
    m->mi = (int *)malloc(n * sizeof(int));
    m->mj = (int *)malloc(n * sizeof(int));
    m->mconf = (float *)malloc(n * sizeof(float));
    m->kp = (float *)malloc(n * 4 * sizeof(float));
    m->h_rmax = (float *)malloc(n * sizeof(float));
    m->h_rarg = (int *)malloc(n * sizeof(int));
    m->h_carg = (int *)malloc(n * sizeof(int));
    ICOREG_API_END
}

/* 3 x 3 convolution of both images of a pair: in holds image 1 at
 * in_stride floats after image 0, out likewise at out_stride. */
static void conv3x3_pair(struct eloftr_model *m, cl_mem in, long in_stride,
                         int C, int H, int W, cl_mem w, cl_mem b, int K,
                         int stride, int act, cl_mem out, long out_stride,
                         cl_mem U = NULL)
{
    struct conv_geom g = ops_geom(3, stride, 1);

    if (U)
        conv3x3_wino_batch(m->ops, 2, in, in_stride, C, H, W, w, U, b, K, act,
                           LEAKY, out, out_stride);
    else
        ops_conv2d_batch(m->ops, 2, in, in_stride, C, H, W, w, b, K, &g, NULL,
                         NULL, NULL, act, LEAKY, out, out_stride);
}

/* The RepVGG backbone on both images of the pair (m->img: image 1 at
 * H W floats after image 0): 1/2 features into f1p, 1/4 into f2p, 1/8
 * into xp, each layer one launch for the pair. eloftr.c:367-394. */
static void backbone(struct eloftr_model *m)
{
    cl_mem in = m->img;
    long in_stride = (long)m->H * m->W;
    int l = 0, Hc = m->H, Wc = m->W;

    for (int s = 0; s < 4; s++)
        for (int b = 0; b < stage_blocks[s]; b++, l++) {
            const int st = m->bstride[l], last = b == stage_blocks[s] - 1;
            const int Ho = Hc / st, Wo = Wc / st;
            const long out_stride = (long)m->bcout[l] * Ho * Wo;
            cl_mem out;

            if (last && s == 1)
                out = m->f1p;
            else if (last && s == 2)
                out = m->f2p;
            else if (last && s == 3)
                out = m->xp;
            else
                out = in == m->s_a ? m->s_b : m->s_a;
            conv3x3_pair(m, in, in_stride, m->bcin[l], Hc, Wc, m->bw[l],
                         m->bb[l], m->bcout[l], st, ACT_RELU, out, out_stride,
                         m->bU[l]);
            Hc = Ho;
            Wc = Wo;
            in = out;
            in_stride = out_stride;
        }
}

/* One aggregated attention block (eloftr.c:405-449) for nimg images at
 * once: image i of X (256 x h x w maps, nimg of them one after the other)
 * attends to image i of Y and is updated in place. The self-attention
 * blocks of a pair run with nimg = 2 (both images' maps are contiguous
 * in xp); cross-attention runs image by image, as the reference orders
 * it.
 *
 * The reference's sequence, with its layout changes folded away: the
 * aggregation, pooling, transposes to tokens and LayerNorms are one
 * kernel; o_proj and fc1's message half are one product (their weights
 * multiplied at load) on the aggregated tokens, written channel-major (the
 * token-major attention output as the transposed operand); its 4x
 * upsampling is added inside fc1's product with x; the MLP runs on
 * channel-major maps, and the MLP LayerNorm is fused with the residual
 * add. */
static void agg_attn(struct eloftr_model *m, const struct eloftr_attn *a,
                     cl_mem X, cl_mem Y, int nimg, int use_rope, cl_mem T = NULL)
{
    struct ops *o = m->ops;
    const int D = ELOFTR_DIM, n = m->h * m->w, na = m->ah * m->aw;
    const int hd = D / HEADS, rows = nimg * na;

    eloftr_aggregate(o, X, Y, nimg, D, m->h, m->w, a->q_agg, a->norm_g,
                     a->norm_b, EPS_LN, m->t_qn, m->t_kvn);
    /* Queries, and keys (columns 0..D-1) with values (D..2D-1) of t_KV,
     * in one launch, the rotary encoding of the queries and keys in its
     * epilogue; row r takes table row r % na: the same positions per
     * image. */
    ops_linear2_rope(o, rows, D, m->t_qn, a->wq, m->t_Q, D, use_rope ? D : 0, m->t_kvn, a->wkv,
                     m->t_KV, 2 * D, use_rope ? D : 0, m->rope, D, na);
    /* Image i's queries attend to image i's keys: one launch for all. */
    ops_attention_batch(o, nimg, ops_mat(m->t_Q, 0, D), (long)na * D,
                        ops_mat(m->t_KV, 0, 2 * D), 2L * na * D,
                        ops_mat(m->t_KV, D, 2 * D), 2L * na * D,
                        ops_mat(m->t_O, 0, D), (long)na * D, na, na, HEADS, hd,
                        1.0f / sqrtf((float)hd), NULL);
    /* P (MLP x na per image) = (fc1[:, D:2D] o_proj) (MLP x D) * O^T, O
     * token-major: fc1's message half on the aggregated tokens. */
    ops_gemm(o, MLP, na, D, ops_mat(a->wmsg, 0, D),
             ops_bmat(m->t_O, 0, D, (long)na * D, 0), 1,
             ops_bmat(m->t_O2, 0, na, (long)MLP * na, 0), nimg, 1, NULL, 0,
             NULL, 0, 1.0f, ACT_NONE, 0);
    /* h1 (MLP x n) = leaky(fc1[:, 0:D] (MLP x D) * x (D x n) + up4(P)):
     * fc1 (MLP x 2D) * [x; up4(message)], the 4x upsampling (ops_resize,
     * scale 4) sampled in the product's epilogue. */
    ops_gemm_upres(o, MLP, n, D, ops_mat(a->fc1, 0, 2 * D),
                   ops_bmat(X, 0, n, (long)D * n, 0),
                   ops_bmat(m->t_h1, 0, n, (long)MLP * n, 0), nimg, m->t_O2,
                   (long)MLP * na, m->ah, m->aw, m->h, m->w, 4, 1, ACT_LEAKY,
                   LEAKY);
    /* h2 (D x n) = fc2 (D x MLP) * h1. */
    ops_gemm(o, D, n, MLP, ops_mat(a->fc2, 0, MLP),
             ops_bmat(m->t_h1, 0, n, (long)MLP * n, 0), 0,
             ops_bmat(m->t_h2, 0, n, (long)D * n, 0), nimg, 1, NULL, 1, NULL,
             0, 1.0f, ACT_NONE, 0);
    eloftr_ln_residual(o, m->t_h2, nimg, D, n, a->mlp_g, a->mlp_b, EPS_LN, X, T);
}

/* eloftr.c:451-463: image 1's cross attention sees image 0's features
 * already updated by this layer. The two self-attention blocks of a layer
 * are independent and run as one. */
static void transformer(struct eloftr_model *m)
{
    for (int l = 0; l < ELOFTR_LAYERS; l++) {
        const bool last = l == ELOFTR_LAYERS - 1;

        agg_attn(m, &m->self_attn[l], m->xp, m->xp, 2, 1);
        /* The last layer also writes the features token-major for the
         * coarse matching (t_tok, t_h1 once its MLP is done). */
        agg_attn(m, &m->cross_attn[l], m->x[0], m->x[1], 1, 0, last ? m->t_tok : NULL);
        agg_attn(m, &m->cross_attn[l], m->x[1], m->x[0], 1, 0, last ? m->t_h1 : NULL);
    }
}

/* Coarse dual-softmax matching by blocks of rows, then mutual maxima
 * above the threshold away from the border (eloftr.c:471-571). */
static void coarse_match(struct eloftr_model *m)
{
    struct ops *o = m->ops;
    const int D = ELOFTR_DIM, n = m->h * m->w, R = m->blk_rows;
    const float alpha = 1.0f / (D * COARSE_T);
    const bool one_block = R >= n;
    /* Both passes read each block of S once (rows and columns together). */
    const bool tiles = eloftr_tiles_ok(m->s_blk, n);

    /* The features arrive token-major in t_tok and t_h1 (transformer). The
     * tile passes start the column statistics from their first block. */
    if (!tiles) {
        ocl_fill(m->ocl, m->col_m, 0, n, -INFINITY);
        ocl_fill(m->ocl, m->col_s, 0, n, 0.0f);
        ocl_fill(m->ocl, m->col_max, 0, n, -1.0f);
        ocl_fill_u32(m->ocl, m->col_arg, 0, n, 0xffffffffu);
    }
    for (int pass = 0; pass < 2; pass++)
        for (int r0 = 0; r0 < n; r0 += R) {
            const int rows = n - r0 < R ? n - r0 : R;

            if (pass == 0 || !one_block)
                ops_gemm(o, rows, n, D, ops_mat(m->t_tok, (long)r0 * D, D),
                         ops_mat(m->t_h1, 0, D), 1, ops_mat(m->s_blk, 0, n), 1,
                         1, NULL, 0, NULL, 0, alpha, ACT_NONE, 0);
            if (pass == 0 && tiles) {
                eloftr_lse_tiles(o, m->s_blk, rows, n, r0, m->row_lse, m->col_m, m->col_s);
            }
            else if (pass == 0) {
                eloftr_row_lse(o, m->s_blk, rows, n, r0, m->row_lse);
                eloftr_col_lse(o, m->s_blk, rows, n, m->col_m, m->col_s);
            }
            else if (tiles) {
                eloftr_conf_tiles(o, m->s_blk, rows, n, r0, m->row_lse, m->col_m, m->col_s,
                                  m->row_max, m->row_arg, m->col_max, m->col_arg);
            }
            else {
                eloftr_conf_row(o, m->s_blk, rows, n, r0, m->row_lse, m->col_m,
                                m->col_s, m->row_max, m->row_arg);
                eloftr_conf_col(o, m->s_blk, rows, n, r0, m->row_lse, m->col_m,
                                m->col_s, m->col_max, m->col_arg);
            }
        }
    /* Mutual selection on the device (eloftr.c:606-636): the matches
     * stay in HBM for fine matching and come back with its results. */
    eloftr_mutual(o, m->row_max, m->row_arg, m->col_arg, m->h, m->w, BORDER, COARSE_THR,
                  m->d_mi, m->d_mj, m->d_mconf, m->m_idx, m->m_count);
}

/* 1 x 1 convolution of both images: W (K, C) times X (C, HW) per image,
 * images C HW / K HW floats apart in X / Y; R (Y's layout) is added when
 * given. */
static void conv1x1_pair(struct eloftr_model *m, cl_mem X, int C, int HW,
                         cl_mem Wt, int K, cl_mem Y, cl_mem R = NULL)
{
    ops_gemm(m->ops, K, HW, C, ops_mat(Wt, 0, C),
             ops_bmat(X, 0, HW, (long)C * HW, 0), 0,
             ops_bmat(Y, 0, HW, (long)K * HW, 0), 2, 1, NULL, 1, R, 0, 1.0f,
             ACT_NONE, 0);
}

/* conv1x1_pair plus the 2x bilinear resize of Rlow (K x HW / 4 per image,
 * K HW / 4 floats apart) as the residual: the reference's ops_resize and
 * residual add after the 1 x 1 convolution, without the upsampled map. */
static void conv1x1_up2_pair(struct eloftr_model *m, cl_mem X, int C, int H, int W,
                             cl_mem Wt, int K, cl_mem Y, cl_mem Rlow)
{
    const long HW = (long)H * W;

    ops_gemm_upres(m->ops, K, (int)HW, C, ops_mat(Wt, 0, C),
                   ops_bmat(X, 0, HW, (long)C * HW, 0), ops_bmat(Y, 0, HW, (long)K * HW, 0),
                   2, Rlow, (long)K * (HW / 4), H / 2, W / 2, H, W, 2, 0, ACT_NONE, 0);
}

/* FPN fusion of both images (eloftr.c:573-604), every layer one launch for
 * the pair (the pair's channels are contiguous). The reference's three 2x
 * resizes are sampled on the fly by their consumers, with the resize's
 * arithmetic: the residuals of the two 1 x 1 convolutions
 * (ops_gemm_upres) and fine matching (eloftr_fine_half). The result is
 * fu_c, the fine maps at half resolution (64, H / 2, W / 2) per image. */
static void fusion(struct eloftr_model *m)
{
    const int h = m->h, w = m->w;
    const int H4 = 2 * h, W4 = 2 * w, H2 = 4 * h, W2 = 4 * w;

    conv1x1_pair(m, m->xp, 256, h * w, m->f_out, 256, m->fu_a);
    conv1x1_up2_pair(m, m->f2p, 128, H4, W4, m->f1_w[0], 256, m->fu_c, m->fu_a);
    conv3x3_pair(m, m->fu_c, 256L * H4 * W4, 256, H4, W4, m->f2_w[0],
                 m->f2_b[0], 256, 1, ACT_LEAKY, m->fu_a, 256L * H4 * W4,
                 m->f2_U[0]);
    conv3x3_pair(m, m->fu_a, 256L * H4 * W4, 256, H4, W4, m->f3_w[0], NULL,
                 128, 1, ACT_NONE, m->fu_b, 128L * H4 * W4, m->f3_U[0]);
    conv1x1_up2_pair(m, m->f1p, 64, H2, W2, m->f1_w[1], 128, m->fu_a, m->fu_b);
    conv3x3_pair(m, m->fu_a, 128L * H2 * W2, 128, H2, W2, m->f2_w[1],
                 m->f2_b[1], 128, 1, ACT_LEAKY, m->fu_b, 128L * H2 * W2,
                 m->f2_U[1]);
    conv3x3_pair(m, m->fu_b, 128L * H2 * W2, 128, H2, W2, m->f3_w[1], NULL, 64,
                 1, ACT_NONE, m->fu_c, 64L * H2 * W2, m->f3_U[1]);
    /* The reference resizes fu_c 2x into the fine maps here; fine
     * matching samples that resize on the fly instead, and finep is
     * written only when asked for (eloftr_fine_maps). */
}

extern "C" void eloftr_fine_maps(struct eloftr_model *m)
{
    ops_resize(m->ops, m->fu_c, 2 * ELOFTR_FINE_DIM, m->H / 2, m->W / 2, m->finep, m->H,
               m->W, 0, 0, 2.0f);
}

/* Fine matching of the device's matches, their count read there. */
static void fine_match(struct eloftr_model *m)
{
    eloftr_fine_half_count(m->ops, m->fine_h[0], m->fine_h[1], m->H, m->W, m->m_idx,
                           m->m_count, m->nmax, FINE_T, m->m_out);
}

/* The one read-back of a pair: the count, the matches and their refined
 * positions. */
static void collect_matches(struct eloftr_model *m)
{
    int cnt[2];

    ocl_read(m->ocl, m->m_count, 0, cnt, sizeof(cnt));
    if (cnt[1])
        icoreg_fatal("ELoFTR: a row argmax is out of range");
    m->nm = cnt[0];
    if (m->nm > 0) {
        ocl_read(m->ocl, m->d_mi, 0, m->mi, (size_t)m->nm * sizeof(int));
        ocl_read(m->ocl, m->d_mj, 0, m->mj, (size_t)m->nm * sizeof(int));
        ocl_read(m->ocl, m->d_mconf, 0, m->mconf, (size_t)m->nm * sizeof(float));
        ocl_read(m->ocl, m->m_out, 0, m->kp, (size_t)m->nm * 4 * sizeof(float));
    }
}

static void dump_dev(struct eloftr_model *m, const char *dir, int tile,
                     const char *what, cl_mem b, size_t floats)
{
    char path[4096];
    float *v = (float *)malloc(floats * sizeof(float));
    FILE *fp;

    ocl_read(m->ocl, b, 0, v, floats * sizeof(float));
    snprintf(path, sizeof(path), "%s/tile%03d_eloftr_%s.f32", dir, tile, what);
    if (!(fp = fopen(path, "wb")) ||
        fwrite(v, sizeof(float), floats, fp) != floats) {
        free(v);
        if (fp)
            fclose(fp);
        icoreg_fatal("Unable to write debug dump <%s>", path);
    }
    fclose(fp);
    free(v);
}

static void match_stages(struct eloftr_model *m, cl_mem dev0, cl_mem dev1,
                         const char *dump, int tile, bool collect)
{
    const size_t n = (size_t)m->h * m->w, hw = (size_t)m->H * m->W;

    need_floats(dev0, 0, (long long)hw, "eloftr_match", "image 0");
    need_floats(dev1, 0, (long long)hw, "eloftr_match", "image 1");
    if (dev0 != m->img)
        ocl_copy(m->ocl, dev0, 0, m->img, 0, hw * sizeof(float));
    ocl_copy(m->ocl, dev1, 0, m->img, hw * sizeof(float), hw * sizeof(float));
    backbone(m);
    if (dump) {
        dump_dev(m, dump, tile, "backbone_0", m->x[0], ELOFTR_DIM * n);
        dump_dev(m, dump, tile, "backbone_1", m->x[1], ELOFTR_DIM * n);
    }
    transformer(m);
    if (dump) {
        dump_dev(m, dump, tile, "coarse_0", m->x[0], ELOFTR_DIM * n);
        dump_dev(m, dump, tile, "coarse_1", m->x[1], ELOFTR_DIM * n);
    }
    coarse_match(m);
    fusion(m);
    if (dump) {
        eloftr_fine_maps(m);
        dump_dev(m, dump, tile, "fine_0", m->fine[0], ELOFTR_FINE_DIM * hw);
        dump_dev(m, dump, tile, "fine_1", m->fine[1], ELOFTR_FINE_DIM * hw);
    }
    fine_match(m);
    if (collect)
        collect_matches(m);
}

extern "C" void eloftr_match_device(struct eloftr_model *m, cl_mem dev0,
                                    cl_mem dev1)
{
    ICOREG_API_BEGIN
    match_stages(m, dev0, dev1, NULL, 0, true);
    ICOREG_API_END
}

extern "C" void eloftr_match_enqueue(struct eloftr_model *m, cl_mem dev0, cl_mem dev1)
{
    ICOREG_API_BEGIN
    match_stages(m, dev0, dev1, NULL, 0, false);
    ICOREG_API_END
}

extern "C" void eloftr_match_collect(struct eloftr_model *m)
{
    ICOREG_API_BEGIN
    collect_matches(m);
    ICOREG_API_END
}

extern "C" void eloftr_match(struct eloftr_model *m, const float *grey0,
                             const float *grey1, const char *dump, int tile)
{
    ICOREG_API_BEGIN
    const size_t hw = (size_t)m->H * m->W;

    /* Image 1 passes through the first fusion buffer, free until the
     * fusion, on its way to the pair's input buffer. */
    ocl_write(m->ocl, m->img, 0, grey0, hw * sizeof(float));
    ocl_write(m->ocl, m->fu_a, 0, grey1, hw * sizeof(float));
    match_stages(m, m->img, m->fu_a, dump, tile, true);
    ICOREG_API_END
}

extern "C" void eloftr_free(struct eloftr_model *m)
{
    cl_mem *all[] = {
        &m->f1[0],   &m->f1[1],   &m->f2[0],   &m->f2[1], &m->x[0],
        &m->x[1],    &m->fine[0], &m->fine[1], &m->fine_h[0], &m->fine_h[1],
        &m->img,     &m->s_a,
        &m->s_b,     &m->f1p,     &m->f2p,     &m->xp,    &m->finep,
        &m->t_qn,    &m->t_kvn,   &m->t_Q,     &m->t_KV,  &m->t_O,
        &m->t_O2,    &m->t_tok,   &m->t_h1,    &m->t_h2,  &m->rope,
        &m->s_blk,   &m->row_lse, &m->col_m,   &m->col_s, &m->row_max,
        &m->row_arg, &m->col_max, &m->col_arg, &m->fu_a,  &m->fu_b,
        &m->fu_c,    &m->m_idx,   &m->m_out,   &m->f_out, &m->d_mi,
        &m->d_mj,    &m->d_mconf, &m->m_count};

    if (m->ocl && m->ocl->stream)
        ocl_finish(m->ocl);
    for (size_t i = 0; i < sizeof(all) / sizeof(all[0]); i++)
        ocl_release(all[i]);
    for (int l = 0; l < ELOFTR_BLOCKS; l++) {
        ocl_release(&m->bw[l]);
        ocl_release(&m->bb[l]);
        ocl_release(&m->bU[l]);
    }
    for (int l = 0; l < ELOFTR_LAYERS; l++) {
        struct eloftr_attn *a[2] = {&m->self_attn[l], &m->cross_attn[l]};

        for (int j = 0; j < 2; j++) {
            cl_mem *f[] = {&a[j]->q_agg, &a[j]->norm_g, &a[j]->norm_b,
                           &a[j]->wq,    &a[j]->wkv,
                           &a[j]->wmsg,  &a[j]->fc1,    &a[j]->fc2,
                           &a[j]->mlp_g, &a[j]->mlp_b};

            for (size_t i = 0; i < sizeof(f) / sizeof(f[0]); i++)
                ocl_release(f[i]);
        }
    }
    for (int i = 0; i < 2; i++) {
        ocl_release(&m->f1_w[i]);
        ocl_release(&m->f2_w[i]);
        ocl_release(&m->f2_b[i]);
        ocl_release(&m->f3_w[i]);
        ocl_release(&m->f2_U[i]);
        ocl_release(&m->f3_U[i]);
    }
    free(m->mi);
    free(m->mj);
    free(m->mconf);
    free(m->kp);
    free(m->h_rmax);
    free(m->h_rarg);
    free(m->h_carg);
    memset(m, 0, sizeof(*m));
}

/* SPDX-License-Identifier: Unlicense */

/* RoMa driver on the HIP path: weight folding at load, work buffers and
 * the stage schedule of one tile pair. The model, its constants and the
 * order of operations are those of the reference (roma.c:42-1435 of
 * i.coregistration.opencl, itself following romatch and DINOv2), because
 * the results must be the same; every stage runs on this build's kernels
 * (ops.h, icoreg_kernels.h). Departures, none of which changes a result
 * beyond float32 rounding:
 *  - the two images of a pair go through VGG19-BN and DINOv2 together:
 *    one batched launch per convolution, and the ViT's token rows of
 *    both images stacked (2 x 1601 rows per GEMM, one attention launch
 *    per image);
 *  - attention is the blockwise kernel (ops_attention) instead of full
 *    16 x 1601 x 1601 score matrices, softmax and two batched GEMMs;
 *  - DINOv2's projection to 512 channels is computed token-major (the
 *    Gaussian process's layout) and transposed for the refiner at 1/16;
 *  - the Gaussian-process solve stays on the device in double precision
 *    (roma_gp_solve) instead of a host Cholesky;
 *  - the position embedding and the GP basis are made at alloc for the
 *    coarse side in use (560 by default, settable for tests);
 *  - the input pair is uploaded once per match as given and resampled
 *    (antialiased bicubic, ImageNet normalisation) on the device for
 *    each pass (roma_prepare), and the certainty sigmoid, the bounds
 *    test and v2's standard deviation run on the device before the
 *    results are read (roma_epilogue, roma_sd). */

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "common.h"
#include "conv.h"
#include "icoreg_kernels.h"
#include "roma.h"

using icoreg::need_floats;

#define EPS_BN 1e-5f
#define EPS_LN_VIT 1e-6f /* DINOv2 */
#define EPS_LN_DEC 1e-5f /* coordinate decoder (nn.LayerNorm default) */
#define VIT_HEADS 16
#define DEC_HEADS 8
#define MLP_RATIO 4
#define GP_DIM 512
#define GP_T 0.2f
#define GP_NOISE 0.1f
#define COS_EPS 1e-6f
#define VIT_GRID 37 /* DINOv2's position embeddings: 518 / 14 */
#define NCLS (ROMA_CLS_RES * ROMA_CLS_RES)

/* Refiners of the outdoor model (roma.c:56-63): scale, features per
 * image, displacement embedding, local correlation radius; projection
 * inputs per scale. */
static const int ref_scale[ROMA_SCALES] = {16, 8, 4, 2, 1};
static const int ref_feat[ROMA_SCALES] = {512, 512, 256, 64, 9};
static const int ref_emb[ROMA_SCALES] = {128, 64, 32, 16, 6};
static const int ref_radius[ROMA_SCALES] = {7, 3, 2, 0, 0};
static const int proj_in_ch[ROMA_SCALES] = {1024, 512, 256, 128, 64};

/* RoMa v2's refiners (roma.c:444-450): scale, input, features,
 * embedding, radius. */
static const int ref2_scale[ROMA2_SCALES] = {4, 2, 1};
static const int ref2_in[ROMA2_SCALES] = {256, 128, 64};
static const int ref2_feat[ROMA2_SCALES] = {192, 48, 12};
static const int ref2_emb[ROMA2_SCALES] = {79, 23, 8};
static const int ref2_radius[ROMA2_SCALES] = {3, 1, 0};

/* VGG19-BN features: convolutions per block and their widths. */
static const int vgg_blocks[4] = {2, 2, 4, 4};
static const int vgg_width[4] = {64, 128, 256, 512};

/* ---- loading --------------------------------------------------------- */

static float *read_host(struct pth_file *pf, const char *name, int ndim,
                        const long *shape)
{
    return pth_read_f32(pf, pth_require(pf, name, ndim, shape));
}

static cl_mem upload(struct roma_model *m, const float *v, size_t n,
                     const char *what)
{
    return ocl_upload(m->ocl, v, n * sizeof(float), what);
}

static cl_mem load_dev(struct roma_model *m, struct pth_file *pf,
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

/* Convolution <conv> (bias optional) followed by BatchNorm <bn>, folded
 * and uploaded (roma.c:118-143). */
static void load_conv_bn(struct roma_model *m, struct pth_file *pf,
                         const char *conv, const char *bn, int co, int ndim,
                         const long *shape, cl_mem *w_out, cl_mem *b_out)
{
    char name[256];
    long per = 1, bs[1] = {co};
    float *w, *b;

    for (int d = 1; d < ndim; d++)
        per *= shape[d];
    snprintf(name, sizeof(name), "%s.weight", conv);
    w = read_host(pf, name, ndim, shape);
    snprintf(name, sizeof(name), "%s.bias", conv);
    if (pth_find(pf, name))
        b = read_host(pf, name, 1, bs);
    else
        b = (float *)calloc(co, sizeof(float));
    fold(pf, bn, co, per, w, b);
    *w_out = upload(m, w, (size_t)co * per, conv);
    *b_out = upload(m, b, co, conv);
    free(w);
    free(b);
}

/* Transformer block <pre> (roma.c:145-211): layer scales (ls1, ls2)
 * folded into proj and fc2 per output channel when ls is set. */
static void load_block(struct roma_model *m, struct pth_file *pf,
                       const char *pre, int D, int qkv_bias, int ls,
                       struct roma_block *b)
{
    char name[256];
    long v1[1] = {D}, sqkv[2] = {3L * D, D}, s3[1] = {3L * D};
    long sp[2] = {D, D}, s1[2] = {(long)MLP_RATIO * D, D};
    long sb1[1] = {(long)MLP_RATIO * D}, s2[2] = {D, (long)MLP_RATIO * D};

#define LD(field, suffix, nd, shape)                                           \
    snprintf(name, sizeof(name), "%s.%s", pre, suffix);                        \
    b->field = load_dev(m, pf, name, nd, shape)
    LD(n1g, "norm1.weight", 1, v1);
    LD(n1b, "norm1.bias", 1, v1);
    LD(qkv_w, "attn.qkv.weight", 2, sqkv);
    if (qkv_bias) {
        LD(qkv_b, "attn.qkv.bias", 1, s3);
    }
    else
        b->qkv_b = NULL;
    LD(n2g, "norm2.weight", 1, v1);
    LD(n2b, "norm2.bias", 1, v1);
    LD(fc1_w, "mlp.fc1.weight", 2, s1);
    LD(fc1_b, "mlp.fc1.bias", 1, sb1);
#undef LD
    for (int j = 0; j < 2; j++) {
        const char *wn = j ? "mlp.fc2" : "attn.proj";
        const int in = j ? MLP_RATIO * D : D;
        float *w, *bias;

        snprintf(name, sizeof(name), "%s.%s.weight", pre, wn);
        w = read_host(pf, name, 2, j ? s2 : sp);
        snprintf(name, sizeof(name), "%s.%s.bias", pre, wn);
        bias = read_host(pf, name, 1, v1);
        if (ls) {
            float *g;

            snprintf(name, sizeof(name), "%s.ls%d.gamma", pre, j + 1);
            g = read_host(pf, name, 1, v1);
            for (int i = 0; i < D; i++) {
                for (int c = 0; c < in; c++)
                    w[(size_t)i * in + c] *= g[i];
                bias[i] *= g[i];
            }
            free(g);
        }
        if (j) {
            b->fc2_w = upload(m, w, (size_t)D * in, "fc2");
            b->fc2_b = upload(m, bias, D, "fc2");
        }
        else {
            b->proj_w = upload(m, w, (size_t)D * in, "proj");
            b->proj_b = upload(m, bias, D, "proj");
        }
        free(w);
        free(bias);
    }
}

/* The first nblk blocks of VGG19-BN under <pre>.<index> (convolution,
 * BatchNorm, ReLU per layer, one index per pooling). roma.c:213-238. */
static void load_vgg(struct roma_model *m, struct pth_file *pf,
                     const char *pre, int nblk, cl_mem *w, cl_mem *b,
                     int *cin_out, int *cout_out, cl_mem *U)
{
    int l = 0, idx = 0, cin = 3;

    for (int blk = 0; blk < nblk; blk++) {
        for (int j = 0; j < vgg_blocks[blk]; j++, l++) {
            const int co = vgg_width[blk];
            long shape[4] = {co, cin, 3, 3};
            char conv[96], bn[96];

            snprintf(conv, sizeof(conv), "%s.%d", pre, idx);
            snprintf(bn, sizeof(bn), "%s.%d", pre, idx + 1);
            load_conv_bn(m, pf, conv, bn, co, 4, shape, &w[l], &b[l]);
            /* Same-size 3 x 3 filters in Winograd form, once (the passes
             * would otherwise transform them on every call). */
            U[l] = conv_wino_supported(3, 3, 1, 1, 1, 1, 1, 1, 1, cin, co, 1, 1)
                       ? conv_wino_prepare(m->ops, w[l], co, cin)
                       : NULL;
            cin_out[l] = cin;
            cout_out[l] = co;
            cin = co;
            idx += 3;
        }
        idx++;
    }
}

static void load_dino(struct roma_model *m, struct pth_file *pf)
{
    long sw[4] = {ROMA_VIT_DIM, 3, ROMA_PATCH, ROMA_PATCH};
    long v1[1] = {ROMA_VIT_DIM}, sc[3] = {1, 1, ROMA_VIT_DIM};
    long sp[3] = {1, VIT_GRID * VIT_GRID + 1, ROMA_VIT_DIM};

    m->patch_w = load_dev(m, pf, "patch_embed.proj.weight", 4, sw);
    m->patch_b = load_dev(m, pf, "patch_embed.proj.bias", 1, v1);
    m->cls = load_dev(m, pf, "cls_token", 3, sc);
    m->pos_host = read_host(pf, "pos_embed", 3, sp);
    for (int i = 0; i < ROMA_VIT_DEPTH; i++) {
        char pre[32];

        snprintf(pre, sizeof(pre), "blocks.%d", i);
        load_block(m, pf, pre, ROMA_VIT_DIM, 1, 1, &m->vit[i]);
    }
    m->norm_g = load_dev(m, pf, "norm.weight", 1, v1);
    m->norm_b = load_dev(m, pf, "norm.bias", 1, v1);
}

/* rows x cols (row-major) into prow x pcol, zero padded; frees v. */
static float *pad2(float *v, long rows, long cols, long prow, long pcol)
{
    float *o = (float *)calloc((size_t)prow * pcol, sizeof(float));

    if (!o)
        icoreg_fatal("RoMa: out of host memory");
    for (long r = 0; r < rows; r++)
        memcpy(o + (size_t)r * pcol, v + (size_t)r * cols, (size_t)cols * sizeof(float));
    free(v);
    return o;
}

/* ConvRefiner blocks (block1, hidden_blocks.*) of cin channels under pre:
 * depthwise conv + BatchNorm names dw / bn, pointwise name pw; uploaded
 * padded to r->cp channels (zero weights and biases). */
static void load_refiner_blocks(struct roma_model *m, struct pth_file *pf,
                                const char *pre, const char *dw,
                                const char *bn, const char *pw,
                                struct roma_refiner *r)
{
    char blk[128], name[200];
    const long c = r->cin, cp = r->cp;

    for (int b = 0; b <= ROMA_HIDDEN; b++) {
        long sdw[4] = {c, 1, 5, 5}, spw[4] = {c, c, 1, 1}, sb[1] = {c};
        float *w, *bias;

        if (b == 0)
            snprintf(blk, sizeof(blk), "%s.block1", pre);
        else
            snprintf(blk, sizeof(blk), "%s.hidden_blocks.%d", pre, b - 1);
        /* Depthwise 5 x 5 with its BatchNorm folded in (load_conv_bn). */
        snprintf(name, sizeof(name), "%s.%s.weight", blk, dw);
        w = read_host(pf, name, 4, sdw);
        snprintf(name, sizeof(name), "%s.%s.bias", blk, dw);
        bias = pth_find(pf, name) ? read_host(pf, name, 1, sb)
                                  : (float *)calloc((size_t)c, sizeof(float));
        snprintf(name, sizeof(name), "%s.%s", blk, bn);
        fold(pf, name, (int)c, 25, w, bias);
        w = pad2(w, c, 25, cp, 25);
        bias = pad2(bias, 1, c, 1, cp);
        snprintf(name, sizeof(name), "%s.%s", blk, dw);
        r->dw_w[b] = upload(m, w, (size_t)cp * 25, name);
        r->dw_b[b] = upload(m, bias, cp, name);
        free(w);
        free(bias);
        snprintf(name, sizeof(name), "%s.%s.weight", blk, pw);
        w = pad2(read_host(pf, name, 4, spw), c, c, cp, cp);
        snprintf(name, sizeof(name), "%s.%s.bias", blk, pw);
        bias = pad2(read_host(pf, name, 1, sb), 1, c, 1, cp);
        r->pw_w[b] = upload(m, w, (size_t)cp * cp, name);
        r->pw_b[b] = upload(m, bias, cp, name);
        free(w);
        free(bias);
    }
}

/* roma.c:353-398. */
static void load_refiner(struct roma_model *m, struct pth_file *pf, int s)
{
    struct roma_refiner *r = &m->ref[s];
    char pre[64], name[128];
    int corr;

    r->scale = ref_scale[s];
    r->feat = ref_feat[s];
    r->emb = ref_emb[s];
    r->radius = ref_radius[s];
    corr = r->radius ? (2 * r->radius + 1) * (2 * r->radius + 1) : 0;
    r->cin = 2 * r->feat + r->emb + corr;
    r->cp = (r->cin + 3) / 4 * 4;
    r->nout = 3;
    snprintf(pre, sizeof(pre), "decoder.conv_refiner.%d", r->scale);
    load_refiner_blocks(m, pf, pre, "0", "1", "3", r);
    {
        long so[4] = {3, r->cin, 1, 1}, sob[1] = {3};
        long se[4] = {r->emb, 2, 1, 1}, seb[1] = {r->emb};

        snprintf(name, sizeof(name), "%s.out_conv.weight", pre);
        {
            float *w = pad2(read_host(pf, name, 4, so), 3, r->cin, 3, r->cp);

            r->out_w = upload(m, w, 3 * (size_t)r->cp, name);
            free(w);
        }
        snprintf(name, sizeof(name), "%s.out_conv.bias", pre);
        r->out_b = load_dev(m, pf, name, 1, sob);
        snprintf(name, sizeof(name), "%s.disp_emb.weight", pre);
        r->emb_w = load_dev(m, pf, name, 4, se);
        snprintf(name, sizeof(name), "%s.disp_emb.bias", pre);
        r->emb_b = load_dev(m, pf, name, 1, seb);
    }
}

extern "C" void roma_load(struct roma_model *m, struct ops *ops,
                          struct pth_file *pf, struct pth_file *dino)
{
    ICOREG_API_BEGIN
    long so[2] = {NCLS + 1, ROMA_DEC_DIM}, sob[1] = {NCLS + 1};
    long sgw[4] = {GP_DIM, 2, 1, 1}, sgb[1] = {GP_DIM};

    memset(m, 0, sizeof(*m));
    m->ops = ops;
    m->ocl = ops->ocl;
    m->imagenet = 1;
    m->coarse = ROMA_COARSE;
    pth_strip_prefix(pf, "matcher.model.");
    load_vgg(m, pf, "encoder.cnn.layers", 4, m->vgg_w, m->vgg_b, m->vgg_cin,
             m->vgg_cout, m->vgg_U);
    load_dino(m, dino);
    for (int s = 0; s < ROMA_SCALES; s++) {
        long shape[4] = {ref_feat[s], proj_in_ch[s], 1, 1};
        char conv[64], bn[64];

        m->proj_in[s] = proj_in_ch[s];
        m->proj_out[s] = ref_feat[s];
        snprintf(conv, sizeof(conv), "decoder.proj.%d.0", ref_scale[s]);
        snprintf(bn, sizeof(bn), "decoder.proj.%d.1", ref_scale[s]);
        load_conv_bn(m, pf, conv, bn, ref_feat[s], 4, shape, &m->proj_w[s],
                     &m->proj_b[s]);
    }
    m->gp_w = read_host(pf, "decoder.gps.16.pos_conv.weight", 4, sgw);
    m->gp_b = read_host(pf, "decoder.gps.16.pos_conv.bias", 1, sgb);
    for (int i = 0; i < ROMA_DEC_DEPTH; i++) {
        char pre[64];

        snprintf(pre, sizeof(pre), "decoder.embedding_decoder.blocks.%d", i);
        load_block(m, pf, pre, ROMA_DEC_DIM, 0, 0, &m->dec[i]);
    }
    m->to_out_w =
        load_dev(m, pf, "decoder.embedding_decoder.to_out.weight", 2, so);
    m->to_out_b =
        load_dev(m, pf, "decoder.embedding_decoder.to_out.bias", 1, sob);
    for (int s = 0; s < ROMA_SCALES; s++)
        load_refiner(m, pf, s);
    ICOREG_API_END
}

/* roma.c:452-532: input projection, blocks, the warp and confidence
 * heads stacked into one 6-output 1 x 1 convolution. */
static void load_refiner2(struct roma_model *m, struct pth_file *pf, int j)
{
    struct roma_refiner *r = &m->ref2[j];
    char pre[64], name[128];
    long sp[2] = {ref2_feat[j], ref2_in[j]}, spb[1] = {ref2_feat[j]};
    int corr;

    r->scale = ref2_scale[j];
    r->feat = ref2_feat[j];
    r->emb = ref2_emb[j];
    r->radius = ref2_radius[j];
    corr = r->radius ? (2 * r->radius + 1) * (2 * r->radius + 1) : 0;
    r->cin = 2 * r->feat + r->emb + corr;
    r->cp = (r->cin + 3) / 4 * 4;
    r->nout = 6;
    snprintf(pre, sizeof(pre), "refiners.%d", r->scale);
    snprintf(name, sizeof(name), "%s.proj.weight", pre);
    m->proj2_w[j] = load_dev(m, pf, name, 2, sp);
    snprintf(name, sizeof(name), "%s.proj.bias", pre);
    m->proj2_b[j] = load_dev(m, pf, name, 1, spb);
    m->proj2_in[j] = ref2_in[j];
    load_refiner_blocks(m, pf, pre, "conv_depthwise", "norm", "conv_pointwise",
                        r);
    {
        long se[4] = {r->emb, 2, 1, 1}, seb[1] = {r->emb};
        long sw[4] = {2, r->cin, 1, 1}, swb[1] = {2};
        long sc[4] = {4, r->cin, 1, 1}, scb[1] = {4};
        float *w = (float *)malloc(6 * (size_t)r->cin * sizeof(float));
        float bias[6], *part;

        snprintf(name, sizeof(name), "%s.disp_emb.weight", pre);
        r->emb_w = load_dev(m, pf, name, 4, se);
        snprintf(name, sizeof(name), "%s.disp_emb.bias", pre);
        r->emb_b = load_dev(m, pf, name, 1, seb);
        snprintf(name, sizeof(name), "%s.warp_head.weight", pre);
        part = read_host(pf, name, 4, sw);
        memcpy(w, part, 2 * (size_t)r->cin * sizeof(float));
        free(part);
        snprintf(name, sizeof(name), "%s.confidence_head.weight", pre);
        part = read_host(pf, name, 4, sc);
        memcpy(w + 2 * (size_t)r->cin, part, 4 * (size_t)r->cin * sizeof(float));
        free(part);
        snprintf(name, sizeof(name), "%s.warp_head.bias", pre);
        part = read_host(pf, name, 1, swb);
        bias[0] = part[0];
        bias[1] = part[1];
        free(part);
        snprintf(name, sizeof(name), "%s.confidence_head.bias", pre);
        part = read_host(pf, name, 1, scb);
        for (int k = 0; k < 4; k++)
            bias[2 + k] = part[k];
        free(part);
        w = pad2(w, 6, r->cin, 6, r->cp);
        r->out_w = upload(m, w, 6 * (size_t)r->cp, "heads");
        r->out_b = upload(m, bias, 6, "heads");
        free(w);
    }
}

extern "C" void roma_load_v2(struct roma_model *m, struct pth_file *pf)
{
    ICOREG_API_BEGIN
    if (m->H)
        icoreg_fatal("roma_load_v2 after roma_alloc");
    load_vgg(m, pf, "refiner_features.layers", 3, m->vgg2_w, m->vgg2_b,
             m->vgg2_cin, m->vgg2_cout, m->vgg2_U);
    for (int j = 0; j < ROMA2_SCALES; j++)
        load_refiner2(m, pf, j);
    m->v2 = 1;
    ICOREG_API_END
}

extern "C" void roma_set_coarse(struct roma_model *m, int side)
{
    ICOREG_API_BEGIN
    if (side < 56 || side % 56)
        icoreg_fatal("RoMa coarse side %d is not a positive multiple of 56",
                     side);
    if (m->H)
        icoreg_fatal("roma_set_coarse after roma_alloc");
    m->coarse = side;
    ICOREG_API_END
}

/* ---- alloc ----------------------------------------------------------- */

/* PyTorch's bicubic convolution weights (A = -0.75) at fraction t. */
static void cubic_weights(double t, double w[4])
{
    const double A = -0.75;
    double x;

    x = t + 1;
    w[0] = ((A * x - 5 * A) * x + 8 * A) * x - 4 * A;
    x = t;
    w[1] = ((A + 2) * x - (A + 3)) * x * x + 1;
    x = 1 - t;
    w[2] = ((A + 2) * x - (A + 3)) * x * x + 1;
    x = 2 - t;
    w[3] = ((A * x - 5 * A) * x + 8 * A) * x - 4 * A;
}

/* DINOv2's interpolate_pos_encoding (roma.c:255-298): the 37 x 37 patch
 * embeddings resized bicubically with F.interpolate's scale_factor
 * semantics, factor (c16 + 0.1) / 37 (source step 37 / (c16 + 0.1)),
 * border-clamped taps; the class embedding first. */
static float *interp_pos(const float *pos, int c16)
{
    const int D = ROMA_VIT_DIM;
    float *out = (float *)malloc((size_t)(c16 * c16 + 1) * D * sizeof(float));
    const double inv = VIT_GRID / (c16 + 0.1);

    memcpy(out, pos, D * sizeof(float));
    for (int oy = 0; oy < c16; oy++)
        for (int ox = 0; ox < c16; ox++) {
            const double ry = inv * (oy + 0.5) - 0.5, rx = inv * (ox + 0.5) - 0.5;
            const int iy = (int)floor(ry), ix = (int)floor(rx);
            double wy[4], wx[4];
            int ty[4], tx[4];
            float *o = out + (size_t)(1 + oy * c16 + ox) * D;

            cubic_weights(ry - iy, wy);
            cubic_weights(rx - ix, wx);
            for (int i = 0; i < 4; i++) {
                ty[i] = iy - 1 + i < 0 ? 0
                        : iy - 1 + i > VIT_GRID - 1 ? VIT_GRID - 1
                                                    : iy - 1 + i;
                tx[i] = ix - 1 + i < 0 ? 0
                        : ix - 1 + i > VIT_GRID - 1 ? VIT_GRID - 1
                                                    : ix - 1 + i;
            }
            for (int c = 0; c < D; c++) {
                double s = 0;

                for (int i = 0; i < 4; i++)
                    for (int j = 0; j < 4; j++)
                        s += wy[i] * wx[j] *
                             pos[(size_t)(1 + ty[i] * VIT_GRID + tx[j]) * D + c];
                o[c] = (float)s;
            }
        }
    return out;
}

/* GP basis of B's coarse grid: cos(8 pi pos_conv(x, y)) at the c16 x c16
 * cell centres, token-major (n16 x 512). roma.c:326-350. */
static float *gp_basis(const struct roma_model *m)
{
    const int c = m->c16;
    float *f = (float *)malloc((size_t)m->n16 * GP_DIM * sizeof(float));

    for (int i = 0; i < m->n16; i++) {
        const float x = -1.0f + 1.0f / c + (i % c) * (2.0f - 2.0f / c) / (c - 1);
        const float y = -1.0f + 1.0f / c + (i / c) * (2.0f - 2.0f / c) / (c - 1);

        for (int d = 0; d < GP_DIM; d++) {
            const float v = m->gp_w[2 * d] * x + m->gp_w[2 * d + 1] * y + m->gp_b[d];

            f[(size_t)i * GP_DIM + d] = cosf(8.0f * (float)M_PI * v);
        }
    }
    return f;
}

static cl_mem walloc(struct roma_model *m, size_t floats, const char *what)
{
    return ocl_alloc(m->ocl, floats * sizeof(float), what);
}

static size_t max_sz(size_t a, size_t b) { return a > b ? a : b; }

/* Side of scale index s (16, 8, .. 1) for a pass of side n. */
static int side(const struct roma_model *m, int n, int s)
{
    (void)m;
    return s == 0 ? n / ROMA_PATCH : n / ref_scale[s];
}

extern "C" void roma_alloc(struct roma_model *m, int H, int W)
{
    ICOREG_API_BEGIN
    size_t hm, dmax = 0;
    float *t;

    if (H <= 0 || W <= 0 || H % ROMA_MULTIPLE || W % ROMA_MULTIPLE)
        icoreg_fatal("RoMa tile %d x %d is not a multiple of %d", H, W,
                     ROMA_MULTIPLE);
    if (m->H)
        icoreg_fatal("roma_alloc called twice");
    m->H = H;
    m->W = W;
    m->c16 = m->coarse / ROMA_PATCH;
    m->n16 = m->c16 * m->c16;
    m->ntok = m->n16 + 1;
    m->hm = H > m->coarse ? H : m->coarse;
    m->wm = W > m->coarse ? W : m->coarse;
    hm = (size_t)m->hm * m->wm;
    const size_t n16 = m->n16, ntok = m->ntok, D = ROMA_VIT_DIM;

    m->img = walloc(m, 2 * 3 * hm, "image pair");
    m->v_a = walloc(m, 2 * 64 * hm, "VGG");
    m->v_b = walloc(m, 2 * 64 * hm, "VGG");
    for (int s = 0; s < ROMA_SCALES; s++) {
        const size_t cells = s == 0 ? n16
                                    : (size_t)(m->hm / ref_scale[s]) *
                                          (m->wm / ref_scale[s]);
        const size_t feat = s == 0 ? GP_DIM : ref_feat[s];

        m->pstride[s] = (long)(feat * cells);
        m->P[s] = walloc(m, 2 * feat * cells, "projected features");
        for (int k = 0; k < 2; k++)
            m->Pv[s][k] = ocl_wrap((float *)m->P[s]->ptr + k * feat * cells,
                                   feat * cells * sizeof(float));
    }
    m->t_x = walloc(m, 2 * ntok * D, "tokens");
    m->t_n = walloc(m, 2 * ntok * D, "tokens");
    m->t_qkv = walloc(m, 2 * ntok * 3 * D, "qkv");
    m->t_o = walloc(m, 2 * ntok * D, "attention");
    m->t_h = walloc(m, 2 * ntok * MLP_RATIO * D, "mlp");
    m->t_out = walloc(m, n16 * (NCLS + 1), "anchor logits");
    m->g_y = walloc(m, 2 * n16 * GP_DIM, "GP tokens");
    m->g_nx = walloc(m, n16, "norms");
    m->g_ny = walloc(m, n16, "norms");
    m->g_kyy = walloc(m, n16 * n16, "GP kernel");
    m->g_kxy = walloc(m, n16 * n16, "GP kernel");
    m->g_f = walloc(m, n16 * GP_DIM, "GP solve");
    m->gp_work = ocl_alloc(m->ocl, roma_gp_work_bytes(m->n16, GP_DIM),
                           "GP solve");
    m->gp_info = ocl_alloc(m->ocl, sizeof(int), "GP status");
    t = gp_basis(m);
    m->gp_basis = upload(m, t, n16 * GP_DIM, "GP basis");
    free(t);
    t = interp_pos(m->pos_host, m->c16);
    m->pos = upload(m, t, ntok * D, "pos_embed");
    free(t);
    /* Refiner inputs at every scale of both passes. */
    for (int p = 0; p < 2; p++)
        for (int s = p; s < ROMA_SCALES; s++) {
            const int ph = p ? H : m->coarse, pw = p ? W : m->coarse;
            const size_t n = (size_t)side(m, ph, s) * side(m, pw, s);

            dmax = max_sz(dmax, (size_t)m->ref[s].cp * n);
        }
    if (m->v2) {
        for (int p = 0; p < 2; p++)
            for (int s = 0; s < ROMA2_SCALES; s++) {
                const int ph = p ? H : m->coarse, pw = p ? W : m->coarse;
                const size_t n =
                    (size_t)(ph / ref2_scale[s]) * (pw / ref2_scale[s]);

                dmax = max_sz(dmax, (size_t)m->ref2[s].cp * n);
            }
        for (int s = 0; s < ROMA2_SCALES; s++) {
            const size_t cells = (size_t)(m->hm / ref2_scale[s]) *
                                 (m->wm / ref2_scale[s]);
            const size_t feat = ref2_feat[s];

            m->p2stride[s] = (long)(feat * cells);
            m->P2[s] = walloc(m, 2 * feat * cells, "projected features");
            for (int k = 0; k < 2; k++)
                m->P2v[s][k] =
                    ocl_wrap((float *)m->P2[s]->ptr + k * feat * cells,
                             feat * cells * sizeof(float));
        }
        for (int k = 0; k < 2; k++)
            m->cf[k] = walloc(m, 4 * hm, "confidence");
    }
    m->d_a = walloc(m, dmax, "refiner");
    m->d_b = walloc(m, dmax, "refiner");
    m->d_c = walloc(m, 6 * hm, "refiner");
    for (int k = 0; k < 2; k++) {
        m->fl[k] = walloc(m, 2 * hm, "warp");
        m->ce[k] = walloc(m, hm, "certainty");
    }
    m->cert16 = walloc(m, n16, "coarse certainty");
    m->lowres = walloc(m, (size_t)H * W, "coarse certainty");
    m->flow = (float *)malloc(2 * (size_t)H * W * sizeof(float));
    m->cert = (float *)malloc((size_t)H * W * sizeof(float));
    m->sd = m->v2 ? (float *)malloc((size_t)H * W * sizeof(float)) : NULL;
    m->raw = walloc(m, 2 * 3 * (size_t)H * W, "input pair");
    ICOREG_API_END
}

/* ---- stages ---------------------------------------------------------- */

/* Pre-norm transformer block on the token rows X (R = nimg * N rows of D)
 * in place, attention within each image's N rows. roma.c:692-713. */
static void block(struct roma_model *m, const struct roma_block *b, int nimg,
                  int N, int D, int heads, float eps)
{
    struct ops *o = m->ops;
    const long R = (long)nimg * N;
    const int hd = D / heads;

    ops_layernorm(o, R, D, m->t_x, m->t_n, b->n1g, b->n1b, eps, ACT_NONE, 0);
    ops_linear(o, (int)R, D, 3 * D, m->t_n, 0, b->qkv_w, b->qkv_b, m->t_qkv, 0,
               ACT_NONE, 0, 0);
    /* Each image's tokens attend within the image: one launch for all. */
    ops_attention_batch(o, nimg, ops_mat(m->t_qkv, 0, 3 * D), 3L * N * D,
                        ops_mat(m->t_qkv, D, 3 * D), 3L * N * D,
                        ops_mat(m->t_qkv, 2 * D, 3 * D), 3L * N * D,
                        ops_mat(m->t_o, 0, D), (long)N * D, N, N, heads, hd,
                        1.0f / sqrtf((float)hd), NULL);
    ops_linear(o, (int)R, D, D, m->t_o, 0, b->proj_w, b->proj_b, m->t_x, 0,
               ACT_NONE, 0, 1);
    ops_layernorm(o, R, D, m->t_x, m->t_n, b->n2g, b->n2b, eps, ACT_NONE, 0);
    ops_linear(o, (int)R, D, MLP_RATIO * D, m->t_n, 0, b->fc1_w, b->fc1_b,
               m->t_h, 0, ACT_GELU, 0, 0);
    ops_linear(o, (int)R, MLP_RATIO * D, D, m->t_h, 0, b->fc2_w, b->fc2_b,
               m->t_x, 0, ACT_NONE, 0, 1);
}

/* DINOv2 on a pair of normalised (3, coarse, coarse) images (roma.c:715-738)
 * and the 1/16 projection (decoder.proj.16): the GP tokens g_y (2, n16,
 * 512) and the refiner features P[0] (2, 512, n16); the final normed
 * tokens stay in t_n. */
static void dino_pair(struct roma_model *m, cl_mem pair)
{
    struct ops *o = m->ops;
    struct conv_geom g = ops_geom(ROMA_PATCH, ROMA_PATCH, 0);
    const int D = ROMA_VIT_DIM, n16 = m->n16, ntok = m->ntok;
    const long img = 3L * m->coarse * m->coarse;

    ops_conv2d_batch(o, 2, pair, img, 3, m->coarse, m->coarse, m->patch_w,
                     m->patch_b, D, &g, NULL, NULL, NULL, ACT_NONE, 0, m->t_h,
                     (long)D * n16);
    ops_transpose(o, m->t_h, m->t_o, 2, D, n16);
    for (int k = 0; k < 2; k++) {
        ocl_copy(m->ocl, m->cls, 0, m->t_x, (size_t)k * ntok * D * 4,
                 (size_t)D * 4);
        ocl_copy(m->ocl, m->t_o, (size_t)k * n16 * D * 4, m->t_x,
                 ((size_t)k * ntok + 1) * D * 4, (size_t)n16 * D * 4);
    }
    ops_axpby(o, m->t_x, m->t_x, 1.0f, m->pos, 1.0f, 2L * ntok * D,
              (long)ntok * D);
    for (int i = 0; i < ROMA_VIT_DEPTH; i++)
        block(m, &m->vit[i], 2, ntok, D, VIT_HEADS, EPS_LN_VIT);
    ops_layernorm(o, 2L * ntok, D, m->t_x, m->t_n, m->norm_g, m->norm_b,
                  EPS_LN_VIT, ACT_NONE, 0);
    /* g_y[k] = patch tokens of image k (rows 1..n16) W^T + b. */
    ops_gemm(o, n16, GP_DIM, D, ops_bmat(m->t_n, D, D, (long)ntok * D, 0),
             ops_bmat(m->proj_w[0], 0, D, 0, 0), 1,
             ops_bmat(m->g_y, 0, GP_DIM, (long)n16 * GP_DIM, 0), 2, 1,
             m->proj_b[0], 0, NULL, 0, 1.0f, ACT_NONE, 0);
    ops_transpose(o, m->g_y, m->P[0], 2, n16, GP_DIM);
}

/* Gaussian-process posterior (roma.c:870-896): K_yy, K_xy cosine
 * kernels, F = (K_yy + 0.1 I)^-1 basis on the device, mu = K_xy F into
 * t_x columns 0..511 and A's tokens into columns 512..1023 (the
 * decoder's input). */
/* The GP solve on the basis (K_yy, already formed) and the posterior
 * mean mu = K_xy F into the decoder input's first GP_DIM columns; events:
 * roma_gp_solve_events instead of roma_gp_solve. */
static void gp_posterior(struct roma_model *m, bool events)
{
    struct ops *o = m->ops;
    const int n16 = m->n16;

    ocl_copy(m->ocl, m->gp_basis, 0, m->g_f, 0, (size_t)n16 * GP_DIM * 4);
    (events ? roma_gp_solve_events : roma_gp_solve)(o, m->g_kyy, n16, GP_NOISE, m->g_f,
                                                    GP_DIM, m->gp_work, m->gp_info);
    ops_gemm(o, n16, GP_DIM, n16, ops_mat(m->g_kxy, 0, n16),
             ops_mat(m->g_f, 0, GP_DIM), 0, ops_mat(m->t_x, 0, ROMA_DEC_DIM),
             1, 1, NULL, 0, NULL, 0, 1.0f, ACT_NONE, 0);
}

static void gp(struct roma_model *m)
{
    struct ops *o = m->ops;
    const int n16 = m->n16;
    const long gb = (long)n16 * GP_DIM;

    roma_row_norm(o, m->g_y, n16, GP_DIM, m->g_nx);
    {
        cl_mem yb = ocl_wrap((float *)m->g_y->ptr + gb, gb * sizeof(float));

        roma_row_norm(o, yb, n16, GP_DIM, m->g_ny);
        ocl_release(&yb);
    }
    ops_gemm(o, n16, n16, GP_DIM, ops_mat(m->g_y, gb, GP_DIM),
             ops_mat(m->g_y, gb, GP_DIM), 1, ops_mat(m->g_kyy, 0, n16), 1, 1,
             NULL, 0, NULL, 0, 1.0f, ACT_NONE, 0);
    roma_cos_exp(o, m->g_kyy, m->g_ny, m->g_ny, n16, n16, GP_T, COS_EPS);
    ops_gemm(o, n16, n16, GP_DIM, ops_mat(m->g_y, 0, GP_DIM),
             ops_mat(m->g_y, gb, GP_DIM), 1, ops_mat(m->g_kxy, 0, n16), 1, 1,
             NULL, 0, NULL, 0, 1.0f, ACT_NONE, 0);
    roma_cos_exp(o, m->g_kxy, m->g_nx, m->g_ny, n16, n16, GP_T, COS_EPS);
    gp_posterior(m, false);
    ocl_copy_rect(m->ocl, m->g_y, 0, GP_DIM * 4, m->t_x, GP_DIM * 4,
                  ROMA_DEC_DIM * 4, GP_DIM * 4, n16);
}

/* Coordinate decoder and the coarse warp (roma.c:898-919) into fl[0],
 * ce[0]. */
static void decoder(struct roma_model *m)
{
    struct ops *o = m->ops;

    for (int i = 0; i < ROMA_DEC_DEPTH; i++)
        block(m, &m->dec[i], 1, m->n16, ROMA_DEC_DIM, DEC_HEADS, EPS_LN_DEC);
    ops_linear(o, m->n16, ROMA_DEC_DIM, NCLS + 1, m->t_x, 0, m->to_out_w,
               m->to_out_b, m->t_out, 0, ACT_NONE, 0, 0);
    roma_cls_to_flow(o, m->t_out, NCLS + 1, NCLS, ROMA_CLS_RES, m->n16,
                     m->fl[0], m->ce[0]);
}

/* The GP status once the stream has run. If a diagonal block's
 * in-kernel wait gave up (info = -1: the solve's second stream could not
 * run beside it), the solve and the posterior are run again with stream
 * event waits, which cannot give up. */
static void gp_check(struct roma_model *m)
{
    int info = 0;

    ocl_read(m->ocl, m->gp_info, 0, &info, sizeof(info));
    if (info < 0) {
        m->gp_retries++;
        gp_posterior(m, true);
        ocl_read(m->ocl, m->gp_info, 0, &info, sizeof(info));
        if (info < 0)
            icoreg_fatal("RoMa: Gaussian process solve: internal wait failed");
    }
    if (info)
        icoreg_fatal("RoMa: Gaussian process kernel not positive definite "
                     "(column %d)",
                     info - 1);
}

/* VGG19-BN (first nblk blocks) on the image pair in m->img (2 x 3 x H x
 * W, normalised); after block b, its features through projection
 * (pw[r], pb[r]: pin -> pout channels, r = the scale index of block b)
 * into the pair buffer dst[r] (image B at dstride[r]). roma.c:740-768,
 * 997-1027. */
static void vgg_pair(struct roma_model *m, cl_mem src, int nblk, const cl_mem *w,
                     const cl_mem *U, const cl_mem *b, const int *cin, const int *cout,
                     const int *scale_of_block, const cl_mem *pw,
                     const cl_mem *pb, const int *pin, const int *pout,
                     const cl_mem *dst, const long *dstride, int H, int W)
{
    struct ops *o = m->ops;
    struct conv_geom g = ops_geom(3, 1, 1);
    cl_mem in = src, out;
    int l = 0, h = H, wd = W;

    for (int blk = 0; blk < nblk; blk++) {
        const int r = scale_of_block[blk];
        const long hw = (long)h * wd;

        for (int j = 0; j < vgg_blocks[blk]; j++, l++) {
            out = in == m->v_a ? m->v_b : m->v_a;
            if (U[l])
                conv3x3_wino_batch(o, 2, in, (long)cin[l] * hw, cin[l], h, wd, w[l], U[l],
                                   b[l], cout[l], ACT_RELU, 0, out, (long)cout[l] * hw);
            else
                ops_conv2d_batch(o, 2, in, (long)cin[l] * hw, cin[l], h, wd, w[l],
                                 b[l], cout[l], &g, NULL, NULL, NULL, ACT_RELU, 0,
                                 out, (long)cout[l] * hw);
            in = out;
        }
        ops_gemm(o, pout[r], (int)hw, pin[r], ops_bmat(pw[r], 0, pin[r], 0, 0),
                 ops_bmat(in, 0, (int)hw, (long)pin[r] * hw, 0), 0,
                 ops_bmat(dst[r], 0, (int)hw, dstride[r], 0), 2, 1, pb[r], 1,
                 NULL, 0, 1.0f, ACT_NONE, 0);
        if (blk < nblk - 1) {
            out = in == m->v_a ? m->v_b : m->v_a;
            ops_pool2d(o, in, 2 * vgg_width[blk], h, wd, 2, 2, 0, 1, out);
            in = out;
            h /= 2;
            wd /= 2;
        }
    }
}

static void vgg(struct roma_model *m, int H, int W, cl_mem src)
{
    static const int sob[4] = {4, 3, 2, 1};

    vgg_pair(m, src, 4, m->vgg_w, m->vgg_U, m->vgg_b, m->vgg_cin, m->vgg_cout, sob,
             m->proj_w, m->proj_b, m->proj_in, m->proj_out, m->P, m->pstride,
             H, W);
}

static void vgg2(struct roma_model *m, int H, int W)
{
    static const int sob[3] = {2, 1, 0};
    int pout[ROMA2_SCALES];

    for (int j = 0; j < ROMA2_SCALES; j++)
        pout[j] = m->ref2[j].feat;
    vgg_pair(m, m->img, 3, m->vgg2_w, m->vgg2_U, m->vgg2_b, m->vgg2_cin, m->vgg2_cout, sob,
             m->proj2_w, m->proj2_b, m->proj2_in, pout, m->P2, m->p2stride, H,
             W);
}

/* One ConvRefiner on an hs x ws grid (roma.c:921-995, 1029-1104): input
 * d = [f_A, f_B at the warp, displacement embedding, local correlation],
 * nine depthwise + pointwise blocks, the output convolution into d_c. */
static void refiner_body(struct roma_model *m, const struct roma_refiner *r,
                         cl_mem fa, cl_mem fb, int hs, int ws, float fx,
                         float fy, cl_mem fl)
{
    struct ops *o = m->ops;
    const int n = hs * ws;

    ocl_copy(m->ocl, fa, 0, m->d_a, 0, (size_t)r->feat * n * 4);
    roma_warp_sample(o, fb, r->feat, hs, ws, fl, m->d_a, r->feat);
    roma_disp(o, fl, hs, ws, fx, fy, m->d_c);
    ops_conv1x1(o, m->d_c, 0, 2, n, r->emb_w, r->emb_b, r->emb, m->d_a,
                2L * r->feat * n, ACT_NONE, 0);
    if (r->radius)
        roma_local_corr(o, fa, fb, r->feat, hs, ws, r->radius, fl, m->d_a,
                        2 * r->feat + r->emb);
    /* The padding channels (cin .. cp) start at zero and stay zero. */
    if (r->cp > r->cin)
        ocl_fill(m->ocl, m->d_a, (size_t)r->cin * n, (size_t)(r->cp - r->cin) * n, 0.0f);
    cl_mem src = m->d_a;

    if (r->cp <= 32 && r->cp % 8 == 0) {
        /* Few channels: each block in one pass, alternating buffers. */
        cl_mem dst = m->d_b;

        for (int b = 0; b <= ROMA_HIDDEN; b++) {
            roma_dwpw_small(o, src, r->cp, hs, ws, r->dw_w[b], r->dw_b[b], r->pw_w[b],
                            r->pw_b[b], dst);
            cl_mem t = src;

            src = dst;
            dst = t;
        }
    }
    else
        for (int b = 0; b <= ROMA_HIDDEN; b++) {
            roma_dwconv5(o, m->d_a, r->cp, hs, ws, r->dw_w[b], r->dw_b[b], m->d_b);
            ops_conv1x1(o, m->d_b, 0, r->cp, n, r->pw_w[b], r->pw_b[b], r->cp,
                        m->d_a, 0, ACT_NONE, 0);
        }
    ops_conv1x1(o, src, 0, r->cp, n, r->out_w, r->out_b, r->nout, m->d_c, 0,
                ACT_NONE, 0);
}

static void refine(struct roma_model *m, int s, int hs, int ws, int Hf, int Wf,
                   float sf, cl_mem fl, cl_mem ce)
{
    const struct roma_refiner *r = &m->ref[s];
    const float fac = 40.0f / 32.0f * sf;

    refiner_body(m, r, m->Pv[s][0], m->Pv[s][1], hs, ws, fac, fac, fl);
    roma_update(m->ops, fl, ce, m->d_c, hs * ws, (float)r->scale, (float)Wf,
                (float)Hf);
}

static void refine2(struct roma_model *m, int j, int hs, int ws, int Hp, int Wp,
                    cl_mem fl, cl_mem cf)
{
    const struct roma_refiner *r = &m->ref2[j];

    refiner_body(m, r, m->P2v[j][0], m->P2v[j][1], hs, ws,
                 (float)Wp / ROMA2_ANCHOR, (float)Hp / ROMA2_ANCHOR, fl);
    roma2_update(m->ops, fl, cf, m->d_c, hs * ws, (float)ws, (float)hs);
}

/* ---- dumps (the reference's names, roma.c:1188-1227) --------------------- */

static void dump_host(const char *dir, int tile, const char *what,
                      const float *v, size_t floats)
{
    char path[4096];
    FILE *fp;

    snprintf(path, sizeof(path), "%s/tile%03d_roma_%s.f32", dir, tile, what);
    if (!(fp = fopen(path, "wb")) ||
        fwrite(v, sizeof(float), floats, fp) != floats) {
        if (fp)
            fclose(fp);
        icoreg_fatal("Unable to write debug dump <%s>", path);
    }
    fclose(fp);
}

static void dump_dev(struct roma_model *m, const char *dir, int tile,
                     const char *what, cl_mem b, size_t off, size_t floats)
{
    float *v = (float *)malloc(floats * sizeof(float));

    ocl_read(m->ocl, b, off * sizeof(float), v, floats * sizeof(float));
    dump_host(dir, tile, what, v, floats);
    free(v);
}

/* The pass-0 DINOv2 features of image k as the reference dumps them:
 * (1024, n16) channel-major normed patch tokens. */
static void dump_dino(struct roma_model *m, const char *dir, int tile)
{
    const size_t D = ROMA_VIT_DIM, n16 = m->n16, ntok = m->ntok;
    float *t = (float *)malloc(2 * ntok * D * sizeof(float));
    float *o = (float *)malloc(D * n16 * sizeof(float));

    ocl_read(m->ocl, m->t_n, 0, t, 2 * ntok * D * sizeof(float));
    for (int k = 0; k < 2; k++) {
        for (size_t i = 0; i < n16; i++)
            for (size_t c = 0; c < D; c++)
                o[c * n16 + i] = t[(k * ntok + 1 + i) * D + c];
        dump_host(dir, tile, k ? "dino_1" : "dino_0", o, D * n16);
    }
    free(t);
    free(o);
}

static void dump_gp(struct roma_model *m, const char *dir, int tile)
{
    const size_t n16 = m->n16;
    float *t = (float *)malloc(n16 * ROMA_DEC_DIM * sizeof(float));
    float *o = (float *)malloc(n16 * GP_DIM * sizeof(float));

    ocl_read(m->ocl, m->t_x, 0, t, n16 * ROMA_DEC_DIM * sizeof(float));
    for (size_t i = 0; i < n16; i++)
        memcpy(o + i * GP_DIM, t + i * ROMA_DEC_DIM, GP_DIM * sizeof(float));
    dump_host(dir, tile, "gp", o, n16 * GP_DIM);
    free(t);
    free(o);
}

/* ---- the pass ------------------------------------------------------------- */

/* RoMa's refiners s0 .. s1 - 1 of pass p (size Hp x Wp), resizing the
 * warp and certainty between scales. roma.c:1229-1256. */
static void refiners(struct roma_model *m, int p, int s0, int s1, int Hp,
                     int Wp, float sf, int *cur, const char *dump, int tile)
{
    for (int s = s0; s < s1; s++) {
        const int hs = side(m, Hp, s), ws = side(m, Wp, s);

        refine(m, s, hs, ws, Hp, Wp, sf, m->fl[*cur], m->ce[*cur]);
        if (p == 0 && s == 0)
            ocl_copy(m->ocl, m->ce[*cur], 0, m->cert16, 0,
                     (size_t)hs * ws * 4);
        if (dump) {
            char what[64];

            snprintf(what, sizeof(what), "p%d_s%d_flow", p, ref_scale[s]);
            dump_dev(m, dump, tile, what, m->fl[*cur], 0, 2 * (size_t)hs * ws);
            snprintf(what, sizeof(what), "p%d_s%d_cert", p, ref_scale[s]);
            dump_dev(m, dump, tile, what, m->ce[*cur], 0, (size_t)hs * ws);
        }
        if (s < s1 - 1) {
            const int hn = side(m, Hp, s + 1), wn = side(m, Wp, s + 1);

            ops_resize(m->ops, m->fl[*cur], 2, hs, ws, m->fl[!*cur], hn, wn, 0,
                       0, 0.0f);
            ops_resize(m->ops, m->ce[*cur], 1, hs, ws, m->ce[!*cur], hn, wn, 0,
                       0, 0.0f);
            *cur = !*cur;
        }
    }
}

/* RoMa v2's refiners of pass p from the warp and confidence on the
 * current h x w grid; zero_prec clears the precision first (before the
 * second pass). roma.c:1268-1303. */
static void refiners2(struct roma_model *m, int p, int Hp, int Wp, int *h,
                      int *w, int *cur, int zero_prec, const char *dump,
                      int tile)
{
    for (int j = 0; j < ROMA2_SCALES; j++) {
        const int hs = Hp / ref2_scale[j], ws = Wp / ref2_scale[j];
        const size_t n = (size_t)*h * *w;

        if (zero_prec && j == 0)
            ocl_fill(m->ocl, m->cf[*cur], n, 3 * n, 0.0f);
        ops_resize(m->ops, m->fl[*cur], 2, *h, *w, m->fl[!*cur], hs, ws, 0, 0,
                   0.0f);
        ops_resize(m->ops, m->cf[*cur], 4, *h, *w, m->cf[!*cur], hs, ws, 0, 0,
                   0.0f);
        *cur = !*cur;
        refine2(m, j, hs, ws, Hp, Wp, m->fl[*cur], m->cf[*cur]);
        if (dump) {
            char what[64];

            snprintf(what, sizeof(what), "p%d_v2s%d_flow", p, ref2_scale[j]);
            dump_dev(m, dump, tile, what, m->fl[*cur], 0, 2 * (size_t)hs * ws);
            snprintf(what, sizeof(what), "p%d_v2s%d_conf", p, ref2_scale[j]);
            dump_dev(m, dump, tile, what, m->cf[*cur], 0, 4 * (size_t)hs * ws);
        }
        *h = hs;
        *w = ws;
    }
}

/* Both images (3, H, W) in 0..1 into m->raw, once per match. */
static void upload_raw(struct roma_model *m, const float *imgA, const float *imgB)
{
    const size_t p = 3 * (size_t)m->H * m->W * sizeof(float);

    ocl_write(m->ocl, m->raw, 0, imgA, p);
    ocl_write(m->ocl, m->raw, p, imgB, p);
}

/* Inputs of a pass: both images resampled to h x w (and normalised) on
 * the device into m->img. */
static void prepare_pair(struct roma_model *m, int h, int w)
{
    roma_prepare(m->ops, m->raw, 2, m->H, m->W, m->img, h, w, m->imagenet);
}

static void match_v2(struct roma_model *m, int cur, const char *dump, int tile)
{
    const size_t hw = (size_t)m->H * m->W;
    int h = side(m, m->coarse, 1), w = side(m, m->coarse, 1);
    const size_t n = (size_t)h * w;

    ocl_fill(m->ocl, m->cf[cur], 0, 4 * n, 0.0f);
    ocl_copy(m->ocl, m->ce[cur], 0, m->cf[cur], 0, n * 4);
    refiners2(m, 0, m->coarse, m->coarse, &h, &w, &cur, 0, dump, tile);
    prepare_pair(m, m->H, m->W);
    if (dump) {
        dump_dev(m, dump, tile, "in_f_0", m->img, 0, 3 * hw);
        dump_dev(m, dump, tile, "in_f_1", m->img, 3 * hw, 3 * hw);
    }
    vgg2(m, m->H, m->W);
    refiners2(m, 1, m->H, m->W, &h, &w, &cur, 1, dump, tile);
    /* cf[cur]: the certainty logit, then the three precision entries. */
    roma_sd(m->ops, m->cf[cur], (long)hw, m->lowres, (long)hw);
    roma_epilogue(m->ops, m->fl[cur], m->cf[cur], NULL, (long)hw);
    ocl_read(m->ocl, m->fl[cur], 0, m->flow, 2 * hw * sizeof(float));
    ocl_read(m->ocl, m->cf[cur], 0, m->cert, hw * sizeof(float));
    ocl_read(m->ocl, m->lowres, 0, m->sd, hw * sizeof(float));
    if (dump) {
        dump_host(dump, tile, "flow", m->flow, 2 * hw);
        dump_host(dump, tile, "cert", m->cert, hw);
        dump_host(dump, tile, "sd", m->sd, hw);
    }
}

extern "C" void roma_coarse_device(struct roma_model *m, cl_mem pair)
{
    ICOREG_API_BEGIN
    if (!m->H)
        icoreg_fatal("roma_coarse_device before roma_alloc");
    need_floats(pair, 0, 2L * 3 * m->coarse * m->coarse, "roma_coarse_device",
                "pair");
    dino_pair(m, pair);
    gp(m);
    decoder(m);
    ICOREG_API_END
}

extern "C" void roma_refine_device(struct roma_model *m, cl_mem pair,
                                   cl_mem flow8, cl_mem cert8)
{
    ICOREG_API_BEGIN
    const char *op = "roma_refine_device";
    const int h8 = side(m, m->H, 1), w8 = side(m, m->W, 1);
    const float sf = sqrtf((float)m->H * m->W) / m->coarse;
    int cur = 0;

    if (!m->H)
        icoreg_fatal("%s before roma_alloc", op);
    if (m->v2)
        icoreg_fatal("%s: RoMa's own (v1) refiners only", op);
    need_floats(pair, 0, 2L * 3 * m->H * m->W, op, "pair");
    need_floats(flow8, 0, 2L * h8 * w8, op, "flow8");
    need_floats(cert8, 0, (long)h8 * w8, op, "cert8");
    vgg(m, m->H, m->W, pair);
    ocl_copy(m->ocl, flow8, 0, m->fl[0], 0, 2 * (size_t)h8 * w8 * 4);
    ocl_copy(m->ocl, cert8, 0, m->ce[0], 0, (size_t)h8 * w8 * 4);
    refiners(m, 1, 1, ROMA_SCALES, m->H, m->W, sf, &cur, NULL, 0);
    m->last = cur;
    ICOREG_API_END
}

extern "C" void roma_match(struct roma_model *m, const float *imgA,
                           const float *imgB, const char *dump, int tile)
{
    ICOREG_API_BEGIN
    const size_t hw = (size_t)m->H * m->W;
    const size_t pc = 3 * (size_t)m->coarse * m->coarse;
    const float sf = sqrtf((float)m->H * m->W) / m->coarse;
    int cur = 0;

    if (!m->H)
        icoreg_fatal("roma_match before roma_alloc");
    /* Coarse pass. */
    upload_raw(m, imgA, imgB);
    prepare_pair(m, m->coarse, m->coarse);
    vgg(m, m->coarse, m->coarse, m->img);
    if (m->v2)
        vgg2(m, m->coarse, m->coarse);
    dino_pair(m, m->img);
    if (dump) {
        dump_dev(m, dump, tile, "in_c_0", m->img, 0, pc);
        dump_dev(m, dump, tile, "in_c_1", m->img, pc, pc);
        dump_dino(m, dump, tile);
    }
    gp(m);
    gp_check(m);
    if (dump)
        dump_gp(m, dump, tile);
    decoder(m);
    if (dump) {
        dump_dev(m, dump, tile, "cls_flow", m->fl[0], 0, 2 * (size_t)m->n16);
        dump_dev(m, dump, tile, "cls_cert", m->ce[0], 0, m->n16);
    }
    refiners(m, 0, 0, m->v2 ? 2 : ROMA_SCALES, m->coarse, m->coarse, 1.0f,
             &cur, dump, tile);
    if (m->v2) {
        match_v2(m, cur, dump, tile);
        goto done;
    }
    /* Fine pass at the tile's size from the coarse pass's finest warp. */
    prepare_pair(m, m->H, m->W);
    if (dump) {
        dump_dev(m, dump, tile, "in_f_0", m->img, 0, 3 * hw);
        dump_dev(m, dump, tile, "in_f_1", m->img, 3 * hw, 3 * hw);
    }
    vgg(m, m->H, m->W, m->img);
    ops_resize(m->ops, m->fl[cur], 2, m->coarse, m->coarse, m->fl[!cur],
               side(m, m->H, 1), side(m, m->W, 1), 0, 0, 0.0f);
    ops_resize(m->ops, m->ce[cur], 1, m->coarse, m->coarse, m->ce[!cur],
               side(m, m->H, 1), side(m, m->W, 1), 0, 0, 0.0f);
    cur = !cur;
    refiners(m, 1, 1, ROMA_SCALES, m->H, m->W, sf, &cur, dump, tile);
    ops_resize(m->ops, m->cert16, 1, m->c16, m->c16, m->lowres, m->H, m->W, 0,
               0, 0.0f);
    roma_epilogue(m->ops, m->fl[cur], m->ce[cur], m->lowres, (long)hw);
    ocl_read(m->ocl, m->fl[cur], 0, m->flow, 2 * hw * sizeof(float));
    ocl_read(m->ocl, m->ce[cur], 0, m->cert, hw * sizeof(float));
    if (dump) {
        dump_host(dump, tile, "flow", m->flow, 2 * hw);
        dump_host(dump, tile, "cert", m->cert, hw);
    }
done:;
    ICOREG_API_END
}

/* ---- free ------------------------------------------------------------------- */

static void release_block(struct roma_block *b)
{
    cl_mem *all[] = {&b->n1g,    &b->n1b,    &b->qkv_w, &b->qkv_b,
                     &b->proj_w, &b->proj_b, &b->n2g,   &b->n2b,
                     &b->fc1_w,  &b->fc1_b,  &b->fc2_w, &b->fc2_b};

    for (size_t i = 0; i < sizeof(all) / sizeof(all[0]); i++)
        ocl_release(all[i]);
}

static void release_refiner(struct roma_refiner *r)
{
    for (int b = 0; b <= ROMA_HIDDEN; b++) {
        ocl_release(&r->dw_w[b]);
        ocl_release(&r->dw_b[b]);
        ocl_release(&r->pw_w[b]);
        ocl_release(&r->pw_b[b]);
    }
    ocl_release(&r->out_w);
    ocl_release(&r->out_b);
    ocl_release(&r->emb_w);
    ocl_release(&r->emb_b);
}

extern "C" void roma_free(struct roma_model *m)
{
    cl_mem *all[] = {&m->patch_w, &m->patch_b,  &m->cls,     &m->norm_g,
                     &m->norm_b,  &m->pos,      &m->to_out_w, &m->to_out_b,
                     &m->img,     &m->v_a,      &m->v_b,     &m->t_x,
                     &m->t_n,     &m->t_qkv,    &m->t_o,     &m->t_h,
                     &m->t_out,   &m->g_y,      &m->g_nx,    &m->g_ny,
                     &m->g_kyy,   &m->g_kxy,    &m->g_f,     &m->gp_basis,
                     &m->gp_work, &m->gp_info,  &m->d_a,     &m->d_b,
                     &m->d_c,     &m->fl[0],    &m->fl[1],   &m->ce[0],
                     &m->ce[1],   &m->cf[0],    &m->cf[1],   &m->cert16,
                     &m->lowres,  &m->raw};

    if (m->ocl && m->ocl->stream)
        ocl_finish(m->ocl);
    for (size_t i = 0; i < sizeof(all) / sizeof(all[0]); i++)
        ocl_release(all[i]);
    for (int i = 0; i < 16; i++) {
        ocl_release(&m->vgg_w[i]);
        ocl_release(&m->vgg_b[i]);
        ocl_release(&m->vgg_U[i]);
    }
    for (int i = 0; i < 8; i++) {
        ocl_release(&m->vgg2_w[i]);
        ocl_release(&m->vgg2_b[i]);
        ocl_release(&m->vgg2_U[i]);
    }
    for (int i = 0; i < ROMA_VIT_DEPTH; i++)
        release_block(&m->vit[i]);
    for (int i = 0; i < ROMA_DEC_DEPTH; i++)
        release_block(&m->dec[i]);
    for (int s = 0; s < ROMA_SCALES; s++) {
        ocl_release(&m->proj_w[s]);
        ocl_release(&m->proj_b[s]);
        ocl_release(&m->Pv[s][0]);
        ocl_release(&m->Pv[s][1]);
        ocl_release(&m->P[s]);
        release_refiner(&m->ref[s]);
    }
    for (int s = 0; s < ROMA2_SCALES; s++) {
        ocl_release(&m->proj2_w[s]);
        ocl_release(&m->proj2_b[s]);
        ocl_release(&m->P2v[s][0]);
        ocl_release(&m->P2v[s][1]);
        ocl_release(&m->P2[s]);
        release_refiner(&m->ref2[s]);
    }
    free(m->pos_host);
    free(m->gp_w);
    free(m->gp_b);
    free(m->flow);
    free(m->cert);
    free(m->sd);
    memset(m, 0, sizeof(*m));
}

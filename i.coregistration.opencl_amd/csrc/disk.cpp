/* SPDX-License-Identifier: Unlicense */

/* DISK driver on the HIP path: the U-Net of kornia.feature.DISK, heatmap
 * NMS, top-n selection and descriptor gather, with the layer plan,
 * constants and order of operations of the reference (disk.c:23-273 of
 * i.coregistration.opencl), because the keypoints must be the same.
 * Every convolution is a 5 x 5, stride 1, pad 2 one-group convolution,
 * which ops_conv2d runs as the direct MFMA kernel with the InstanceNorm +
 * PReLU of the block applied to its input as it is loaded. Unlike the
 * reference, the down path writes its skip outputs straight into the up
 * path's concatenation buffers, and the top-n selection runs on the
 * device (disk_topn), so a detection syncs once, to read the keypoints. */

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "common.h"
#include "disk.h"
#include "icoreg_kernels.h"

/* Unet(in_features=3, size=5, down=[16, 32, 64, 64, 64],
 * up=[64, 64, 64, 129]) (disk.c:23-31): down blocks 0-4, up blocks 0-3;
 * every block but the first normalises and gates its input, down blocks
 * 1-4 average-pool first, up blocks upsample the bottom input and
 * concatenate the skip connection. */
static const int layer_cin[DISK_LAYERS] = {3, 16, 32, 64, 64, 128, 128, 96, 80};
static const int layer_cout[DISK_LAYERS] = {16, 32, 64, 64,           64,
                                            64, 64, 64, DISK_DESC + 1};

static cl_mem upload_tensor(struct disk_model *m, struct pth_file *pf,
                            const char *name, int ndim, const long *shape)
{
    const struct pth_tensor *t = pth_require(pf, name, ndim, shape);
    float *v = pth_read_f32(pf, t);
    cl_mem buf = ocl_upload(m->ocl, v, pth_numel(t) * sizeof(float), name);

    free(v);
    return buf;
}

extern "C" void disk_load(struct disk_model *m, struct ops *ops,
                          struct pth_file *pf)
{
    ICOREG_API_BEGIN
    char name[128];

    memset(m, 0, sizeof(*m));
    m->ocl = ops->ocl;
    m->ops = ops;
    for (int l = 0; l < DISK_LAYERS; l++) {
        long wshape[4] = {layer_cout[l], layer_cin[l], 5, 5};
        long bshape[1] = {layer_cout[l]}, ashape[1] = {layer_cin[l]};
        const bool down = l < 5;
        const int idx = down ? l : l - 5;

        m->cin[l] = layer_cin[l];
        m->cout[l] = layer_cout[l];
#define NAME(sub, what)                                                        \
    (down ? snprintf(name, sizeof(name), "unet.path_down.%d.1.%d.%s", idx,     \
                     sub, what)                                                \
          : snprintf(name, sizeof(name), "unet.path_up.%d.conv.%d.%s", idx,    \
                     sub, what))
        NAME(3, "weight");
        m->w[l] = upload_tensor(m, pf, name, 4, wshape);
        NAME(3, "bias");
        m->b[l] = upload_tensor(m, pf, name, 1, bshape);
        if (l > 0) {
            NAME(1, "weight");
            m->alpha[l] = upload_tensor(m, pf, name, 1, ashape);
        }
#undef NAME
    }
    ICOREG_API_END
}

extern "C" void disk_alloc(struct disk_model *m, int H, int W, int nmax)
{
    ICOREG_API_BEGIN
    const size_t px = (size_t)H * W;

    if (H <= 0 || W <= 0 || H % DISK_MULTIPLE || W % DISK_MULTIPLE)
        icoreg_fatal("DISK tile %d x %d is not a multiple of %d", H, W,
                     DISK_MULTIPLE);
    if (nmax < 1)
        icoreg_fatal("DISK: keypoint capacity %d", nmax);
    m->H = H;
    m->W = W;
    m->nmax = nmax;
    m->input = ocl_alloc(m->ocl, 3 * px * sizeof(float), "input");
    for (int l = 0; l < 4; l++) {
        const size_t plane = px >> (2 * l);

        m->cat[l] = ocl_alloc(m->ocl, (64 + layer_cout[l]) * plane * sizeof(float),
                              "concatenation");
        m->f[l] = ocl_wrap((float *)m->cat[l]->ptr + 64 * plane,
                           layer_cout[l] * plane * sizeof(float));
    }
    m->f[4] = ocl_alloc(m->ocl, layer_cout[4] * (px >> 8) * sizeof(float), "down features");
    for (int k = 0; k < 3; k++)
        m->u[k] = ocl_alloc(m->ocl, 64 * (px >> (2 * (3 - k))) * sizeof(float),
                            "up features");
    m->tmp = ocl_alloc(m->ocl, 64 * (px >> 8) * sizeof(float), "pooled");
    m->out = ocl_alloc(m->ocl, (DISK_DESC + 1) * px * sizeof(float), "output");
    m->mean = ocl_alloc(m->ocl, 128 * sizeof(float), "mean");
    m->rstd = ocl_alloc(m->ocl, 128 * sizeof(float), "rstd");
    m->mask = ocl_alloc(m->ocl, px, "nms mask");
    m->valid = ocl_alloc(m->ocl, px, "valid mask");
    m->xy = ocl_alloc(m->ocl, 2 * (size_t)nmax * sizeof(int), "keypoints");
    m->score = ocl_alloc(m->ocl, (size_t)nmax * sizeof(float), "scores");
    m->count = ocl_alloc(m->ocl, sizeof(int), "keypoint count");
    m->desc = ocl_alloc(m->ocl, (size_t)nmax * DISK_DESC * sizeof(float),
                        "descriptors");
    m->topn_work = ocl_alloc(m->ocl, disk_topn_work_bytes(H, W), "top-n");
    ICOREG_API_END
}

/* Layer l on in (cin, H, W) into out (cout, H, W); every layer but the
 * first normalises and gates its input with m->mean / rstd. */
static void conv(struct disk_model *m, int l, cl_mem in, int H, int W,
                 cl_mem out)
{
    struct conv_geom g = ops_geom(5, 1, 2);

    if (l > 0)
        ops_conv2d(m->ops, in, m->cin[l], H, W, m->w[l], m->b[l], m->cout[l],
                   &g, m->mean, m->rstd, m->alpha[l], ACT_NONE, 0, out);
    else
        ops_conv2d(m->ops, in, m->cin[l], H, W, m->w[l], m->b[l], m->cout[l],
                   &g, NULL, NULL, NULL, ACT_NONE, 0, out);
}

extern "C" int disk_detect(struct disk_model *m, const float *img, int H,
                           int W, int h, int w, int n, float thresh,
                           const unsigned char *valid, int *xy, float *score,
                           float *desc)
{
    ICOREG_API_BEGIN
    const size_t px = (size_t)H * W;
    const long off = (long)DISK_DESC * (long)px;
    int nk = 0;

    if (H > m->H || W > m->W || px > (size_t)m->H * m->W || H % DISK_MULTIPLE ||
        W % DISK_MULTIPLE)
        icoreg_fatal("DISK tile %d x %d does not fit its buffers", H, W);
    if (h < 0 || w < 0 || h > H || w > W)
        icoreg_fatal("DISK crop %d x %d outside the %d x %d tile", h, w, H, W);
    if (n > m->nmax)
        n = m->nmax;
    if (n < 0)
        n = 0;
    ocl_write(m->ocl, m->input, 0, img, 3 * px * sizeof(float));
    if (valid && (size_t)h * w > 0)
        ocl_write(m->ocl, m->valid, 0, valid, (size_t)h * w);

    /* Down path (disk.c:186-200): block lev average-pools block lev - 1's
     * output (into its own level's concatenation buffer, whose first 64
     * channels the up path fills only later) and writes its output into
     * the skip part of that buffer. */
    conv(m, 0, m->input, H, W, m->f[0]);
    for (int lev = 1; lev < 5; lev++) {
        const int c = layer_cout[lev - 1], hh = H >> lev, ww = W >> lev;
        cl_mem t = lev < 4 ? m->cat[lev] : m->tmp;

        ops_avgpool2(m->ops, m->f[lev - 1], c, H >> (lev - 1), W >> (lev - 1),
                     t);
        ops_chan_stats(m->ops, t, c, hh * ww, 1e-5f, m->mean, m->rstd);
        conv(m, lev, t, hh, ww, m->f[lev]);
    }
    /* Up path (disk.c:202-218): bottom input upsampled into the first 64
     * channels of the concatenation, the skip connection already after
     * it. */
    for (int j = 0; j < 4; j++) {
        const int l = 5 + j, lvl = 3 - j, hh = H >> lvl, ww = W >> lvl;
        cl_mem bot = j == 0 ? m->f[4] : m->u[j - 1];
        const int cb = 64, ch = layer_cout[lvl];
        const size_t plane = (size_t)hh * ww;

        ops_resize(m->ops, bot, cb, hh / 2, ww / 2, m->cat[lvl], hh, ww, 0, 0,
                   2.0f);
        ops_chan_stats(m->ops, m->cat[lvl], cb + ch, (int)plane, 1e-5f, m->mean,
                       m->rstd);
        conv(m, l, m->cat[lvl], hh, ww, j < 3 ? m->u[j] : m->out);
    }
    /* Heatmap NMS on the h x w crop, top-n (disk.c:220-253), descriptors;
     * then the keypoints come back. */
    disk_nms5x5(m->ops, m->out, off, W, h, w, thresh, m->mask);
    disk_topn(m->ops, m->out, off, W, h, w, m->mask, valid ? m->valid : NULL, n, m->xy,
              m->score, m->count, m->topn_work);
    disk_gather_desc_count(m->ops, m->out, H, W, DISK_DESC, m->xy, m->count, n, m->desc);
    ocl_read(m->ocl, m->count, 0, &nk, sizeof(int));
    if (nk > 0) {
        ocl_read(m->ocl, m->xy, 0, xy, 2 * (size_t)nk * sizeof(int));
        ocl_read(m->ocl, m->score, 0, score, (size_t)nk * sizeof(float));
        ocl_read(m->ocl, m->desc, 0, desc, (size_t)nk * DISK_DESC * sizeof(float));
    }
    return nk;
    ICOREG_API_END_RET(0)
}

extern "C" void disk_free(struct disk_model *m)
{
    if (m->ocl && m->ocl->stream)
        ocl_finish(m->ocl);
    for (int k = 0; k < DISK_LAYERS; k++) {
        ocl_release(&m->w[k]);
        ocl_release(&m->b[k]);
        ocl_release(&m->alpha[k]);
    }
    ocl_release(&m->input);
    for (int k = 0; k < 5; k++)
        ocl_release(&m->f[k]);
    for (int k = 0; k < 4; k++)
        ocl_release(&m->cat[k]);
    for (int k = 0; k < 3; k++)
        ocl_release(&m->u[k]);
    ocl_release(&m->tmp);
    ocl_release(&m->out);
    ocl_release(&m->mean);
    ocl_release(&m->rstd);
    ocl_release(&m->mask);
    ocl_release(&m->valid);
    ocl_release(&m->xy);
    ocl_release(&m->score);
    ocl_release(&m->count);
    ocl_release(&m->desc);
    ocl_release(&m->topn_work);
    memset(m, 0, sizeof(*m));
}

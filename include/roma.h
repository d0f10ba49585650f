/* SPDX-License-Identifier: Unlicense */

/* RoMa dense matcher on one MI355X.
 *
 * The API is the reference's (roma.h:9-128 of i.coregistration.opencl):
 * roma_load / roma_load_v2 / roma_alloc / roma_match / roma_free and the
 * struct fields its caller reads (net.flow, cert, sd, H, W, imagenet;
 * matcher_roma.c:45-54, 107, 154). The buffer plan behind them is this
 * build's: both images of a pair run through VGG19-BN and DINOv2 as one
 * batch (token rows of the two images stacked), the Gaussian-process
 * solve runs on the device in double precision, and every stage stays
 * resident in HBM until the host epilogue. */

#ifndef ICOREG_ROMA_H
#define ICOREG_ROMA_H

#include "ops.h"
#include "pth_loader.h"

#ifdef __cplusplus
extern "C" {
#endif

#define ROMA_MULTIPLE 8   /* Tile sides: VGG features down to 1/8. */
#define ROMA_COARSE 560   /* Side of the coarse pass (training size). */
#define ROMA_PATCH 14     /* DINOv2 patch size. */
#define ROMA_VIT_DIM 1024 /* DINOv2 ViT-L/14 width. */
#define ROMA_VIT_DEPTH 24 /* DINOv2 blocks. */
#define ROMA_DEC_DIM 1024 /* Coordinate decoder width (GP 512 + 512). */
#define ROMA_DEC_DEPTH 5  /* Coordinate decoder blocks. */
#define ROMA_CLS_RES 64   /* Coarse warp classes: 64 x 64 anchors. */
#define ROMA_SCALES 5     /* Refiners at 1/16, 1/8, 1/4, 1/2, 1/1. */
#define ROMA_HIDDEN 8     /* Hidden blocks per refiner. */
#define ROMA2_SCALES 3    /* RoMa v2's refiners at 1/4, 1/2, 1/1. */
#define ROMA2_ANCHOR 512  /* Their displacement scale: side / 512. */

/* One pre-norm transformer block (DINOv2's or the coordinate decoder's),
 * DINOv2's layer scales folded into proj and fc2 (roma.h:22-29). */
struct roma_block {
    cl_mem n1g, n1b, qkv_w, qkv_b, proj_w, proj_b;
    cl_mem n2g, n2b, fc1_w, fc1_b, fc2_w, fc2_b;
};

/* One ConvRefiner (roma.h:31-41): block1 and ROMA_HIDDEN hidden blocks
 * of depthwise 5 x 5 (BatchNorm folded) + ReLU + 1 x 1; out_conv to 3
 * outputs (v1) or 6 (v2: warp head and confidence head). */
struct roma_refiner {
    /* cp: cin rounded up to a multiple of 4; the blocks and the output
     * convolution run on cp channels, the padding channels zero (zero
     * weights and biases), so that every weight row is 16-byte aligned. */
    int scale, feat, emb, radius, cin, nout, cp;
    cl_mem dw_w[ROMA_HIDDEN + 1], dw_b[ROMA_HIDDEN + 1];
    cl_mem pw_w[ROMA_HIDDEN + 1], pw_b[ROMA_HIDDEN + 1];
    cl_mem out_w, out_b, emb_w, emb_b;
};

struct roma_model {
    struct ops *ops;
    struct ocl_backend *ocl;
    /* Inputs normalised with the ImageNet mean and deviation (RoMa's
     * transforms); set to 0 for weights trained on 0..1. */
    int imagenet;
    /* Side of the coarse pass: ROMA_COARSE unless changed with
     * roma_set_coarse before roma_alloc (a multiple of 56). */
    int coarse;
    int c16, n16, ntok; /* coarse / 14, its square, + the class token */

    /* Weights. VGG19-BN (16 convolutions, BatchNorm folded). */
    cl_mem vgg_w[16], vgg_b[16];
    int vgg_cin[16], vgg_cout[16];
    cl_mem vgg_U[16]; /* the same filters in Winograd form (NULL: direct) */
    /* DINOv2: patch embedding, class token, final norm; the position
     * embedding is interpolated to the coarse grid at alloc. */
    cl_mem patch_w, patch_b, cls, norm_g, norm_b, pos;
    float *pos_host; /* (1 + 37 * 37) x 1024 as loaded */
    struct roma_block vit[ROMA_VIT_DEPTH];
    /* Projections per scale (BatchNorm folded), GP, decoder, refiners. */
    cl_mem proj_w[ROMA_SCALES], proj_b[ROMA_SCALES];
    int proj_in[ROMA_SCALES], proj_out[ROMA_SCALES];
    float *gp_w, *gp_b; /* pos_conv (512 x 2, 512), host */
    struct roma_block dec[ROMA_DEC_DEPTH];
    cl_mem to_out_w, to_out_b;
    struct roma_refiner ref[ROMA_SCALES];
    /* RoMa v2's refiners and their VGG19-BN (roma_load_v2). */
    int v2;
    cl_mem vgg2_w[8], vgg2_b[8];
    int vgg2_cin[8], vgg2_cout[8];
    cl_mem vgg2_U[8];
    cl_mem proj2_w[ROMA2_SCALES], proj2_b[ROMA2_SCALES];
    int proj2_in[ROMA2_SCALES];
    struct roma_refiner ref2[ROMA2_SCALES];

    /* Work buffers for tiles of H x W (multiples of ROMA_MULTIPLE);
     * hm x wm is the larger of the tile and the coarse pass. Pair
     * buffers hold image A then image B. */
    int H, W, hm, wm;
    cl_mem img;           /* 2 x 3 x hm x wm */
    cl_mem v_a, v_b;      /* 2 x 64 x hm x wm VGG activations */
    /* Projected features per scale: image A, then image B at a fixed
     * offset (the largest pass's size); Pv / P2v are views of each. */
    cl_mem P[ROMA_SCALES], P2[ROMA2_SCALES];
    cl_mem Pv[ROMA_SCALES][2], P2v[ROMA2_SCALES][2];
    long pstride[ROMA_SCALES], p2stride[ROMA2_SCALES];
    cl_mem t_x, t_n, t_qkv, t_o, t_h, t_out; /* token buffers */
    cl_mem g_y, g_nx, g_ny, g_kyy, g_kxy, g_f, gp_basis, gp_work, gp_info;
    cl_mem d_a, d_b, d_c, fl[2], ce[2], cf[2], cert16, lowres;
    /* Last run, host side (roma.h:92-104): flow (2, H, W) normalised to
     * -1..1 in image B, certainty (H, W) in 0..1, and with v2 the
     * predicted standard deviation sd (H, W) in cells. */
    float *flow, *cert, *sd;
    cl_mem raw; /* 2 x 3 x H x W: the pair as given, resampled on the device */
    int last;           /* fl / ce index holding roma_refine_device's result */
    int gp_retries;     /* GP solves re-run after the in-kernel wait gave up */
};

/* Read the weights: RoMa's RegressionMatcher state dict (names as
 * roma_outdoor.pth; MatchAnything's "matcher.model." prefix stripped)
 * and DINOv2 ViT-L/14; fold BatchNorms and layer scales, upload. Fatal
 * on a missing tensor or a shape mismatch. roma.h:106-112. */
void roma_load(struct roma_model *m, struct ops *ops, struct pth_file *pf,
               struct pth_file *dino);

/* RoMa v2's refiners and their VGG19-BN (refiners.*, refiner_features.*),
 * after roma_load and before roma_alloc. roma.h:114-118. */
void roma_load_v2(struct roma_model *m, struct pth_file *pf);

/* Extension with no counterpart in the reference: the side of the
 * coarse pass (default ROMA_COARSE = 560, a multiple of 56), for tests
 * at small sizes. Before roma_alloc. */
void roma_set_coarse(struct roma_model *m, int side);

/* Work buffers for tiles of H x W. roma.h:120-121. */
void roma_alloc(struct roma_model *m, int H, int W);

/* Dense warp of image A onto image B, both (3, H, W) in 0..1: results in
 * m->flow, m->cert (and m->sd with v2). With dump set (a folder), the
 * inputs and intermediate tensors of tile number tile are written there
 * as tileNNN_roma_<what>.f32, the reference's names. roma.h:123-127. */
void roma_match(struct roma_model *m, const float *imgA, const float *imgB,
                const char *dump, int tile);

/* Extension: the coarse forward of a pair already on the device — two
 * normalised (3, coarse, coarse) images back to back in pair —
 * DINOv2 x 2, Gaussian process, coordinate decoder and cls_to_flow,
 * leaving the 1/14 warp and certainty logit in fl[0], ce[0]. The timed
 * unit of the benchmark. */
void roma_coarse_device(struct roma_model *m, cl_mem pair);

/* Extension: the fine pass of roma_match (roma.c:1404-1412) on a pair
 * already on the device — two normalised (3, H, W) images back to back
 * in pair, H x W the allocated tile — from a warp flow8 (2, H / 8, W / 8)
 * and certainty logit cert8 (H / 8 x W / 8): VGG19-BN on both images,
 * then the refiners at 1/8, 1/4, 1/2 and 1/1 with their resizes. The
 * warp and certainty logit at full size are left in fl[last], ce[last].
 * RoMa's own refiners only (no roma_load_v2). The timed unit of the
 * refiner benchmark. */
void roma_refine_device(struct roma_model *m, cl_mem pair, cl_mem flow8,
                        cl_mem cert8);

void roma_free(struct roma_model *m);

#ifdef __cplusplus
}
#endif

#endif /* ICOREG_ROMA_H */

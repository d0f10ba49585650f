/* SPDX-License-Identifier: Unlicense */

/* ORACLE — test infrastructure only.
 *
 * A plain-C CPU restatement of the kernels of i.coregistration.opencl's
 * matcher tensor path (ops.cl, eloftr_kernels.cl, roma_kernels.cl,
 * disk_kernels.cl) and of the network schedules that drive them, in
 * float32 following each kernel's own arithmetic. It is the checker of
 * the HIP library: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it. The product never links or calls it.
 *
 * Pinning (how each function is known to be right, not just retyped):
 *  - generic ops: tests/golden/ holds outputs of torch float64 closed
 *    forms (F.conv2d, F.layer_norm, F.scaled_dot_product_attention,
 *    F.grid_sample, F.interpolate, ...) on the exact inputs of the
 *    reference's tests/ops_check.c (same xorshift64 stream and cases);
 *  - eloftr coarse / fine: brute-force torch float64 (full score matrix,
 *    softmax over both axes, first argmax; per-match windows) on small
 *    seeded inputs;
 *  - RoMa / DISK kernels: torch closed forms (grid_sample with shifted
 *    grids, depthwise conv2d, softplus, max_pool neighbourhoods) and
 *    brute force.
 * Functions without such a check say "parity unpinned" below.
 *
 * Conventions: tensors are contiguous float arrays, offsets in floats,
 * the same argument meaning as the reference's ops.h. */

#ifndef ICOREG_ORACLE_H
#define ICOREG_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The xorshift64 stream of tests/ops_check.c:33-42 (seed
 * 88172645463325252). */
void orc_rng_seed(uint64_t s);
uint64_t orc_rng_state(void);
float orc_urand(float lo, float hi);
void orc_rand_fill(float *v, long n, float lo, float hi);

/* ops.cl:23-37 */
float orc_act(float v, int act, float slope);

/* ops.cl:39-138: batched C = act(alpha A op(B) + bias) + R. R at roff of
 * buffer R with C's layout; R may alias C. */
void orc_gemm(int M, int N, int K, const float *A, long aoff, int lda,
              long sa0, long sa1, const float *B, long boff, int ldb,
              long sb0, long sb1, int transb, float *C, long coff, int ldc,
              long sc0, long sc1, int nb, int nb1, const float *bias,
              int biasrow, const float *R, long roff, float alpha, int act,
              float slope);

/* ops.cl:389-448 (covers conv5x5 :319-387 and im2col + GEMM, which
 * compute the same sums). */
void orc_conv2d(const float *in, int C, int H, int W, const float *w,
                const float *b, int K, int kh, int kw, int sy, int sx, int py,
                int px, int dy, int dx, int groups, const float *mean,
                const float *rstd, const float *alpha, int act, float slope,
                float *out);

void orc_chan_stats(const float *x, int C, int HW, float eps, float *mean,
                    float *rstd);                              /* :450-492 */
void orc_chan_affine(const float *X, float *Y, int C, int HW,
                     const float *mean, const float *rstd, const float *g,
                     const float *b, int act, float slope);    /* :494-519 */
void orc_prelu(const float *X, float *Y, int C, int HW,
               const float *alpha);                            /* :521-532 */
void orc_act_map(const float *X, float *Y, long n, int act,
                 float slope);                                 /* :534-542 */
void orc_layernorm(long rows, int C, const float *X, float *Y, const float *g,
                   const float *b, float eps, int act, float slope); /* :544 */
void orc_softmax_rows(float *S, long rows, int L, float scale); /* :580-602 */
/* ops.cl:604-687; kmask bytes (NULL: none). */
void orc_attention(const float *Q, long qoff, int ldq, const float *K,
                   long koff, int ldk, const float *V, long voff, int ldv,
                   float *O, long ooff, int ldo, int Nq, int Nk, int nh, int d,
                   float scale, const unsigned char *kmask);
void orc_rope(float *X, long off, int ld, long rows, int nh, int d, int npos,
              const float *cs, int interleaved);               /* :689-716 */
void orc_resize(const float *in, int C, int h, int w, float *out, int H, int W,
                int coff, int align_corners, float scale);     /* :718-754 */
void orc_grid_sample(const float *in, int C, int H, int W, const float *grid,
                     int n, int align_corners, float *out);    /* :756-793 */
void orc_unfold(const float *in, int C, int H, int W, int kh, int kw, int sy,
                int sx, int py, int px, float *out);           /* :795-816 */
void orc_avgpool2(const float *in, int C, int H, int W, float *out);
void orc_pool2d(const float *in, int C, int H, int W, int k, int s, int p,
                int max, float *out);                          /* :832-860 */
void orc_transpose(const float *in, float *out, int B, int R, int C);
void orc_axpby(float *out, const float *a, float alpha, const float *b,
               float beta, long n, long bmod);                 /* :882-893 */
/* ops.c:612-626 */
void orc_fold_bn(float *w, float *b, int K, long per, const float *gamma,
                 const float *beta, const float *mean, const float *var,
                 float eps);

/* ---- ELoFTR (eloftr_kernels.cl, eloftr.c) ------------------------------ */

/* Coarse dual-softmax statistics and argmaxes of the n x n score matrix
 * S = alpha F0 F1^T (F0, F1 token-major n x D), eloftr_kernels.cl:10-144
 * as scheduled by eloftr.c:498-548 (row blocks of blk rows): row_max,
 * row_arg, col_arg (n each). Also returns the row and column margins
 * (top-1 minus top-2 confidence) and the column maximum confidence when
 * those pointers are not NULL. */
void orc_eloftr_coarse(const float *F0, const float *F1, int n, int D,
                       float alpha, int blk, float *row_max, int *row_arg,
                       int *col_arg, float *row_margin, float *col_margin,
                       float *col_max);

/* Host mutual / threshold / border selection, eloftr.c:552-566. Returns
 * the match count; mi, mj, mconf sized n. */
int orc_eloftr_select(const float *row_max, const int *row_arg,
                      const int *col_arg, int h, int w, float thr, int border,
                      int *mi, int *mj, float *mconf);

/* Two-stage fine matching, eloftr_kernels.cl:146-295: f0, f1 (64, H, W),
 * cells (x0, y0, x1, y1) per match, out (x0, y0, x1, y1) per match.
 * margin (NULL or M floats) gets the first-stage top-2 margin. */
void orc_eloftr_fine(const float *f0, const float *f1, int H, int W,
                     const int *cells, int M, float T, float *out,
                     float *margin);

/* ---- RoMa (roma_kernels.cl) -------------------------------------------- */

void orc_roma_row_norm(const float *X, int rows, int C, float *out);
void orc_roma_cos_exp(float *S, const float *nx, const float *ny, int N, int M,
                      float T, float eps);
void orc_roma_cls_to_flow(const float *L, int ld, int C, int res, int n,
                          float *flow, float *cert);
void orc_roma_warp_sample(const float *in, int C, int H, int W,
                          const float *flow, float *out, int coff);
void orc_roma_local_corr(const float *f1, const float *f2, int C, int H,
                         int W, int r, const float *flow, float *out,
                         int coff);
void orc_roma_disp(const float *flow, int H, int W, float fx, float fy,
                   float *out);
void orc_roma_update(float *flow, float *cert, const float *d, int n,
                     float scale, float Wf, float Hf);
void orc_roma2_update(float *flow, float *conf, const float *d, int n, float W,
                      float H);
void orc_roma_dwconv5(const float *in, int C, int H, int W, const float *w,
                      const float *bias, float *out);

/* A named weight array (the safetensors tensors, float32). */
struct orc_named {
    const char *name;
    const float *data;
    long numel;
};

/* Outputs of orc_eloftr_forward; NULL pointers are skipped (but row_max,
 * row_arg, col_arg, mi, mj, mconf and kp are required, n or 4 n long). */
struct orc_eloftr_out {
    float *backbone[2], *coarse[2]; /* 256 x n each */
    float *row_max, *row_margin, *col_margin;
    int *row_arg, *col_arg;
    int nm;
    int *mi, *mj;
    float *mconf, *kp, *fine_margin;
    float *fine[2]; /* 64 x H x W each */
    float *col_max;
};

/* The whole Efficient LoFTR pass of eloftr.c:654-681 on grey H x W
 * images; returns the match count. */
int orc_eloftr_forward(const struct orc_named *weights, int nweights,
                       const float *grey0, const float *grey1, int H, int W,
                       float pos_scale, struct orc_eloftr_out *out);

/* ---- DISK (disk_kernels.cl, disk.c) ------------------------------------ */

/* disk_kernels.cl:8-35: mask (h x w) of strict 5 x 5 maxima above
 * thresh of heat (row stride W), border 2 never. */
void orc_disk_nms5x5(const float *heat, int W, int h, int w, float thresh,
                     unsigned char *mask);
/* disk_kernels.cl:37-60. */
void orc_disk_gather_desc(const float *feat, int H, int W, int D,
                          const int *xy, int n, float *desc);
/* The host top-n of disk.c:228-253 on the NMS mask (h x w) and valid
 * (or NULL): returns the count, xy / score in raster order. */
int orc_disk_topn(const float *heat, int W, int h, int w,
                  const unsigned char *mask, const unsigned char *valid, int n,
                  int *xy, float *score);
/* disk_detect (disk.c:164-273) on a (3, H, W) image: returns the keypoint
 * count; out_full (129 x H x W, or NULL) gets the U-Net output. */
int orc_disk_detect(const struct orc_named *weights, int nweights,
                    const float *img, int H, int W, int h, int w, int n,
                    float thresh, const unsigned char *valid, int *xy,
                    float *score, float *desc, float *out_full);

/* ---- AdaLAM's nearest-neighbour search (adalam.c:38-116) --------------- */

/* Per row of d1 (n1 x dim): the first index of the nearest row of d2
 * (n2 x dim) by squared distance, and the ratio of the two smallest
 * distances (second clamped to 1e-3); per row of d2, when nn21 is not
 * NULL, the first index of the nearest row of d1. */
void orc_adalam_nearest(const float *d1, int n1, const float *d2, int n2,
                        int dim, int *nn12, float *score, int *nn21);

/* One pre-norm ViT block (DINOv2's, roma.c:675-713) on X (N x 1024) in
 * place; w[12] = norm1 g, b; qkv W, b; proj W, b; norm2 g, b; fc1 W, b;
 * fc2 W, b, layer scale folded into proj and fc2. */
void orc_vit_block(const float *const w[12], float *X, int N, int heads,
                   float eps);

/* OpenMP threads of the oracle's parallel loops. */
int orc_threads(void);
void orc_set_threads(int n);

/* ---- RoMa network (roma.c) ------------------------------------------------ */

/* Host input preparation, roma.c:1106-1186: (3, H, W) resampled to (3, h,
 * w) with Pillow's antialiased bicubic filter, ImageNet-normalised when
 * imagenet is set. */
void orc_roma_prepare(const float *in, int H, int W, float *out, int h, int w,
                      int imagenet);

/* Outputs of orc_roma_forward; NULL pointers are skipped, flow (2 H W)
 * and cert (H W) are required. scale_flow[p][s]: the warp after the
 * refiner of scale index s (16, 8, 4, 2, 1) in pass p (0: coarse). */
struct orc_roma_out {
    float *dino[2];          /* 1024 x n16 normed patch tokens */
    float *gp;               /* n16 x 512 posterior mean */
    float *logits;           /* n16 x 4097 */
    float *cls_flow, *cls_cert;
    float *scale_flow[2][5];
    float *flow, *cert, *sd; /* sd (v2 only) may be NULL */
};

/* RoMa's match (roma.c:1351-1435) on (3, H, W) images in 0..1 with a
 * coarse pass of side coarse (a multiple of 56); v2 weights (nv2 > 0)
 * switch to RoMa v2's refiners. cls_flow_in (2 n16, or NULL) replaces
 * the decoder's coarse warp before the refiners. Returns 0, or 1 + the
 * column at which the GP kernel was not positive definite. */
int orc_roma_forward(const struct orc_named *weights, int nweights,
                     const struct orc_named *dino, int ndino,
                     const struct orc_named *v2, int nv2, const float *imgA,
                     const float *imgB, int H, int W, int coarse, int imagenet,
                     const float *cls_flow_in, struct orc_roma_out *out);

/* RoMa's coarse forward alone (roma.c:715-919: DINOv2 on both images,
 * GP, decoder, cls_to_flow) on (3, coarse, coarse) images already
 * ImageNet-normalised: cls_flow (2 n16), cls_cert (n16). Returns the GP
 * status (0, or 1 + the failing column). */
int orc_roma_coarse(const struct orc_named *weights, int nweights,
                    const struct orc_named *dino, int ndino, const float *pairA,
                    const float *pairB, int coarse, float *cls_flow, float *cls_cert);

/* The fine pass alone (roma.c:1404-1413, the v1 refiners of scales 8 .. 1)
 * on (3, H, W) images already ImageNet-normalised, from the 1/8 warp flow8
 * (2, H/8, W/8) and certainty logit cert8 (H/8, W/8); coarse sets the
 * displacement scale sqrt(H W) / coarse. out->flow (2 H W) and out->cert
 * (H W) get the last refiner's warp and logit (no epilogue),
 * out->scale_flow[1][s] (s = 1 .. 4, when set) the warp after each scale.
 * Returns 0. */
int orc_roma_refine(const struct orc_named *weights, int nweights,
                    const struct orc_named *dino, int ndino, const float *pairA,
                    const float *pairB, int H, int W, int coarse, const float *flow8,
                    const float *cert8, struct orc_roma_out *out);

#ifdef __cplusplus
}
#endif

#endif /* ICOREG_ORACLE_H */

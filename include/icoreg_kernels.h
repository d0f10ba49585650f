/* SPDX-License-Identifier: Unlicense */

/* Model kernels of the matcher tensor path: one C launcher per kernel of
 * the reference's eloftr_kernels.cl, roma_kernels.cl and
 * disk_kernels.cl (i.coregistration.opencl), replacing the drivers'
 * ocl_kernel lookups and SETARG / ops_run launches (eloftr.c:255-259,
 * 510-546, 625-633). Same arguments and meaning as the OpenCL kernels,
 * device buffers as cl_mem, every access checked on the host, fatal
 * errors naming the call. Asynchronous on the backend's stream. */

#ifndef ICOREG_KERNELS_H
#define ICOREG_KERNELS_H

#include "ops.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- ELoFTR (eloftr_kernels.cl) ---------------------------------------- */

/* Log-sum-exp of each of the rows rows of a score block S (rows x N,
 * row-major) into lse[r0 + r]. eloftr_kernels.cl:10-44. */
void eloftr_row_lse(struct ops *o, cl_mem S, int rows, int N, int r0,
                    cl_mem lse);

/* Running column maximum cm and sum of exponentials cs (N each), merged
 * with this block's R rows. eloftr_kernels.cl:46-66. */
void eloftr_col_lse(struct ops *o, cl_mem S, int R, int N, cl_mem cm,
                    cl_mem cs);

/* Row maximum and first argmax of the dual-softmax confidence
 * exp(s - lse_row) exp(s - (cm + log cs)) of each row of the block, into
 * rmax[r0 + r], rarg[r0 + r] (int). eloftr_kernels.cl:68-113. */
void eloftr_conf_row(struct ops *o, cl_mem S, int rows, int N, int r0,
                     cl_mem lse, cl_mem cm, cl_mem cs, cl_mem rmax,
                     cl_mem rarg);

/* Running column maximum and first argmax (global row index) of the
 * confidence over blocks of rows taken in increasing order: cmax, carg
 * (int) hold the state between blocks (start at -1, -1).
 * eloftr_kernels.cl:115-144. */
void eloftr_conf_col(struct ops *o, cl_mem S, int R, int N, int r0, cl_mem lse,
                     cl_mem cm, cl_mem cs, cl_mem cmax, cl_mem carg);

/* The form eloftr_match runs (no counterpart among the reference's
 * kernels, which launch the four above one after the other): the first
 * pass of a block, eloftr_row_lse and eloftr_col_lse in one read of S,
 * and the second, eloftr_conf_row and eloftr_conf_col in one read of S;
 * same arguments, states and results. With r0 == 0 the column state
 * (cm, cs; cmax, carg) is started by the call itself, with no prior fill.
 * N % 4 == 0 and S 16-byte aligned. */
void eloftr_lse_block(struct ops *o, cl_mem S, int R, int N, int r0, cl_mem lse,
                      cl_mem cm, cl_mem cs);
void eloftr_conf_block(struct ops *o, cl_mem S, int R, int N, int r0, cl_mem lse,
                       cl_mem cm, cl_mem cs, cl_mem rmax, cl_mem rarg, cl_mem cmax,
                       cl_mem carg);

/* Two-stage fine matching of M coarse matches: f0, f1 (64, H, W) fine
 * features, cells (int4: x0, y0, x1, y1 per match), T the second-stage
 * temperature, out (float4: x0, y0, x1, y1 per match, the reference's
 * pixel convention). eloftr_kernels.cl:146-295. */
void eloftr_fine(struct ops *o, cl_mem f0, cl_mem f1, int H, int W,
                 cl_mem cells, int M, float T, cl_mem out);

/* No counterpart in the reference: eloftr_fine on the fine features at
 * half resolution, for the ELoFTR driver. f0, f1 (64, H / 2, W / 2) stand
 * for their 2x bilinear resize (64, H, W) (ops_resize, pixel centres),
 * sampled in the windows with the resize's own arithmetic, so that the
 * result is eloftr_fine's on the resized maps without writing them (the
 * reference resizes before fine matching, eloftr.c:604). H and W even. */
void eloftr_fine_half(struct ops *o, cl_mem f0, cl_mem f1, int H, int W,
                      cl_mem cells, int M, float T, cl_mem out);

/* No counterpart in the reference: eloftr_fine_half for the first
 * *count of at most nmax matches, the count read on the device (the
 * driver's matches never come back to the host before fine matching). */
void eloftr_fine_half_count(struct ops *o, cl_mem f0, cl_mem f1, int H, int W,
                            cl_mem cells, cl_mem count, int nmax, float T, cl_mem out);

/* The mutual nearest-neighbour selection of eloftr.c:606-636 on the
 * device: cell i (of h x w) is kept with j = row_arg[i] when row_max[i] >
 * thr, col_arg[j] == i and both cells lie at least border cells inside;
 * kept matches in raster order into mi, mj, mconf (n each) and cells
 * (int4 x0, y0, x1, y1); count[0] = their number, count[1] = 1 if a row
 * argmax was out of range. */
void eloftr_mutual(struct ops *o, cl_mem row_max, cl_mem row_arg, cl_mem col_arg, int h,
                   int w, int border, float thr, cl_mem mi, cl_mem mj, cl_mem mconf,
                   cl_mem cells, cl_mem count);

/* ---- RoMa (roma_kernels.cl) ----------------------------------------------
 * Warps are channel-major (2, n): x then y, normalised to -1..1 with
 * align_corners = 0 (cell centres at -1 + (2 i + 1) / size). */

/* nimg images (3, H, W) in 0..1, consecutive in `in`, resampled to
 * (3, h, w) into `out` with Pillow's antialiased bicubic filter (Keys'
 * cubic, a = -0.5, support scaled by the reduction; width pass first,
 * sums in double) and ImageNet-normalised when imagenet is set: the
 * host's prepare of roma.c:1106-1186. Reductions up to 15.5x per axis.
 * Uses the ops work buffer. */
void roma_prepare(struct ops *o, cl_mem in, int nimg, int H, int W, cl_mem out,
                  int h, int w, int imagenet);

/* The host epilogue of roma.c:1328-1349,1413-1429 on hw cells in place:
 * certainty c -= 0.5 low where low < 0 (low may be NULL: v2),
 * sigmoid, 0 where the warp leaves [-1, 1]^2; warp (2, hw) clamped. */
void roma_epilogue(struct ops *o, cl_mem flow, cl_mem cert, cl_mem low, long hw);

/* RoMa v2's standard deviation (roma.c:1330-1339): det = p0 p2 - p1^2 of
 * the precision planes (3, hw) at float offset poff of prec, in double;
 * det^-0.25, or NaN where det <= 0. */
void roma_sd(struct ops *o, cl_mem prec, long poff, cl_mem sd, long hw);

/* Euclidean norm of each row of X (rows x C). roma_kernels.cl:9-23. */
void roma_row_norm(struct ops *o, cl_mem X, int rows, int C, cl_mem out);

/* In place on S (N x M): exp((S / (nx[i] ny[j] + eps) - 1) / T), RoMa's
 * cosine kernel. roma_kernels.cl:25-38. */
void roma_cos_exp(struct ops *o, cl_mem S, cl_mem nx, cl_mem ny, int N, int M,
                  float T, float eps);

/* Per token (row of L with ld floats: C = res^2 anchor logits, then the
 * certainty logit): first argmax, softmax over the anchors, its mode and
 * four neighbours (indices clamped to 0..C-1), probability-weighted mean
 * anchor position into flow (2, n), certainty logit into cert (n).
 * roma_kernels.cl:40-102. */
void roma_cls_to_flow(struct ops *o, cl_mem L, int ld, int C, int res, int n,
                      cl_mem flow, cl_mem cert);

/* in (C, H, W) sampled bilinearly (zero padding) at the warp flow (2, n)
 * of the same grid (n = H W) into channels coff.. of out (*, n).
 * roma_kernels.cl:104-141. */
void roma_warp_sample(struct ops *o, cl_mem in, int C, int H, int W,
                      cl_mem flow, cl_mem out, int coff);

/* Local correlation: for each cell and window offset k = (a, b) of
 * (2 r + 1)^2 (a the row), f1 (C, n) / sqrt(C) dotted with f2 (C, H, W)
 * sampled at the warp shifted by (b - r, a - r) cells, into channels
 * coff + k of out. C <= 1024, r <= 7. roma_kernels.cl:143-192. */
void roma_local_corr(struct ops *o, cl_mem f1, cl_mem f2, int C, int H, int W,
                     int r, cl_mem flow, cl_mem out, int coff);

/* Displacement input (fx, fy) * (warp - own cell centre) into out (2, n).
 * roma_kernels.cl:194-208. */
void roma_disp(struct ops *o, cl_mem flow, int H, int W, float fx, float fy,
               cl_mem out);

/* flow += scale d / (4 Wf, 4 Hf); cert += d2 (d: 3 x n).
 * roma_kernels.cl:210-224. */
void roma_update(struct ops *o, cl_mem flow, cl_mem cert, cl_mem d, int n,
                 float scale, float Wf, float Hf);

/* RoMa v2: flow += d / (4 W, 4 H); conf (4, n) += overlap logit and the
 * precision (l00^2, l00 l10, l10^2 + l11^2) of the Cholesky factor with
 * softplus diagonal (threshold 20) + 1e-6. roma_kernels.cl:226-250. */
void roma2_update(struct ops *o, cl_mem flow, cl_mem conf, cl_mem d, int n,
                  float W, float H);

/* Depthwise 5 x 5, stride 1, zero padding 2, bias, ReLU on (C, H, W)
 * (weights (C, 25)). roma_kernels.cl:252-284. */
void roma_dwconv5(struct ops *o, cl_mem in, int C, int H, int W, cl_mem w,
                  cl_mem bias, cl_mem out);

/* No counterpart among the reference's kernels: a refiner block on C = 8,
 * 16, 24 or 32 channels in one pass, out = pw (C x C) relu(dw5(in) + db)
 * + pb, the same result as roma_dwconv5 followed by ops_conv1x1 (to
 * float32 rounding) without the intermediate map. in and out must not
 * overlap. */
void roma_dwpw_small(struct ops *o, cl_mem in, int C, int H, int W, cl_mem dw,
                     cl_mem db, cl_mem pw, cl_mem pb, cl_mem out);

/* ---- DISK (disk_kernels.cl) -------------------------------------------- */

/* Keypoint candidates of the heatmap (float offset off of heat, row
 * stride W) cropped to h x w: mask (h x w bytes) = 1 where the cell is
 * strictly greater than its 24 neighbours in the 5 x 5 window and than
 * thresh; the 2-cell border never. disk_kernels.cl:8-35. */
void disk_nms5x5(struct ops *o, cl_mem heat, long off, int W, int h, int w,
                 float thresh, cl_mem mask);

/* Descriptors: channels 0..D-1 of feat (D + 1, H, W) at the n keypoints
 * xy (int x, y pairs), L2-normalised (eps 1e-12) into desc (n x D).
 * disk_kernels.cl:37-60. */
void disk_gather_desc(struct ops *o, cl_mem feat, int H, int W, int D,
                      cl_mem xy, int n, cl_mem desc);

/* The top-n selection of disk_detect on the device (the reference does
 * it on the host, disk.c:228-253): among the cells of mask (h x w bytes,
 * 1 = NMS maximum) that valid (h x w bytes, or NULL) allows, the cut is
 * the (n+1)-th highest heat value, or the lowest when there are no more
 * than n; the cells strictly above it are kept in raster order: xy (x, y
 * int pairs, capacity n) and score, their number into count (one int on
 * the device). heat as for disk_nms5x5. work holds
 * disk_topn_work_bytes(h, w) bytes. No counterpart among the reference's
 * kernels. */
size_t disk_topn_work_bytes(int h, int w);
void disk_topn(struct ops *o, cl_mem heat, long off, int W, int h, int w,
               cl_mem mask, cl_mem valid, int n, cl_mem xy, cl_mem score,
               cl_mem count, cl_mem work);

/* disk_gather_desc for the keypoints disk_topn left on the device: their
 * number in count (one int, at most nmax), xy within h x w by
 * construction. No counterpart among the reference's kernels. */
void disk_gather_desc_count(struct ops *o, cl_mem feat, int H, int W, int D,
                            cl_mem xy, cl_mem count, int nmax, cl_mem desc);

/* Extension with no counterpart among the reference's kernels: the
 * Gaussian-process solve that roma.c:770-836 runs on the host in double
 * precision, on the device in double precision. F (n x d floats) is
 * replaced by (K + noise I)^-1 F, K (n x n floats, symmetric, its lower
 * triangle read). work holds roma_gp_work_bytes(n, d) bytes; info (one
 * int, cleared by the call) gets 1 + the first column whose pivot is
 * not positive, the reference's "not positive definite" failure, for
 * the caller to check once the stream has run. The call runs on the
 * library's stream and on its second stream (joined back before it
 * returns to the stream). Each diagonal block waits inside its kernel for
 * the other stream's trailing update, and each panel's first products
 * inside theirs for the diagonal block; those waits are bounded (about
 * 0.1 s), and info = -1 reports that one gave up, which can happen only
 * if the other stream's work could not run meanwhile (both streams of two
 * concurrent solves mapped onto shared hardware queues, or a GPU
 * time-sliced away for that long). The result is then not valid: F has
 * been overwritten, so the caller restores it and calls
 * roma_gp_solve_events, as roma_match does. */
size_t roma_gp_work_bytes(int n, int d);
void roma_gp_solve(struct ops *o, cl_mem K, int n, float noise, cl_mem F,
                   int d, cl_mem work, cl_mem info);
/* The same solve with the two streams waiting through stream events
 * (no in-kernel wait, so info is never -1): the form used under stream
 * capture, and the fallback after info = -1. Same arithmetic and results;
 * about 0.1 ms slower at n = 1600 (the command processor's event waits on
 * the critical path). */
void roma_gp_solve_events(struct ops *o, cl_mem K, int n, float noise,
                          cl_mem F, int d, cl_mem work, cl_mem info);

#ifdef __cplusplus
}
#endif

#endif /* ICOREG_KERNELS_H */

/* SPDX-License-Identifier: Unlicense */

/* Fused kernels of the ELoFTR driver that have no counterpart among the
 * reference's kernels: they replace a chain of its generic operations
 * with one launch of the same result. */

#ifndef ICOREG_ELOFTR_FUSED_H
#define ICOREG_ELOFTR_FUSED_H

#include "ops.h"

/* X (nb, C, n) += LayerNorm over the C <= 256 channels of each of the n tokens
 * of M (nb, C, n), gain g and bias b (C each), epsilon eps: the
 * LayerNorm of the MLP output and the residual add that end an
 * aggregated-attention block (eloftr.c:445-448 of i.coregistration.opencl:
 * ops_layernorm on token-major rows, transpose back, ops_axpby). T (or
 * NULL; C % 64 == 0, 16-byte aligned) also receives the result
 * token-major, (nb, n, C): the transpose that precedes the coarse
 * matching (eloftr.c:471-480). */
void eloftr_ln_residual(struct ops *o, cl_mem M, int nb, int C, int n,
                        cl_mem g, cl_mem b, float eps, cl_mem X, cl_mem T);

/* Tokens of an aggregated-attention block for nb images of C = 256
 * channels (h x w maps, multiples of 4; image k of X and Y C h w floats
 * after image k - 1): Q (nb, h/4 * w/4, C) = LayerNorm of the depthwise
 * 4 x 4 stride-4 aggregation of X with wq (C, 1, 4, 4); KV (same shape)
 * = LayerNorm of the 4 x 4 max pooling of Y; the LayerNorm's gain g and
 * bias b shared (eloftr.c:411-423: ops_conv2d, ops_pool2d, two
 * transposes, two ops_layernorm). */
void eloftr_aggregate(struct ops *o, cl_mem X, cl_mem Y, int nb, int C, int h,
                      int w, cl_mem wq, cl_mem g, cl_mem b, float eps,
                      cl_mem Q, cl_mem KV);

/* The coarse dual softmax of a block of R rows of S (rows r0.., N
 * columns) in one read of S per pass: eloftr_row_lse and eloftr_col_lse
 * together (eloftr_lse_tiles), then eloftr_conf_row and eloftr_conf_col
 * together (eloftr_conf_tiles); same arguments and running states as
 * those four (eloftr_kernels.cl:9-144 of i.coregistration.opencl).
 * eloftr_tiles_ok: N % 4 == 0 and S 16-byte aligned, which both need. */
bool eloftr_tiles_ok(cl_mem S, int N);
void eloftr_lse_tiles(struct ops *o, cl_mem S, int R, int N, int r0, cl_mem lse, cl_mem cm,
                      cl_mem cs);
void eloftr_conf_tiles(struct ops *o, cl_mem S, int R, int N, int r0, cl_mem lse, cl_mem cm,
                       cl_mem cs, cl_mem rmax, cl_mem rarg, cl_mem cmax, cl_mem carg);

#endif /* ICOREG_ELOFTR_FUSED_H */

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
 * ops_layernorm on token-major rows, transpose back, ops_axpby). */
void eloftr_ln_residual(struct ops *o, cl_mem M, int nb, int C, int n,
                        cl_mem g, cl_mem b, float eps, cl_mem X);

#endif /* ICOREG_ELOFTR_FUSED_H */

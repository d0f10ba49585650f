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

/* Two-stage fine matching of M coarse matches: f0, f1 (64, H, W) fine
 * features, cells (int4: x0, y0, x1, y1 per match), T the second-stage
 * temperature, out (float4: x0, y0, x1, y1 per match, the reference's
 * pixel convention). eloftr_kernels.cl:146-295. */
void eloftr_fine(struct ops *o, cl_mem f0, cl_mem f1, int H, int W,
                 cl_mem cells, int M, float T, cl_mem out);

#ifdef __cplusplus
}
#endif

#endif /* ICOREG_KERNELS_H */

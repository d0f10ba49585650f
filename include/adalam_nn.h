/* SPDX-License-Identifier: Unlicense */

/* AdaLAM's brute-force nearest-neighbour search on the GPU: the static
 * nearest() of adalam.c:38-116 (i.coregistration.opencl), which
 * adalam_match (adalam.c:326) calls before its host filtering. Same
 * arguments and results: per row of d1 (n1 x dim, row-major) the first
 * index of the nearest row of d2 (n2 x dim) by squared distance
 * |a|^2 + |b|^2 - 2 a.b, Lowe's ratio of the two smallest distances
 * with the second clamped to 1e-3 (a tie gives 1), and, when nn21 is
 * not NULL, per row of d2 the first index of the nearest row of d1.
 * Distances are float32 with the dot products summed in another order
 * than the host loop, so indices agree wherever the two smallest
 * distances differ by more than float32 rounding. No distance matrix
 * is stored (the host loop keeps n1 x n2 floats). */

#ifndef ICOREG_ADALAM_NN_H
#define ICOREG_ADALAM_NN_H

#include <stddef.h>

#include "ops.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of the work buffer adalam_nearest needs for n1 x n2. */
size_t adalam_nearest_work_bytes(int n1, int n2);

/* Device form, on the ops stream: d1, d2 float32; nn12 (n1 int), score
 * (n1 float32), nn21 (n2 int, or NULL); work of
 * adalam_nearest_work_bytes(n1, n2) bytes. The descriptors DISK leaves
 * on the device can be passed as they are. */
void adalam_nearest(struct ops *o, cl_mem d1, int n1, cl_mem d2, int n2, int dim,
                    cl_mem nn12, cl_mem score, cl_mem nn21, cl_mem work);

/* Host form, a drop-in for nearest(d1, n1, d2, n2, dim, nn12, score,
 * nn21) (adalam.c:38-40) given a device: uploads, runs, reads back,
 * synchronises. */
void adalam_nearest_host(struct ops *o, const float *d1, int n1, const float *d2, int n2,
                         int dim, int *nn12, float *score, int *nn21);

#ifdef __cplusplus
}
#endif

#endif /* ICOREG_ADALAM_NN_H */

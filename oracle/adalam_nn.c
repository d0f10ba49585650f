/* SPDX-License-Identifier: Unlicense */

/* ORACLE — test infrastructure only (see oracle.h): the brute-force
 * nearest-neighbour search in front of AdaLAM, adalam.c:38-116 of
 * i.coregistration.opencl (kornia's dist_matrix plus Lowe's ratio). */

#include <float.h>
#include <stdlib.h>

#include "oracle.h"

/* Squared distances |a|^2 + |b|^2 - 2 a.b in float32 with the norms and
 * dot products summed in k order (adalam.c:46-80); per d1 the first
 * index of the smallest distance and the ratio of the two smallest
 * (the second clamped to 1e-3, adalam.c:71-83); per d2, when nn21 is
 * not NULL, the first index of the smallest distance over d1
 * (adalam.c:85-96). */
void orc_adalam_nearest(const float *d1, int n1, const float *d2, int n2,
                        int dim, int *nn12, float *score, int *nn21)
{
    float *q1 = malloc(((size_t)n1 + 1) * sizeof(float));
    float *q2 = malloc(((size_t)n2 + 1) * sizeof(float));
    float *dm = nn21 ? malloc(((size_t)n1 * n2 + 1) * sizeof(float)) : NULL;
    int i, j, k;

    for (i = 0; i < n1; i++) {
        float s = 0;

        for (k = 0; k < dim; k++)
            s += d1[(size_t)i * dim + k] * d1[(size_t)i * dim + k];
        q1[i] = s;
    }
    for (j = 0; j < n2; j++) {
        float s = 0;

        for (k = 0; k < dim; k++)
            s += d2[(size_t)j * dim + k] * d2[(size_t)j * dim + k];
        q2[j] = s;
    }
#pragma omp parallel for private(j, k) schedule(static)
    for (i = 0; i < n1; i++) {
        const float *a = d1 + (size_t)i * dim;
        float best = FLT_MAX, second = FLT_MAX;
        int bj = 0;

        for (j = 0; j < n2; j++) {
            const float *b = d2 + (size_t)j * dim;
            float dot = 0, d;

            for (k = 0; k < dim; k++)
                dot += a[k] * b[k];
            d = q1[i] + q2[j] - 2.0f * dot;
            if (dm)
                dm[(size_t)i * n2 + j] = d;
            if (d < best) {
                second = best;
                best = d;
                bj = j;
            }
            else if (d < second)
                second = d;
        }
        nn12[i] = bj;
        score[i] = best / (second > 1e-3f ? second : 1e-3f);
    }
    if (nn21)
        for (j = 0; j < n2; j++) {
            float best = FLT_MAX;
            int bi = 0;

            for (i = 0; i < n1; i++)
                if (dm[(size_t)i * n2 + j] < best) {
                    best = dm[(size_t)i * n2 + j];
                    bi = i;
                }
            nn21[j] = bi;
        }
    free(dm);
    free(q1);
    free(q2);
}

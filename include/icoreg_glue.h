/* SPDX-License-Identifier: Unlicense */

/* Glue for bindings that cannot see C struct layouts (ctypes, cgo
 * without the headers): allocation of the model structs and read access
 * to their results and intermediate buffers. No counterpart in the
 * reference, whose callers are C and read the struct fields directly;
 * these functions add nothing to the computation. */

#ifndef ICOREG_GLUE_H
#define ICOREG_GLUE_H

#include "eloftr.h"
#include "pth_loader.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Zeroed structs on the heap, freed with free() after *_free / pth_close. */
struct pth_file *icoreg_pth_new(void);
struct eloftr_model *icoreg_eloftr_new(void);
void icoreg_struct_delete(void *p);

/* Results of the last eloftr_match: match count, host arrays (owned by
 * the model), coarse statistics (n = (H / 8) (W / 8) each). */
int icoreg_eloftr_result(const struct eloftr_model *m, const int **mi,
                         const int **mj, const float **mconf,
                         const float **kp);
int icoreg_eloftr_coarse_stats(const struct eloftr_model *m,
                               const float **row_max, const int **row_arg,
                               const int **col_arg);
void icoreg_eloftr_set_pos_scale(struct eloftr_model *m, float s);

/* A named device buffer of the model: "x0", "x1" (1/8 features, 256 x
 * n), "fine0", "fine1" (64 x H x W), "f1_0", "f2_0", ... Returns NULL for
 * an unknown name. */
cl_mem icoreg_eloftr_buffer(const struct eloftr_model *m, const char *name);

#ifdef __cplusplus
}
#endif

#endif /* ICOREG_GLUE_H */

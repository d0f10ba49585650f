/* SPDX-License-Identifier: Unlicense */

/* Glue for bindings that cannot see C struct layouts (ctypes, cgo
 * without the headers): allocation of the model structs and read access
 * to their results and intermediate buffers. No counterpart in the
 * reference, whose callers are C and read the struct fields directly;
 * these functions add nothing to the computation. */

#ifndef ICOREG_GLUE_H
#define ICOREG_GLUE_H

#include "disk.h"
#include "eloftr.h"
#include "pth_loader.h"
#include "roma.h"

#ifdef __cplusplus
extern "C" {
#endif

/* sizeof(struct ocl_backend) and sizeof(struct ops), so that a binding
 * that mirrors their layouts can check them. */
size_t icoreg_sizeof_backend(void);
size_t icoreg_sizeof_ops(void);

/* Zeroed structs on the heap, freed with free() after *_free / pth_close. */
struct pth_file *icoreg_pth_new(void);
struct eloftr_model *icoreg_eloftr_new(void);
void icoreg_struct_delete(void *p);

/* Results of the last eloftr_match: match count, host arrays (owned by
 * the model); coarse statistics (n = (H / 8) (W / 8) each), read from the
 * device into the model's host copies on each call. */
int icoreg_eloftr_result(const struct eloftr_model *m, const int **mi,
                         const int **mj, const float **mconf,
                         const float **kp);
int icoreg_eloftr_coarse_stats(struct eloftr_model *m,
                               const float **row_max, const int **row_arg,
                               const int **col_arg);
void icoreg_eloftr_set_pos_scale(struct eloftr_model *m, float s);

/* A named device buffer of the model: "x0", "x1" (1/8 features, 256 x
 * n), "fine0", "fine1" (64 x H x W, written from the last match's
 * half-resolution maps by this request), "fineh0", "fineh1" (those maps,
 * 64 x H/2 x W/2), "f1_0", "f2_0", ... Returns NULL for an unknown name. */
cl_mem icoreg_eloftr_buffer(struct eloftr_model *m, const char *name);

struct roma_model *icoreg_roma_new(void);
struct disk_model *icoreg_disk_new(void);

/* A named device buffer of a DISK model: "out" (129 x H x W: descriptor
 * channels then the heatmap), "mask" (NMS bytes); NULL otherwise. */
cl_mem icoreg_disk_buffer(const struct disk_model *m, const char *name);

/* Results of the last roma_match: H x W, host arrays owned by the model
 * (sd NULL without v2). */
int icoreg_roma_result(const struct roma_model *m, const float **flow,
                       const float **cert, const float **sd);

/* A named device buffer of the model: "fl0", "fl1", "ce0", "ce1", "cf0",
 * "cf1", "t_out", "g_y", "g_f", "t_x", "cert16", "P0" .. "P4"; NULL for an
 * unknown name. */
cl_mem icoreg_roma_buffer(const struct roma_model *m, const char *name);

/* 1 + the first failing GP pivot of the last solve, 0 if it succeeded
 * (waits for the stream). */
int icoreg_roma_gp_info(struct roma_model *m);
/* Index (0 or 1) of the fl / ce buffers holding roma_refine_device's
 * result. */
int icoreg_roma_last(const struct roma_model *m);

void icoreg_roma_set_imagenet(struct roma_model *m, int on);

/* Test hooks of the GP solve's in-kernel waits (roma_gp_solve): their
 * poll limit (0: the default, about 0.1 s) and whether the panel flags
 * are set at all (0: never, so every waiting diagonal kernel and every
 * panel's first products give up after spin_max polls and report info =
 * -1). Process-wide; for tests of the give-up path and of roma_match's
 * recovery. */
void icoreg_gp_test_wait(int spin_max, int set_flags);
/* Which Winograd form the same-size 3 x 3 convolutions take: 0 each
 * shape's own choice (the default), 2 F(2 x 2, 3 x 3) or 4 F(4 x 4, 3 x 3)
 * wherever that form applies. Process-wide; for tests and measurements. */
void icoreg_conv_wino_form(int form);
/* The form (4 or 2; 0: not a Winograd shape) the library gives a 3 x 3,
 * stride 1, padding 1 convolution of nb contiguous C x H x W images to K
 * channels on o's device, under the current icoreg_conv_wino_form. */
int icoreg_conv_wino_choice(struct ops *o, int nb, int C, int H, int W, int K);
/* How many times roma_match has re-run a GP solve through
 * roma_gp_solve_events after the in-kernel wait gave up. */
int icoreg_roma_gp_retries(const struct roma_model *m);

#ifdef __cplusplus
}
#endif

#endif /* ICOREG_GLUE_H */

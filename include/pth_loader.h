/* SPDX-License-Identifier: Unlicense */

/* Checkpoint reader of the model drivers: the API of the reference's
 * pth_loader.h (pth_loader.h:9-61 of i.coregistration.opencl) over the
 * three formats its pth_loader.c reads: torch.save zip archives (stored
 * entries, Zip64 included), legacy torch.save pickle streams and
 * safetensors files. float32, float16 and bfloat16 tensors are indexed
 * (read back as float32); integer and boolean tensors are left out.
 * Pickles are interpreted without executing anything. Every format or
 * lookup problem is a fatal error. */

#ifndef ICOREG_PTH_LOADER_H
#define ICOREG_PTH_LOADER_H

#include <stddef.h>
#include <stdio.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PTH_MAX_DIMS 8

enum pth_dtype { PTH_F32, PTH_F16, PTH_BF16, PTH_OTHER };

struct pth_tensor {
    char *name;
    int ndim;
    long shape[PTH_MAX_DIMS];
    long stride[PTH_MAX_DIMS]; /* In elements. */
    long storage_offset;       /* In elements. */
    enum pth_dtype dtype;
    long data_offset;     /* Byte offset of the storage in the file. */
    size_t storage_bytes; /* Byte size of the storage. */
};

struct pth_file {
    FILE *fp;
    char *path;
    int ntensors;
    struct pth_tensor *tensors;
};

/* Open and index a checkpoint (pth_loader.h:36-38). */
void pth_open(struct pth_file *pf, const char *path);

/* The tensor called name, or NULL (pth_loader.h:40-41). */
const struct pth_tensor *pth_find(const struct pth_file *pf, const char *name);

/* Like pth_find, fatal if missing or if the shape does not match the
 * ndim leading entries of shape (-1 matches anything). */
const struct pth_tensor *pth_require(const struct pth_file *pf,
                                     const char *name, int ndim,
                                     const long *shape);

/* Remove prefix from the names that start with it; returns their count. */
int pth_strip_prefix(struct pth_file *pf, const char *prefix);

long pth_numel(const struct pth_tensor *t);

/* Total data bytes of the tensors whose names start with prefix. */
double pth_bytes(const struct pth_file *pf, const char *prefix);

/* The tensor as a newly malloc'ed float32 array (free with free()). */
float *pth_read_f32(const struct pth_file *pf, const struct pth_tensor *t);

void pth_close(struct pth_file *pf);

#ifdef __cplusplus
}
#endif

#endif /* ICOREG_PTH_LOADER_H */

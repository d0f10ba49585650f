/* SPDX-License-Identifier: Unlicense */

/* DISK local features on one MI355X.
 *
 * The API is the reference's (disk.h:10-52 of i.coregistration.opencl):
 * disk_load / disk_alloc / disk_detect / disk_free, called unchanged by
 * matcher_disk.c:39-58. The U-Net of kornia.feature.DISK (5 x 5 kernels,
 * down 16-32-64-64-64, up 64-64-64-129, InstanceNorm + PReLU on each
 * block's input) runs on this build's direct 5 x 5 convolution on the
 * matrix cores with the normalisation fused into its input loads; the
 * heatmap NMS, the top-n selection (on the host in the reference) and
 * the descriptor gather are HIP kernels (icoreg_kernels.h); the host
 * reads back only the keypoints. */

#ifndef ICOREG_DISK_H
#define ICOREG_DISK_H

#include "ocl_backend.h"
#include "ops.h"
#include "pth_loader.h"

#ifdef __cplusplus
extern "C" {
#endif

#define DISK_DESC 128    /* Descriptor dimension. */
#define DISK_LAYERS 9    /* Five down blocks, four up blocks. */
#define DISK_MULTIPLE 16 /* Input sides must be multiples of this. */

struct disk_model {
    struct ocl_backend *ocl;
    struct ops *ops;
    int cin[DISK_LAYERS], cout[DISK_LAYERS];
    cl_mem w[DISK_LAYERS], b[DISK_LAYERS], alpha[DISK_LAYERS];
    /* Work buffers for tiles of up to H x W cells. cat[l] is the up
     * path's concatenation at level l (64 upsampled channels, then the
     * skip connection); f[l] (l < 4) is a view of its skip part, where
     * the down path writes, so no copy joins them. */
    int H, W, nmax;
    cl_mem input, f[5], u[3], cat[4], tmp, out, mean, rstd, mask, valid;
    cl_mem xy, score, count, desc, topn_work;
};

/* Read the DISK weights ("unet.path_down.*", "unet.path_up.*" of the
 * extractor state dict) and upload them. Fatal on a missing tensor or a
 * shape mismatch. disk.h:34-38. */
void disk_load(struct disk_model *m, struct ops *ops, struct pth_file *pf);

/* Work buffers for tiles of up to H x W cells (multiples of
 * DISK_MULTIPLE) and up to nmax keypoints. disk.h:40-42. */
void disk_alloc(struct disk_model *m, int H, int W, int nmax);

/* Keypoints of img, a (3, H, W) image in 0..1 whose content covers its
 * top-left h x w cells: 5 x 5 NMS on the heatmap cropped to h x w, cells
 * above thresh, then the n highest in raster order (kornia
 * heatmap_to_keypoints), skipping cells where valid is 0 when valid is
 * not NULL; xy (x, y pairs), score and L2-normalised descriptors (n x
 * DISK_DESC). Returns the keypoint count. disk.h:44-50. */
int disk_detect(struct disk_model *m, const float *img, int H, int W, int h,
                int w, int n, float thresh, const unsigned char *valid, int *xy,
                float *score, float *desc);

void disk_free(struct disk_model *m);

#ifdef __cplusplus
}
#endif

#endif /* ICOREG_DISK_H */

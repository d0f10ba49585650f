/* SPDX-License-Identifier: Unlicense */

/* Efficient LoFTR on one MI355X: RepVGG backbone (folded 3 x 3 convs on
 * the implicit-GEMM MFMA kernel), aggregated-attention transformer with
 * 2D RoPE (MFMA flash attention), coarse dual-softmax matching with
 * mutual nearest selection, FPN fusion and two-stage fine matching.
 *
 * The API is the reference's (eloftr.h:9-82 of i.coregistration.opencl):
 * eloftr_load / eloftr_alloc / eloftr_match / eloftr_free and the result
 * fields its matcher reads (nm, mi, mj, mconf, kp, pos_scale, H, W,
 * matcher_eloftr.c:49-101). The buffer plan behind them is this build's
 * own. */

#ifndef ICOREG_ELOFTR_H
#define ICOREG_ELOFTR_H

#include "ops.h"
#include "pth_loader.h"

#ifdef __cplusplus
extern "C" {
#endif

#define ELOFTR_MULTIPLE 32   /* Tile sides: 1/8 features, aggregated by 4. */
#define ELOFTR_DIM 256       /* Coarse feature dimension. */
#define ELOFTR_FINE_DIM 64   /* Fine feature dimension. */
#define ELOFTR_BLOCKS 21     /* RepVGG blocks: 1 + 2 + 4 + 14. */
#define ELOFTR_LAYERS 4      /* Transformer layers (self + cross each). */
#define ELOFTR_TRAIN_RES 832 /* Training resolution of the "npe". */

struct eloftr_attn {
    cl_mem q_agg;          /* Depthwise 4 x 4 (256, 1, 4, 4). */
    cl_mem norm_g, norm_b; /* LayerNorm of the aggregated tokens. */
    cl_mem wq;             /* (256, 256), no bias. */
    /* fc1[:, 256:512] o_proj (512, 256): the message's route into fc1. */
    cl_mem wmsg;
    cl_mem wkv;            /* k_proj over v_proj: (512, 256), no bias. */
    cl_mem fc1, fc2;       /* (512, 512), (256, 512), no bias. */
    cl_mem mlp_g, mlp_b;   /* LayerNorm after the MLP. */
};

struct eloftr_model {
    struct ops *ops;
    struct ocl_backend *ocl;
    /* RepVGG blocks folded into 3 x 3 convolutions with bias. */
    cl_mem bw[ELOFTR_BLOCKS], bb[ELOFTR_BLOCKS];
    int bcin[ELOFTR_BLOCKS], bcout[ELOFTR_BLOCKS], bstride[ELOFTR_BLOCKS];
    struct eloftr_attn self_attn[ELOFTR_LAYERS], cross_attn[ELOFTR_LAYERS];
    /* Fine fusion: out_conv (x / 16 folded), then per block out_conv1
     * 1 x 1, out_conv2 3 x 3 with BatchNorm folded, out_conv3 3 x 3. */
    cl_mem f_out, f1_w[2], f2_w[2], f2_b[2], f3_w[2];
    /* The stride-1 3 x 3 filters in Winograd form (NULL where the
     * convolution runs direct): backbone blocks, then f2_w, f3_w. */
    cl_mem bU[ELOFTR_BLOCKS], f2_U[2], f3_U[2];

    /* Scale of the RoPE positions (1; the authors' "npe": 832 / long
     * side), set before eloftr_alloc. */
    float pos_scale;
    int H, W, h, w, ah, aw, nmax;
    /* Work buffers (eloftr_alloc). Both images of the pair sit in one
     * allocation (img, s_a, s_b, f1p, f2p, xp, finep, fu_*: image 1 right
     * after image 0), so that the backbone and the fusion run each layer
     * once for the pair; f1[k], f2[k], x[k], fine[k] are views of image k.
     * finep is written only on request (eloftr_fine_maps); fine matching
     * reads the half-resolution maps fine_h[k] (views of fu_c). */
    cl_mem img, s_a, s_b, f1p, f2p, xp, finep;
    cl_mem f1[2], f2[2], x[2], fine[2], fine_h[2];
    cl_mem t_qn, t_kvn, t_Q, t_KV, t_O, t_O2, t_tok, t_h1, t_h2,
        rope;
    cl_mem s_blk, row_lse, col_m, col_s, row_max, row_arg, col_max, col_arg;
    cl_mem fu_a, fu_b, fu_c, m_idx, m_out;
    cl_mem d_mi, d_mj, d_mconf, m_count; /* the matches on the device */
    int blk_rows;
    /* Last match: coarse matches (cell indices i, j and confidence) and
     * their refined positions (x0, y0, x1, y1 per match, pixel index -
     * 3.5 as the reference). */
    int nm;
    int *mi, *mj;
    float *mconf, *kp;
    /* Host copies of the coarse statistics of the last match (n each):
     * row maximum, row argmax, column argmax (read on request by
     * icoreg_eloftr_coarse_stats). */
    float *h_rmax;
    int *h_rarg, *h_carg;
};

/* Read the weights (safetensors with the names of
 * EfficientLoFTRForKeypointMatching), fold BatchNorms and RepVGG
 * branches in double precision, upload. Fatal on any missing tensor or
 * shape mismatch. eloftr.h:62-66. */
void eloftr_load(struct eloftr_model *m, struct ops *ops, struct pth_file *pf);

/* Work buffers for tiles of H x W cells (multiples of ELOFTR_MULTIPLE). */
void eloftr_alloc(struct eloftr_model *m, int H, int W);

/* Match two grey H x W images (values in 0..1): coarse mutual matches
 * above 0.2 confidence away from the border, refined by the fine stage;
 * results in nm, mi, mj, mconf, kp. With dump (a folder), writes
 * tileNNN_eloftr_{backbone,coarse,fine}_{0,1}.f32 as the reference. */
void eloftr_match(struct eloftr_model *m, const float *grey0,
                  const float *grey1, const char *dump, int tile);

/* eloftr_match on a pair already in device memory (dev0, dev1: H x W
 * floats each): the same stages with no image upload; the mutual
 * selection and the fine stage run on the device, and the only host
 * transfer is the final read of the matches. */
void eloftr_match_device(struct eloftr_model *m, cl_mem dev0, cl_mem dev1);

/* eloftr_match_device split in two (no counterpart in the reference):
 * enqueue queues every stage on the library's stream with no host
 * transfer or synchronisation (so it can be recorded as a HIP graph,
 * ocl_graph_begin / ocl_graph_end); collect waits and reads the matches
 * into nm, mi, mj, mconf, kp. */
void eloftr_match_enqueue(struct eloftr_model *m, cl_mem dev0, cl_mem dev1);
void eloftr_match_collect(struct eloftr_model *m);

void eloftr_free(struct eloftr_model *m);
/* Write finep (fine[0], fine[1]: 64 x H x W each), the 2x bilinear resize
 * of the last match's half-resolution fine maps (eloftr.c:604); the
 * matcher itself samples that resize on the fly and does not need it. */
void eloftr_fine_maps(struct eloftr_model *m);

#ifdef __cplusplus
}
#endif

#endif /* ICOREG_ELOFTR_H */

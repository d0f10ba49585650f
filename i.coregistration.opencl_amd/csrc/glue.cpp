/* SPDX-License-Identifier: Unlicense */

/* Struct allocation and result access for bindings (icoreg_glue.h). */

#include <stdlib.h>
#include <string.h>

#include "icoreg_glue.h"

extern "C" size_t icoreg_sizeof_backend(void) { return sizeof(struct ocl_backend); }

extern "C" size_t icoreg_sizeof_ops(void) { return sizeof(struct ops); }

extern "C" struct pth_file *icoreg_pth_new(void)
{
    return (struct pth_file *)calloc(1, sizeof(struct pth_file));
}

extern "C" struct eloftr_model *icoreg_eloftr_new(void)
{
    return (struct eloftr_model *)calloc(1, sizeof(struct eloftr_model));
}

extern "C" void icoreg_struct_delete(void *p) { free(p); }

extern "C" int icoreg_eloftr_result(const struct eloftr_model *m,
                                    const int **mi, const int **mj,
                                    const float **mconf, const float **kp)
{
    *mi = m->mi;
    *mj = m->mj;
    *mconf = m->mconf;
    *kp = m->kp;
    return m->nm;
}

extern "C" int icoreg_eloftr_coarse_stats(struct eloftr_model *m,
                                          const float **row_max,
                                          const int **row_arg,
                                          const int **col_arg)
{
    const size_t n = (size_t)m->h * m->w;

    ocl_read(m->ocl, m->row_max, 0, m->h_rmax, n * sizeof(float));
    ocl_read(m->ocl, m->row_arg, 0, m->h_rarg, n * sizeof(int));
    ocl_read(m->ocl, m->col_arg, 0, m->h_carg, n * sizeof(int));
    *row_max = m->h_rmax;
    *row_arg = m->h_rarg;
    *col_arg = m->h_carg;
    return (int)n;
}

extern "C" void icoreg_eloftr_set_pos_scale(struct eloftr_model *m, float s)
{
    m->pos_scale = s;
}

extern "C" cl_mem icoreg_eloftr_buffer(struct eloftr_model *m, const char *name)
{
    static const struct {
        const char *name;
        size_t off;
    } tab[] = {
        {"x0", offsetof(struct eloftr_model, x[0])},
        {"x1", offsetof(struct eloftr_model, x[1])},
        {"fine0", offsetof(struct eloftr_model, fine[0])},
        {"fine1", offsetof(struct eloftr_model, fine[1])},
        {"fineh0", offsetof(struct eloftr_model, fine_h[0])},
        {"fineh1", offsetof(struct eloftr_model, fine_h[1])},
        {"f1_0", offsetof(struct eloftr_model, f1[0])},
        {"f1_1", offsetof(struct eloftr_model, f1[1])},
        {"f2_0", offsetof(struct eloftr_model, f2[0])},
        {"f2_1", offsetof(struct eloftr_model, f2[1])},
        {"row_lse", offsetof(struct eloftr_model, row_lse)},
        {"col_m", offsetof(struct eloftr_model, col_m)},
        {"col_s", offsetof(struct eloftr_model, col_s)},
    };

    /* The full-resolution fine maps are written on request only. */
    if ((strcmp(name, "fine0") == 0 || strcmp(name, "fine1") == 0) && m->fu_c && m->finep)
        eloftr_fine_maps(m);
    for (size_t i = 0; i < sizeof(tab) / sizeof(tab[0]); i++)
        if (strcmp(tab[i].name, name) == 0)
            return *(const cl_mem *)((const char *)m + tab[i].off);
    return NULL;
}

extern "C" struct roma_model *icoreg_roma_new(void)
{
    return (struct roma_model *)calloc(1, sizeof(struct roma_model));
}

extern "C" int icoreg_roma_result(const struct roma_model *m,
                                  const float **flow, const float **cert,
                                  const float **sd)
{
    *flow = m->flow;
    *cert = m->cert;
    *sd = m->sd;
    return m->H * m->W;
}

extern "C" cl_mem icoreg_roma_buffer(const struct roma_model *m,
                                     const char *name)
{
    static const struct {
        const char *name;
        size_t off;
    } tab[] = {
        {"fl0", offsetof(struct roma_model, fl[0])},
        {"fl1", offsetof(struct roma_model, fl[1])},
        {"ce0", offsetof(struct roma_model, ce[0])},
        {"ce1", offsetof(struct roma_model, ce[1])},
        {"cf0", offsetof(struct roma_model, cf[0])},
        {"cf1", offsetof(struct roma_model, cf[1])},
        {"t_out", offsetof(struct roma_model, t_out)},
        {"t_x", offsetof(struct roma_model, t_x)},
        {"t_n", offsetof(struct roma_model, t_n)},
        {"g_y", offsetof(struct roma_model, g_y)},
        {"g_f", offsetof(struct roma_model, g_f)},
        {"g_kyy", offsetof(struct roma_model, g_kyy)},
        {"cert16", offsetof(struct roma_model, cert16)},
        {"img", offsetof(struct roma_model, img)},
        {"P0", offsetof(struct roma_model, P[0])},
        {"P1", offsetof(struct roma_model, P[1])},
        {"P2", offsetof(struct roma_model, P[2])},
        {"P3", offsetof(struct roma_model, P[3])},
        {"P4", offsetof(struct roma_model, P[4])},
    };

    for (size_t i = 0; i < sizeof(tab) / sizeof(tab[0]); i++)
        if (strcmp(tab[i].name, name) == 0)
            return *(const cl_mem *)((const char *)m + tab[i].off);
    return NULL;
}

extern "C" int icoreg_roma_last(const struct roma_model *m) { return m->last; }

extern "C" int icoreg_roma_gp_retries(const struct roma_model *m) { return m->gp_retries; }

extern "C" int icoreg_roma_gp_info(struct roma_model *m)
{
    int info = 0;

    ocl_read(m->ocl, m->gp_info, 0, &info, sizeof(info));
    return info;
}

extern "C" void icoreg_roma_set_imagenet(struct roma_model *m, int on)
{
    m->imagenet = on;
}

extern "C" struct disk_model *icoreg_disk_new(void)
{
    return (struct disk_model *)calloc(1, sizeof(struct disk_model));
}

extern "C" cl_mem icoreg_disk_buffer(const struct disk_model *m,
                                     const char *name)
{
    if (strcmp(name, "out") == 0)
        return m->out;
    if (strcmp(name, "mask") == 0)
        return m->mask;
    return NULL;
}

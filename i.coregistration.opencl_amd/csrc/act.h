/* SPDX-License-Identifier: Unlicense */

/* Activations applied after the bias (the contract of apply_act,
 * ops.cl:23-37 of i.coregistration.opencl): exact GELU through erff,
 * GELU tanh approximation through tanhf, ReLU, LeakyReLU. */

#ifndef ICOREG_ACT_H
#define ICOREG_ACT_H

#include <hip/hip_runtime.h>

#include "ops.h"

/* Rotary rotation of the pair (a, b) by (cos, sin) = rot, the order of
 * operations fixed so that every kernel that applies it rounds alike. */
__device__ __forceinline__ void icoreg_rope_pair(float a, float b, float2 rot, float &x0,
                                                 float &x1)
{
    x0 = fmaf(a, rot.x, -(b * rot.y));
    x1 = fmaf(a, rot.y, b * rot.x);
}

__device__ __forceinline__ float icoreg_act(float v, int act, float slope)
{
    switch (act) {
    case ACT_GELU:
        return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
    case ACT_RELU:
        return fmaxf(v, 0.0f);
    case ACT_LEAKY:
        return v >= 0.0f ? v : slope * v;
    case ACT_GELU_TANH:
        return 0.5f * v *
               (1.0f + tanhf(0.79788456080286536f * (v + 0.044715f * v * v * v)));
    default:
        return v;
    }
}

#endif /* ICOREG_ACT_H */

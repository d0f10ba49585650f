/* SPDX-License-Identifier: Unlicense */

/* Wave64 reductions by cross-lane exchange (DPP / ds_swizzle through
 * __shfl_xor), and block-level reductions over 4 waves. */

#ifndef ICOREG_REDUCE_H
#define ICOREG_REDUCE_H

#include <hip/hip_runtime.h>

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

/* (value, index) maximum with ties to the lowest index: associative and
 * commutative, so any reduction order gives the first argmax. */
__device__ __forceinline__ void argmax_merge(float &v, int &i, float v2, int i2)
{
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

__device__ __forceinline__ void wave_argmax(float &v, int &i)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v2 = __shfl_xor(v, o, 64);
        const int i2 = __shfl_xor(i, o, 64);

        argmax_merge(v, i, v2, i2);
    }
}

/* Sum over a block of nw waves; red holds nw floats. Every thread gets
 * the total. */
template <int NW>
__device__ __forceinline__ float block_sum(float v, float *red)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;

    v = wave_sum(v);
    if (lane == 0)
        red[w] = v;
    __syncthreads();
    v = 0.0f;
#pragma unroll
    for (int k = 0; k < NW; k++)
        v += red[k];
    __syncthreads();
    return v;
}

template <int NW>
__device__ __forceinline__ float block_max(float v, float *red)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;

    v = wave_max(v);
    if (lane == 0)
        red[w] = v;
    __syncthreads();
    v = red[0];
#pragma unroll
    for (int k = 1; k < NW; k++)
        v = fmaxf(v, red[k]);
    __syncthreads();
    return v;
}

#endif /* ICOREG_REDUCE_H */

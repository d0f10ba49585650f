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

/* The same reductions for waves whose 64 lanes are all active, without
 * the LDS crossbar: DPP exchanges inside each 16-lane row (quad
 * permutations, half-row and row mirrors), then the four row results read
 * into scalar registers. Every lane gets the result (uniform). */
__device__ __forceinline__ float dpp_f(float v, int ctrl)
{
    /* ctrl is one of the constants below (the builtin wants a constant). */
    switch (ctrl) {
    case 0xB1:
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v),
                                                                  0xB1, 0xF, 0xF, false));
    case 0x4E:
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v),
                                                                  0x4E, 0xF, 0xF, false));
    case 0x141:
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v),
                                                                  0x141, 0xF, 0xF, false));
    default:
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v),
                                                                  0x140, 0xF, 0xF, false));
    }
}

__device__ __forceinline__ float lane_f(float v, int l)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

/* quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror. */
__device__ __forceinline__ float wave_sum_full(float v)
{
    v += dpp_f(v, 0xB1);
    v += dpp_f(v, 0x4E);
    v += dpp_f(v, 0x141);
    v += dpp_f(v, 0x140);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

__device__ __forceinline__ float wave_max_full(float v)
{
    v = fmaxf(v, dpp_f(v, 0xB1));
    v = fmaxf(v, dpp_f(v, 0x4E));
    v = fmaxf(v, dpp_f(v, 0x141));
    v = fmaxf(v, dpp_f(v, 0x140));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
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

__device__ __forceinline__ int dpp_i(int v, int ctrl)
{
    switch (ctrl) {
    case 0xB1:
        return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
    case 0x4E:
        return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
    case 0x141:
        return __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false);
    default:
        return __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false);
    }
}

/* wave_argmax for fully active waves (DPP, then the four rows' results
 * through scalar registers); every lane gets the result. */
__device__ __forceinline__ void wave_argmax_full(float &v, int &i)
{
    const int ctl[4] = {0xB1, 0x4E, 0x141, 0x140};

#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float v2 = dpp_f(v, ctl[k]);
        const int i2 = dpp_i(i, ctl[k]);

        argmax_merge(v, i, v2, i2);
    }
    {
        float bv = lane_f(v, 0);
        int bi = __builtin_amdgcn_readlane(i, 0);

#pragma unroll
        for (int l = 16; l < 64; l += 16)
            argmax_merge(bv, bi, lane_f(v, l), __builtin_amdgcn_readlane(i, l));
        v = bv;
        i = bi;
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

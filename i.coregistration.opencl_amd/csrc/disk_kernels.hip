/* SPDX-License-Identifier: Unlicense */

/* DISK's own kernels on gfx950: the 5 x 5 non-maxima suppression of the
 * heatmap and the descriptor gather. Contracts of disk_kernels.cl:8-60
 * (i.coregistration.opencl).
 *
 *  - NMS: 32 x 8 output cells per block, the (12 x 36) heat patch staged
 *    in LDS once, so each heat value is read from HBM about 1.6 times
 *    instead of 25;
 *  - gather: one wave64 per keypoint, lanes over the descriptor
 *    channels, the squared norm by a cross-lane reduction, coalesced
 *    descriptor rows. */

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdlib.h>

#include "common.h"
#include "icoreg_kernels.h"
#include "reduce.h"

using namespace icoreg;

__global__ void fill_int_kernel(int *p, int n, int v)
{
    const int i = blockIdx.x * 64 + threadIdx.x;

    if (i < n)
        p[i] = v;
}

#define NMS_TX 32
#define NMS_TY 8

__global__ void __launch_bounds__(256)
    nms5x5_kernel(const float *__restrict__ heat, int W, int h, int w,
                  float thresh, unsigned char *__restrict__ mask)
{
    __shared__ float t[NMS_TY + 4][NMS_TX + 5];
    const int lx = threadIdx.x & (NMS_TX - 1), ly = threadIdx.x / NMS_TX;
    const int x0 = blockIdx.x * NMS_TX, y0 = blockIdx.y * NMS_TY;
    const int x = x0 + lx, y = y0 + ly;

    for (int e = threadIdx.x; e < (NMS_TY + 4) * (NMS_TX + 4); e += 256) {
        const int yy = y0 - 2 + e / (NMS_TX + 4), xx = x0 - 2 + e % (NMS_TX + 4);

        t[e / (NMS_TX + 4)][e % (NMS_TX + 4)] =
            yy >= 0 && yy < h && xx >= 0 && xx < w
                ? heat[(long long)yy * W + xx]
                : -INFINITY;
    }
    __syncthreads();
    if (x >= w || y >= h)
        return;
    if (x < 2 || y < 2 || x >= w - 2 || y >= h - 2) {
        mask[(long long)y * w + x] = 0;
        return;
    }
    {
        const float v = t[ly + 2][lx + 2];
        bool keep = v > thresh;

#pragma unroll
        for (int dy = 0; dy < 5; dy++)
#pragma unroll
            for (int dx = 0; dx < 5; dx++)
                if (dy != 2 || dx != 2)
                    keep = keep && v > t[ly + dy][lx + dx];
        mask[(long long)y * w + x] = keep ? 1 : 0;
    }
}

/* n, or the count on the device when ncount is set (keypoints k >= it
 * do nothing). */
__global__ void __launch_bounds__(256)
    gather_desc_kernel(const float *__restrict__ feat, long long plane,
                       int D, const int *__restrict__ xy, int n, int W,
                       float *__restrict__ desc, const int *__restrict__ ncount)
{
    const int lane = threadIdx.x & 63;
    const int k = blockIdx.x * 4 + (threadIdx.x >> 6);
    long long off;
    float ss = 0.0f, inv;

    if (ncount)
        n = min(n, *ncount);
    if (k >= n)
        return;
    off = (long long)xy[2 * k + 1] * W + xy[2 * k];
    for (int d = lane; d < D; d += 64) {
        const float v = feat[d * plane + off];

        ss = fmaf(v, v, ss);
    }
    ss = wave_sum(ss);
    inv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
    for (int d = lane; d < D; d += 64)
        desc[(long long)k * D + d] = feat[d * plane + off] * inv;
}

extern "C" void disk_nms5x5(struct ops *o, cl_mem heat, long off, int W, int h,
                            int w, float thresh, cl_mem mask)
{
    ICOREG_API_BEGIN
    const char *op = "disk_nms5x5";

    if (h < 0 || w < 0 || W < w || off < 0)
        icoreg_fatal("%s: invalid crop %d x %d of width %d", op, h, w, W);
    if ((long long)h * w == 0)
        return;
    need_floats(heat, off, (long long)(h - 1) * W + w, op, "heat");
    need_bytes(mask, 0, (long long)h * w, op, "mask");
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(nms5x5_kernel,
                       dim3((unsigned)((w + NMS_TX - 1) / NMS_TX),
                            (unsigned)((h + NMS_TY - 1) / NMS_TY)),
                       dim3(256), 0, stream_of(o->ocl), cfptr(heat) + off, W, h,
                       w, thresh, (unsigned char *)mask->ptr);
    launch_check(op);
    ICOREG_API_END
}

extern "C" void disk_gather_desc(struct ops *o, cl_mem feat, int H, int W,
                                 int D, cl_mem xy, int n, cl_mem desc)
{
    ICOREG_API_BEGIN
    const char *op = "disk_gather_desc";
    const long long plane = (long long)H * W;

    if (H < 1 || W < 1 || D < 1 || n < 0)
        icoreg_fatal("%s: invalid sizes H=%d W=%d D=%d n=%d", op, H, W, D, n);
    if (n == 0)
        return;
    need_floats(feat, 0, (long long)D * plane, op, "feat");
    need_bytes(xy, 0, 8LL * n, op, "xy");
    need_floats(desc, 0, (long long)n * D, op, "desc");
    {
        /* Keypoint coordinates are host data the caller uploaded: check
         * them before they index the feature planes. */
        int *h_xy = (int *)malloc(8 * (size_t)n);

        ocl_read(o->ocl, xy, 0, h_xy, 8 * (size_t)n);
        for (int k = 0; k < n; k++)
            if (h_xy[2 * k] < 0 || h_xy[2 * k] >= W || h_xy[2 * k + 1] < 0 ||
                h_xy[2 * k + 1] >= H) {
                const int x = h_xy[2 * k], y = h_xy[2 * k + 1];

                free(h_xy);
                icoreg_fatal("%s: keypoint %d at (%d, %d) outside %d x %d", op,
                             k, x, y, W, H);
            }
        free(h_xy);
    }
    prof_scope ps(o->ocl, op);
    hipLaunchKernelGGL(gather_desc_kernel, dim3((unsigned)((n + 3) / 4)),
                       dim3(256), 0, stream_of(o->ocl), cfptr(feat), plane, D,
                       (const int *)xy->ptr, n, W, fptr(desc), nullptr);
    launch_check(op);
    ICOREG_API_END
}

extern "C" void disk_gather_desc_count(struct ops *o, cl_mem feat, int H, int W, int D,
                                       cl_mem xy, cl_mem count, int nmax, cl_mem desc)
{
    ICOREG_API_BEGIN
    const char *op = "disk_gather_desc_count";
    const long long plane = (long long)H * W;

    if (H < 1 || W < 1 || D < 1 || nmax < 0)
        icoreg_fatal("%s: invalid sizes H=%d W=%d D=%d nmax=%d", op, H, W, D, nmax);
    if (nmax == 0)
        return;
    need_floats(feat, 0, (long long)D * plane, op, "feat");
    need_bytes(xy, 0, 8LL * nmax, op, "xy");
    need_bytes(count, 0, 4, op, "count");
    need_floats(desc, 0, (long long)nmax * D, op, "desc");
    prof_scope ps(o->ocl, "disk_gather_desc");
    hipLaunchKernelGGL(gather_desc_kernel, dim3((unsigned)((nmax + 3) / 4)),
                       dim3(256), 0, stream_of(o->ocl), cfptr(feat), plane, D,
                       (const int *)xy->ptr, nmax, W, fptr(desc),
                       (const int *)count->ptr);
    launch_check(op);
    ICOREG_API_END
}

/* ---- top-n selection ------------------------------------------------------------------ */

/* The cells kept by disk.c:228-253 are those of the NMS mask (and valid)
 * whose heat exceeds the cut, in raster order; the cut is the (n+1)-th
 * highest candidate (the lowest if there are no more than n). On the
 * device: per row the candidate count, an exclusive scan over rows, the
 * candidates written in raster order (value, cell), an exact radix
 * select of the cut over the candidates' order-preserving 32-bit keys
 * (four 8-bit passes, one work-group), and the compaction of the
 * candidates above the cut (float comparison, as the host loop's). */

__device__ __forceinline__ unsigned topn_key(float v)
{
    const unsigned u = __float_as_uint(v);

    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ bool topn_cand(const unsigned char *__restrict__ mask,
                                          const unsigned char *__restrict__ valid, long long i)
{
    return mask[i] && (!valid || valid[i]);
}

/* counts[y] = candidates of row y. */
__global__ void __launch_bounds__(256)
    topn_count_kernel(const unsigned char *__restrict__ mask,
                      const unsigned char *__restrict__ valid, int w,
                      int *__restrict__ counts)
{
    __shared__ int red[4];
    const int y = blockIdx.x, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int c = 0;

    for (int x = threadIdx.x; x < w; x += 256)
        c += topn_cand(mask, valid, (long long)y * w + x) ? 1 : 0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        c += __shfl_xor(c, o);
    if (lane == 0)
        red[wv] = c;
    __syncthreads();
    if (threadIdx.x == 0)
        counts[y] = red[0] + red[1] + red[2] + red[3];
}

/* Exclusive scan of the h row counts into offs, the total into offs[h];
 * one work-group, 1024 rows per round with a carry. */
__global__ void __launch_bounds__(1024)
    topn_scan_kernel(const int *__restrict__ counts, int h, int *__restrict__ offs)
{
    __shared__ int wsum[16];
    __shared__ int carry;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;

    if (tid == 0)
        carry = 0;
    __syncthreads();
    for (int r0 = 0; r0 < h; r0 += 1024) {
        const int v = r0 + tid < h ? counts[r0 + tid] : 0;
        int x = v;

#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(x, o);

            if (lane >= o)
                x += t;
        }
        if (lane == 63)
            wsum[wv] = x;
        __syncthreads();
        int before = carry;

        for (int q = 0; q < wv; q++)
            before += wsum[q];
        if (r0 + tid < h)
            offs[r0 + tid] = before + x - v;
        __syncthreads();
        if (tid == 1023)
            carry = before + x;
        __syncthreads();
    }
    if (tid == 0)
        offs[h] = carry;
}

/* The candidates of row y at offs[y] on, x increasing: heat value and
 * cell index y * w + x. */
__global__ void __launch_bounds__(256)
    topn_write_kernel(const unsigned char *__restrict__ mask,
                      const unsigned char *__restrict__ valid,
                      const float *__restrict__ heat, int W, int w,
                      const int *__restrict__ offs, float *__restrict__ cval,
                      int *__restrict__ ccell)
{
    __shared__ int wcnt[4];
    const int y = blockIdx.x, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int base = offs[y];

    for (int x0 = 0; x0 < w; x0 += 256) {
        const int x = x0 + threadIdx.x;
        const bool f = x < w && topn_cand(mask, valid, (long long)y * w + x);
        const unsigned long long b = __ballot(f);
        const int rank = __popcll(b & ((1ull << lane) - 1));

        if (lane == 0)
            wcnt[wv] = __popcll(b);
        __syncthreads();
        int pos = base + rank;

        for (int q = 0; q < wv; q++)
            pos += wcnt[q];
        if (f) {
            cval[pos] = heat[(long long)y * W + x];
            ccell[pos] = y * w + x;
        }
        base += wcnt[0] + wcnt[1] + wcnt[2] + wcnt[3];
        __syncthreads();
    }
}

/* Radix select of the cut and compaction; one work-group of 1024. */
__global__ void __launch_bounds__(1024)
    topn_select_kernel(const float *__restrict__ cval, const int *__restrict__ ccell,
                       const int *__restrict__ offs, int h, int w, int n,
                       int *__restrict__ xy, float *__restrict__ score,
                       int *__restrict__ count)
{
    __shared__ unsigned hist[256];
    __shared__ unsigned sel[2]; /* prefix, remaining rank */
    __shared__ int wcnt[16];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int N = offs[h];
    unsigned prefix = 0, pmask = 0;

    if (N == 0) {
        if (tid == 0)
            *count = 0;
        return;
    }
    if (tid == 0) {
        sel[0] = 0;
        sel[1] = (unsigned)(N > n ? n + 1 : N); /* rank from the top, 1-based */
    }
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;

        if (tid < 256)
            hist[tid] = 0;
        __syncthreads();
        for (int i = tid; i < N; i += 1024) {
            const unsigned kk = topn_key(cval[i]);

            if ((kk & pmask) == prefix)
                atomicAdd(&hist[(kk >> shift) & 255], 1u);
        }
        __syncthreads();
        /* Wave 0 finds the digit holding the remaining rank, from the top
         * digit down: lane l sums digits 255 - 4 l .. 252 - 4 l, a suffix
         * scan over the lanes, then the lane that crosses the rank walks
         * its four digits. */
        if (wv == 0) {
            const unsigned k = sel[1];
            unsigned s4 = 0;

            for (int q = 0; q < 4; q++)
                s4 += hist[255 - 4 * lane - q];
            unsigned incl = s4;

#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const unsigned t = __shfl_up(incl, o);

                if (lane >= o)
                    incl += t;
            }
            const unsigned excl = incl - s4;

            if (excl < k && k <= incl) {
                unsigned acc = excl;

                for (int q = 0; q < 4; q++) {
                    const int d = 255 - 4 * lane - q;
                    const unsigned c = hist[d];

                    if (k <= acc + c) {
                        sel[0] = prefix | ((unsigned)d << shift);
                        sel[1] = k - acc;
                        break;
                    }
                    acc += c;
                }
            }
        }
        __syncthreads();
        prefix = sel[0];
        pmask |= 0xFFu << shift;
        __syncthreads();
    }
    /* prefix is the cut's key: back to the float. */
    const unsigned ck = prefix;
    const float cut = __uint_as_float((ck & 0x80000000u) ? (ck & 0x7FFFFFFFu) : ~ck);
    int base = 0;

    for (int i0 = 0; i0 < N; i0 += 1024) {
        const int i = i0 + tid;
        const bool f = i < N && cval[i] > cut;
        const unsigned long long b = __ballot(f);
        const int rank = __popcll(b & ((1ull << lane) - 1));

        if (lane == 0)
            wcnt[wv] = __popcll(b);
        __syncthreads();
        int pos = base + rank;

        for (int q = 0; q < wv; q++)
            pos += wcnt[q];
        if (f && pos < n) {
            const int cell = ccell[i];

            xy[2 * pos] = cell % w;
            xy[2 * pos + 1] = cell / w;
            score[pos] = cval[i];
        }
        for (int q = 0; q < 16; q++)
            base += wcnt[q];
        __syncthreads();
    }
    if (tid == 0)
        *count = base < n ? base : n;
}

extern "C" size_t disk_topn_work_bytes(int h, int w)
{
    const size_t rows = (size_t)(h > 0 ? h : 0), cells = rows * (size_t)(w > 0 ? w : 0);

    return ((2 * rows + 1) * sizeof(int) + 255) / 256 * 256 + cells * 8;
}

extern "C" void disk_topn(struct ops *o, cl_mem heat, long off, int W, int h, int w,
                          cl_mem mask, cl_mem valid, int n, cl_mem xy, cl_mem score,
                          cl_mem count, cl_mem work)
{
    ICOREG_API_BEGIN
    const char *op = "disk_topn";
    hipStream_t st = stream_of(o->ocl);

    if (h < 0 || w < 0 || W < w || off < 0 || n < 0)
        icoreg_fatal("%s: invalid sizes h=%d w=%d W=%d n=%d", op, h, w, W, n);
    count32((long long)h * w, op);
    need_bytes(count, 0, 4, op, "count");
    if ((long long)h * w == 0 || n == 0) {
        hipLaunchKernelGGL(fill_int_kernel, dim3(1), dim3(64), 0, st, (int *)count->ptr, 1, 0);
        launch_check(op);
        return;
    }
    need_floats(heat, off, (long long)(h - 1) * W + w, op, "heat");
    need_bytes(mask, 0, (long long)h * w, op, "mask");
    if (valid)
        need_bytes(valid, 0, (long long)h * w, op, "valid");
    need_bytes(xy, 0, 8LL * n, op, "xy");
    need_floats(score, 0, n, op, "score");
    need_bytes(work, 0, (long long)disk_topn_work_bytes(h, w), op, "work");
    {
        int *counts = (int *)work->ptr, *offs = counts + h;
        char *cand = (char *)work->ptr + ((2 * (size_t)h + 1) * sizeof(int) + 255) / 256 * 256;
        float *cval = (float *)cand;
        int *ccell = (int *)(cand + (size_t)h * w * 4);
        const unsigned char *vm = valid ? (const unsigned char *)valid->ptr : nullptr;
        const unsigned char *mk = (const unsigned char *)mask->ptr;

        prof_scope ps(o->ocl, op);
        hipLaunchKernelGGL(topn_count_kernel, dim3((unsigned)h), dim3(256), 0, st, mk, vm, w,
                           counts);
        hipLaunchKernelGGL(topn_scan_kernel, dim3(1), dim3(1024), 0, st, (const int *)counts,
                           h, offs);
        hipLaunchKernelGGL(topn_write_kernel, dim3((unsigned)h), dim3(256), 0, st, mk, vm,
                           cfptr(heat) + off, W, w, (const int *)offs, cval, ccell);
        hipLaunchKernelGGL(topn_select_kernel, dim3(1), dim3(1024), 0, st,
                           (const float *)cval, (const int *)ccell, (const int *)offs, h, w,
                           n, (int *)xy->ptr, fptr(score), (int *)count->ptr);
    }
    launch_check(op);
    ICOREG_API_END
}

/* SPDX-License-Identifier: Unlicense */

/* Internal helpers of the HIP library: the fatal-error guard of public
 * entry points, HIP status checks, host-side bounds checks of kernel
 * accesses, and per-name launch timing. */

#ifndef ICOREG_COMMON_H
#define ICOREG_COMMON_H

#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>

#include "hip_backend.h"
#include "ops.h"

namespace icoreg {

/* Thrown by icoreg_fatal in ICOREG_FATAL_RECORD mode, caught by the
 * outermost ICOREG_API_BEGIN/END of a public call. */
struct fatal_error : std::runtime_error {
    explicit fatal_error(const std::string &m) : std::runtime_error(m) {}
};

/* Depth of public calls on this thread, so that only the outermost one
 * swallows a fatal error (drivers call public ops internally). */
struct api_depth {
    api_depth();
    ~api_depth();
    bool outermost() const;
};

void record_error(const char *msg);

/* Fatal unless e == hipSuccess. */
void hip_check(hipError_t e, const char *what);

/* Fatal if [off, off + n) floats do not fit in buffer b (NULL b with
 * n > 0 is fatal too). what names the operation and the operand. */
void need_floats(cl_mem b, long long off, long long n, const char *op,
                 const char *operand);
/* Same in bytes. */
void need_bytes(cl_mem b, long long off, long long n, const char *op,
                const char *operand);
/* Element counts handed to kernels as int (ops.c:79-84). */
int count32(long long n, const char *what);

inline float *fptr(cl_mem b) { return b ? (float *)b->ptr : nullptr; }
inline const float *cfptr(cl_mem b) { return b ? (const float *)b->ptr : nullptr; }

/* Launch timing when ocl->profile is set: begin records a start event,
 * end a stop event, synchronises, and adds the time under name. */
struct prof_scope {
    prof_scope(struct ocl_backend *ocl, const char *name);
    ~prof_scope();
    struct ocl_backend *ocl;
    const char *name;
    hipEvent_t e0, e1;
};

inline hipStream_t stream_of(struct ocl_backend *ocl)
{
    return (hipStream_t)ocl->stream;
}

/* Channels per thread of the bilinear sampling kernels (warp sampling,
 * grid_sample): 8, or 4 when that leaves fewer idle slots in the last
 * group of C channels. */
inline int sample_cg(int C) { return (C + 3) / 4 * 4 - C < (C + 7) / 8 * 8 - C ? 4 : 8; }

/* The backend's second stream (made on first use) and event i of its
 * pool (disable-timing events, made on first use, i < 4096). */
hipStream_t aux_stream_of(struct ocl_backend *ocl);
hipEvent_t aux_event(struct ocl_backend *ocl, int i);

/* Check the launch just queued (launch-configuration errors). */
void launch_check(const char *what);

/* The ops work buffer (struct ops.scratch), grown to at least bytes.
 * Growing synchronises the stream first (the old buffer may be in use). */
cl_mem scratch_get(struct ops *o, size_t bytes);

} // namespace icoreg

#define ICOREG_API_BEGIN                                                       \
    icoreg::api_depth icoreg_depth_;                                           \
    try {
#define ICOREG_API_END                                                         \
    }                                                                          \
    catch (const icoreg::fatal_error &e)                                       \
    {                                                                          \
        if (!icoreg_depth_.outermost())                                        \
            throw;                                                             \
    }

#define ICOREG_API_END_RET(v)                                                  \
    }                                                                          \
    catch (const icoreg::fatal_error &e)                                       \
    {                                                                          \
        if (!icoreg_depth_.outermost())                                        \
            throw;                                                             \
    }                                                                          \
    return v;

#endif /* ICOREG_COMMON_H */

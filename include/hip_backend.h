/* SPDX-License-Identifier: Unlicense */

/* Device backend of the matcher tensor path on one AMD Instinct MI355X
 * (gfx950) through the HIP runtime: one device, one in-order stream for
 * every launch, hipMalloc-resident buffers, blocking host transfers (and,
 * beside them, optional uploads on a copy stream: ocl_write_async).
 *
 * Drop-in for the OpenCL backend of i.coregistration.opencl
 * (ocl_backend.h:15-61): the identifiers its callers use are kept
 * (struct ocl_backend, ocl_init, ocl_alloc, ocl_write, ...), so that
 * ops.h and the model drivers keep their text. There is no OpenCL
 * runtime behind them and no fallback: a machine without a HIP device
 * fails in ocl_init with a message naming the call.
 *
 * cl_mem is a handle to a device buffer {device pointer, byte size};
 * the byte size lets every operation check its accesses on the host
 * before a launch (see ops.h). */

#ifndef ICOREG_HIP_BACKEND_H
#define ICOREG_HIP_BACKEND_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Scalar types of the reference's kernel arguments (cl_platform.h
 * names, fixed widths). */
typedef int32_t cl_int;
typedef uint32_t cl_uint;
typedef int64_t cl_long;
typedef uint64_t cl_ulong;
typedef float cl_float;

/* A device buffer: hipMalloc'd storage (owned) or a view of memory
 * owned by someone else (ocl_wrap). */
struct ocl_buf {
    void *ptr;
    size_t bytes;
    int owned;
};
typedef struct ocl_buf *cl_mem;

/* Replaces ocl_backend.h:15-27. platform/device/context/queue/program
 * have no HIP counterpart beyond the device ordinal and the stream. */
struct ocl_backend {
    int device;            /* HIP device ordinal. */
    void *stream;          /* hipStream_t, default priority. */
    char device_name[256]; /* e.g. "AMD Instinct MI355X". */
    char platform_name[256];
    cl_ulong max_alloc;  /* Largest single buffer accepted by ocl_alloc. */
    cl_ulong global_mem; /* Device memory in bytes. */
    int is_gpu;
    int profile; /* Per-launch timing (I_COREGISTRATION_OPENCL_PROFILE). */
    int cu_count;
    char arch[64]; /* gcnArchName, e.g. "gfx950:sramecc+:xnack-". */
    /* A second in-order stream (default priority) and a pool of events,
     * made on first use by operations that run independent work beside
     * the main stream and join it back before they return (the GP solve);
     * released by ocl_free. */
    void *aux_stream;
    void *aux_events;
    int aux_nevents;
    /* The copy stream of ocl_write_async (default priority), its ring of
     * OCL_COPY_TICKETS events and the number of copies queued on it, made
     * on first use; released by ocl_free. */
    void *copy_stream;
    void *copy_events;
    long long copy_tickets;
};

/* Select the device and create the stream. device_opt: "auto", "gpu"
 * or a device ordinal ("0", "1", ...); "cpu" is refused (no CPU
 * device on this path). platform_opt is accepted and ignored (one
 * runtime). Fatal if no HIP device is found or the device is not
 * gfx950. Replaces ocl_backend.h:36-37. */
void ocl_init(struct ocl_backend *ocl, const char *device_opt,
              const char *platform_opt);

/* No counterpart in the reference (the reference has no graphs): the
 * launches and device copies queued on the library's stream between
 * ocl_graph_begin and ocl_graph_end are recorded, not run, into a HIP
 * graph that ocl_graph_launch replays on the stream. Calls that allocate,
 * read, write or synchronise are errors while recording (run the work
 * once before recording, so that the ops work buffer has its size). The
 * graph holds the buffer addresses of the recording. */
void ocl_graph_begin(struct ocl_backend *ocl);
void *ocl_graph_end(struct ocl_backend *ocl);
void ocl_graph_launch(struct ocl_backend *ocl, void *graph);
void ocl_graph_free(void *graph);

/* Synchronize, destroy the stream, reset the struct. */
void ocl_free(struct ocl_backend *ocl);

/* Name of a HIP error code (hipGetErrorName). ocl_backend.h:42. */
const char *ocl_errstr(cl_int err);

/* Fatal unless err is hipSuccess, the message naming what.
 * ocl_backend.h:45. */
void ocl_check(cl_int err, const char *what);

/* Device buffer of n bytes (n = 0 gives 4 bytes), fatal above max_alloc
 * or on failure. ocl_backend.h:48. */
cl_mem ocl_alloc(struct ocl_backend *ocl, size_t n, const char *what);

/* Allocate and fill from host memory. ocl_backend.h:51-52. */
cl_mem ocl_upload(struct ocl_backend *ocl, const void *src, size_t n,
                  const char *what);

/* Blocking transfers of n bytes at byte offset off (ocl_backend.c:
 * 304-318): they return once the stream has completed them and every
 * launch queued before them. */
void ocl_write(struct ocl_backend *ocl, cl_mem dst, size_t off, const void *src,
               size_t n);
void ocl_read(struct ocl_backend *ocl, cl_mem src, size_t off, void *dst,
              size_t n);

/* No counterpart in the reference, whose tile loop writes each tile with
 * a blocking transfer and then computes it (main.c:796-809 through
 * matcher.run, ocl_backend.c:304-311): host-to-device copies that run
 * beside the library's stream, so that a caller can upload the next tile
 * while the current one computes (see eloftr_match_enqueue,
 * roma_coarse_device).
 *
 * ocl_host_alloc: n bytes of page-locked host memory (hipHostMalloc), the
 * kind of source a copy needs to overlap anything; ocl_host_free frees it.
 *
 * ocl_write_async: queue n bytes from src to dst at byte offset off on the
 * backend's copy stream and return the copy's ticket (>= 0). The copy
 * does not wait for launches already queued on the library's stream, so
 * dst's range must not be one they still read (upload into a second
 * buffer).
 *
 * ocl_write_join: launches queued on the library's stream after this call
 * see the copy's data (the stream waits on the device; the host does not
 * block).
 *
 * ocl_write_wait: the host blocks until the copy is done; src may then be
 * rewritten.
 *
 * A ticket stays valid while fewer than OCL_COPY_TICKETS later copies have
 * been queued; an older one is an error. All three are errors while a
 * graph is being recorded (ocl_graph_begin). */
#define OCL_COPY_TICKETS 64
void *ocl_host_alloc(struct ocl_backend *ocl, size_t n);
void ocl_host_free(void *p);
long long ocl_write_async(struct ocl_backend *ocl, cl_mem dst, size_t off, const void *src,
                          size_t n);
void ocl_write_join(struct ocl_backend *ocl, long long ticket);
void ocl_write_wait(struct ocl_backend *ocl, long long ticket);

/* Free a buffer and NULL the handle. ocl_backend.h:61. */
void ocl_release(cl_mem *m);

/* New entry points for the raw cl* calls of the reference's drivers
 * (clEnqueueCopyBuffer eloftr.c:399, roma.c:654, disk.c:202;
 * clEnqueueCopyBufferRect roma.c:668; clEnqueueFillBuffer roma.c:1262):
 * asynchronous on the stream, byte offsets and sizes, bounds-checked. */
void ocl_copy(struct ocl_backend *ocl, cl_mem src, size_t soff, cl_mem dst,
              size_t doff, size_t bytes);
/* rows x width bytes from src (row pitch spitch bytes, from soff) to dst
 * (row pitch dpitch bytes, from doff). */
void ocl_copy_rect(struct ocl_backend *ocl, cl_mem src, size_t soff,
                   size_t spitch, cl_mem dst, size_t doff, size_t dpitch,
                   size_t width, size_t rows);
/* Fill n floats from float offset off with value (a fill kernel, so the
 * call can sit inside a captured graph). */
void ocl_fill(struct ocl_backend *ocl, cl_mem buf, size_t off, size_t n,
              float value);
/* Same for 32-bit words given by their bit pattern (int -1: 0xffffffff). */
void ocl_fill_u32(struct ocl_backend *ocl, cl_mem buf, size_t off, size_t n,
                  uint32_t bits);
/* Wait for everything queued on the stream. */
void ocl_finish(struct ocl_backend *ocl);

/* A handle on memory owned elsewhere (for example a torch tensor's
 * storage): ocl_release frees the handle, not the memory. */
cl_mem ocl_wrap(void *ptr, size_t bytes);

/* ---- Error convention ------------------------------------------------
 * The reference's G_fatal_error ends the process with a message naming
 * the failed call (ocl_backend.c:80-85, ops.c:79-84). That is the
 * default here too (ICOREG_FATAL_EXIT). With ICOREG_FATAL_RECORD (for
 * bindings and tests), a fatal error instead abandons the outermost
 * public call it happened in, which returns normally; the message is
 * kept for icoreg_last_error() until icoreg_clear_error(). */
#define ICOREG_FATAL_EXIT 0
#define ICOREG_FATAL_RECORD 1
void icoreg_set_fatal_mode(int mode);
const char *icoreg_last_error(void);
void icoreg_clear_error(void);
/* Report a fatal error (printf format). Does not return. */
void icoreg_fatal(const char *fmt, ...)
#ifdef __GNUC__
    __attribute__((format(printf, 1, 2), noreturn))
#endif
    ;

/* ---- Timing ------------------------------------------------------------
 * HIP events on the backend's stream: ocl_event_record returns an event
 * index (0..1023, reused after ocl_event_reset), ocl_event_ms the time
 * between two recorded events once both completed. */
int ocl_event_record(struct ocl_backend *ocl);
float ocl_event_ms(struct ocl_backend *ocl, int ev0, int ev1);
void ocl_event_reset(struct ocl_backend *ocl);

/* Per-launch timing table (the reference's ops_run profiling, ops.c:
 * 25-67), filled when ocl->profile is set: 1 synchronises after every
 * launch (the reference's mode); 2 records event pairs on the stream
 * without synchronising and resolves them in icoreg_prof_flush, so that
 * a timed region is not disturbed. Entry i: name, total ms, launches;
 * icoreg_prof_entry returns 0 past the end. */
int icoreg_prof_entry(int i, const char **what, double *ms, long *calls);
int icoreg_prof_flush(void);
void icoreg_prof_reset(void);

#ifdef __cplusplus
}
#endif

#endif /* ICOREG_HIP_BACKEND_H */

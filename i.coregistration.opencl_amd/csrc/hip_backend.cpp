/* SPDX-License-Identifier: Unlicense */

/* HIP device backend: device selection, the stream, buffers, blocking
 * transfers, copies and fills, the fatal-error convention and launch
 * timing. Replaces ocl_backend.c of i.coregistration.opencl (device
 * selection :210-262, alloc :275-293, write/read :304-318, release
 * :331-337) for one HIP device. */

#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <string>

#include "common.h"
#include "hip_backend.h"

/* ---- fatal errors ----------------------------------------------------- */

static int fatal_mode = ICOREG_FATAL_EXIT;
static thread_local std::string last_error;
static thread_local int depth = 0;

namespace icoreg {

api_depth::api_depth() { depth++; }
api_depth::~api_depth() { depth--; }
bool api_depth::outermost() const { return depth == 1; }

void record_error(const char *msg) { last_error = msg; }

void hip_check(hipError_t e, const char *what)
{
    if (e != hipSuccess)
        icoreg_fatal("HIP: %s failed: %s (%d)", what, hipGetErrorName(e),
                     (int)e);
}

void need_bytes(cl_mem b, long long off, long long n, const char *op,
                const char *operand)
{
    if (n <= 0)
        return;
    if (!b || !b->ptr)
        icoreg_fatal("%s: %s is NULL but %lld bytes are accessed", op, operand,
                     n);
    if (off < 0 || (unsigned long long)(off + n) > b->bytes)
        icoreg_fatal("%s: %s accessed at bytes [%lld, %lld) of a %zu-byte "
                     "buffer",
                     op, operand, off, off + n, b->bytes);
}

void need_floats(cl_mem b, long long off, long long n, const char *op,
                 const char *operand)
{
    need_bytes(b, off * 4, n * 4, op, operand);
}

int count32(long long n, const char *what)
{
    if (n < 0 || n > 0x7fffffffLL)
        icoreg_fatal("HIP: %s of %lld elements exceeds 2^31", what, n);
    return (int)n;
}

void launch_check(const char *what)
{
    hipError_t e = hipGetLastError();

    if (e != hipSuccess)
        icoreg_fatal("HIP: launch of %s failed: %s (%d)", what,
                     hipGetErrorName(e), (int)e);
}

} // namespace icoreg

extern "C" void icoreg_set_fatal_mode(int mode) { fatal_mode = mode; }

extern "C" const char *icoreg_last_error(void) { return last_error.c_str(); }

extern "C" void icoreg_clear_error(void) { last_error.clear(); }

extern "C" void icoreg_fatal(const char *fmt, ...)
{
    char buf[1024];
    va_list ap;

    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (fatal_mode == ICOREG_FATAL_RECORD && depth > 0) {
        last_error = buf;
        throw icoreg::fatal_error(buf);
    }
    fprintf(stderr, "ERROR: %s\n", buf);
    fflush(stderr);
    exit(EXIT_FAILURE);
}

/* ---- profiling table (ops.c:25-67) ------------------------------------- */

static struct {
    const char *what;
    double ms;
    long calls;
} prof[64];
static int nprof;
static std::mutex prof_mu;

/* Asynchronous event pairs (profile mode 2): recorded around each launch
 * without synchronising, resolved by icoreg_prof_flush. */
#define NPAIRS 65536
static struct {
    hipEvent_t e0, e1;
    const char *what;
} pairs[NPAIRS];
static int npairs;

namespace icoreg {

void prof_add(const char *what, double ms)
{
    int i;

    std::lock_guard<std::mutex> lk(prof_mu);
    for (i = 0; i < nprof && strcmp(prof[i].what, what) != 0; i++)
        ;
    if (i == nprof && nprof < 64)
        prof[nprof++].what = what;
    if (i < 64) {
        prof[i].ms += ms;
        prof[i].calls++;
    }
}

prof_scope::prof_scope(struct ocl_backend *o, const char *n)
    : ocl(o), name(n), e0(nullptr), e1(nullptr)
{
    if (!ocl || !ocl->profile)
        return;
    if (ocl->profile == 2) {
        if (npairs >= NPAIRS)
            return;
        if (!pairs[npairs].e0) {
            hip_check(hipEventCreate(&pairs[npairs].e0), "hipEventCreate");
            hip_check(hipEventCreate(&pairs[npairs].e1), "hipEventCreate");
        }
        e0 = pairs[npairs].e0;
        e1 = pairs[npairs].e1;
        pairs[npairs].what = n;
        npairs++;
        hip_check(hipEventRecord(e0, stream_of(ocl)), "hipEventRecord");
        return;
    }
    hip_check(hipEventCreate(&e0), "hipEventCreate");
    hip_check(hipEventCreate(&e1), "hipEventCreate");
    hip_check(hipEventRecord(e0, stream_of(ocl)), "hipEventRecord");
}

prof_scope::~prof_scope()
{
    float ms = 0;

    if (!e0)
        return;
    if (ocl->profile == 2) {
        (void)hipEventRecord(e1, stream_of(ocl));
        return;
    }
    if (hipEventRecord(e1, stream_of(ocl)) != hipSuccess ||
        hipEventSynchronize(e1) != hipSuccess ||
        hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
        ms = 0;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    prof_add(name, ms);
}

} // namespace icoreg

extern "C" void ops_report(void)
{
    int i;

    for (i = 0; i < nprof; i++)
        fprintf(stderr, "%-24s %10.3f ms %8ld calls\n", prof[i].what,
                prof[i].ms, prof[i].calls);
}

/* Profile table access for bindings: entry i (name, total ms, calls);
 * returns 0 past the end. */
extern "C" int icoreg_prof_entry(int i, const char **what, double *ms,
                                 long *calls)
{
    if (i < 0 || i >= nprof)
        return 0;
    *what = prof[i].what;
    *ms = prof[i].ms;
    *calls = prof[i].calls;
    return 1;
}

extern "C" void icoreg_prof_reset(void)
{
    std::lock_guard<std::mutex> lk(prof_mu);
    nprof = 0;
    npairs = 0;
    memset(prof, 0, sizeof(prof));
}

/* Resolve the event pairs of profile mode 2 into the table (waits for
 * the last one); returns the number of launches resolved. */
extern "C" int icoreg_prof_flush(void)
{
    int n = npairs, i;

    for (i = 0; i < n; i++) {
        float ms = 0;

        if (hipEventSynchronize(pairs[i].e1) != hipSuccess ||
            hipEventElapsedTime(&ms, pairs[i].e0, pairs[i].e1) != hipSuccess)
            ms = 0;
        icoreg::prof_add(pairs[i].what, ms);
    }
    npairs = 0;
    return n;
}

/* ---- device selection -------------------------------------------------- */

extern "C" const char *ocl_errstr(cl_int err)
{
    return hipGetErrorName((hipError_t)err);
}

extern "C" void ocl_check(cl_int err, const char *what)
{
    ICOREG_API_BEGIN
    if (err != 0)
        icoreg_fatal("HIP: %s failed: %s (%d)", what, ocl_errstr(err), err);
    ICOREG_API_END
}

extern "C" void ocl_init(struct ocl_backend *ocl, const char *device_opt,
                         const char *platform_opt)
{
    ICOREG_API_BEGIN
    int n = 0, dev = 0;
    hipDeviceProp_t p;
    hipStream_t s;

    (void)platform_opt;
    memset(ocl, 0, sizeof(*ocl));
    if (device_opt && strcmp(device_opt, "cpu") == 0)
        icoreg_fatal("HIP: device <cpu> requested: this path runs on the "
                     "GPU only");
    if (device_opt && strcmp(device_opt, "auto") != 0 &&
        strcmp(device_opt, "gpu") != 0) {
        char *end;

        dev = (int)strtol(device_opt, &end, 10);
        if (*end || dev < 0)
            icoreg_fatal("Invalid device option <%s>", device_opt);
    }
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        icoreg_fatal("HIP: no usable GPU device found");
    if (dev >= n)
        icoreg_fatal("HIP: device %d requested, %d present", dev, n);
    icoreg::hip_check(hipSetDevice(dev), "hipSetDevice");
    icoreg::hip_check(hipGetDeviceProperties(&p, dev),
                      "hipGetDeviceProperties");
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        icoreg_fatal("HIP: device %d is %s; this library is built for gfx950 "
                     "(MI355X) only",
                     dev, p.gcnArchName);
    icoreg::hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking),
                      "hipStreamCreate");
    ocl->device = dev;
    ocl->stream = (void *)s;
    snprintf(ocl->device_name, sizeof(ocl->device_name), "%s", p.name);
    snprintf(ocl->platform_name, sizeof(ocl->platform_name), "HIP %d",
             HIP_VERSION);
    snprintf(ocl->arch, sizeof(ocl->arch), "%s", p.gcnArchName);
    ocl->global_mem = p.totalGlobalMem;
    ocl->max_alloc = p.totalGlobalMem;
    ocl->is_gpu = 1;
    ocl->cu_count = p.multiProcessorCount;
    ocl->profile = getenv("I_COREGISTRATION_OPENCL_PROFILE") != NULL;
    ICOREG_API_END
}

static void destroy_events(void);

#define AUX_MAXEV 4096

namespace icoreg {

hipStream_t aux_stream_of(struct ocl_backend *ocl)
{
    if (!ocl->aux_stream) {
        hipStream_t s;

        hip_check(hipSetDevice(ocl->device), "hipSetDevice");
        hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate (aux)");
        ocl->aux_stream = (void *)s;
    }
    return (hipStream_t)ocl->aux_stream;
}

hipEvent_t aux_event(struct ocl_backend *ocl, int i)
{
    if (i < 0 || i >= AUX_MAXEV)
        icoreg_fatal("aux_event: index %d (at most %d events)", i, AUX_MAXEV);
    if (i >= ocl->aux_nevents) {
        const int m = i + 1 > 2 * ocl->aux_nevents ? i + 1 : 2 * ocl->aux_nevents;
        const int nn = m < AUX_MAXEV ? m : AUX_MAXEV;
        hipEvent_t *ev = (hipEvent_t *)realloc(ocl->aux_events, nn * sizeof(hipEvent_t));

        if (!ev)
            icoreg_fatal("aux_event: out of host memory");
        ocl->aux_events = ev;
        for (int k = ocl->aux_nevents; k < nn; k++) {
            hip_check(hipEventCreateWithFlags(&ev[k], hipEventDisableTiming), "hipEventCreate");
            ocl->aux_nevents = k + 1;
        }
    }
    return ((hipEvent_t *)ocl->aux_events)[i];
}

} // namespace icoreg

extern "C" void ocl_free(struct ocl_backend *ocl)
{
    ICOREG_API_BEGIN
    if (ocl->stream) {
        (void)hipStreamSynchronize((hipStream_t)ocl->stream);
        if (ocl->aux_stream)
            (void)hipStreamSynchronize((hipStream_t)ocl->aux_stream);
        destroy_events();
        for (int k = 0; k < ocl->aux_nevents; k++)
            (void)hipEventDestroy(((hipEvent_t *)ocl->aux_events)[k]);
        free(ocl->aux_events);
        if (ocl->aux_stream)
            (void)hipStreamDestroy((hipStream_t)ocl->aux_stream);
        if (ocl->copy_stream) {
            (void)hipStreamSynchronize((hipStream_t)ocl->copy_stream);
            for (int k = 0; k < OCL_COPY_TICKETS; k++)
                (void)hipEventDestroy(((hipEvent_t *)ocl->copy_events)[k]);
            free(ocl->copy_events);
            (void)hipStreamDestroy((hipStream_t)ocl->copy_stream);
        }
        (void)hipStreamDestroy((hipStream_t)ocl->stream);
    }
    memset(ocl, 0, sizeof(*ocl));
    ICOREG_API_END
}

/* ---- buffers -------------------------------------------------------- */

extern "C" cl_mem ocl_alloc(struct ocl_backend *ocl, size_t n,
                            const char *what)
{
    cl_mem m = nullptr;
    ICOREG_API_BEGIN
    void *p = nullptr;
    hipError_t e;

    if (n == 0)
        n = 4;
    if (n > ocl->max_alloc)
        icoreg_fatal("HIP: buffer <%s> needs %lu MiB, more than the device "
                     "maximum allocation of %lu MiB (reduce batch= or "
                     "tile_size=)",
                     what, (unsigned long)(n >> 20),
                     (unsigned long)(ocl->max_alloc >> 20));
    e = hipMalloc(&p, n);
    if (e != hipSuccess)
        icoreg_fatal("HIP: allocating %lu MiB for <%s> failed: %s",
                     (unsigned long)(n >> 20), what, hipGetErrorName(e));
    m = (cl_mem)calloc(1, sizeof(*m));
    m->ptr = p;
    m->bytes = n;
    m->owned = 1;
    ICOREG_API_END_RET(m)
}

extern "C" cl_mem ocl_wrap(void *ptr, size_t bytes)
{
    cl_mem m = (cl_mem)calloc(1, sizeof(*m));

    m->ptr = ptr;
    m->bytes = bytes;
    m->owned = 0;
    return m;
}

extern "C" void ocl_write(struct ocl_backend *ocl, cl_mem dst, size_t off,
                          const void *src, size_t n)
{
    ICOREG_API_BEGIN
    if (n == 0)
        return;
    icoreg::need_bytes(dst, (long long)off, (long long)n, "ocl_write",
                       "destination");
    icoreg::hip_check(hipMemcpyAsync((char *)dst->ptr + off, src, n,
                                     hipMemcpyHostToDevice,
                                     icoreg::stream_of(ocl)),
                      "hipMemcpyAsync (write)");
    icoreg::hip_check(hipStreamSynchronize(icoreg::stream_of(ocl)),
                      "hipStreamSynchronize (write)");
    ICOREG_API_END
}

/* ---- copies beside the stream ----------------------------------------- */

namespace {

/* Fatal while the library's stream is being recorded into a graph: a
 * copy on another stream would not be part of it. */
void not_capturing(struct ocl_backend *ocl, const char *what)
{
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;

    icoreg::hip_check(hipStreamIsCapturing(icoreg::stream_of(ocl), &st), "hipStreamIsCapturing");
    if (st != hipStreamCaptureStatusNone)
        icoreg_fatal("%s: not allowed while a graph is being recorded", what);
}

hipEvent_t copy_event(struct ocl_backend *ocl, long long ticket, const char *what)
{
    if (ticket < 0 || ticket >= ocl->copy_tickets ||
        ticket < ocl->copy_tickets - OCL_COPY_TICKETS)
        icoreg_fatal("%s: ticket %lld is not one of the last %d copies (%lld queued)", what,
                     ticket, OCL_COPY_TICKETS, ocl->copy_tickets);
    return ((hipEvent_t *)ocl->copy_events)[ticket % OCL_COPY_TICKETS];
}

} // namespace

extern "C" void *ocl_host_alloc(struct ocl_backend *ocl, size_t n)
{
    void *p = nullptr;
    ICOREG_API_BEGIN
    icoreg::hip_check(hipSetDevice(ocl->device), "hipSetDevice");
    icoreg::hip_check(hipHostMalloc(&p, n ? n : 4, hipHostMallocDefault), "hipHostMalloc");
    ICOREG_API_END_RET(p)
}

extern "C" void ocl_host_free(void *p)
{
    if (p)
        (void)hipHostFree(p);
}

extern "C" long long ocl_write_async(struct ocl_backend *ocl, cl_mem dst, size_t off,
                                     const void *src, size_t n)
{
    long long t = -1;
    ICOREG_API_BEGIN
    not_capturing(ocl, "ocl_write_async");
    icoreg::need_bytes(dst, (long long)off, (long long)n, "ocl_write_async", "destination");
    if (!ocl->copy_stream) {
        hipStream_t cs;
        hipEvent_t *ev = (hipEvent_t *)calloc(OCL_COPY_TICKETS, sizeof(hipEvent_t));

        if (!ev)
            icoreg_fatal("ocl_write_async: out of host memory");
        icoreg::hip_check(hipSetDevice(ocl->device), "hipSetDevice");
        for (int k = 0; k < OCL_COPY_TICKETS; k++)
            icoreg::hip_check(hipEventCreateWithFlags(&ev[k], hipEventDisableTiming),
                              "hipEventCreate (copy)");
        icoreg::hip_check(hipStreamCreateWithFlags(&cs, hipStreamNonBlocking),
                          "hipStreamCreate (copy)");
        ocl->copy_events = ev;
        ocl->copy_stream = (void *)cs;
    }
    {
        hipStream_t cs = (hipStream_t)ocl->copy_stream;
        hipEvent_t ev = ((hipEvent_t *)ocl->copy_events)[ocl->copy_tickets % OCL_COPY_TICKETS];

        if (n)
            icoreg::hip_check(hipMemcpyAsync((char *)dst->ptr + off, src, n,
                                             hipMemcpyHostToDevice, cs),
                              "hipMemcpyAsync (write_async)");
        icoreg::hip_check(hipEventRecord(ev, cs), "hipEventRecord (write_async)");
        t = ocl->copy_tickets++;
    }
    ICOREG_API_END_RET(t)
}

extern "C" void ocl_write_join(struct ocl_backend *ocl, long long ticket)
{
    ICOREG_API_BEGIN
    not_capturing(ocl, "ocl_write_join");
    icoreg::hip_check(hipStreamWaitEvent(icoreg::stream_of(ocl),
                                         copy_event(ocl, ticket, "ocl_write_join"), 0),
                      "hipStreamWaitEvent (write_join)");
    ICOREG_API_END
}

extern "C" void ocl_write_wait(struct ocl_backend *ocl, long long ticket)
{
    ICOREG_API_BEGIN
    not_capturing(ocl, "ocl_write_wait");
    icoreg::hip_check(hipEventSynchronize(copy_event(ocl, ticket, "ocl_write_wait")),
                      "hipEventSynchronize (write_wait)");
    ICOREG_API_END
}

extern "C" cl_mem ocl_upload(struct ocl_backend *ocl, const void *src,
                             size_t n, const char *what)
{
    cl_mem m = nullptr;
    ICOREG_API_BEGIN
    m = ocl_alloc(ocl, n, what);
    ocl_write(ocl, m, 0, src, n);
    ICOREG_API_END_RET(m)
}

extern "C" void ocl_read(struct ocl_backend *ocl, cl_mem src, size_t off,
                         void *dst, size_t n)
{
    ICOREG_API_BEGIN
    if (n == 0)
        return;
    icoreg::need_bytes(src, (long long)off, (long long)n, "ocl_read",
                       "source");
    icoreg::hip_check(hipMemcpyAsync(dst, (char *)src->ptr + off, n,
                                     hipMemcpyDeviceToHost,
                                     icoreg::stream_of(ocl)),
                      "hipMemcpyAsync (read)");
    icoreg::hip_check(hipStreamSynchronize(icoreg::stream_of(ocl)),
                      "hipStreamSynchronize (read)");
    ICOREG_API_END
}

extern "C" void ocl_release(cl_mem *m)
{
    if (!m || !*m)
        return;
    if ((*m)->owned && (*m)->ptr)
        (void)hipFree((*m)->ptr);
    free(*m);
    *m = nullptr;
}

/* n 16-byte units from a to b, grid-stride. */
__global__ void __launch_bounds__(256)
    copy16_kernel(const uint4 *__restrict__ a, uint4 *__restrict__ b, long n)
{
    long i = (long)blockIdx.x * 256 + threadIdx.x;
    const long stride = (long)gridDim.x * 256;

    for (; i < n; i += stride)
        b[i] = a[i];
}

/* Device-to-device copies whose ends and size are 16-byte aligned go
 * through copy16_kernel (16-byte loads and stores, about 6.3 TB/s at
 * 24 MB on MI355X, where the runtime's copy reached 3.7); others through
 * hipMemcpyAsync. */
extern "C" void ocl_copy(struct ocl_backend *ocl, cl_mem src, size_t soff,
                         cl_mem dst, size_t doff, size_t bytes)
{
    ICOREG_API_BEGIN
    if (bytes == 0)
        return;
    icoreg::need_bytes(src, (long long)soff, (long long)bytes, "ocl_copy",
                       "source");
    icoreg::need_bytes(dst, (long long)doff, (long long)bytes, "ocl_copy",
                       "destination");
    icoreg::prof_scope ps(ocl, "copy");
    {
        const char *a = (const char *)src->ptr + soff;
        char *b = (char *)dst->ptr + doff;

        if ((((uintptr_t)a | (uintptr_t)b | bytes) & 15) == 0) {
            const long n = (long)(bytes / 16);
            const long blocks = (n + 255) / 256 < 8192 ? (n + 255) / 256 : 8192;

            hipLaunchKernelGGL(copy16_kernel, dim3((unsigned)blocks), dim3(256), 0,
                               icoreg::stream_of(ocl), (const uint4 *)a, (uint4 *)b, n);
            icoreg::launch_check("copy");
        }
        else
            icoreg::hip_check(hipMemcpyAsync(b, a, bytes, hipMemcpyDeviceToDevice,
                                             icoreg::stream_of(ocl)),
                              "hipMemcpyAsync (copy)");
    }
    ICOREG_API_END
}

extern "C" void ocl_copy_rect(struct ocl_backend *ocl, cl_mem src, size_t soff,
                              size_t spitch, cl_mem dst, size_t doff,
                              size_t dpitch, size_t width, size_t rows)
{
    ICOREG_API_BEGIN
    if (width == 0 || rows == 0)
        return;
    if (width > spitch || width > dpitch)
        icoreg_fatal("ocl_copy_rect: width %zu exceeds a pitch (%zu, %zu)",
                     width, spitch, dpitch);
    icoreg::need_bytes(src, (long long)soff,
                       (long long)((rows - 1) * spitch + width),
                       "ocl_copy_rect", "source");
    icoreg::need_bytes(dst, (long long)doff,
                       (long long)((rows - 1) * dpitch + width),
                       "ocl_copy_rect", "destination");
    icoreg::prof_scope ps(ocl, "copy_rect");
    icoreg::hip_check(hipMemcpy2DAsync((char *)dst->ptr + doff, dpitch,
                                       (const char *)src->ptr + soff, spitch,
                                       width, rows, hipMemcpyDeviceToDevice,
                                       icoreg::stream_of(ocl)),
                      "hipMemcpy2DAsync");
    ICOREG_API_END
}

__global__ void __launch_bounds__(256)
    fill_kernel(uint32_t *p, long n, uint32_t v)
{
    long i = (long)blockIdx.x * 256 + threadIdx.x;
    long stride = (long)gridDim.x * 256;

    for (; i < n; i += stride)
        p[i] = v;
}

extern "C" void ocl_fill_u32(struct ocl_backend *ocl, cl_mem buf, size_t off,
                             size_t n, uint32_t bits)
{
    ICOREG_API_BEGIN
    long blocks;

    if (n == 0)
        return;
    icoreg::need_bytes(buf, 4LL * (long long)off, 4LL * (long long)n,
                       "ocl_fill", "buffer");
    blocks = (long)((n + 255) / 256);
    if (blocks > 8192)
        blocks = 8192;
    icoreg::prof_scope ps(ocl, "fill");
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       icoreg::stream_of(ocl), (uint32_t *)buf->ptr + off,
                       (long)n, bits);
    icoreg::launch_check("fill");
    ICOREG_API_END
}

extern "C" void ocl_fill(struct ocl_backend *ocl, cl_mem buf, size_t off,
                         size_t n, float value)
{
    uint32_t bits;

    memcpy(&bits, &value, 4);
    ocl_fill_u32(ocl, buf, off, n, bits);
}

extern "C" void ocl_finish(struct ocl_backend *ocl)
{
    ICOREG_API_BEGIN
    icoreg::hip_check(hipStreamSynchronize(icoreg::stream_of(ocl)),
                      "hipStreamSynchronize");
    ICOREG_API_END
}

/* ---- graphs ----------------------------------------------------------- */

extern "C" void ocl_graph_begin(struct ocl_backend *ocl)
{
    ICOREG_API_BEGIN
    icoreg::hip_check(hipStreamBeginCapture(icoreg::stream_of(ocl),
                                            hipStreamCaptureModeThreadLocal),
                      "hipStreamBeginCapture");
    ICOREG_API_END
}

extern "C" void *ocl_graph_end(struct ocl_backend *ocl)
{
    hipGraphExec_t exec = nullptr;
    ICOREG_API_BEGIN
    hipGraph_t g = nullptr;

    icoreg::hip_check(hipStreamEndCapture(icoreg::stream_of(ocl), &g), "hipStreamEndCapture");
    {
        const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);

        (void)hipGraphDestroy(g);
        icoreg::hip_check(e, "hipGraphInstantiate");
    }
    ICOREG_API_END_RET((void *)exec)
}

extern "C" void ocl_graph_launch(struct ocl_backend *ocl, void *graph)
{
    ICOREG_API_BEGIN
    if (!graph)
        icoreg_fatal("ocl_graph_launch: no graph");
    icoreg::hip_check(hipGraphLaunch((hipGraphExec_t)graph, icoreg::stream_of(ocl)),
                      "hipGraphLaunch");
    ICOREG_API_END
}

extern "C" void ocl_graph_free(void *graph)
{
    if (graph)
        (void)hipGraphExecDestroy((hipGraphExec_t)graph);
}

/* ---- events ----------------------------------------------------------- */

#define NEVENTS 1024
static hipEvent_t events[NEVENTS];
static int nevents_used;

static void destroy_events(void)
{
    int i;

    for (i = 0; i < NEVENTS; i++)
        if (events[i]) {
            (void)hipEventDestroy(events[i]);
            events[i] = nullptr;
        }
    nevents_used = 0;
}

extern "C" int ocl_event_record(struct ocl_backend *ocl)
{
    int k = -1;
    ICOREG_API_BEGIN
    if (nevents_used >= NEVENTS)
        icoreg_fatal("ocl_event_record: more than %d events without "
                     "ocl_event_reset",
                     NEVENTS);
    k = nevents_used++;
    if (!events[k])
        icoreg::hip_check(hipEventCreate(&events[k]), "hipEventCreate");
    icoreg::hip_check(hipEventRecord(events[k], icoreg::stream_of(ocl)),
                      "hipEventRecord");
    ICOREG_API_END_RET(k)
}

extern "C" float ocl_event_ms(struct ocl_backend *ocl, int ev0, int ev1)
{
    float ms = -1.0f;
    ICOREG_API_BEGIN
    (void)ocl;
    if (ev0 < 0 || ev1 < 0 || ev0 >= nevents_used || ev1 >= nevents_used)
        icoreg_fatal("ocl_event_ms: events %d, %d not recorded", ev0, ev1);
    icoreg::hip_check(hipEventSynchronize(events[ev1]), "hipEventSynchronize");
    icoreg::hip_check(hipEventElapsedTime(&ms, events[ev0], events[ev1]),
                      "hipEventElapsedTime");
    ICOREG_API_END_RET(ms)
}

extern "C" void ocl_event_reset(struct ocl_backend *ocl)
{
    (void)ocl;
    nevents_used = 0;
}

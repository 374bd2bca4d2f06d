// Device management for the C host: device selection, allocations, copies, streams.
// Errors are reported as negative return codes with a per-thread message (sdy_last_error).
#include <cxxabi.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include "sdy_internal.h"
#include "sdy_shim.h"

static thread_local char g_err[512];
static int g_inited = 0;
static int g_n_cu = 0;
static size_t g_mem = 0;

extern "C" const char *sdy_last_error(void) { return g_err; }

extern "C" int sdy_fail(int rc, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return rc;
}

static int hip_fail(hipError_t e, const char *what) {
    return sdy_fail(-2, "%s: %s (%s)", what, hipGetErrorString(e), hipGetErrorName(e));
}

#define HIPCK(call, what)                                   \
    do {                                                    \
        hipError_t e_ = (call);                             \
        if (e_ != hipSuccess) return hip_fail(e_, what);    \
    } while (0)

thread_local const void *sdy_last_kernel_fn = nullptr;

// Demangled name of the kernel noted last by this thread (e.g. "void k_matvec_ring<14, 3, 8>(MvArgs)"),
// or "" when none: benchmarks label their roofline with the kernel the dispatch actually chose.
extern "C" const char *sdy_last_kernel(void) {
    static thread_local char name[256];
    name[0] = '\0';
    if (!sdy_last_kernel_fn) return name;
    const char *mangled = hipKernelNameRefByPtr(sdy_last_kernel_fn, nullptr);
    if (!mangled) return name;
    int status = -1;
    char *d = abi::__cxa_demangle(mangled, nullptr, nullptr, &status);
    snprintf(name, sizeof name, "%s", status == 0 && d ? d : mangled);
    free(d);
    return name;
}

extern "C" int sdy_check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, what);
    return 0;
}

// Raises the dynamic-LDS limit of kernel fn to `bytes` when *granted is below it (the limit counts
// dynamic bytes only; a kernel's static LDS comes on top, so the request is exact, not the maximum).
extern "C" int sdy_lds_limit(const void *fn, size_t bytes, size_t *granted) {
    if (bytes <= 64 * 1024 || bytes <= *granted) return 0;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return sdy_fail(-2, "dynamic LDS of %zu bytes refused: %s", bytes, hipGetErrorString(e));
    }
    *granted = bytes;
    return 0;
}

extern "C" int sdy_init(void) {
    if (g_inited) return 0;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n < 1)
        return sdy_fail(-3, "no HIP device available (%s): this library computes on an MI355X (gfx950) GPU",
                        e != hipSuccess ? hipGetErrorString(e) : "0 devices");
    HIPCK(hipSetDevice(0), "hipSetDevice");
    hipDeviceProp_t p;
    HIPCK(hipGetDeviceProperties(&p, 0), "hipGetDeviceProperties");
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return sdy_fail(-3, "device 0 is %s; the kernels are built for gfx950 only", p.gcnArchName);
    g_n_cu = p.multiProcessorCount;
    g_mem = p.totalGlobalMem;
    g_inited = 1;
    return sdy_attn_split_scratch_setup();
}

extern "C" int sdy_device_info(int *n_cu, size_t *mem_total) {
    int rc = sdy_init();
    if (rc) return rc;
    if (n_cu) *n_cu = g_n_cu;
    if (mem_total) *mem_total = g_mem;
    return 0;
}

extern "C" int sdy_mem_info(size_t *free_bytes, size_t *total_bytes) {
    int rc = sdy_init();
    if (rc) return rc;
    size_t f = 0, t = 0;
    HIPCK(hipMemGetInfo(&f, &t), "hipMemGetInfo");
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return 0;
}

extern "C" int sdy_malloc(void **p, size_t n) {
    int rc = sdy_init();
    if (rc) return rc;
    *p = nullptr;
    if (n == 0) n = 256;
    hipError_t e = hipMalloc(p, n);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return sdy_fail(SDY_ERR_ALLOC, "device allocation of %.1f MB failed: %s", n / 1e6, hipGetErrorString(e));
    }
    return 0;
}

extern "C" int sdy_free(void *p) {
    if (!p) return 0;
    HIPCK(hipFree(p), "hipFree");
    return 0;
}

extern "C" int sdy_host_alloc(void **p, size_t n) {
    int rc = sdy_init();
    if (rc) return rc;
    HIPCK(hipHostMalloc(p, n ? n : 64, hipHostMallocDefault), "hipHostMalloc");
    return 0;
}

extern "C" int sdy_host_alloc_mapped(void **host, void **dev, size_t n) {
    int rc = sdy_init();
    if (rc) return rc;
    *host = *dev = nullptr;
    // coarse-grained (non-coherent): the GPU may keep the lines in its caches, which suits weights
    // written once at load and then only read
    hipError_t e = hipHostMalloc(host, n ? n : 64, hipHostMallocMapped | hipHostMallocNonCoherent);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *host = nullptr;
        return sdy_fail(SDY_ERR_ALLOC, "pinned host allocation of %.1f MB failed: %s", n / 1e6, hipGetErrorString(e));
    }
    if ((e = hipHostGetDevicePointer(dev, *host, 0)) != hipSuccess) {
        (void)hipHostFree(*host);
        *host = *dev = nullptr;
        return sdy_fail(-2, "hipHostGetDevicePointer: %s", hipGetErrorString(e));
    }
    return 0;
}

extern "C" int sdy_host_free(void *p) {
    if (!p) return 0;
    HIPCK(hipHostFree(p), "hipHostFree");
    return 0;
}

extern "C" int sdy_h2d(void *dst, const void *src, size_t n, sdy_stream s) {
    if (!n) return 0;
    HIPCK(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, (hipStream_t)s), "copy to device");
    return 0;
}

extern "C" int sdy_d2h(void *dst, const void *src, size_t n, sdy_stream s) {
    if (!n) return 0;
    HIPCK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, (hipStream_t)s), "copy to host");
    return 0;
}

extern "C" int sdy_d2d(void *dst, const void *src, size_t n, sdy_stream s) {
    if (!n) return 0;
    HIPCK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, (hipStream_t)s), "device copy");
    return 0;
}

extern "C" int sdy_memset(void *p, int v, size_t n, sdy_stream s) {
    if (!n) return 0;
    HIPCK(hipMemsetAsync(p, v, n, (hipStream_t)s), "memset");
    return 0;
}

extern "C" int sdy_sync(sdy_stream s) {
    HIPCK(hipStreamSynchronize((hipStream_t)s), "stream synchronize");
    return 0;
}

extern "C" int sdy_stream_new(sdy_stream *s) {
    int rc = sdy_init();
    if (rc) return rc;
    hipStream_t st;
    HIPCK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hipStreamCreate");
    *s = (sdy_stream)st;
    return 0;
}

extern "C" int sdy_stream_free(sdy_stream s) {
    if (!s) return 0;
    HIPCK(hipStreamDestroy((hipStream_t)s), "hipStreamDestroy");
    return 0;
}

// ---- events (timing on a given stream)
extern "C" int sdy_event_new(void **ev) {
    int rc = sdy_init();
    if (rc) return rc;
    hipEvent_t e;
    HIPCK(hipEventCreate(&e), "hipEventCreate");
    *ev = (void *)e;
    return 0;
}

extern "C" int sdy_event_record(void *ev, sdy_stream s) {
    HIPCK(hipEventRecord((hipEvent_t)ev, (hipStream_t)s), "hipEventRecord");
    return 0;
}

extern "C" int sdy_event_elapsed(float *ms, void *e0, void *e1) {
    HIPCK(hipEventSynchronize((hipEvent_t)e1), "hipEventSynchronize");
    HIPCK(hipEventElapsedTime(ms, (hipEvent_t)e0, (hipEvent_t)e1), "hipEventElapsedTime");
    return 0;
}

extern "C" int sdy_event_free(void *ev) {
    if (!ev) return 0;
    HIPCK(hipEventDestroy((hipEvent_t)ev), "hipEventDestroy");
    return 0;
}

// ---- graphs: the kernels issued on a stream between begin and end are recorded once and
// replayed with one launch. Relaxed capture mode: other threads may keep using HIP meanwhile.
extern "C" int sdy_graph_begin(sdy_stream s) {
    HIPCK(hipStreamBeginCapture((hipStream_t)s, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
    return 0;
}

extern "C" int sdy_graph_end(sdy_stream s, void **exec) {
    hipGraph_t g = nullptr;
    HIPCK(hipStreamEndCapture((hipStream_t)s, &g), "hipStreamEndCapture");
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    *exec = (void *)ge;
    return 0;
}

// Ends a capture that failed part-way; the partial graph is discarded.
extern "C" void sdy_graph_abort(sdy_stream s) {
    hipGraph_t g = nullptr;
    if (hipStreamEndCapture((hipStream_t)s, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
    (void)hipGetLastError();
}

extern "C" int sdy_graph_launch(void *exec, sdy_stream s) {
    HIPCK(hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)s), "hipGraphLaunch");
    return 0;
}

extern "C" int sdy_graph_free(void *exec) {
    if (!exec) return 0;
    HIPCK(hipGraphExecDestroy((hipGraphExec_t)exec), "hipGraphExecDestroy");
    return 0;
}

// ---- HBM read-bandwidth probe: every byte of buf read once, as fast as a pure read stream goes:
// each workgroup reads a contiguous slice (n16 / grid 16-byte elements) with non-temporal 16-byte
// loads, 4 KiB per workgroup and load instruction, eight loads of a lane in flight before their data
// is used, over 8 workgroups of 256 threads per CU; the last workgroup also reads the remainder. A
// sweep of read patterns over 4 GiB on MI355X put this one (slices per workgroup: 7.0-7.2 TB/s) above
// the grid-strided form of the weight kernels (consecutive waves on consecutive KiB, every wave's
// loads in flight a grid apart: 5.9-6.8 TB/s by grid size). An XOR of the data is kept live so the
// loads are not removed.
typedef unsigned int membw_u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void k_membw_read(const membw_u32x4 *__restrict__ p, size_t n16, unsigned *sink) {
    constexpr int U = 8;
    const size_t per = n16 / gridDim.x, stride = blockDim.x;
    const membw_u32x4 *q = p + blockIdx.x * per;
    const size_t end = blockIdx.x + 1 == gridDim.x ? n16 - blockIdx.x * per : per;
    size_t i = threadIdx.x;
    unsigned acc = 0;
    for (; i + (U - 1) * stride < end; i += U * stride) {
        membw_u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = __builtin_nontemporal_load(q + i + u * stride);
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < end; i += stride) {
        const membw_u32x4 v = __builtin_nontemporal_load(q + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

// The same read stream grid-strided (consecutive waves on consecutive KiB, four loads of a lane in
// flight a grid apart) over 2 workgroups of 256 threads per CU: on buffers of a few hundred MB read
// back to back, where each launch's ramp and tail weigh more, the faster of the two.
__global__ __launch_bounds__(256) void k_membw_read_strided(const membw_u32x4 *__restrict__ p, size_t n16,
                                                            unsigned *sink) {
    constexpr int U = 4;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    unsigned acc = 0;
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        membw_u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const membw_u32x4 v = __builtin_nontemporal_load(p + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

extern "C" int sdy_membw_read_strided(const void *buf, size_t bytes, void *sink, sdy_stream s) {
    int rc = sdy_init();
    if (rc) return rc;
    hipLaunchKernelGGL(k_membw_read_strided, dim3((unsigned)(g_n_cu * 2)), dim3(256), 0, (hipStream_t)s,
                       (const membw_u32x4 *)buf, bytes / 16, (unsigned *)sink);
    return sdy_check_launch("membw_read_strided");
}

extern "C" int sdy_membw_read(const void *buf, size_t bytes, void *sink, sdy_stream s) {
    int rc = sdy_init();
    if (rc) return rc;
    hipLaunchKernelGGL(k_membw_read, dim3((unsigned)(g_n_cu * 8)), dim3(256), 0, (hipStream_t)s,
                       (const membw_u32x4 *)buf, bytes / 16, (unsigned *)sink);
    return sdy_check_launch("membw_read");
}

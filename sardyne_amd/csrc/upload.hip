// Pipelined weight upload: GGUF mapping -> pinned host slots -> device slots -> repacked planes.
//
// The reference reads its weights straight from the file mapping (csrc/gguf.c, csrc/model_llama.c:
// 321-406), with gguf_prefetch / moe_prefetch advising the kernel to read ahead (csrc/gguf.c:322-328,
// csrc/model_llama.c:710-721). Here every weight is copied once into HBM at load, through a ring of
// n_slots slots:
//   1. a pool of host threads copies the next rows of a tensor from the mapping into a free pinned
//      slot, after advising the kernel (POSIX_MADV_WILLNEED) to read the rows that follow;
//   2. the slot goes to its device slot by DMA on the copy stream;
//   3. the work stream waits for that copy and repacks the rows into the matrix's planes; an event
//      after the repack frees the slot.
// So the host copy of slot k + 1, the DMA of slot k and the repack of slot k - 1 overlap. The
// GEMM exactness checks of the uploaded rows are queued at sdy_uploader_finish, with their flags
// read back in one synchronisation.
#include <hip/hip_runtime.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <time.h>
#include <unistd.h>

#include <vector>

#include "sdy_internal.h"
#include "sdy_shim.h"

namespace {

constexpr int MAX_SLOTS = 8;
constexpr int MAX_THREADS = 32;

double now_s() {
    timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

struct CopyJob {
    uint8_t *dst;
    const uint8_t *src;
    size_t n;
};

void *copy_part(void *arg) {
    const CopyJob *j = static_cast<const CopyJob *>(arg);
    memcpy(j->dst, j->src, j->n);
    return nullptr;
}

// memcpy split over up to n_threads threads (the calling thread takes the first part)
void parallel_copy(uint8_t *dst, const uint8_t *src, size_t n, int n_threads) {
    const size_t min_part = size_t(1) << 20;
    int parts = n_threads;
    if ((size_t)parts * min_part > n) parts = (int)(n / min_part) > 0 ? (int)(n / min_part) : 1;
    if (parts <= 1) {
        memcpy(dst, src, n);
        return;
    }
    const size_t step = (n / parts + 4095) & ~size_t(4095);
    CopyJob jobs[MAX_THREADS];
    pthread_t th[MAX_THREADS];
    bool started[MAX_THREADS] = {};
    int np = 0;
    for (size_t off = 0; off < n && np < MAX_THREADS; off += step, np++) {
        jobs[np] = CopyJob{dst + off, src + off, off + step < n ? step : n - off};
        if (np > 0) started[np] = pthread_create(&th[np], nullptr, copy_part, &jobs[np]) == 0;
    }
    copy_part(&jobs[0]);
    for (int i = 1; i < np; i++) {
        if (started[i]) pthread_join(th[i], nullptr);
        else copy_part(&jobs[i]);  // thread creation failed: copy here
    }
}

// advise the kernel to read [p, p + n) of a file mapping ahead (page-aligned; errors ignored: a
// pointer that is not a mapping simply gets no advice)
void advise_ahead(const void *p, size_t n) {
    if (!n) return;
    const long page = sysconf(_SC_PAGESIZE);
    const uintptr_t a = (uintptr_t)p & ~(uintptr_t)(page - 1), e = (uintptr_t)p + n;
    posix_madvise((void *)a, e - a, POSIX_MADV_WILLNEED);
}

struct Check {
    sdy_mat *m;
    long r0, n;
};

}  // namespace

struct sdy_uploader {
    int n_slots = 0, n_threads = 1, next = 0;
    size_t slot_bytes = 0;
    void *host[MAX_SLOTS] = {};
    void *dev[MAX_SLOTS] = {};
    hipEvent_t copied[MAX_SLOTS] = {}, freed[MAX_SLOTS] = {};
    bool busy[MAX_SLOTS] = {};
    hipStream_t copy = nullptr;
    sdy_stream work = nullptr;
    std::vector<Check> checks;
    double bytes = 0, host_copy_s = 0, slot_wait_s = 0;
};

#define UPCK(expr, what)                                                                                  \
    do {                                                                                                  \
        hipError_t e_ = (expr);                                                                           \
        if (e_ != hipSuccess) return sdy_fail(-2, "upload: %s: %s", what, hipGetErrorString(e_));       \
    } while (0)

extern "C" int sdy_uploader_new(sdy_uploader **out, size_t slot_bytes, int n_slots, int n_threads, sdy_stream work) {
    *out = nullptr;
    if (n_slots < 2 || n_slots > MAX_SLOTS || slot_bytes < (size_t(1) << 20))
        return sdy_fail(-1, "uploader: %d slots of %zu bytes (2..%d slots of at least 1 MiB)", n_slots, slot_bytes,
                        MAX_SLOTS);
    sdy_uploader *u = new (std::nothrow) sdy_uploader();
    if (!u) return sdy_fail(-1, "uploader: out of memory");
    u->n_slots = n_slots;
    u->slot_bytes = slot_bytes;
    u->n_threads = n_threads < 1 ? 1 : n_threads > MAX_THREADS ? MAX_THREADS : n_threads;
    u->work = work;
    int rc = 0;
    if (hipStreamCreateWithFlags(&u->copy, hipStreamNonBlocking) != hipSuccess) rc = sdy_fail(-2, "uploader: stream");
    for (int k = 0; !rc && k < n_slots; k++) {
        if (hipHostMalloc(&u->host[k], slot_bytes, hipHostMallocDefault) != hipSuccess ||
            hipMalloc(&u->dev[k], slot_bytes) != hipSuccess ||
            hipEventCreateWithFlags(&u->copied[k], hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&u->freed[k], hipEventDisableTiming) != hipSuccess)
            rc = sdy_fail(-2, "uploader: slot %d of %zu bytes", k, slot_bytes);
    }
    if (rc) {
        sdy_uploader_free(u);
        return rc;
    }
    *out = u;
    return 0;
}

extern "C" int sdy_uploader_rows(sdy_uploader *u, sdy_mat *m, long r0, long n, long step, long grp, long gstride,
                                 const void *host_raw) {
    if (n < 0 || r0 < 0 || step < 1 || grp < 1 || gstride < 0) return sdy_fail(-1, "upload: bad row map");
    if (n == 0) return 0;
    const size_t row = sdy_raw_row_bytes(m->type, m->n_in);
    // rows per slot: whole groups when the map repeats per group, so each slot starts a group
    long per = (long)(u->slot_bytes / row);
    if (grp < n) per = per / grp * grp;
    if (per < 1)
        return sdy_fail(-1, "upload: %ld rows of %zu bytes (a group of the map) exceed the %zu-byte slot",
                        grp < n ? grp : 1, row, u->slot_bytes);
    const uint8_t *src = static_cast<const uint8_t *>(host_raw);
    for (long i0 = 0; i0 < n; i0 += per) {
        const long cnt = n - i0 < per ? n - i0 : per;
        const size_t bytes = (size_t)cnt * row;
        const int k = u->next;
        u->next = (k + 1) % u->n_slots;
        if (u->busy[k]) {  // the slot's previous repack must be done before its buffers are reused
            const double t0 = now_s();
            UPCK(hipEventSynchronize(u->freed[k]), "waiting for a slot");
            u->slot_wait_s += now_s() - t0;
        }
        if (i0 + cnt < n) advise_ahead(src + (size_t)(i0 + cnt) * row, (size_t)((n - i0 - cnt) < per ? n - i0 - cnt : per) * row);
        const double t0 = now_s();
        parallel_copy(static_cast<uint8_t *>(u->host[k]), src + (size_t)i0 * row, bytes, u->n_threads);
        u->host_copy_s += now_s() - t0;
        UPCK(hipMemcpyAsync(u->dev[k], u->host[k], bytes, hipMemcpyHostToDevice, u->copy), "copy to device");
        UPCK(hipEventRecord(u->copied[k], u->copy), "event");
        UPCK(hipStreamWaitEvent((hipStream_t)u->work, u->copied[k], 0), "stream wait");
        // the chunk's first destination row (i0 is a multiple of grp, or the map has one group)
        const long base = r0 + (i0 / grp) * gstride + (i0 % grp) * step;
        const int rc = sdy_mat_repack_async(m, base, cnt, step, grp, gstride, u->dev[k], u->work);
        if (rc) return rc;
        UPCK(hipEventRecord(u->freed[k], (hipStream_t)u->work), "event");
        u->busy[k] = true;
        u->bytes += (double)bytes;
    }
    if (m->gemm_ok) {
        const long span = r0 + ((n - 1) / grp) * gstride + (grp - 1 < n - 1 ? grp - 1 : n - 1) * step;
        u->checks.push_back(Check{m, r0, span - r0 + 1});
    }
    return 0;
}

extern "C" int sdy_uploader_finish(sdy_uploader *u) {
    if (!u) return 0;
    const size_t nc = u->checks.size();
    int *flags = nullptr, rc = 0;
    if (nc) {
        if ((rc = sdy_malloc((void **)&flags, nc * sizeof(int)))) return rc;
        rc = sdy_memset(flags, 0, nc * sizeof(int), u->work);
        for (size_t i = 0; !rc && i < nc; i++)
            rc = sdy_gemm_check_rows_async(u->checks[i].m, u->checks[i].r0, u->checks[i].n, flags + i, u->work);
    }
    std::vector<int> bad(nc ? nc : 1, 0);
    if (!rc && nc) rc = sdy_d2h(bad.data(), flags, nc * sizeof(int), u->work);
    if (!rc) rc = sdy_sync(u->work);
    if (flags) sdy_free(flags);
    if (rc) return rc;
    for (size_t i = 0; i < nc; i++)
        if (bad[i]) u->checks[i].m->gemm_ok = 2;
    u->checks.clear();
    for (int k = 0; k < u->n_slots; k++) u->busy[k] = false;
    return 0;
}

extern "C" void sdy_uploader_stats(const sdy_uploader *u, double *bytes, double *host_copy_s, double *slot_wait_s) {
    if (bytes) *bytes = u ? u->bytes : 0;
    if (host_copy_s) *host_copy_s = u ? u->host_copy_s : 0;
    if (slot_wait_s) *slot_wait_s = u ? u->slot_wait_s : 0;
}

extern "C" int sdy_uploader_free(sdy_uploader *u) {
    if (!u) return 0;
    int rc = 0;
    if (u->work) rc = sdy_uploader_finish(u);
    if (u->copy) hipStreamSynchronize(u->copy);
    for (int k = 0; k < MAX_SLOTS; k++) {
        if (u->host[k]) hipHostFree(u->host[k]);
        if (u->dev[k]) hipFree(u->dev[k]);
        if (u->copied[k]) hipEventDestroy(u->copied[k]);
        if (u->freed[k]) hipEventDestroy(u->freed[k]);
    }
    if (u->copy) hipStreamDestroy(u->copy);
    delete u;
    return rc;
}

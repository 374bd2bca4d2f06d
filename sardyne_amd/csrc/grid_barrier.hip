// Measurement of the synchronisation that a persistent decode kernel (one launch per layer or per
// step, workgroups owning fixed slices of every matrix) would pay at each of a layer's five
// dependent phases, against the kernel boundary it would replace. Not on the decode path: the
// benchmark's grid_barrier workload runs it.
//
// A co-resident grid (cooperative launch) runs `rounds` grid barriers. Before each one every
// workgroup stores 64 floats of the round's data; after it, it reads another workgroup's and counts
// the values that are not the ones stored (the check that the barrier publishes data across the
// eight XCDs, whose L2 caches are not coherent with each other). Barrier forms:
//   flat       one agent-scope arrival counter for the grid, polled by every workgroup; data with
//              agent-scope (sc1) stores and loads;
//   two_level  a counter per XCD (the XCD of a workgroup read from its XCC_ID hardware register),
//              the last arrival of each XCD adds to one grid counter and, once all XCDs have,
//              releases its XCD through a flag; data with sc1 stores and loads;
//   fenced     two_level with the memory model's release/acquire done by the XCD leaders alone:
//              members store their data plainly (it waits in their XCD's L2), the leader writes its
//              L2 back (agent-scope release fence) before the grid arrival and invalidates it
//              (acquire) after; members read with L1-bypassing loads.
// Optionally the other three waves of every workgroup stream a buffer meanwhile (non-temporal
// 16-byte loads, as the weight matvecs do): the barrier latency while HBM is busy, which is what a
// persistent kernel prefetching its next phase's weights across the barrier would see.
//
// Every wait polls at most SPIN times; a timeout raises an abort flag that ends every other wait,
// so the grid always drains.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "sardyne.h"
#include "sdy_device.h"
#include "sdy_internal.h"
#include "sdy_shim.h"

namespace {

typedef unsigned int gb_u32x4 __attribute__((ext_vector_type(4)));

struct BarCtl {
    unsigned census[8 * 32];  // workgroups per XCD (one 128-byte line each)
    unsigned xc[8 * 32];      // per-XCD arrival counters
    unsigned xf[8 * 32];      // per-XCD release flags (the round number)
    unsigned gc[32];          // grid counter (two-level) / census arrivals and rounds (flat)
    unsigned abort_[32];
    unsigned err[32];         // [0] timeouts, [1] mismatches
};

constexpr unsigned SPIN = 1u << 20;

SDY_DEV unsigned ld_ag(unsigned *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
SDY_DEV void st_ag(unsigned *p, unsigned v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
SDY_DEV unsigned add_ag(unsigned *p, unsigned v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
SDY_DEV void stf_ag(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
SDY_DEV float ldf_ag(float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// waits until *p >= v: agent-scope loads (RMW: an atomic add of a run-time zero, for the census,
// whose lines no local atomic has refreshed); false on timeout or abort
template <bool RMW>
SDY_DEV bool wait_ge(unsigned *p, unsigned v, BarCtl *c, unsigned zero) {
    for (unsigned i = 0; i < SPIN; i++) {
        const unsigned x = RMW ? add_ag(p, zero) : ld_ag(p);
        if ((int)(x - v) >= 0) return true;
        if ((i & 63) == 63 && ld_ag(c->abort_)) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    st_ag(c->abort_, 1);
    add_ag(c->err, 1);
    return false;
}

struct BarArgs {
    BarCtl *c;
    float *data;              // [2][grid][64]: the round's data, by round parity
    int rounds, mode;         // mode: SDY_BARRIER_FLAT, _TWO_LEVEL, _FENCED
    const gb_u32x4 *stream;   // buffer streamed by waves 1..3 (or null)
    long stream_n;            // its 16-byte elements
    int stream_passes;
    long long *ts;            // [rounds + 1] wall-clock stamps of workgroup 0
    unsigned long long *stream_end;  // latest wall-clock stamp at which a streaming wave finished
    unsigned *sink;
    unsigned zero;            // 0, unknown to the compiler
};

__global__ __launch_bounds__(256) void k_barrier_probe(BarArgs a) {
    BarCtl *c = a.c;
    const int G = (int)gridDim.x, bx = (int)blockIdx.x, wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
    __shared__ unsigned s_ok, s_cnt, s_nx;
    if (wave != 0) {
        if (!a.stream) return;
        const long nw = (long)G * 3, w = (long)bx * 3 + (wave - 1), per = a.stream_n / nw;
        const gb_u32x4 *p = a.stream + w * per;
        unsigned acc = 0;
        for (int pass = 0; pass < a.stream_passes; pass++)
            for (long i = lane; i < per; i += 64 * 8) {
                gb_u32x4 v[8];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const long k = i + j * 64 < per ? i + j * 64 : i;
                    v[j] = __builtin_nontemporal_load(p + k);
                }
#pragma unroll
                for (int j = 0; j < 8; j++) acc ^= v[j].x ^ v[j].w;
            }
        if (acc == 0x12345678u) a.sink[0] = acc;
        if (lane == 0) atomicMax(a.stream_end, (unsigned long long)wall_clock64());
        return;
    }
    const unsigned zero = __builtin_amdgcn_readfirstlane(a.zero);
    const unsigned xcc = __builtin_amdgcn_s_getreg((20) | (0 << 6) | ((16 - 1) << 11)) & 7u;  // HW_REG_XCC_ID
    // census: every workgroup counts itself on its XCD before it arrives, then reads all counts
    if (lane == 0) {
        add_ag(&c->census[xcc * 32], 1);
        add_ag(c->gc, 1);
        bool ok = wait_ge<true>(c->gc, (unsigned)G, c, zero);
        unsigned n = 0;
        for (int x = 0; x < 8; x++) n += add_ag(&c->census[x * 32], zero) ? 1u : 0u;
        s_cnt = add_ag(&c->census[xcc * 32], zero);
        s_nx = n;
        s_ok = ok;
    }
    __builtin_amdgcn_wave_barrier();
    if (!s_ok) return;
    const unsigned ncnt = s_cnt, nx = s_nx;
    if (bx == 0 && lane == 0) a.ts[0] = (long long)wall_clock64();
    for (int r = 1; r <= a.rounds; r++) {
        float *slot = a.data + ((size_t)(r & 1) * G + bx) * 64 + lane;
        const float val = (float)(r * 1000 + bx) + (float)lane * 0.001f;
        if (a.mode == SDY_BARRIER_FENCED) *slot = val;
        else stf_ag(slot, val);
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
        if (lane == 0) {
            bool ok;
            if (a.mode == SDY_BARRIER_FLAT) {
                add_ag(c->gc, 1);
                ok = wait_ge<false>(c->gc, (unsigned)G * (r + 1), c, zero);
            } else {
                const unsigned o = add_ag(&c->xc[xcc * 32], 1);
                if (o == ncnt * r - 1) {  // the XCD's last arrival
                    if (a.mode == SDY_BARRIER_FENCED) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
                    add_ag(c->gc, 1);
                    ok = wait_ge<false>(c->gc, (unsigned)G + nx * r, c, zero);
                    if (a.mode == SDY_BARRIER_FENCED) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                    st_ag(&c->xf[xcc * 32], (unsigned)r);
                } else {
                    ok = wait_ge<false>(&c->xf[xcc * 32], (unsigned)r, c, zero);
                }
            }
            s_ok = ok;
        }
        __builtin_amdgcn_wave_barrier();
        if (!s_ok) return;
        const int src = (bx + r * 37 + 1) % G;
        float *ps = a.data + ((size_t)(r & 1) * G + src) * 64 + lane;
        const float v = a.mode == SDY_BARRIER_FENCED
                            ? __hip_atomic_load(ps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                            : ldf_ag(ps);
        if (v != (float)(r * 1000 + src) + (float)lane * 0.001f) add_ag(c->err + 1, 1);
        // (the data is double-buffered by round parity: a writer of round r + 2 has passed barrier r + 1,
        // which every reader of round r reaches only after its read)
        __builtin_amdgcn_s_waitcnt(0);
        if (bx == 0 && lane == 0) a.ts[r] = (long long)wall_clock64();
    }
}

__global__ void k_empty_boundary() {}

}  // namespace

extern "C" int sdy_grid_barrier_probe(int n_wg, int rounds, int mode, int stream_mb, sdy_barrier_stats *out) {
    int rc = sdy_init();
    if (rc) return rc;
    if (!out || n_wg < 8 || rounds < 1 || rounds > 100000 || mode < SDY_BARRIER_FLAT || mode > SDY_BARRIER_FENCED ||
        stream_mb < 0 || stream_mb > 65536)
        return sdy_fail(-1, "grid_barrier_probe: bad arguments");
    int per_cu = 0, n_cu = 0, wclk = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)k_barrier_probe, 256, 0);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, 0);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&wclk, hipDeviceAttributeWallClockRate, 0);
    if (e != hipSuccess) return sdy_fail(-2, "grid_barrier_probe: %s", hipGetErrorString(e));
    if (n_wg > per_cu * n_cu)
        return sdy_fail(-1, "grid_barrier_probe: %d workgroups exceed the %d the GPU holds at once", n_wg, per_cu * n_cu);
    BarCtl *c = nullptr;
    float *data = nullptr;
    long long *ts = nullptr;
    unsigned *sink = nullptr;
    void *stream = nullptr;
    const size_t sbytes = (size_t)stream_mb << 20;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if ((rc = sdy_malloc((void **)&c, sizeof(BarCtl))) || (rc = sdy_malloc((void **)&data, (size_t)2 * n_wg * 64 * 4)) ||
        (rc = sdy_malloc((void **)&ts, ((size_t)rounds + 1) * 8)) || (rc = sdy_malloc((void **)&sink, 64)) ||
        (sbytes && (rc = sdy_malloc(&stream, sbytes))))
        goto done;
    if ((e = hipMemset(c, 0, sizeof(BarCtl))) != hipSuccess || (e = hipMemset(sink, 0, 64)) != hipSuccess ||
        (sbytes && (e = hipMemset(stream, 1, sbytes)) != hipSuccess) || (e = hipEventCreate(&e0)) != hipSuccess ||
        (e = hipEventCreate(&e1)) != hipSuccess) {
        rc = sdy_fail(-2, "grid_barrier_probe: %s", hipGetErrorString(e));
        goto done;
    }
    {
        BarArgs a{c, data, rounds, mode, (const gb_u32x4 *)stream, (long)(sbytes / 16), sbytes ? 4 : 0, ts,
                  (unsigned long long *)(sink + 2), sink, 0u};
        void *kp[] = {&a};
        SDY_NOTE_KERNEL(k_barrier_probe);
        if ((e = hipEventRecord(e0, 0)) != hipSuccess ||
            (e = hipLaunchCooperativeKernel((const void *)k_barrier_probe, dim3(n_wg), dim3(256), kp, 0, 0)) !=
                hipSuccess ||
            (e = hipEventRecord(e1, 0)) != hipSuccess || (e = hipEventSynchronize(e1)) != hipSuccess) {
            rc = sdy_fail(-2, "grid_barrier_probe: %s", hipGetErrorString(e));
            goto done;
        }
        float ms = 0.0f;
        BarCtl hc;
        std::vector<long long> h((size_t)rounds + 1);
        unsigned long long send = 0;
        if ((e = hipEventElapsedTime(&ms, e0, e1)) != hipSuccess ||
            (e = hipMemcpy(&hc, c, sizeof hc, hipMemcpyDeviceToHost)) != hipSuccess ||
            (e = hipMemcpy(h.data(), ts, h.size() * 8, hipMemcpyDeviceToHost)) != hipSuccess ||
            (e = hipMemcpy(&send, sink + 2, 8, hipMemcpyDeviceToHost)) != hipSuccess) {
            rc = sdy_fail(-2, "grid_barrier_probe: %s", hipGetErrorString(e));
            goto done;
        }
        out->timeouts = hc.err[0];
        out->mismatches = hc.err[1];
        out->kernel_ms = ms;
        out->rounds_done = 0;
        std::vector<double> d, ds;
        for (int r = 1; r <= rounds && !hc.err[0]; r++) {
            if (!h[r]) break;
            const double us = (double)(h[r] - h[r - 1]) * 1000.0 / wclk;
            d.push_back(us);
            if (sbytes && (unsigned long long)h[r] <= send) ds.push_back(us);
        }
        out->rounds_done = (int)d.size();
        auto median = [](std::vector<double> v) {
            if (v.empty()) return 0.0;
            std::sort(v.begin(), v.end());
            return v[v.size() / 2];
        };
        auto mean = [](const std::vector<double> &v) {
            double s = 0;
            for (double x : v) s += x;
            return v.empty() ? 0.0 : s / v.size();
        };
        out->us_median = (float)median(d);
        out->us_mean = (float)mean(d);
        out->us_mean_streaming = (float)mean(ds);
        out->rounds_streaming = (int)ds.size();
    }
done:
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    sdy_free(c);
    sdy_free(data);
    sdy_free(ts);
    sdy_free(sink);
    sdy_free(stream);
    return rc;
}

// The kernel boundary: n empty kernels back to back on one stream, recorded as a graph and replayed
// (as the decode step is), and issued eagerly; the mean time per kernel in each case.
extern "C" int sdy_kernel_boundary_us(int n, float *us_graph, float *us_eager) {
    int rc = sdy_init();
    if (rc) return rc;
    if (n < 1 || n > 100000 || !us_graph || !us_eager) return sdy_fail(-1, "kernel_boundary_us: bad arguments");
    hipStream_t st = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    void *exec = nullptr;
    float ms = 0.0f;
    hipError_t e = hipStreamCreate(&st);
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e != hipSuccess) {
        rc = sdy_fail(-2, "kernel_boundary_us: %s", hipGetErrorString(e));
        goto done;
    }
    if ((rc = sdy_graph_begin((sdy_stream)st))) goto done;
    for (int i = 0; i < n; i++) hipLaunchKernelGGL(k_empty_boundary, dim3(1), dim3(64), 0, st);
    if ((rc = sdy_graph_end((sdy_stream)st, &exec))) goto done;
    for (int rep = 0; rep < 3 && !rc; rep++) {  // the last of three replays
        if ((rc = sdy_graph_launch(exec, (sdy_stream)st))) break;
        if ((e = hipEventRecord(e0, st)) != hipSuccess || (rc = sdy_graph_launch(exec, (sdy_stream)st)) ||
            (e = hipEventRecord(e1, st)) != hipSuccess || (e = hipEventSynchronize(e1)) != hipSuccess ||
            (e = hipEventElapsedTime(&ms, e0, e1)) != hipSuccess)
            break;
    }
    if (!rc && e != hipSuccess) rc = sdy_fail(-2, "kernel_boundary_us: %s", hipGetErrorString(e));
    if (rc) goto done;
    *us_graph = ms * 1000.0f / n;
    if ((e = hipEventRecord(e0, st)) == hipSuccess) {
        for (int i = 0; i < n; i++) hipLaunchKernelGGL(k_empty_boundary, dim3(1), dim3(64), 0, st);
        e = hipEventRecord(e1, st);
    }
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e != hipSuccess) rc = sdy_fail(-2, "kernel_boundary_us: %s", hipGetErrorString(e));
    else *us_eager = ms * 1000.0f / n;
done:
    if (exec) sdy_graph_free(exec);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (st) (void)hipStreamDestroy(st);
    return rc;
}

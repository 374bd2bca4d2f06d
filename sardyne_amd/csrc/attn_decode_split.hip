// One-launch decode attention for one token, split over positions (within tolerance of the
// reference, not its bits).
//
// The reference's op_attention_head (csrc/ops.c:405-414) computes, per query head, the scores
// q.k_j / sqrt(head_dim) over every cached position j, one softmax over all of them, and the
// weighted sum of the V rows in position order. This kernel computes the same softmax-weighted sum
// as a split over chunks of CHUNK = 32 positions (the flash-decoding form):
//
//   workgroup (chunk c, kv head g), 256 threads:
//     - q/k RMSNorm (qwen3) and RoPE of the group's n_rep query heads, and of the new k when the
//       chunk holds the token's own position (that workgroup also writes the new K/V to the cache);
//     - the chunk's K and V rows staged in LDS, scores s = q.k * (1/sqrtf(head_dim)) per (head,
//       position), the chunk maximum m, e = exp(s - m), l = sum e and acc = sum e * v;
//     - (m, l, acc) stored as the chunk's partial;
//   the last workgroup of the group to finish (a counter per kv head; the partials are exchanged
//   with agent-scope atomic stores and loads) merges the chunks in ascending order: M = max m_c,
//   L = sum l_c exp(m_c - M),
//   out = sum acc_c exp(m_c - M) / L, and writes the Q8_K blocks of its heads' outputs.
//
// Every sum has a fixed order (no float atomics), so results are deterministic run to run. They
// differ from the reference's in rounding only (exp of chunk-relative scores, f32 partial sums);
// the engine's bit-exact path (k_attn_scores + k_attn_decode_softmax + k_attn_decode_wv) stays
// available for comparisons.
//
// sdy_attn_decode_split_noalloc is the same computation for callers that cannot allocate (code
// under graph capture, serving loops): its partials and counters live in this file's `scratch`
// array, a static device array every GPU the library runs on holds until the process ends.
#include "sdy_attn_dev.h"
#include "sdy_device.h"
#include "sdy_internal.h"
#include "sdy_ops.h"
#include "sdy_quant_dev.h"
#include "sdy_shim.h"

namespace {

constexpr int CHUNK = 32;    // positions per workgroup: one per lane of a half-wave
constexpr int MERGE_ROUND = 16;  // chunks whose partials the merge loads at a time
constexpr int MAX_REP = 16;  // query heads per kv head

struct SplitArgs {
    const float *q, *k, *v;          // the token's raw q [n_head][HD], k and v [n_kv_head][HD]
    const float *q_norm, *k_norm;    // per-head RMSNorm weights (qwen3) or null
    float eps;
    const float *rope_cos, *rope_sin;
    const int32_t *step;             // step[1] = the token's position
    int n_head, n_kv_head, interleaved, n_chunk_max, max_seq;
    float *k_cache, *v_cache;        // [n_kv_head][max_seq][HD]
    long head_stride;                // max_seq * HD
    float *part;                     // [n_head][n_chunk_max][HD + 4]: m, l, -, -, acc[HD]
    unsigned *count;                 // [n_kv_head] arrivals, zero between launches
    float scale;                     // 1 / sqrtf(HD)
    float *out;                      // [n_head][HD]
    uint8_t *xq;                     // Q8_K blocks of out (or null)
};

// agent-scope relaxed float store / load: coherent across the XCDs without a fence
SDY_DEV void st_agent(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
SDY_DEV float ld_agent(const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

template <int HD>
__global__ __launch_bounds__(256) void k_attn_decode_split(SplitArgs a) {
    constexpr int KS = HD + 4;       // K rows in LDS: 16-byte aligned, consecutive rows on other banks
    constexpr int L4 = HD / 4;       // float4 per row
    constexpr int HPP = 256 / L4;    // heads per pass of the weighted sum (thread = head, float4 of dims)
    extern __shared__ __align__(16) float sm[];
    float *ks = sm;                          // [CHUNK][KS]
    float *vs = ks + CHUNK * KS;             // [CHUNK][HD]
    float *qs = vs + CHUNK * HD;             // [n_rep][HD]
    float *ps = qs + MAX_REP * HD;           // [n_rep][CHUNK]
    float *mls = ps + MAX_REP * CHUNK;       // [n_rep][2]: m, l
    __shared__ int s_last;

    const int c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n_rep = a.n_head / a.n_kv_head;
    const int pos = a.step[1];
    // a position outside the cache: every workgroup returns before it writes or counts anything
    // (the output is left as it was, the counters stay at zero for the next call)
    if (pos < 0 || pos >= a.max_seq) return;
    const int n_kv = pos + 1, n_chunk = (n_kv + CHUNK - 1) / CHUNK;
    if (c >= n_chunk) return;  // beyond the token's position: no work, not counted
    const int p0 = c * CHUNK, np = min(CHUNK, n_kv - p0);
    const bool own = p0 + np == n_kv;  // this chunk holds the token's own position (the last row)
    const int n_cached = own ? np - 1 : np;

    // K and V rows of the cached positions, all loads issued before any use
    const float4 *kc = reinterpret_cast<const float4 *>(a.k_cache + g * a.head_stride + (size_t)p0 * HD);
    const float4 *vc = reinterpret_cast<const float4 *>(a.v_cache + g * a.head_stride + (size_t)p0 * HD);
    constexpr int PER = CHUNK * L4 / 256;  // float4 of K (and of V) per thread
    float4 kr[PER], vr[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int f = tid + 256 * i, row = f / L4;
        if (row < n_cached) {
            kr[i] = kc[f];
            vr[i] = vc[f];
        }
    }
    // the group's query heads, and the new k / v when this chunk holds the token's position
    const float *cs = a.rope_cos + (size_t)pos * (HD / 2), *sn = a.rope_sin + (size_t)pos * (HD / 2);
    for (int r = wave; r < n_rep; r += 4) {
        const float *src = a.q + (size_t)(g * n_rep + r) * HD;
        for (int i = lane; i < HD; i += 64) qs[r * HD + i] = src[i];
        sdy_wave_sync();
        sdy_norm_rope<HD>(qs + r * HD, a.q_norm, a.eps, cs, sn, a.interleaved, lane);
    }
    if (own && wave == 3) {
        float *kn = ks + (np - 1) * KS;
        const float *ksrc = a.k + (size_t)g * HD, *vsrc = a.v + (size_t)g * HD;
        for (int i = lane; i < HD; i += 64) {
            kn[i] = ksrc[i];
            vs[(np - 1) * HD + i] = vsrc[i];
        }
        sdy_wave_sync();
        sdy_norm_rope<HD>(kn, a.k_norm, a.eps, cs, sn, a.interleaved, lane);
        float *kw = a.k_cache + g * a.head_stride + (size_t)pos * HD;
        float *vw = a.v_cache + g * a.head_stride + (size_t)pos * HD;
        for (int i = lane; i < HD; i += 64) {
            kw[i] = kn[i];
            vw[i] = vs[(np - 1) * HD + i];
        }
    }
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int f = tid + 256 * i, row = f / L4, col = f - row * L4;
        if (row < n_cached) {
            *reinterpret_cast<float4 *>(ks + row * KS + 4 * col) = kr[i];
            *reinterpret_cast<float4 *>(vs + row * HD + 4 * col) = vr[i];
        }
    }
    __syncthreads();

    // scores, chunk maximum and exponentials: each half-wave takes one head (wave w: heads 2w, 2w + 1,
    // then 2w + 8, ...), lane = position
    const int half = lane >> 5, j = lane & 31;
    for (int r0 = 2 * wave; r0 < n_rep; r0 += 8) {
        const int r = r0 + half;
        const bool on = r < n_rep;
        float s = -INFINITY;
        if (on && j < np) {
            const float4 *kp = reinterpret_cast<const float4 *>(ks + j * KS);
            const float4 *qp = reinterpret_cast<const float4 *>(qs + r * HD);
            float d0 = 0.f, d1 = 0.f, d2 = 0.f, d3 = 0.f;
#pragma unroll 8
            for (int i = 0; i < L4; i++) {
                const float4 kk = kp[i], qq = qp[i];
                d0 = fmaf(qq.x, kk.x, d0);
                d1 = fmaf(qq.y, kk.y, d1);
                d2 = fmaf(qq.z, kk.z, d2);
                d3 = fmaf(qq.w, kk.w, d3);
            }
            s = ((d0 + d1) + (d2 + d3)) * a.scale;
        }
        float m = s;
        for (int off = 16; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        const float e = on && j < np ? __expf(s - m) : 0.0f;
        float l = e;
        for (int off = 16; off >= 1; off >>= 1) l += __shfl_xor(l, off);
        if (on) {
            ps[r * CHUNK + j] = e;
            if (j == 0) {
                mls[2 * r] = m;
                mls[2 * r + 1] = l;
            }
        }
    }
    __syncthreads();

    // partial weighted V: thread = (head, float4 of dims), positions in order, eight positions'
    // LDS reads in flight at a time
    const int d4 = tid % L4;
    for (int r = tid / L4; r < n_rep; r += HPP) {
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        const float *pr = ps + r * CHUNK;
        const float *vcol = vs + 4 * d4;
        int j = 0;
        for (; j + 8 <= np; j += 8) {
            float p[8];
            float4 vv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                p[u] = pr[j + u];
                vv[u] = *reinterpret_cast<const float4 *>(vcol + (j + u) * HD);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                acc.x = fmaf(p[u], vv[u].x, acc.x);
                acc.y = fmaf(p[u], vv[u].y, acc.y);
                acc.z = fmaf(p[u], vv[u].z, acc.z);
                acc.w = fmaf(p[u], vv[u].w, acc.w);
            }
        }
        for (; j < np; j++) {
            const float p = pr[j];
            const float4 vv = *reinterpret_cast<const float4 *>(vcol + j * HD);
            acc.x = fmaf(p, vv.x, acc.x);
            acc.y = fmaf(p, vv.y, acc.y);
            acc.z = fmaf(p, vv.z, acc.z);
            acc.w = fmaf(p, vv.w, acc.w);
        }
        float *pp = a.part + ((size_t)(g * n_rep + r) * a.n_chunk_max + c) * (HD + 4);
        st_agent(pp + 4 + 4 * d4 + 0, acc.x);
        st_agent(pp + 4 + 4 * d4 + 1, acc.y);
        st_agent(pp + 4 + 4 * d4 + 2, acc.z);
        st_agent(pp + 4 + 4 * d4 + 3, acc.w);
        if (d4 == 0) {
            st_agent(pp, mls[2 * r]);
            st_agent(pp + 1, mls[2 * r + 1]);
        }
    }

    // hand-off: the group's last workgroup to arrive merges. The partials are written and read with
    // agent-scope accesses (sc1: past the non-coherent per-XCD L2s), and the arrival is an agent-scope
    // acquire-release increment by one thread after the workgroup's barrier: its release writes back
    // this XCD's L2 before the count moves (the workgroup's stores are ordered before it by the
    // barrier), and the last arrival's acquire invalidates its L2 before the merge reads the partials.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const unsigned done = __hip_atomic_fetch_add(a.count + g, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = done == (unsigned)(n_chunk - 1);
        if (s_last) __hip_atomic_store(a.count + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;

    // merge of the group's heads over its chunks, in ascending chunk order: rounds of MERGE_ROUND
    // chunks whose loads are all issued before use, folded with the running maximum
    // (M' = max(M, m_c), L and o rescaled by exp(M - M')); the result goes to LDS (qs, no longer
    // needed) for the Q8_K blocks and to out
    for (int r = tid / L4; r < n_rep; r += HPP) {
        const float *pb = a.part + (size_t)(g * n_rep + r) * a.n_chunk_max * (HD + 4);
        float M = -INFINITY, L = 0.f;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int c0 = 0; c0 < n_chunk; c0 += MERGE_ROUND) {
            float mv[MERGE_ROUND], lv[MERGE_ROUND];
            float4 av[MERGE_ROUND];
#pragma unroll
            for (int u = 0; u < MERGE_ROUND; u++) {
                const int cc = c0 + u < n_chunk ? c0 + u : c0;
                const float *pc = pb + cc * (HD + 4);
                mv[u] = ld_agent(pc);
                lv[u] = ld_agent(pc + 1);
                av[u] = make_float4(ld_agent(pc + 4 + 4 * d4), ld_agent(pc + 5 + 4 * d4), ld_agent(pc + 6 + 4 * d4),
                                    ld_agent(pc + 7 + 4 * d4));
            }
            float Mr = M;
#pragma unroll
            for (int u = 0; u < MERGE_ROUND; u++)
                if (c0 + u < n_chunk) Mr = fmaxf(Mr, mv[u]);
            const float sc = __expf(M - Mr);  // 0 on the first round (M = -inf)
            L *= sc;
            o.x *= sc;
            o.y *= sc;
            o.z *= sc;
            o.w *= sc;
#pragma unroll
            for (int u = 0; u < MERGE_ROUND; u++) {
                if (c0 + u >= n_chunk) break;
                const float w = __expf(mv[u] - Mr);
                L = fmaf(lv[u], w, L);
                o.x = fmaf(av[u].x, w, o.x);
                o.y = fmaf(av[u].y, w, o.y);
                o.z = fmaf(av[u].z, w, o.z);
                o.w = fmaf(av[u].w, w, o.w);
            }
            M = Mr;
        }
        const float inv = 1.0f / L;
        o.x *= inv;
        o.y *= inv;
        o.z *= inv;
        o.w *= inv;
        *reinterpret_cast<float4 *>(qs + r * HD + 4 * d4) = o;
        *reinterpret_cast<float4 *>(a.out + (size_t)(g * n_rep + r) * HD + 4 * d4) = o;
    }
    if (a.xq) {
        // the group's n_rep * HD outputs are whole Q8_K blocks (checked at launch): one per wave pass
        __syncthreads();
        const int n_blk = n_rep * HD / 256, blk0 = g * n_rep * HD / 256;
        for (int b = wave; b < n_blk; b += 4) {
            const float4 x4 = *reinterpret_cast<const float4 *>(qs + b * 256 + 4 * lane);
            const float xs[4] = {x4.x, x4.y, x4.z, x4.w};
            sdy_q8k_block(xs, lane, a.xq + (size_t)(blk0 + b) * 292);
        }
    }
}

size_t split_lds(int hd) {
    return sizeof(float) * ((size_t)CHUNK * (hd + 4) + (size_t)CHUNK * hd + (size_t)MAX_REP * hd +
                            (size_t)MAX_REP * CHUNK + 2 * MAX_REP);
}

template <int HD>
int launch_split(const SplitArgs &A, hipStream_t st) {
    static size_t granted = 0;
    const size_t lds = split_lds(HD);
    int rc = sdy_lds_limit((const void *)k_attn_decode_split<HD>, lds, &granted);
    if (rc) return rc;
    SDY_NOTE_KERNEL((k_attn_decode_split<HD>));
    hipLaunchKernelGGL((k_attn_decode_split<HD>), dim3(A.n_chunk_max, A.n_kv_head), dim3(256), lds, st, A);
    return sdy_check_launch("attn_decode_split");
}

__global__ void k_zero_u32(unsigned *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

}  // namespace

// The no-alloc entry point's scratch: partials of at most SCRATCH_PART_FLOATS floats (4 MiB), then
// SCRATCH_COUNTERS arrival counters. In host code the name is only a stand-in for the symbol: its
// device address on the current GPU comes from hipGetSymbolAddress (scratch_dev below).
constexpr size_t SCRATCH_PART_FLOATS = size_t(1) << 20;
constexpr int SCRATCH_COUNTERS = 256;
static __device__ __align__(256) float scratch[SCRATCH_PART_FLOATS + SCRATCH_COUNTERS];
constexpr int SCRATCH_MAX_DEVICES = 64;
static float *scratch_dev[SCRATCH_MAX_DEVICES];  // per device: the address of `scratch` there, once set up

// Looks up `scratch` on the current device (once per device) and clears its counters. Called by
// sdy_init for the device it selects, and by the no-alloc entry point's first call on another one.
extern "C" int sdy_attn_split_scratch_setup(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return sdy_fail(-2, "scratch setup: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= SCRATCH_MAX_DEVICES)
        return sdy_fail(-1, "scratch setup: device %d beyond the %d the table holds", dev, SCRATCH_MAX_DEVICES);
    if (scratch_dev[dev]) return 0;
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return sdy_fail(-2, "scratch setup: hipGetSymbolAddress: %s", hipGetErrorString(e));
    float *base = static_cast<float *>(p);
    hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(SCRATCH_COUNTERS), 0, 0,
                       reinterpret_cast<unsigned *>(base + SCRATCH_PART_FLOATS), SCRATCH_COUNTERS);
    if ((e = hipGetLastError()) != hipSuccess || (e = hipDeviceSynchronize()) != hipSuccess)
        return sdy_fail(-2, "scratch setup: clearing the counters: %s", hipGetErrorString(e));
    scratch_dev[dev] = base;
    return 0;
}

extern "C" int sdy_attn_decode_split_ok(int n_head, int n_kv_head, int hd) {
    return (hd == 64 || hd == 128) && n_kv_head >= 1 && n_head % n_kv_head == 0 && n_head / n_kv_head <= MAX_REP;
}

extern "C" size_t sdy_attn_decode_split_floats(int n_head, int hd, int max_seq) {
    return (size_t)n_head * ((max_seq + CHUNK - 1) / CHUNK) * (hd + 4);
}

extern "C" int sdy_attn_decode_split(const float *q, const float *k, const float *v, const float *q_norm,
                                     const float *k_norm, float eps, const float *rope_cos, const float *rope_sin,
                                     const int32_t *step_dev, int n_head, int n_kv_head, int hd, int interleaved,
                                     float *k_cache, float *v_cache, long head_stride, int max_seq, float *part,
                                     unsigned *count, float *out, void *xq_q8k, sdy_stream s) {
    if (!sdy_attn_decode_split_ok(n_head, n_kv_head, hd))
        return sdy_fail(-1, "attn_decode_split: head_dim %d with %d heads / %d kv heads not supported", hd, n_head,
                        n_kv_head);
    if (xq_q8k && (n_head / n_kv_head * hd) % 256)
        return sdy_fail(-1, "attn_decode_split: a kv group's %d outputs are not whole Q8_K blocks",
                        n_head / n_kv_head * hd);
    SplitArgs A = {};
    A.q = q;
    A.k = k;
    A.v = v;
    A.q_norm = q_norm;
    A.k_norm = k_norm;
    A.eps = eps;
    A.rope_cos = rope_cos;
    A.rope_sin = rope_sin;
    A.step = step_dev;
    A.n_head = n_head;
    A.n_kv_head = n_kv_head;
    A.interleaved = interleaved;
    A.n_chunk_max = (max_seq + CHUNK - 1) / CHUNK;
    A.max_seq = max_seq;
    A.k_cache = k_cache;
    A.v_cache = v_cache;
    A.head_stride = head_stride;
    A.part = part;
    A.count = count;
    A.scale = 1.0f / sqrtf((float)hd);
    A.out = out;
    A.xq = (uint8_t *)xq_q8k;
    return hd == 128 ? launch_split<128>(A, (hipStream_t)s) : launch_split<64>(A, (hipStream_t)s);
}

extern "C" int sdy_attn_decode_split_noalloc(const float *q, const float *k, const float *v, const float *q_norm,
                                             const float *k_norm, float eps, const float *rope_cos,
                                             const float *rope_sin, const int32_t *step_dev, int n_head, int n_kv_head,
                                             int hd, int interleaved, float *k_cache, float *v_cache, long head_stride,
                                             int max_seq, float *out, void *xq_q8k, sdy_stream s) {
    if (!sdy_attn_decode_split_ok(n_head, n_kv_head, hd))
        return sdy_fail(-1, "attn_decode_split_noalloc: head_dim %d with %d heads / %d kv heads not supported", hd,
                        n_head, n_kv_head);
    const size_t need = sdy_attn_decode_split_floats(n_head, hd, max_seq);
    if (need > SCRATCH_PART_FLOATS || n_kv_head > SCRATCH_COUNTERS)
        return sdy_fail(-1, "attn_decode_split_noalloc: %d heads x %d positions (head_dim %d) need %zu floats of "
                        "partials and %d counters, beyond the fixed scratch of %zu floats and %d counters",
                        n_head, max_seq, hd, need, n_kv_head, SCRATCH_PART_FLOATS, SCRATCH_COUNTERS);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SCRATCH_MAX_DEVICES)
        return sdy_fail(-1, "attn_decode_split_noalloc: no usable current device");
    if (!scratch_dev[dev]) {
        // the first call on a device that sdy_init did not select sets the scratch up, which launches
        // and waits on the null stream: not allowed while the caller's stream is being captured
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing((hipStream_t)s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
            return sdy_fail(-1, "attn_decode_split_noalloc: device %d is not set up and the stream is being "
                                "captured: call sdy_init with this device current (or this entry point once "
                                "outside capture) first", dev);
        const int rc = sdy_attn_split_scratch_setup();
        if (rc) return rc;
    }
    float *base = scratch_dev[dev];
    return sdy_attn_decode_split(q, k, v, q_norm, k_norm, eps, rope_cos, rope_sin, step_dev, n_head, n_kv_head, hd,
                                 interleaved, k_cache, v_cache, head_stride, max_seq, base,
                                 reinterpret_cast<unsigned *>(base + SCRATCH_PART_FLOATS), out, xq_q8k, s);
}

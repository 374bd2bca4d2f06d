// gfx950 kernels of the quantized-weight path: device weight layout (repack), dequantisation,
// activation quantisers and the decode / small-batch matvec.
//
// Device weight layout. Every quantized matrix is split into "planes" so that each lane of a
// wave64 reads its share of a row with one 16-byte load per plane and the 64 lanes of a load
// instruction cover 1 KiB of contiguous HBM. The unit of work is a 64-element slice of a row
// ("unit"; 4 units per 256-element K-quant super-block, 2 blocks per unit for the 32-element
// types). Plane p of a matrix is [n_rows][per-row bytes] and the byte count of all planes
// together equals the GGUF size (plus padding of odd 32-element blocks), so HBM traffic is the
// format's own bytes:
//
//   Q4_K  QA: qs[32j..32j+16) of sub-block pair j (16 B/unit)   QB: qs[32j+16..32j+32) (16 B/unit)
//         H : d, dmin, scales[12] as stored (16 B/super-block)
//   Q6_K  N0, N1: 32 bytes/unit of low nibbles; byte i holds element i (low) and i+32 (high)
//         HB: 16 bytes/unit; byte i holds the two high bits of elements i, i+16, i+32, i+48
//         SC: scales[16] as stored (16 B/super-block)   D: f16 d (2 B/super-block)
//         The six-bit values are the stored ones, only their bits are regrouped per unit.
//   Q8_0  Q0..Q3: the 64 int8 quants of blocks 2u, 2u+1 (16 B each)   D: both f16 scales (4 B/unit)
//   Q4_0  P0, P1: qs of blocks 2u, 2u+1   D: 4 B/unit
//   Q5_0  P0, P1: qs   QH: qh of both blocks (8 B/unit)   D: 4 B/unit
//
// Numerics (the reference's csrc/quant.c:191-235 and csrc/quant.h:84-91): integer parts of a
// super-block are exact int32 sums (v_dot4c_i32_i8 + quad reduction), and the fp32 combine
// acc + (yd*d*isum - yd*dmin*msum) runs in super-block order with contraction disabled, so the
// Q4_K / Q6_K matvec reproduces the reference's float result bit for bit. Q8_0/Q4_0/Q5_0 blocks
// contribute (float)isum*(dw*dx) as the reference's scalar kernel does; two blocks of a unit are
// summed first, then units in order (the reference's AVX2 order differs again; parity for these
// types is by tolerance).
#include "sdy_device.h"
#include "sdy_shim.h"
#include "sdy_internal.h"
#include "sdy_quant_dev.h"
#include "sdy_norm_dev.h"
#include "sdy_route_dev.h"

namespace {

constexpr int WAVES = 4;  // waves per workgroup of the matvec
constexpr int THREADS = 64 * WAVES;

struct Planes {
    const uint8_t *p[5];
    int n_in, T, nb;  // elements per row, units per row, 32/256-element blocks per row
};

SDY_DEV uint4 ld16(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }
SDY_DEV uint32_t ld4(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }
// Weight loads: every weight byte is read once per matvec, so full-line plane loads are issued
// non-temporal (streamed past the caches). Sub-line planes that neighbouring waves share (the
// Q6_K d plane: 32 bytes per iteration) keep normal loads so the line is fetched once.
typedef unsigned int sdy_u32x4 __attribute__((ext_vector_type(4)));
SDY_DEV uint4 ldw16(const uint8_t *p) {
    sdy_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const sdy_u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
SDY_DEV uint32_t ldw4(const uint8_t *p) { return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p)); }
SDY_DEV uint16_t ldw2(const uint8_t *p) { return *reinterpret_cast<const uint16_t *>(p); }

// ------------------------------------------------------------------------------------ repack

// Row map of an upload: source row i goes to destination row (i / grp) * gstride + (i % grp) * step
// of the planes in dst (step 2 interleaves two matrices; grp/gstride repeat that per expert).
struct RowMap {
    long step, grp, gstride;
};

// The destination planes' row-0 addresses, passed by value.
struct DstPlanes {
    uint8_t *p[5];
    SDY_DEV uint8_t *operator[](int i) const { return p[i]; }
};

// Whole-record stores of bytes assembled in registers (a matrix in host memory takes the stores over
// the host link, where single-byte writes would each be a transaction of their own).
template <int N>
SDY_DEV void st_bytes(uint8_t *dst, const uint8_t (&b)[N]) {
    uint32_t w[N / 4];
#pragma unroll
    for (int k = 0; k < N / 4; k++)
        w[k] = b[4 * k] | (uint32_t)b[4 * k + 1] << 8 | (uint32_t)b[4 * k + 2] << 16 | (uint32_t)b[4 * k + 3] << 24;
    if constexpr (N == 16) *reinterpret_cast<uint4 *>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
    else if constexpr (N == 8) *reinterpret_cast<uint2 *>(dst) = make_uint2(w[0], w[1]);
    else *reinterpret_cast<uint32_t *>(dst) = w[0];
}

template <int WT>
__global__ void k_repack(const uint8_t *__restrict__ src, size_t src_row, Planes P, DstPlanes dst, long n_rows,
                         RowMap map) {
    long gid = blockIdx.x * (long)blockDim.x + threadIdx.x;
    long srow = gid / P.T;
    int u = (int)(gid - srow * P.T);
    if (srow >= n_rows) return;
    const uint8_t *r = src + srow * src_row;
    const long row = (srow / map.grp) * map.gstride + (srow % map.grp) * map.step;
    if constexpr (WT == SDY_Q4_K) {
        int s = u >> 2, j = u & 3;
        const uint8_t *sb = r + 144 * s;
        uint8_t a[16], b[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            a[i] = sb[16 + 32 * j + i];
            b[i] = sb[16 + 32 * j + 16 + i];
        }
        st_bytes(dst[0] + (row * P.T + u) * 16, a);
        st_bytes(dst[1] + (row * P.T + u) * 16, b);
        if (j == 0) {
            uint8_t h[16];
#pragma unroll
            for (int i = 0; i < 16; i++) h[i] = sb[i];
            st_bytes(dst[2] + (row * P.nb + s) * 16, h);
        }
    } else if constexpr (WT == SDY_Q6_K) {
        int s = u >> 2, j = u & 3;
        const uint8_t *sb = r + 210 * s;
        // six-bit value of super-block element e (csrc/quant.c:62-75)
        auto lo4 = [&](int e) -> int {
            int half = e >> 7, ee = e & 127, l = ee & 31, k = ee >> 5;
            int b = sb[64 * half + l + ((k & 1) ? 32 : 0)];
            return (k >= 2) ? (b >> 4) : (b & 15);
        };
        auto hi2 = [&](int e) -> int {
            int half = e >> 7, ee = e & 127, l = ee & 31, k = ee >> 5;
            return (sb[128 + 32 * half + l] >> (2 * k)) & 3;
        };
        int base = 64 * j;
        uint8_t n0[16], n1[16], hb[16];
#pragma unroll
        for (int i = 0; i < 32; i++) {
            uint8_t v = (uint8_t)(lo4(base + i) | (lo4(base + i + 32) << 4));
            if (i < 16) n0[i] = v;
            else n1[i - 16] = v;
        }
#pragma unroll
        for (int i = 0; i < 16; i++) {
            int v = 0;
            for (int k = 0; k < 4; k++) v |= hi2(base + i + 16 * k) << (2 * k);
            hb[i] = (uint8_t)v;
        }
        st_bytes(dst[0] + (row * P.T + u) * 16, n0);
        st_bytes(dst[1] + (row * P.T + u) * 16, n1);
        st_bytes(dst[2] + (row * P.T + u) * 16, hb);
        if (j == 0) {
            uint8_t sc[16];
#pragma unroll
            for (int i = 0; i < 16; i++) sc[i] = sb[192 + i];
            st_bytes(dst[3] + (row * P.nb + s) * 16, sc);
            *reinterpret_cast<uint16_t *>(dst[4] + (row * P.nb + s) * 2) = (uint16_t)(sb[208] | sb[209] << 8);
        }
    } else {
        // 32-element types: blocks 2u and 2u+1 (the second may be absent when the row has an odd
        // number of blocks: zero quants and zero scale).
        constexpr int BB = WT == SDY_Q8_0 ? 34 : WT == SDY_Q4_0 ? 18 : 22;
        constexpr int QOFF = WT == SDY_Q8_0 ? 2 : WT == SDY_Q4_0 ? 2 : 6;
        uint8_t d[4];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            int b = 2 * u + h;
            bool ok = b < P.nb;
            const uint8_t *blk = r + (size_t)BB * (ok ? b : 0);
            d[2 * h] = ok ? blk[0] : 0;
            d[2 * h + 1] = ok ? blk[1] : 0;
            if constexpr (WT == SDY_Q8_0) {
                uint8_t q0[16], q1[16];
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    q0[i] = ok ? blk[QOFF + i] : 0;
                    q1[i] = ok ? blk[QOFF + 16 + i] : 0;
                }
                st_bytes(dst[2 * h] + (row * P.T + u) * 16, q0);
                st_bytes(dst[2 * h + 1] + (row * P.T + u) * 16, q1);
            } else {
                uint8_t q[16];
#pragma unroll
                for (int i = 0; i < 16; i++) q[i] = ok ? blk[QOFF + i] : 0;
                st_bytes(dst[h] + (row * P.T + u) * 16, q);
                if constexpr (WT == SDY_Q5_0) {
                    uint8_t qh[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) qh[i] = ok ? blk[2 + i] : 0;
                    st_bytes(dst[2] + (row * P.T + u) * 8 + 4 * h, qh);
                }
            }
        }
        st_bytes(dst[4] + (row * P.T + u) * 4, d);
    }
}

// ------------------------------------------------------------------------------------ dequant

// Six-bit scale (is_min = 0) or min (is_min = 1) of Q4_K sub-block k from the 12 scale bytes
// (csrc/quant.h:72-80).
SDY_DEV int q4k_scale(const uint8_t *s, int k, int is_min) {
    if (k < 4) return s[k + 4 * is_min] & 63;
    return is_min ? ((s[k + 4] >> 4) | ((s[k] >> 6) << 4)) : ((s[k + 4] & 15) | ((s[k - 4] >> 6) << 4));
}

template <int WT>
__global__ void k_dequant(Planes P, const int32_t *__restrict__ idx, long r0, long n, float *__restrict__ out) {
    long gid = blockIdx.x * (long)blockDim.x + threadIdx.x;
    long i = gid / P.T;
    int u = (int)(gid - i * P.T);
    if (i >= n) return;
    long row = idx ? (long)idx[i] : r0 + i;
    float *o = out + i * P.n_in + 64 * u;
    int n_el = P.n_in - 64 * u < 64 ? P.n_in - 64 * u : 64;
    if constexpr (WT == SDY_Q4_K) {
        int s = u >> 2, j = u & 3;
        uint8_t qa[16], qb[16], h[16];
        *reinterpret_cast<uint4 *>(qa) = ld16(P.p[0] + (row * P.T + u) * 16);
        *reinterpret_cast<uint4 *>(qb) = ld16(P.p[1] + (row * P.T + u) * 16);
        *reinterpret_cast<uint4 *>(h) = ld16(P.p[2] + (row * P.nb + s) * 16);
        float d = sdy_h2f((uint16_t)(h[0] | (h[1] << 8))), dmin = sdy_h2f((uint16_t)(h[2] | (h[3] << 8)));
        for (int half = 0; half < 2; half++) {
            int k = 2 * j + half;
            float d1 = d * (float)q4k_scale(h + 4, k, 0);
            float m1 = dmin * (float)q4k_scale(h + 4, k, 1);
            for (int l = 0; l < 32; l++) {
                int b = l < 16 ? qa[l] : qb[l - 16];
                int q = half ? (b >> 4) : (b & 15);
                float p = d1 * (float)q;
                o[32 * half + l] = p - m1;
            }
        }
    } else if constexpr (WT == SDY_Q6_K) {
        int s = u >> 2, j = u & 3;
        uint8_t nb8[32], hb[16];
        *reinterpret_cast<uint4 *>(nb8) = ld16(P.p[0] + (row * P.T + u) * 16);
        *reinterpret_cast<uint4 *>(nb8 + 16) = ld16(P.p[1] + (row * P.T + u) * 16);
        *reinterpret_cast<uint4 *>(hb) = ld16(P.p[2] + (row * P.T + u) * 16);
        const int8_t *sc = reinterpret_cast<const int8_t *>(P.p[3] + (row * P.nb + s) * 16);
        const uint8_t *dp = P.p[4] + (row * P.nb + s) * 2;
        float d = sdy_h2f((uint16_t)(dp[0] | (dp[1] << 8)));
        for (int e = 0; e < 64; e++) {
            int lo = e < 32 ? (nb8[e] & 15) : (nb8[e - 32] >> 4);
            int hi = (hb[e & 15] >> (2 * (e >> 4))) & 3;
            int v = (lo | (hi << 4)) - 32;
            float ds = d * (float)sc[4 * j + (e >> 4)];
            o[e] = ds * (float)v;
        }
    } else {
        const uint8_t *dd = P.p[4] + (row * P.T + u) * 4;
        for (int e = 0; e < n_el; e++) {
            int h = e >> 5, i = e & 31;
            float d = sdy_h2f((uint16_t)(dd[2 * h] | (dd[2 * h + 1] << 8)));
            int v;
            if constexpr (WT == SDY_Q8_0) {
                const uint8_t *q = P.p[2 * h + (i >> 4)] + (row * P.T + u) * 16;
                v = (int8_t)q[i & 15];
            } else {
                const uint8_t *q = P.p[h] + (row * P.T + u) * 16;
                int nib = i < 16 ? (q[i] & 15) : (q[i - 16] >> 4);
                if constexpr (WT == SDY_Q4_0) {
                    v = nib - 8;
                } else {
                    uint32_t qh = ld4(P.p[2] + (row * P.T + u) * 8 + 4 * h);
                    v = (nib | (int)(((qh >> i) & 1u) << 4)) - 16;
                }
            }
            o[e] = (float)v * d;
        }
    }
}

template <int WT>
__global__ void k_dequant_float(const uint8_t *__restrict__ w, int n_in, const int32_t *__restrict__ idx, long r0,
                                long n, float *__restrict__ out) {
    long gid = blockIdx.x * (long)blockDim.x + threadIdx.x;
    long i = gid / n_in;
    int e = (int)(gid - i * n_in);
    if (i >= n) return;
    long row = idx ? (long)idx[i] : r0 + i;
    float v;
    if constexpr (WT == SDY_F32) v = reinterpret_cast<const float *>(w)[row * n_in + e];
    else if constexpr (WT == SDY_F16) v = sdy_h2f(reinterpret_cast<const uint16_t *>(w)[row * n_in + e]);
    else v = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(w)[row * n_in + e] << 16);
    out[i * n_in + e] = v;
}

// ------------------------------------------------------------------------ activation quantisers

// Q8_K (csrc/quant.c:118-144): one wave per 256-element block (four blocks of a row per 256-thread
// workgroup), lane l holds elements 4l..4l+3. With e.y16 set, also the GEMM's expansion of the block.
__global__ __launch_bounds__(256) void k_quant_q8k(const float *__restrict__ x, uint8_t *__restrict__ out, int n_in,
                                                   SdyGemmExp e) {
    const int nb = n_in / 256, s = blockIdx.x * 4 + (threadIdx.x >> 6), t = blockIdx.y, l = threadIdx.x & 63;
    if (s >= nb) return;  // uniform per wave
    const float4 v = *reinterpret_cast<const float4 *>(x + (size_t)t * n_in + 256 * s + 4 * l);
    const float xs[4] = {v.x, v.y, v.z, v.w};
    const SdyQ8kLane r = sdy_q8k_lane(xs, l);
    uint8_t *ob = out + ((size_t)t * nb + s) * 292;
    *reinterpret_cast<uint32_t *>(ob + 4 + 4 * l) = r.packed;
    if ((l & 3) == 0) *reinterpret_cast<int16_t *>(ob + 260 + 2 * (l >> 2)) = (int16_t)r.gsum;
    if (l == 0) *reinterpret_cast<float *>(ob) = r.d;
    if (e.y16) e.put(r, l, (size_t)t * nb + s);
}

// Q8_0 (csrc/quant.c:98-108): one wave per two 32-element blocks, one element per lane.
__global__ void k_quant_q8_0(const float *__restrict__ x, uint8_t *__restrict__ out, int n_in) {
    const int nblk = n_in / 32, t = blockIdx.y, l = threadIdx.x & 31;
    const int b = 2 * blockIdx.x + (threadIdx.x >> 5);
    if (b >= nblk) return;  // uniform per half-wave
    sdy_q8_0_block(x[(size_t)t * n_in + 32 * b + l], l, out + ((size_t)t * nblk + b) * 34);
}

// ------------------------------------------------------------------------------------ matvec

// LDS layout of the staged activations of MT tokens (T units per row):
//   Y  [MT][4][T] x 16 B   y bytes of unit u, 16-byte chunk q (conflict-free ds_read_b128)
//   K-quants: BS [MT][T] x 8 B (bsums 4j..4j+3 of the unit)   YD [MT][nb] floats (Q8_K d)
//   32-element types: DX [MT][T] x 8 B (two f32 scales)   SY [MT][T] x 8 B (two int sums of y)
// followed by one term buffer per wave: [rb rows][MT tokens][nterm] floats.
//
// Work decomposition. Rows are cut into batches of rb rows; the (row, unit) tasks of a batch are
// spread over ceil(rb*T/64) wave iterations (64 lanes, one unit each; a last partial iteration
// leaves lanes idle). Each wave owns one contiguous, balanced range of batches and walks it as one
// flat sequence of iterations, loading the weights of the next iteration while it computes the
// current one, across batch boundaries. At the end of a batch the wave sums the terms of each
// (row, token) in block order (phase 2). rb is the smallest row count with at least 64 tasks, so
// small matrices still spread over every CU.
struct MvArgs {
    Planes P;
    const uint8_t *xq;
    int n_tok;
    float *out;
    long out_stride;
    const float *bias, *resid;
    long row0, row1;
    int rb;      // rows per batch
    int ipb;     // wave iterations per batch = ceil(rb * T / 64)
    int nterm;   // f32 terms per row and token (super-blocks or units)
    int q64, r64;  // 64 / T and 64 % T: advance of a lane's (row, unit) per iteration
    int swiglu;    // rows (2i, 2i+1) are (gate, up) of output i: out[i] = silu(gate) * up
    // Grouped one-token matvec (routed experts, k_matvec_rl with register activations only):
    // blockIdx.y is a slot whose rows are those of expert slot_expert[slot] in a stack of
    // n_slot_exp experts of slot_rows rows each; the slot's activation row starts xq_slot bytes and
    // its output out_slot floats after slot 0's. slot_expert == null: an ordinary matvec.
    const int32_t *slot_expert;
    long slot_rows;
    int n_slot_exp;
    long xq_slot, out_slot;
    // k_matvec_1t: rows per iteration 64/T, (lane * tmag) >> 16 == lane / T for lane < 64, and the
    // iteration count
    int rpi, tmag, n_it;
    // activations quantised by the kernel itself (one token, K-quants): the f32 row px (slot s's at
    // px + s * px_slot in a grouped launch), first RMS-normalised with the weights pnw and peps when
    // pnw is set
    const float *px, *pnw;
    float peps;
    long px_slot;
    // a grouped launch that selects its experts itself: the router's route_ne logits of the token,
    // route_k choices; the choices and their weights are written to route_top / route_wts
    const float *route_logits;
    int route_ne, route_k;
    int32_t *route_top;
    float *route_wts;
};

constexpr bool is_k(int wt) { return wt == SDY_Q4_K || wt == SDY_Q6_K; }

template <int WT, int MT>
__device__ void stage_acts(const MvArgs &a, uint8_t *lds) {
    const int T = a.P.T, nb = a.P.nb, tid = threadIdx.x;
    const int n_tok = a.n_tok;
    if constexpr (is_k(WT)) {
        // Q8_K rows: nb blocks of 292 B; y starts 4 bytes into a block (dword aligned). The loads of
        // 8 rounds go out before their LDS stores (clamped indices: no conditional load).
        const int n_words = n_tok * T * 16;
        for (int i0 = tid; i0 < n_words; i0 += 8 * THREADS) {
            uint32_t v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = i0 + j * THREADS < n_words ? i0 + j * THREADS : n_words - 1;
                const int m = i / (T * 16), r = i - m * T * 16, u = r >> 4, w = r & 15;
                v[j] = ld4(a.xq + ((size_t)m * nb + (u >> 2)) * 292 + 4 + 64 * (u & 3) + 4 * w);
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = i0 + j * THREADS;
                if (i < n_words) {
                    const int m = i / (T * 16), r = i - m * T * 16, u = r >> 4, w = r & 15;
                    *reinterpret_cast<uint32_t *>(lds + ((m * 4 + (w >> 2)) * T + u) * 16 + 4 * (w & 3)) = v[j];
                }
            }
        }
        uint8_t *bs = lds + MT * 4 * T * 16;
        for (int i = tid; i < n_tok * T; i += THREADS) {
            int m = i / T, u = i - m * T;
            const uint8_t *src = a.xq + ((size_t)m * nb + (u >> 2)) * 292 + 260 + 8 * (u & 3);
            *reinterpret_cast<uint2 *>(bs + (m * T + u) * 8) = make_uint2(ld4(src), ld4(src + 4));
        }
        float *yd = reinterpret_cast<float *>(bs + MT * T * 8);
        for (int i = tid; i < n_tok * nb; i += THREADS)
            yd[i] = *reinterpret_cast<const float *>(a.xq + (size_t)i * 292);
    } else {
        // Q8_0 rows: nb blocks of 34 B (2-byte aligned); unit u = blocks 2u, 2u+1 (the second may
        // be missing: zeros)
        for (int i = tid; i < n_tok * T * 16; i += THREADS) {
            int m = i / (T * 16), r = i - m * T * 16, u = r >> 4, w = r & 15;
            int b = 2 * u + (w >> 3);
            uint32_t v = 0;
            if (b < nb) {
                const uint16_t *src =
                    reinterpret_cast<const uint16_t *>(a.xq + ((size_t)m * nb + b) * 34 + 2 + 4 * (w & 7));
                v = (uint32_t)src[0] | ((uint32_t)src[1] << 16);
            }
            *reinterpret_cast<uint32_t *>(lds + ((m * 4 + (w >> 2)) * T + u) * 16 + 4 * (w & 3)) = v;
        }
        float *dx = reinterpret_cast<float *>(lds + MT * 4 * T * 16);
        int *sy = reinterpret_cast<int *>(dx + MT * T * 2);
        for (int i = tid; i < n_tok * T * 2; i += THREADS) {
            int m = i / (T * 2), r = i - m * T * 2;  // r = 2u + h = block index
            float dv = 0.0f;
            int s = 0;
            if (r < nb) {
                const uint8_t *blk = a.xq + ((size_t)m * nb + r) * 34;
                dv = sdy_h2f((uint16_t)(blk[0] | (blk[1] << 8)));
                for (int e = 0; e < 32; e++) s += (int8_t)blk[2 + e];
            }
            dx[m * T * 2 + r] = dv;
            sy[m * T * 2 + r] = s;
        }
    }
}

template <int WT>
struct WRegs {
    uint4 a, b, c, e;
    uint32_t f, g;
};

// Loads one unit of a row given its unit index iu = row * T + u and (K-quants) super-block index
// is = row * nb + u / 4 in the planes.
template <int WT>
SDY_DEV void load_w_at(const Planes &P, uint32_t iu, uint32_t is, uint32_t u, WRegs<WT> &r) {
    const uint32_t ou = iu * 16u;
    if constexpr (WT == SDY_Q4_K) {
        r.a = ldw16(P.p[0] + ou);
        r.b = ldw16(P.p[1] + ou);
        r.c = ldw16(P.p[2] + is * 16u);
    } else if constexpr (WT == SDY_Q6_K) {
        r.a = ldw16(P.p[0] + ou);
        r.b = ldw16(P.p[1] + ou);
        r.c = ldw16(P.p[2] + ou);
        r.f = ldw4(P.p[3] + is * 16u + 4u * (u & 3u));
        r.g = ldw2(P.p[4] + is * 2u);
    } else if constexpr (WT == SDY_Q8_0) {  // (is unused)
        r.a = ldw16(P.p[0] + ou);
        r.b = ldw16(P.p[1] + ou);
        r.c = ldw16(P.p[2] + ou);
        r.e = ldw16(P.p[3] + ou);
        r.f = ldw4(P.p[4] + iu * 4u);
    } else {
        r.a = ldw16(P.p[0] + ou);
        r.b = ldw16(P.p[1] + ou);
        r.f = ldw4(P.p[4] + iu * 4u);
        if constexpr (WT == SDY_Q5_0) {
            const uint8_t *q = P.p[2] + iu * 8u;
            r.c.x = ldw4(q);
            r.c.y = ldw4(q + 4);
        }
    }
}

// Loads one unit of one row (row and unit given as indices into the planes).
template <int WT>
SDY_DEV void load_w(const Planes &P, uint32_t row, uint32_t u, WRegs<WT> &r) {
    const uint32_t ou = (row * (uint32_t)P.T + u) * 16u;
    if constexpr (WT == SDY_Q4_K) {
        r.a = ldw16(P.p[0] + ou);
        r.b = ldw16(P.p[1] + ou);
        r.c = ldw16(P.p[2] + (row * (uint32_t)P.nb + (u >> 2)) * 16u);
    } else if constexpr (WT == SDY_Q6_K) {
        const uint32_t os = row * (uint32_t)P.nb + (u >> 2);
        r.a = ldw16(P.p[0] + ou);
        r.b = ldw16(P.p[1] + ou);
        r.c = ldw16(P.p[2] + ou);
        r.f = ldw4(P.p[3] + os * 16u + 4u * (u & 3u));
        r.g = ldw2(P.p[4] + os * 2u);
    } else if constexpr (WT == SDY_Q8_0) {
        r.a = ldw16(P.p[0] + ou);
        r.b = ldw16(P.p[1] + ou);
        r.c = ldw16(P.p[2] + ou);
        r.e = ldw16(P.p[3] + ou);
        r.f = ldw4(P.p[4] + (row * (uint32_t)P.T + u) * 4u);
    } else {
        r.a = ldw16(P.p[0] + ou);
        r.b = ldw16(P.p[1] + ou);
        r.f = ldw4(P.p[4] + (row * (uint32_t)P.T + u) * 4u);
        if constexpr (WT == SDY_Q5_0) {
            const uint8_t *q = P.p[2] + (row * (uint32_t)P.T + u) * 8u;
            r.c.x = ldw4(q);
            r.c.y = ldw4(q + 4);
        }
    }
}

SDY_DEV uint32_t w4(const uint4 &v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// Scales and mins of the Q4_K sub-block pair (2j, 2j+1) from the 12 scale bytes held in the
// dwords A (bytes 0-3), B (4-7), C (8-11) (csrc/quant.h:72-80), with shifts and masks only (both
// forms computed and one selected: the four lanes of a super-block differ in j, so a branch would
// run both sides anyway).
SDY_DEV void q4k_pair(uint32_t A, uint32_t B, uint32_t C, int j, int &sc0, int &sc1, int &m0, int &m1) {
    const uint32_t sh = (j & 1) ? 16u : 0u;
    const uint32_t a = (A >> sh) & 0xFFFFu, b = (B >> sh) & 0xFFFFu, c = (C >> sh) & 0xFFFFu;
    const uint32_t sc_lo = a & 0x3F3Fu, m_lo = b & 0x3F3Fu;
    const uint32_t sc_hi = (c & 0x0F0Fu) | ((a >> 2) & 0x3030u), m_hi = ((c >> 4) & 0x0F0Fu) | ((b >> 2) & 0x3030u);
    const uint32_t sc = j < 2 ? sc_lo : sc_hi, m = j < 2 ? m_lo : m_hi;
    sc0 = (int)(sc & 255u);
    sc1 = (int)(sc >> 8);
    m0 = (int)(m & 255u);
    m1 = (int)(m >> 8);
}

// One unit of one token: K-quants return the lane's integer parts (isum, msum), the 32-element
// types return the unit's f32 term directly.
template <int WT>
SDY_DEV void unit_dot(const WRegs<WT> &r, const uint4 *Y, uint2 bsp, int u, int &isum, int &msum, float &term,
                      float2 dxp, int2 syp) {
    constexpr uint32_t LO = 0x0F0F0F0Fu;
    if constexpr (WT == SDY_Q4_K) {
        int slo = 0, shi = 0;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            uint32_t qa = w4(r.a, w), qb = w4(r.b, w);
            slo = sdy_dot4((int)(qa & LO), (int)w4(Y[0], w), slo);
            slo = sdy_dot4((int)(qb & LO), (int)w4(Y[1], w), slo);
            shi = sdy_dot4((int)((qa >> 4) & LO), (int)w4(Y[2], w), shi);
            shi = sdy_dot4((int)((qb >> 4) & LO), (int)w4(Y[3], w), shi);
        }
        int sc0, sc1, m0, m1;
        q4k_pair(r.c.y, r.c.z, r.c.w, u & 3, sc0, sc1, m0, m1);
        const int b0 = (int)(int16_t)(bsp.x & 0xFFFFu), b1 = (int)(int16_t)(bsp.x >> 16);
        const int b2 = (int)(int16_t)(bsp.y & 0xFFFFu), b3 = (int)(int16_t)(bsp.y >> 16);
        // 24-bit multiplies (full rate): |slo|, |shi| <= 32 * 15 * 128, scales and mins < 64,
        // |b0 + b1| <= 32 * 128
        isum = __mul24(sc0, slo) + __mul24(sc1, shi);
        msum = __mul24(m0, b0 + b1) + __mul24(m1, b2 + b3);
    } else if constexpr (WT == SDY_Q6_K) {
        int acc0 = -32 * (int)(int16_t)(bsp.x & 0xFFFFu), acc1 = -32 * (int)(int16_t)(bsp.x >> 16);
        int acc2 = -32 * (int)(int16_t)(bsp.y & 0xFFFFu), acc3 = -32 * (int)(int16_t)(bsp.y >> 16);
#pragma unroll
        for (int w = 0; w < 4; w++) {
            uint32_t n0 = w4(r.a, w), n1 = w4(r.b, w), h = w4(r.c, w);
            uint32_t e0 = (n0 & LO) | ((h & 0x03030303u) << 4);
            uint32_t e1 = (n1 & LO) | (((h >> 2) & 0x03030303u) << 4);
            uint32_t e2 = ((n0 >> 4) & LO) | (((h >> 4) & 0x03030303u) << 4);
            uint32_t e3 = ((n1 >> 4) & LO) | (((h >> 6) & 0x03030303u) << 4);
            acc0 = sdy_dot4((int)e0, (int)w4(Y[0], w), acc0);
            acc1 = sdy_dot4((int)e1, (int)w4(Y[1], w), acc1);
            acc2 = sdy_dot4((int)e2, (int)w4(Y[2], w), acc2);
            acc3 = sdy_dot4((int)e3, (int)w4(Y[3], w), acc3);
        }
        int s0 = (int)(int8_t)(r.f & 255u), s1 = (int)(int8_t)((r.f >> 8) & 255u);
        int s2 = (int)(int8_t)((r.f >> 16) & 255u), s3 = (int)(int8_t)(r.f >> 24);
        // 24-bit multiplies: |acc| <= 16 * 63 * 128 + 32 * 16 * 128, |s| <= 128
        isum = __mul24(s0, acc0) + __mul24(s1, acc1) + __mul24(s2, acc2) + __mul24(s3, acc3);
        msum = 0;
    } else {
        int s[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            int acc = 0;
            if constexpr (WT == SDY_Q8_0) {
                const uint4 &qa = h ? r.c : r.a, &qb = h ? r.e : r.b;
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    acc = sdy_dot4((int)w4(qa, w), (int)w4(Y[2 * h], w), acc);
                    acc = sdy_dot4((int)w4(qb, w), (int)w4(Y[2 * h + 1], w), acc);
                }
            } else {
                const uint4 &q = h ? r.b : r.a;
                uint32_t qh = h ? r.c.y : r.c.x;
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    uint32_t lo = w4(q, w) & LO, hi = (w4(q, w) >> 4) & LO;
                    if constexpr (WT == SDY_Q5_0) {
                        lo |= sdy_spread4(qh >> (4 * w));
                        hi |= sdy_spread4(qh >> (16 + 4 * w));
                    }
                    acc = sdy_dot4((int)lo, (int)w4(Y[2 * h], w), acc);
                    acc = sdy_dot4((int)hi, (int)w4(Y[2 * h + 1], w), acc);
                }
                acc -= (WT == SDY_Q4_0 ? 8 : 16) * (h ? syp.y : syp.x);
            }
            s[h] = acc;
        }
        float dw0 = sdy_h2f((uint16_t)(r.f & 0xFFFFu)), dw1 = sdy_h2f((uint16_t)(r.f >> 16));
        float f0 = dw0 * dxp.x, f1 = dw1 * dxp.y;
        float t0 = (float)s[0] * f0, t1 = (float)s[1] * f1;
        term = t0 + t1;
        isum = msum = 0;
    }
}

// YREG: every lane keeps the same unit for the whole kernel (64 % T == 0, one token), so its
// activation slice lives in registers instead of being re-read from LDS.
template <int WT, int MT, bool YREG>
__global__ __launch_bounds__(THREADS) void k_matvec(MvArgs a) {
    extern __shared__ uint8_t lds[];
    const int T = a.P.T, nb = a.P.nb;
    const size_t y_bytes = (size_t)MT * 4 * T * 16;
    const uint8_t *aux_base = lds + y_bytes;  // BS (K) or DX (32-element types)
    const float *yd = reinterpret_cast<const float *>(lds + y_bytes + (size_t)MT * T * 8);
    const int *sy = reinterpret_cast<const int *>(lds + y_bytes + (size_t)MT * T * 8);
    const size_t act_bytes = y_bytes + (size_t)MT * T * 16;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float *terms = reinterpret_cast<float *>(lds + act_bytes) + (size_t)wave * a.rb * MT * a.nterm;

    const int rb = a.rb, ipb = a.ipb, tasks = rb * T;
    const long n_rows = a.row1 - a.row0;
    const long n_batches = (n_rows + rb - 1) / rb;
    const long n_waves = (long)gridDim.x * WAVES, wid = (long)blockIdx.x * WAVES + wave;
    const long b_begin = n_batches * wid / n_waves, b_end = n_batches * (wid + 1) / n_waves;
    const int rl0 = lane / T, u0 = lane - rl0 * T;  // lane's (row, unit) in the first iteration of a batch

    // the lane's task in (batch b, iteration i): rl, u; validity: task < tasks and row < row1
    long b = b_begin;
    int it = 0, rl = rl0, u = u0;
    auto row_of = [&](long bb, int rr) -> long { return a.row0 + bb * rb + rr; };
    auto lane_ok = [&](long bb, int itx, int rr) -> bool {
        return itx * 64 + lane < tasks && row_of(bb, rr) < a.row1;
    };
    // the first weight loads are issued before the activations are staged, so that the two
    // memory latencies overlap
    WRegs<WT> cur, nxt;
    if (b_begin < b_end) {
        long row = lane_ok(b, it, rl) ? row_of(b, rl) : a.row0;
        load_w<WT>(a.P, (uint32_t)(row - 0), (uint32_t)(lane_ok(b, it, rl) ? u : 0), cur);
    }
    stage_acts<WT, MT>(a, lds);
    __syncthreads();
    if (b_begin >= b_end) return;

    uint4 Yr[4];
    uint2 bsr = make_uint2(0u, 0u);
    if constexpr (YREG) {
#pragma unroll
        for (int q = 0; q < 4; q++) Yr[q] = *reinterpret_cast<const uint4 *>(lds + (q * T + u0) * 16);
        if constexpr (is_k(WT)) bsr = *reinterpret_cast<const uint2 *>(aux_base + u0 * 8);
    }

    for (;;) {
        // advance a copy of the position to the next iteration and prefetch it
        long nb_ = b;
        int nit = it + 1, nrl = rl + a.q64, nu = u + a.r64;
        if (nu >= T) {
            nu -= T;
            nrl++;
        }
        if (nit == ipb) {
            nit = 0;
            nb_ = b + 1;
            nrl = rl0;
            nu = u0;
        }
        const bool more = nb_ < b_end;
        if (more) {
            const bool ok = lane_ok(nb_, nit, nrl);
            load_w<WT>(a.P, (uint32_t)(ok ? row_of(nb_, nrl) : a.row0), (uint32_t)(ok ? nu : 0), nxt);
        }
        const bool valid = lane_ok(b, it, rl);
#pragma unroll
        for (int m = 0; m < MT; m++) {
            if (m >= a.n_tok) break;
            uint4 Y[4];
            uint2 bsp = bsr;
            if constexpr (YREG) {
#pragma unroll
                for (int q = 0; q < 4; q++) Y[q] = Yr[q];
            } else {
                const int uu = valid ? u : 0;
#pragma unroll
                for (int q = 0; q < 4; q++) Y[q] = *reinterpret_cast<const uint4 *>(lds + ((m * 4 + q) * T + uu) * 16);
                if constexpr (is_k(WT)) bsp = *reinterpret_cast<const uint2 *>(aux_base + (m * T + uu) * 8);
            }
            int isum, msum;
            float term;
            if constexpr (is_k(WT)) {
                unit_dot<WT>(cur, Y, bsp, u, isum, msum, term, make_float2(0.f, 0.f), make_int2(0, 0));
                isum = sdy_quad_sum(isum);
                if constexpr (WT == SDY_Q4_K) msum = sdy_quad_sum(msum);
                if ((u & 3) == 0 && valid) {
                    const int s = u >> 2;
                    const float ydv = yd[m * nb + s];
                    float t;
                    if constexpr (WT == SDY_Q4_K) {
                        float d = sdy_h2f((uint16_t)(cur.c.x & 0xFFFFu)), dmin = sdy_h2f((uint16_t)(cur.c.x >> 16));
                        float dall = ydv * d, dmn = ydv * dmin;
                        float t1 = dall * (float)isum, t2 = dmn * (float)msum;
                        t = t1 - t2;
                    } else {
                        float d = sdy_h2f((uint16_t)cur.g);
                        float ydd = ydv * d;
                        t = ydd * (float)isum;
                    }
                    terms[(rl * MT + m) * a.nterm + s] = t;
                }
            } else {
                const int uu = valid ? u : 0;
                const float2 dxp = *reinterpret_cast<const float2 *>(aux_base + (m * T + uu) * 8);
                const int2 syp = *reinterpret_cast<const int2 *>(sy + (m * T + uu) * 2);
                unit_dot<WT>(cur, Y, make_uint2(0u, 0u), u, isum, msum, term, dxp, syp);
                if (valid) terms[(rl * MT + m) * a.nterm + u] = term;
            }
        }
        if (it + 1 == ipb) {
            // end of batch b: each lane sums the terms of one (row, token) in block order
            sdy_wave_sync();
            if (a.swiglu) {
                // rb is even and batches start at even rows: each (gate, up) pair is in this batch
                for (int i = lane; i < (rb >> 1) * a.n_tok; i += 64) {
                    int r = 2 * (i / a.n_tok), m = i - (r >> 1) * a.n_tok;
                    long row = row_of(b, r);
                    if (row >= a.row1) continue;
                    const float *tg = terms + (r * MT + m) * a.nterm, *tu = terms + ((r + 1) * MT + m) * a.nterm;
                    float g = 0.0f, up = 0.0f;
                    for (int s = 0; s < a.nterm; s++) {
                        g = g + tg[s];
                        up = up + tu[s];
                    }
                    a.out[(size_t)m * a.out_stride + ((row - a.row0) >> 1)] = sdy_silu_mul1(g, up);
                }
            } else {
                for (int i = lane; i < rb * a.n_tok; i += 64) {
                    int r = i / a.n_tok, m = i - r * a.n_tok;
                    long row = row_of(b, r);
                    if (row >= a.row1) continue;
                    const float *tp = terms + (r * MT + m) * a.nterm;
                    float acc = 0.0f;
                    for (int s = 0; s < a.nterm; s++) acc = acc + tp[s];
                    if (a.bias) acc = acc + a.bias[row];
                    if (a.resid) acc = a.resid[(size_t)m * a.out_stride + row] + acc;
                    a.out[(size_t)m * a.out_stride + row] = acc;
                }
            }
            sdy_wave_sync();
        }
        if (!more) break;
        b = nb_;
        it = nit;
        rl = nrl;
        u = nu;
        cur = nxt;
    }
}

// Row-in-lanes variant: an iteration covers 64/T whole rows, lane = (row rl, unit u) for the whole
// kernel (T <= 64; when T does not divide 64 — K-quants with one token only — lanes past
// (64/T)*T idle). After the quad reduction the super-block terms of a row sit in lanes
// rl*T + 4s; the row sum folds them in block order with lane shuffles (the reference's sequential
// f32 order), so no LDS round trip is needed. 32-element types sum their unit terms with a fixed
// butterfly over the row's T lanes (T a power of two). Waves stride over the iterations and load
// the next iteration's weights while they compute the current one.
// (the body of k_matvec_rl for workgroup bx of a grid of G, routed-expert slot `slot`)
template <int WT, int MT, bool YREG>
SDY_DEV void matvec_rl_body(const MvArgs &a, long G, long bx, int slot) {
    extern __shared__ uint8_t lds[];
    // One token of Q8_K activations in memory: every lane reads the 64 activation bytes of its unit
    // (and the unit's bsums and block scale) straight into registers; no LDS staging, no barrier.
    constexpr bool DIRECT = YREG && is_k(WT) && MT == 1;
    const int T = a.P.T, nb = a.P.nb;
    const size_t y_bytes = (size_t)MT * 4 * T * 16;
    const uint8_t *aux_base = lds + y_bytes;
    const float *yd = reinterpret_cast<const float *>(lds + y_bytes + (size_t)MT * T * 8);
    const int *sy = reinterpret_cast<const int *>(lds + y_bytes + (size_t)MT * T * 8);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rpi = 64 / T;  // rows per iteration
    const int rl_ = lane / T, u = lane - rl_ * T;
    const bool lane_on = rl_ < rpi;   // spare lanes (T not dividing 64) shadow row 0 and store nothing
    const int rl = lane_on ? rl_ : 0;
    // grouped (routed-expert) launch: this workgroup's slot, its expert's first row, activation and output
    long poff = 0;
    const uint8_t *xq = a.xq;
    float *out = a.out;
    if (a.slot_expert) {
        int e = a.slot_expert[slot];
        e = e < 0 ? 0 : (e >= a.n_slot_exp ? a.n_slot_exp - 1 : e);
        poff = (long)e * a.slot_rows;
        xq += (size_t)slot * a.xq_slot;
        out += (size_t)slot * a.out_slot;
    }
    const long n_rows = a.row1 - a.row0;
    const long n_it = (n_rows + rpi - 1) / rpi;
    // Workgroups are dealt round-robin over the 8 XCDs; renumber them so that consecutive work
    // (neighbouring rows) stays on one XCD and its L2.
    const long vblk = (G % 8 == 0) ? (bx % 8) * (G / 8) + bx / 8 : bx;  // a bijection of [0, G)
    const long n_waves = G * WAVES, wid = vblk * WAVES + wave;
    // grid-stride: at any moment the waves of the grid read neighbouring rows, so the whole GPU
    // sweeps each plane front to back
    auto row_at = [&](long itx) -> long { return a.row0 + itx * rpi + rl; };
    auto load_it = [&](long itx, WRegs<WT> &r) {
        long rr = row_at(itx);
        load_w<WT>(a.P, (uint32_t)((rr < a.row1 ? rr : a.row0) + poff), (uint32_t)u, r);
    };
    // the first weight loads go out before anything else, so their latency overlaps the
    // activation loads
    WRegs<WT> A, B;
    if (wid < n_it) load_it(wid, A);

    uint4 Yr[4];
    uint2 bsr = make_uint2(0u, 0u);
    float2 dxr = make_float2(0.f, 0.f);
    int2 syr = make_int2(0, 0);
    float ydr = 0.0f;
    if constexpr (DIRECT) {
        if (wid >= n_it) return;
        const uint8_t *blk = xq + (size_t)(u >> 2) * 292;
        const uint8_t *yb = blk + 4 + 64 * (u & 3);
#pragma unroll
        for (int q = 0; q < 4; q++)
            Yr[q] = make_uint4(ld4(yb + 16 * q), ld4(yb + 16 * q + 4), ld4(yb + 16 * q + 8), ld4(yb + 16 * q + 12));
        bsr = make_uint2(ld4(blk + 260 + 8 * (u & 3)), ld4(blk + 264 + 8 * (u & 3)));
        ydr = *reinterpret_cast<const float *>(blk);
    } else {
        stage_acts<WT, MT>(a, lds);
        __syncthreads();
        if (wid >= n_it) return;
        if constexpr (YREG) {
#pragma unroll
            for (int q = 0; q < 4; q++) Yr[q] = *reinterpret_cast<const uint4 *>(lds + (q * T + u) * 16);
            if constexpr (is_k(WT)) bsr = *reinterpret_cast<const uint2 *>(aux_base + u * 8);
            else {
                dxr = *reinterpret_cast<const float2 *>(aux_base + u * 8);
                syr = *reinterpret_cast<const int2 *>(sy + u * 2);
            }
        }
    }
    auto body = [&](const WRegs<WT> &cur, long itx) {
        const long row = row_at(itx);
        const bool valid = lane_on && row < a.row1;
#pragma unroll
        for (int m = 0; m < MT; m++) {
            if (m >= a.n_tok) break;
            uint4 Y[4];
            uint2 bsp = bsr;
            float2 dxp = dxr;
            int2 syp = syr;
            if constexpr (YREG) {
#pragma unroll
                for (int q = 0; q < 4; q++) Y[q] = Yr[q];
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) Y[q] = *reinterpret_cast<const uint4 *>(lds + ((m * 4 + q) * T + u) * 16);
                if constexpr (is_k(WT)) bsp = *reinterpret_cast<const uint2 *>(aux_base + (m * T + u) * 8);
                else {
                    dxp = *reinterpret_cast<const float2 *>(aux_base + (m * T + u) * 8);
                    syp = *reinterpret_cast<const int2 *>(sy + (m * T + u) * 2);
                }
            }
            int isum, msum;
            float term = 0.0f;
            unit_dot<WT>(cur, Y, bsp, u, isum, msum, term, dxp, syp);
            float acc;
            if constexpr (is_k(WT)) {
                isum = sdy_quad_sum(isum);
                if constexpr (WT == SDY_Q4_K) msum = sdy_quad_sum(msum);
                const float ydv = DIRECT ? ydr : yd[m * nb + (u >> 2)];
                if constexpr (WT == SDY_Q4_K) {
                    float d = sdy_h2f((uint16_t)(cur.c.x & 0xFFFFu)), dmin = sdy_h2f((uint16_t)(cur.c.x >> 16));
                    float dall = ydv * d, dmn = ydv * dmin;
                    float t1 = dall * (float)isum, t2 = dmn * (float)msum;
                    term = t1 - t2;
                } else {
                    float d = sdy_h2f((uint16_t)cur.g);
                    float ydd = ydv * d;
                    term = ydd * (float)isum;
                }
                // sequential fold over the row's super-blocks (lane rl*T reads lanes rl*T + 4s), from
                // the reference's initial 0.0f
                acc = 0.0f + term;
                const int nsb = T >> 2;
                for (int s = 1; s < nsb; s++) acc = acc + __shfl(term, lane + 4 * s);
            } else {
                acc = term;
                for (int off = 1; off < T; off <<= 1) acc = acc + __shfl_xor(acc, off);
            }
            if (a.swiglu) {
                // rows per iteration is even and row0 is even: lane (rl+1)*T holds the up row
                const float up = __shfl(acc, (lane + T) & 63);
                if (u == 0 && (rl & 1) == 0 && valid)
                    out[(size_t)m * a.out_stride + ((row - a.row0) >> 1)] = sdy_silu_mul1(acc, up);
            } else if (u == 0 && valid) {
                if (a.bias) acc = acc + a.bias[row];
                if (a.resid) acc = a.resid[(size_t)m * a.out_stride + row] + acc;
                out[(size_t)m * a.out_stride + row] = acc;
            }
        }
    };
    // ping-pong register buffers: the loads of one iteration stay in flight while the other computes
    const long S = n_waves;
    for (long itx = wid; itx < n_it; itx += 2 * S) {
        if (itx + S < n_it) load_it(itx + S, B);
        body(A, itx);
        if (itx + S >= n_it) break;
        if (itx + 2 * S < n_it) load_it(itx + 2 * S, A);
        body(B, itx + S);
    }
}

template <int WT, int MT, bool YREG>
__global__ __launch_bounds__(THREADS) void k_matvec_rl(MvArgs a) {
    matvec_rl_body<WT, MT, YREG>(a, gridDim.x, blockIdx.x, blockIdx.y);
}

// Two one-token matvecs on the same Q8_K activations in one launch (q|k and v of a layer when v has
// another type): workgroups [0, g1) run the first, [g1, gridDim.x) the second. g1 is a multiple of 8,
// so each part keeps its own XCD-aware numbering.
template <int WT1, int WT2>
__global__ __launch_bounds__(THREADS) void k_matvec_rl_pair(MvArgs a, MvArgs b, int g1) {
    if ((int)blockIdx.x < g1) matvec_rl_body<WT1, 1, true>(a, g1, blockIdx.x, 0);
    else matvec_rl_body<WT2, 1, true>(b, (long)gridDim.x - g1, (long)blockIdx.x - g1, 0);
}

// The Q8_K row of a one-token matvec built in LDS by its workgroup of WV waves from the f32 row x (n
// elements, a multiple of 256, x 16-byte aligned), RMS-normalised first when NORM (nb <= WV NR): the
// bytes that k_quant_q8k (k_norm_quant with NORM) writes — same sum order, same wave quantiser — in
// an aligned layout: y [nb][256] int8, bsums [nb][16] int16, d [nb] f32 (nb * 292 bytes).
// issue() requests the lane's inputs: super-blocks wave + WV k, k < NR (called before the weight
// loads, so that these few bytes do not queue behind the weight stream); build() quantises them into
// LDS, loading further rounds of NR super-blocks per wave when nb > WV NR (without NORM only). Every
// thread of the workgroup calls build(); it ends with a barrier.
template <bool NORM, int NR, int WV = 4>
struct Q8kRow {
    static_assert(!NORM || WV == 4 || WV == 8, "the norm's sum order is that of 256 threads");
    float4 xv[NR], wv[NR];

    SDY_DEV void issue(const float *__restrict__ x, const float *__restrict__ nw, int n) {
        const int nb = n >> 8, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
        for (int k = 0; k < NR; k++) {
            const int sb = wave + WV * k < nb ? wave + WV * k : nb - 1;
            xv[k] = *reinterpret_cast<const float4 *>(x + 256 * sb + 4 * lane);
            if constexpr (NORM) wv[k] = *reinterpret_cast<const float4 *>(nw + 256 * sb + 4 * lane);
        }
    }

    SDY_DEV void build(const float *__restrict__ x, float eps, int n, uint8_t *lds) {
        const int nb = n >> 8, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
        uint32_t *ly = reinterpret_cast<uint32_t *>(lds);
        int16_t *lbs = reinterpret_cast<int16_t *>(lds + (size_t)nb * 256);
        float *ld = reinterpret_cast<float *>(lds + (size_t)nb * 288);
        float scale = 1.0f;
        if constexpr (NORM) {
            // sdy_row_sumsq's order: thread t adds the squares of its float4 chunks t, t + 256, ...
            // (chunk t + 256 k is super-block wave + 4 k, the lane's four elements), then the tree
            __shared__ double sh[4];
            double ss = 0.0;
            auto add = [&](const float4 &v) {
                ss += (double)v.x * (double)v.x;
                ss += (double)v.y * (double)v.y;
                ss += (double)v.z * (double)v.z;
                ss += (double)v.w * (double)v.w;
            };
            if constexpr (WV == 4) {
#pragma unroll
                for (int k = 0; k < NR; k++)
                    if (wave + 4 * k < nb) add(xv[k]);
                ss = sdy_block_sum256(ss, sh);
            } else {
                // eight waves: thread t of the 256-thread order (wave w = t / 64 < 4) takes super-blocks
                // w, w + 4, w + 8, ... in turn; w + 8 k is wave w's k-th, w + 4 + 8 k the k-th of wave
                // w + 4, which passes its chunks through LDS. Waves 0-3 add in that order, then the
                // same tree over their four wave sums
                __shared__ float4 xch[4][NR][64];
                if (wave >= 4) {
#pragma unroll
                    for (int k = 0; k < NR; k++) xch[wave - 4][k][lane] = xv[k];
                }
                __syncthreads();
                if (wave < 4) {
#pragma unroll
                    for (int k = 0; k < NR; k++) {
                        if (wave + 8 * k < nb) add(xv[k]);
                        if (wave + 4 + 8 * k < nb) add(xch[wave][k][lane]);
                    }
                }
                const double v = sdy_wave_sum_f64(ss);
                if (lane == 0 && wave < 4) sh[wave] = v;
                __syncthreads();
                ss = (sh[0] + sh[1]) + (sh[2] + sh[3]);
            }
            scale = (float)(1.0 / sqrt(ss / (double)n + (double)eps));
        }
        for (int s0 = wave; s0 < nb; s0 += WV * NR) {
            if (s0 != wave) {  // a further round (long rows without NORM)
#pragma unroll
                for (int k = 0; k < NR; k++) {
                    const int sb = s0 + WV * k < nb ? s0 + WV * k : nb - 1;
                    xv[k] = *reinterpret_cast<const float4 *>(x + 256 * sb + 4 * lane);
                }
            }
            float xs[NR][4];
#pragma unroll
            for (int k = 0; k < NR; k++) {
                float4 v = xv[k];
                if constexpr (NORM) {
                    const float4 w = wv[k];
                    v = make_float4((v.x * scale) * w.x, (v.y * scale) * w.y, (v.z * scale) * w.z, (v.w * scale) * w.w);
                }
                xs[k][0] = v.x;
                xs[k][1] = v.y;
                xs[k][2] = v.z;
                xs[k][3] = v.w;
            }
            SdyQ8kLane r[NR];
            sdy_q8k_lanes<NR>(xs, lane, r);
#pragma unroll
            for (int k = 0; k < NR; k++) {
                const int sb = s0 + WV * k;
                if (sb < nb) {
                    ly[sb * 64 + lane] = r[k].packed;
                    if ((lane & 3) == 0) lbs[sb * 16 + (lane >> 2)] = (int16_t)r[k].gsum;
                    if (lane == 0) ld[sb] = r[k].d;
                }
            }
        }
        __syncthreads();
    }
};

// The lane's unit u of the activation row in LDS (Q8kRow layout): its 64 y bytes, the bsums of
// its four 16-element groups and the block scale.
SDY_DEV void q8k_unit_lds(const uint8_t *lds, int nb, int u, uint4 (&Yr)[4], uint2 &bsr, float &ydr) {
    const uint8_t *y = lds + (u >> 2) * 256 + 64 * (u & 3);
#pragma unroll
    for (int q = 0; q < 4; q++) Yr[q] = *reinterpret_cast<const uint4 *>(y + 16 * q);
    bsr = *reinterpret_cast<const uint2 *>(lds + (size_t)nb * 256 + (u >> 2) * 32 + 8 * (u & 3));
    ydr = reinterpret_cast<const float *>(lds + (size_t)nb * 288)[u >> 2];
}

// Lane rl*T's sequential fold of the row's nsb <= N super-block terms (lanes rl*T + 4s).
template <int N>
SDY_DEV float rl_fold(float term, int lane, int nsb) {
    float tv[N];
#pragma unroll
    for (int s = 1; s < N; s++) tv[s] = __shfl(term, (lane + 4 * s) & 63);
    float acc = 0.0f + term;
#pragma unroll
    for (int s = 1; s < N; s++)
        if (s < nsb) acc = acc + tv[s];
    return acc;
}

// The row sum of one K-quant unit term per lane (one token, activations in registers): the quad
// reduction leaves super-block s of row rl in lane rl*T + 4s, and lane rl*T folds the terms in
// super-block order from the reference's initial 0.0f. All the lane reads are issued before the
// first add (one LDS round trip), for up to 16 super-blocks (T <= 64); NSB > 0: exactly NSB.
template <int WT, int NSB>
SDY_DEV float rl_row_sum(const WRegs<WT> &cur, const uint4 (&Yr)[4], uint2 bsr, float ydr, int u, int lane, int T) {
    int isum, msum;
    float term = 0.0f;
    unit_dot<WT>(cur, Yr, bsr, u, isum, msum, term, make_float2(0.f, 0.f), make_int2(0, 0));
    isum = sdy_quad_sum(isum);
    if constexpr (WT == SDY_Q4_K) {
        msum = sdy_quad_sum(msum);
        const float d = sdy_h2f((uint16_t)(cur.c.x & 0xFFFFu)), dmin = sdy_h2f((uint16_t)(cur.c.x >> 16));
        const float dall = ydr * d, dmn = ydr * dmin;
        const float t1 = dall * (float)isum, t2 = dmn * (float)msum;
        term = t1 - t2;
    } else {
        const float d = sdy_h2f((uint16_t)cur.g);
        const float ydd = ydr * d;
        term = ydd * (float)isum;
    }
    if constexpr (NSB > 0) return rl_fold<NSB>(term, lane, NSB);
    else return rl_fold<16>(term, lane, T >> 2);
}

// A grouped one-token matvec that routes its token itself (k_matvec_1t with PRO 3): one wave of each
// workgroup runs the router's softmax and top-k over the route_ne logits (the bits of k_moe_route,
// at most 128 experts) and takes slot `slot`'s expert; the writer wave (one in the grid) stores the
// route_k choices and their weights for the kernels that follow.
SDY_DEV int routed_expert(const MvArgs &a, int slot, int lane, bool writer) {
    int my_e;
    float my_p, chosen_sum;
    sdy_moe_route_wave<2>(a.route_logits, a.route_ne, a.route_k, lane, sdy_expf_tab_lane(lane), my_e, my_p,
                          chosen_sum);
    if (writer && lane < a.route_k) {
        a.route_top[lane] = my_e;
        a.route_wts[lane] = my_p / chosen_sum;
    }
    return __builtin_amdgcn_readlane(my_e, slot);
}

// One token, K-quants with at most 64 units per row (every one-token matvec of a decode step but
// the output head): wave w of the S waves of the grid takes the NIT iterations w, w + S, ...,
// w + (NIT - 1) S of 64/T rows each, and issues every load it needs (the weights of all its
// iterations, its unit's activations, the bias and residual of its rows) before its first
// computation, so the wave waits for one memory round trip; the results are stored at the end.
// Same lane layout and arithmetic as k_matvec_rl, so the bits are the same.
// (the body of k_matvec_1t for workgroup bx of a grid of G, routed-expert slot `slot`)
// PRO: 0 the Q8_K row a.xq in memory, 1 the f32 row a.px quantised by the workgroup (into LDS),
// 2 a.px RMS-normalised with a.pnw, then quantised; 3 as 0 in a grouped launch whose workgroups
// select their slot's expert from the router's logits (routed_expert).
// WV waves per workgroup: 4, or 8 for the RMS-normalised row (PRO 2), whose row is then built after
// the weights are requested (with 4 it is built before them; its sum of squares keeps the 256-thread
// order either way).
template <int WT, int NIT, int NSB, int PRO = 0, int WV = WAVES>
SDY_DEV void matvec_1t_body(const MvArgs &a, int G, int bx, int slot) {
    // super-blocks per wave of the workgroup's activation row (n_in 768: 3, 2048: 8, else up to 16)
    constexpr int PRO_NR = WV == 4 ? (NSB == 3 ? 1 : NSB == 8 ? 2 : 4) : (NSB == 3 || NSB == 8 ? 1 : 2);
    constexpr bool ROUTE = PRO == 3;
    constexpr int PK = ROUTE ? 0 : PRO;  // the activation row's kind
    constexpr bool NORM_FIRST = PK == 2 && WV == 4;  // the normalised row built before the weight loads
    const int T = a.P.T;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int rpi = a.rpi;
    const int rl_ = __mul24(lane, a.tmag) >> 16, u = lane - __mul24(rl_, T);
    const bool lane_on = rl_ < rpi;
    const int rl = lane_on ? rl_ : 0;
    const int vblk = (G & 7) == 0 ? (bx & 7) * (G >> 3) + (bx >> 3) : bx;  // XCD-aware renumbering
    const int S = G * WV, wid = vblk * WV + wave;
    int e_routed = 0;
    if constexpr (ROUTE) {
        // wave 0 routes the token and hands its slot's expert to the workgroup (before any wave
        // leaves: the barrier counts them all); one wave per workgroup reading the logits instead of
        // every wave: 30B-A3B decode 465-467 against 461-463 tok/s
        __shared__ int sh_e;
        if (wave == 0) {
            const int e0 = routed_expert(a, slot, lane, bx == 0 && slot == 0);
            if (lane == 0) sh_e = e0;
        }
        __syncthreads();
        e_routed = __builtin_amdgcn_readfirstlane(sh_e);
    }
    if constexpr (PK == 0) {
        if (wid >= a.n_it) return;
    }
    long poff = 0;
    const uint8_t *xq = a.xq;
    float *out = a.out;
    if (a.slot_expert) {
        int e;
        if constexpr (ROUTE) e = e_routed;
        else e = a.slot_expert[slot];
        e = e < 0 ? 0 : (e >= a.n_slot_exp ? a.n_slot_exp - 1 : e);
        poff = (long)e * a.slot_rows;
        xq += (size_t)slot * a.xq_slot;
        out += (size_t)slot * a.out_slot;
    }
    extern __shared__ uint8_t lds_act[];
    Q8kRow<PK == 2, PRO_NR, WV> arow;
    const float *px = a.px + (PK ? (size_t)slot * a.px_slot : 0);
    // (with PRO, waves past the rows still take part in the workgroup's activation row: their rows
    // are all >= row1, so they load row0 and store nothing)
    if constexpr (PK != 0) arow.issue(px, a.pnw, a.P.n_in);
    // load order: the first iteration's weights, the activations, the bias and residual, then the
    // other iterations' weights, so that iteration k waits only for the loads it uses (every load
    // is unconditional, which keeps the compiler's wait counts exact)
    WRegs<WT> R[NIT];
    long row[NIT];
#pragma unroll
    for (int k = 0; k < NIT; k++) row[k] = a.row0 + (long)((wid + k * S) * rpi + rl);
    // unit and super-block indices: the row base is uniform over the wave (scalar arithmetic) and
    // rl * T + u = lane; rows past the end read row0 instead
    const uint32_t le = lane_on ? lane : u, nb = a.P.nb;
    auto load_k = [&](int k) {
        const uint32_t base = (uint32_t)(a.row0 + (long)(wid + k * S) * rpi + poff);
        const uint32_t r0 = (uint32_t)(a.row0 + poff);
        const bool ok = row[k] < a.row1;
        const uint32_t iu = ok ? base * (uint32_t)T + le : r0 * (uint32_t)T + u;
        const uint32_t is = ok ? base * nb + (le >> 2) : r0 * nb + (u >> 2);
        load_w_at<WT>(a.P, iu, is, (uint32_t)u, R[k]);
    };
    uint4 Yr[4];
    uint2 bsr;
    float ydr;
    if constexpr (NORM_FIRST) {
        // the normalised row first: requested before any weight, its loads do not return behind
        // this workgroup's weight stream (measured on the 22016 x 2048 gate|up with the FFN norm
        // and 4-wave workgroups: 9.5 -> 8.9 us against building the row while the weights are in
        // flight)
        arow.build(px, a.peps, a.P.n_in, lds_act);
        q8k_unit_lds(lds_act, a.P.nb, u, Yr, bsr, ydr);
    }
    load_k(0);
    const uint32_t etab = sdy_expf_tab_lane(lane);  // the SwiGLU epilogue's exponential table
    if constexpr (PK == 0) {
        const uint8_t *blk = xq + __mul24(u >> 2, 292);
        const uint8_t *yb = blk + 4 + 64 * (u & 3);
#pragma unroll
        for (int q = 0; q < 4; q++)
            Yr[q] = make_uint4(ld4(yb + 16 * q), ld4(yb + 16 * q + 4), ld4(yb + 16 * q + 8), ld4(yb + 16 * q + 12));
        bsr = make_uint2(ld4(blk + 260 + 8 * (u & 3)), ld4(blk + 264 + 8 * (u & 3)));
        ydr = *reinterpret_cast<const float *>(blk);
    } else {
#pragma unroll
        for (int k = 1; k < NIT; k++) load_k(k);
        if constexpr (PK == 1 || (PK == 2 && !NORM_FIRST)) {
            // the quantiser alone (no norm): every weight load goes out first and the workgroup
            // quantises the row while they are in flight (3B decode 637 -> 646 tok/s against building
            // it first, with the 2048 x 2048 wo); the same for the norm with 8-wave workgroups
            arow.build(px, a.peps, a.P.n_in, lds_act);
            q8k_unit_lds(lds_act, a.P.nb, u, Yr, bsr, ydr);
        }
    }
    // the bias and residual of the lane's rows (an absent one reads a stand-in: the activation row)
    const float *stand_in = PK ? px : reinterpret_cast<const float *>(xq);
    const float *bsrc = a.bias ? a.bias : stand_in;
    const float *rsrc = a.resid ? a.resid : stand_in;
    float bv[NIT], rv[NIT];
#pragma unroll
    for (int k = 0; k < NIT; k++) {
        const int rc = (int)(row[k] < a.row1 ? row[k] : a.row0);
        bv[k] = bsrc[a.bias ? rc : 0];
        rv[k] = rsrc[a.resid ? rc : 0];
    }
    if constexpr (PK == 0) {
#pragma unroll
        for (int k = 1; k < NIT; k++) load_k(k);
    }
    float acc[NIT];
#pragma unroll
    for (int k = 0; k < NIT; k++) acc[k] = rl_row_sum<WT, NSB>(R[k], Yr, bsr, ydr, u, lane, T);
    if (a.swiglu) {
        // rows per iteration and row0 are even: iteration k's output pair p has its gate row in lane
        // 2p*T and its up row in lane (2p+1)*T. Lane j < NIT * rpi/2 gathers output j (iteration
        // j / (rpi/2), pair j % (rpi/2)), so the wave evaluates SiLU once for all its outputs.
        const int npair = rpi >> 1, nout = NIT * npair;
        const int j = lane < nout ? lane : 0;
        int kj = 0;
#pragma unroll
        for (int k = 1; k < NIT; k++)
            if (j >= k * npair) kj = k;
        const int p = j - kj * npair;
        float g = 0.0f, up = 0.0f;
#pragma unroll
        for (int k = 0; k < NIT; k++) {
            const float gk = __shfl(acc[k], 2 * p * T), uk = __shfl(acc[k], (2 * p + 1) * T);
            g = k == kj ? gk : g;
            up = k == kj ? uk : up;
        }
        const long rowj = a.row0 + (long)((wid + kj * S) * rpi + 2 * p);
        const float r = sdy_silu_mul1_reg(g, up, etab);
        if (lane < nout && rowj < a.row1) out[(rowj - a.row0) >> 1] = r;
        return;
    }
#pragma unroll
    for (int k = 0; k < NIT; k++) {
        if (u == 0 && lane_on && row[k] < a.row1) {
            float v = acc[k];
            if (a.bias) v = v + bv[k];
            if (a.resid) v = rv[k] + v;
            out[row[k]] = v;
        }
    }
}

template <int WT, int NIT, int NSB, int PRO, int WV = WAVES>
__global__ __launch_bounds__(64 * WV) void k_matvec_1t(MvArgs a) {
    matvec_1t_body<WT, NIT, NSB, PRO, WV>(a, (int)gridDim.x, (int)blockIdx.x, (int)blockIdx.y);
}

// k_matvec_1t's pair form (see k_matvec_rl_pair), one iteration per wave
template <int WT1, int WT2, int NSB, int PRO, int WV = WAVES>
__global__ __launch_bounds__(64 * WV) void k_matvec_1t_pair(MvArgs a, MvArgs b, int g1) {
    if ((int)blockIdx.x < g1) matvec_1t_body<WT1, 1, NSB, PRO, WV>(a, g1, (int)blockIdx.x, 0);
    else matvec_1t_body<WT2, 1, NSB, PRO, WV>(b, (int)gridDim.x - g1, (int)blockIdx.x - g1, 0);
}

// The routed experts' down projections of one token and their combine in one launch. Workgroup of
// KMAX waves over rpi rows: wave s computes slot s's dots with expert slot_expert[s] as
// k_matvec_1t's grouped form does (the same bits: lane (rl, u) holds unit u of row rl), the
// workgroup exchanges them through LDS, and wave 0 sums the k slots in ascending expert id with the
// weights wts (k_moe_combine's order, op_axpy's per-element form), plus resid, into out. The k
// slots' f32 rows (px, n_in apart: contiguous) are quantised by the workgroup as one row of
// k * n_in elements into LDS (slot s's units follow slot s - 1's).
template <int WT, int NSB, int KMAX>
__global__ __launch_bounds__(64 * KMAX) void k_moe_down_combine(MvArgs a, const float *__restrict__ wts, int k,
                                                                float *out, const float *resid) {
    const int T = a.P.T, n_in = a.P.n_in;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int rpi = a.rpi;
    const int rl_ = __mul24(lane, a.tmag) >> 16, u = lane - __mul24(rl_, T);
    const bool lane_on = rl_ < rpi;
    const int rl = lane_on ? rl_ : 0;
    const int G = (int)gridDim.x, bx = (int)blockIdx.x;
    const int vblk = (G & 7) == 0 ? (bx & 7) * (G >> 3) + (bx >> 3) : bx;  // XCD-aware renumbering
    const long row = a.row0 + (long)vblk * rpi + rl;
    const long rowc = row < a.row1 ? row : a.row0;  // (rows past the end read row0 and store nothing)
    extern __shared__ uint8_t lds_act[];
    // (eight rows of 768: 24 super-blocks, three per wave)
    Q8kRow<false, NSB == 3 ? 3 : 4, KMAX> arow;
    arow.issue(a.px, nullptr, k * n_in);
    __builtin_amdgcn_sched_barrier(0);  // (the row's loads stay ahead of the weights')
    const int sl = wave < k ? wave : k - 1;
    int e = a.slot_expert[sl];
    e = e < 0 ? 0 : (e >= a.n_slot_exp ? a.n_slot_exp - 1 : e);
    WRegs<WT> R;
    const uint32_t nb = a.P.nb, base = (uint32_t)((long)e * a.slot_rows + rowc);
    load_w_at<WT>(a.P, base * (uint32_t)T + (uint32_t)u, base * nb + ((uint32_t)u >> 2), (uint32_t)u, R);
    // (an unconditional load, from a stand-in when there is no residual: a load under a pointer
    // test makes the compiler's wait before the activation row count the weight loads issued ahead
    // of it)
    const float rv = (resid ? resid : a.px)[resid ? rowc : 0];
    // the combine's expert ids and weights, requested with the other loads
    int ids[KMAX];
    float wv[KMAX], yv[KMAX];
#pragma unroll
    for (int i = 0; i < KMAX; i++) {
        const int ii = i < k ? i : 0;
        const int id = a.slot_expert[ii];  // (unconditional loads: the slots past k read slot 0)
        ids[i] = i < k ? id : 0x7fffffff;
        wv[i] = wts[ii];
    }
    arow.build(a.px, 0.0f, k * n_in, lds_act);
    uint4 Yr[4];
    uint2 bsr;
    float ydr;
    q8k_unit_lds(lds_act, k * (int)nb, sl * T + u, Yr, bsr, ydr);
    const float acc = rl_row_sum<WT, NSB>(R, Yr, bsr, ydr, u, lane, T);
    float *xacc = reinterpret_cast<float *>(lds_act + (size_t)k * nb * 292);  // [KMAX][64]
    if (u == 0) xacc[wave * 64 + rl_] = acc;
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int i = 0; i < KMAX; i++) yv[i] = xacc[(i < k ? i : 0) * 64 + rl];
    // ascending expert id (the same order k_moe_combine sorts the triples into)
#pragma unroll
    for (int i = 0; i < KMAX; i++)
#pragma unroll
        for (int j = 0; j + 1 < KMAX - i; j++)
            if (ids[j] > ids[j + 1]) {
                const int ti = ids[j];
                ids[j] = ids[j + 1];
                ids[j + 1] = ti;
                const float tw = wv[j];
                wv[j] = wv[j + 1];
                wv[j + 1] = tw;
                const float ty = yv[j];
                yv[j] = yv[j + 1];
                yv[j + 1] = ty;
            }
    const long dim = a.row1 - a.row0, d = rowc - a.row0;
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < KMAX; i++)
        if (i < k) tot = d < (dim & ~7L) ? fmaf(wv[i], yv[i], tot) : tot + wv[i] * yv[i];
    if (u == 0 && lane_on && row < a.row1) out[row] = resid ? rv + tot : tot;
}

// One token, rows of at most 64 units: K-quants when the rows are too many for k_matvec_1t (the
// output head), and the 32-element types (whose activation row is staged in LDS, as in
// k_matvec_rl, and whose unit terms are summed by k_matvec_rl's butterfly): a grid the GPU holds at
// once, wave w of S taking iterations w, w + S, ...
// (64/T rows each) with NB iterations' weights in flight in a ring of registers. Every load is
// unconditional (rows past the end read row0), so the code is straight-line per round of NB
// iterations and the compiler's wait before each iteration's computation covers only that
// iteration's loads; the slot is refilled right after its computation. Same lane layout and
// arithmetic as k_matvec_1t (the same bits); no SwiGLU epilogue.
// PRO 1 / 2 (K-quants): the workgroup builds the Q8_K row of the f32 input a.px in LDS
// (RMS-normalised first for 2: Q8kRow, the bytes k_quant_q8k / k_norm_quant write) after its waves
// have requested their first NB iterations' weights, which stream meanwhile.
template <int WT, int NB, int NSB, int PRO = 0>
__global__ __launch_bounds__(THREADS) void k_matvec_ring(MvArgs a) {
    extern __shared__ uint8_t lds[];
    const int T = a.P.T;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int rpi = a.rpi;
    const int rl_ = __mul24(lane, a.tmag) >> 16, u = lane - __mul24(rl_, T);
    const bool lane_on = rl_ < rpi;
    const int rl = lane_on ? rl_ : 0;
    const int G = (int)gridDim.x, bx = (int)blockIdx.x;
    const int vblk = (G & 7) == 0 ? (bx & 7) * (G >> 3) + (bx >> 3) : bx;  // XCD-aware renumbering
    const int S = G * WAVES, wid = vblk * WAVES + wave;
    if constexpr (!is_k(WT)) {  // the 32-element types' activation row in LDS (every thread)
        stage_acts<WT, 1>(a, lds);
        __syncthreads();
    }
    static_assert(PRO == 0 || is_k(WT), "in-kernel quantisation of K-quant activations only");
    constexpr int PRO_NR = NSB == 3 ? 1 : NSB == 8 ? 2 : 4;  // the row's super-blocks per wave (nb <= 16)
    Q8kRow<PRO == 2, PRO_NR, WAVES> arow;
    if constexpr (PRO) {
        arow.issue(a.px, a.pnw, a.P.n_in);
        __builtin_amdgcn_sched_barrier(0);  // (the row's loads stay ahead of the weights')
    } else {
        if (wid >= a.n_it) return;
    }
    // this wave's iterations (with PRO, waves past them still build the row with the workgroup)
    const int n_my = wid < a.n_it ? (a.n_it - wid + S - 1) / S : 0;
    const uint32_t le = lane_on ? lane : u, nb = a.P.nb, r0 = (uint32_t)a.row0;
    WRegs<WT> R[NB];
    // iteration i of this wave: rows row0 + (wid + i S) rpi + rl
    auto load_i = [&](int t, int i) {
        const uint32_t base = (uint32_t)(a.row0 + (long)(wid + i * S) * rpi);
        const bool ok = (long)base + rl < a.row1;
        const uint32_t iu = ok ? base * (uint32_t)T + le : r0 * (uint32_t)T + u;
        const uint32_t is = ok ? base * nb + (le >> 2) : r0 * nb + (u >> 2);
        load_w_at<WT>(a.P, iu, is, (uint32_t)u, R[t]);
    };
    load_i(0, 0);
    uint4 Yr[4];
    uint2 bsr = make_uint2(0u, 0u);
    float ydr = 0.0f;
    float2 dxr = make_float2(0.f, 0.f);
    int2 syr = make_int2(0, 0);
    if constexpr (PRO) {
#pragma unroll
        for (int t = 1; t < NB; t++) load_i(t, t);
        arow.build(a.px, a.peps, a.P.n_in, lds);
        q8k_unit_lds(lds, nb, u, Yr, bsr, ydr);
    } else if constexpr (is_k(WT)) {
        const uint8_t *blk = a.xq + __mul24(u >> 2, 292);
        const uint8_t *yb = blk + 4 + 64 * (u & 3);
#pragma unroll
        for (int q = 0; q < 4; q++)
            Yr[q] = make_uint4(ld4(yb + 16 * q), ld4(yb + 16 * q + 4), ld4(yb + 16 * q + 8), ld4(yb + 16 * q + 12));
        bsr = make_uint2(ld4(blk + 260 + 8 * (u & 3)), ld4(blk + 264 + 8 * (u & 3)));
        ydr = *reinterpret_cast<const float *>(blk);
    } else {  // k_matvec_rl's LDS layout (stage_acts)
#pragma unroll
        for (int q = 0; q < 4; q++) Yr[q] = *reinterpret_cast<const uint4 *>(lds + (q * T + u) * 16);
        dxr = *reinterpret_cast<const float2 *>(lds + 4 * T * 16 + u * 8);
        syr = *reinterpret_cast<const int2 *>(lds + 4 * T * 16 + T * 8 + u * 8);
    }
    // the iteration's row sum (K-quants: the in-order super-block fold; else the butterfly over T)
    auto row_sum = [&](const WRegs<WT> &cur) -> float {
        if constexpr (is_k(WT)) {
            return rl_row_sum<WT, NSB>(cur, Yr, bsr, ydr, u, lane, T);
        } else {
            int isum, msum;
            float acc = 0.0f;
            unit_dot<WT>(cur, Yr, bsr, u, isum, msum, acc, dxr, syr);
            for (int off = 1; off < T; off <<= 1) acc = acc + __shfl_xor(acc, off);
            return acc;
        }
    };
    if constexpr (!PRO) {
#pragma unroll
        for (int t = 1; t < NB; t++) load_i(t, t);
    }
    auto finish = [&](float acc, int i) {  // (no SwiGLU epilogue here)
        const long row = a.row0 + (long)(wid + i * S) * rpi + rl;
        const bool valid = lane_on && row < a.row1;
        if (u == 0 && valid) {
            if (a.bias) acc = acc + a.bias[row];
            if (a.resid) acc = a.resid[row] + acc;
            a.out[row] = acc;
        }
    };
    int i0 = 0;
    for (; i0 + NB <= n_my; i0 += NB) {
#pragma unroll
        for (int t = 0; t < NB; t++) {
            const float acc = row_sum(R[t]);
            // an opaque zero that depends on acc: the refill of slot t cannot be issued before the
            // slot's registers are read
            int z;
            asm volatile("s_mov_b32 %0, 0" : "=s"(z) : "v"(acc));
            load_i(t, i0 + t + NB + z);
            finish(acc, i0 + t);
        }
    }
#pragma unroll
    for (int t = 0; t < NB; t++)  // the last n_my - i0 < NB iterations, already in flight
        if (i0 + t < n_my) finish(row_sum(R[t]), i0 + t);
}

// Long rows, one token (K-quants with T > 64 units, e.g. n_in = 11008 with 172 units): a wave owns
// whole rows, lane l handles units l, l + 64, ..., l + 64 (NI - 1) of a row. After the quad
// reduction the term of super-block s = 16k + q sits in lane 4q of pass k, and the row sum folds the
// terms in super-block order with lane reads (the reference's sequential f32 order). Each lane keeps
// the activations of its units in registers (read from memory with the first row's weights). Each
// wave walks its rows one at a time.
// PRO = 1: the f32 row a.px is quantised by the workgroup into LDS (q8k_row_lds) instead of read
// from a.xq. WV waves per workgroup: with 4 the row is built before any weight is requested; with
// 8 (half the workgroups, each quantising the row once) the row's loads go out first, then every
// wave's weights, and the workgroup builds the row while the weights stream (its loads, issued
// first, complete first). Measured on the 3B's 2048 x 11008 down: 8 waves 677 tok/s, 4 waves
// 630-635, 16 waves (128 VGPRs: spills) 611, the quantiser's own launch 659-661.
template <int WT, int NI, int PRO = 0, int WV = WAVES>
__global__ __launch_bounds__(64 * WV) void k_matvec_lr(MvArgs a) {
    // the row's super-blocks per wave in one round: up to 16 NI super-blocks over the WV waves
    constexpr int PRO_NR = (16 * NI + WV - 1) / WV < 12 ? (16 * NI + WV - 1) / WV : 12;
    constexpr bool WFIRST = WV > 4;
    const int T = a.P.T, nb = a.P.nb;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long n_rows = a.row1 - a.row0;
    const long G = gridDim.x, bx = blockIdx.x;
    const long vblk = (G % 8 == 0) ? (bx % 8) * (G / 8) + bx / 8 : bx;  // XCD-aware renumbering
    const long S = G * WV, wid = vblk * WV + wave;
    auto load_row = [&](long r, WRegs<WT> (&R)[NI]) {
#pragma unroll
        for (int k = 0; k < NI; k++) {
            const int u = 64 * k + lane;
            load_w<WT>(a.P, (uint32_t)(a.row0 + r), (uint32_t)(u < T ? u : 0), R[k]);
        }
    };
    WRegs<WT> A[NI];
    extern __shared__ uint8_t lds_act[];
    Q8kRow<false, PRO_NR, WV> arow;
    // (with PRO, waves past the rows still take part in the workgroup's activation row: they load
    // row 0 and run no row)
    if constexpr (PRO) {
        arow.issue(a.px, nullptr, a.P.n_in);
        // (the row's loads stay ahead of the weights': the wait before the row is built then
        // covers only them)
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (!WFIRST) arow.build(a.px, 0.0f, a.P.n_in, lds_act);
    } else {
        if (wid >= n_rows) return;
    }
    const long w0 = wid < n_rows ? wid : 0;
    load_row(w0, A);
    // the bias and residual of the row, requested with its weights (lane 0 stores). Every lane
    // loads (an absent one reads a stand-in: the activation row): a load under a lane or pointer
    // test makes the compiler's wait before the activation row also count the weight loads issued
    // ahead of it, so that the row would wait for the first weights to land
    const float *stand_in = PRO ? a.px : reinterpret_cast<const float *>(a.xq);
    const float *bsrc = a.bias ? a.bias : stand_in, *rsrc = a.resid ? a.resid : stand_in;
    float bv = 0.0f, rv = 0.0f;
    auto load_br = [&](long r) {
        bv = bsrc[a.bias ? a.row0 + r : 0];
        rv = rsrc[a.resid ? a.row0 + r : 0];
    };
    load_br(w0);
    if constexpr (PRO && WFIRST) arow.build(a.px, 0.0f, a.P.n_in, lds_act);
    // the lane's activations (the 64 Q8_K bytes of its unit in each pass, their bsums and the block
    // scale) straight from memory into registers, requested with the first row's weights: no LDS
    // staging, no barrier
    uint4 Yr[NI][4];
    uint2 bsr[NI];
    float ydr[NI];
#pragma unroll
    for (int k = 0; k < NI; k++) {
        const int u = 64 * k + lane, uu = u < T ? u : 0;
        if constexpr (PRO) {
            q8k_unit_lds(lds_act, nb, uu, Yr[k], bsr[k], ydr[k]);
            continue;
        }
        const uint8_t *blk = a.xq + (size_t)(uu >> 2) * 292;
        const uint8_t *yb = blk + 4 + 64 * (uu & 3);
#pragma unroll
        for (int q = 0; q < 4; q++)
            Yr[k][q] = make_uint4(ld4(yb + 16 * q), ld4(yb + 16 * q + 4), ld4(yb + 16 * q + 8), ld4(yb + 16 * q + 12));
        bsr[k] = make_uint2(ld4(blk + 260 + 8 * (uu & 3)), ld4(blk + 264 + 8 * (uu & 3)));
        ydr[k] = *reinterpret_cast<const float *>(blk);
    }
    auto body = [&](const WRegs<WT> (&R)[NI], long r) {
        float term[NI];
#pragma unroll
        for (int k = 0; k < NI; k++) {
            const int u = 64 * k + lane, uu = u < T ? u : 0;
            int isum, msum;
            float dummy = 0.0f;
            unit_dot<WT>(R[k], Yr[k], bsr[k], uu, isum, msum, dummy, make_float2(0.f, 0.f), make_int2(0, 0));
            isum = sdy_quad_sum(isum);
            if constexpr (WT == SDY_Q4_K) msum = sdy_quad_sum(msum);
            const float ydv = ydr[k];
            if constexpr (WT == SDY_Q4_K) {
                float d = sdy_h2f((uint16_t)(R[k].c.x & 0xFFFFu)), dmin = sdy_h2f((uint16_t)(R[k].c.x >> 16));
                float dall = ydv * d, dmn = ydv * dmin;
                float t1 = dall * (float)isum, t2 = dmn * (float)msum;
                term[k] = t1 - t2;
            } else {
                float d = sdy_h2f((uint16_t)R[k].g);
                float ydd = ydv * d;
                term[k] = ydd * (float)isum;
            }
        }
        // fold in super-block order: super-block 16k + q is in lane 4q of pass k. The lanes past
        // the row's super-blocks hold +0 and are folded too, with no test per step: the sum starts
        // at +0, so it is never -0, and adding +0 leaves it as it is
#pragma unroll
        for (int k = 0; k < NI; k++)
            if (16 * k + (lane >> 2) >= nb) term[k] = 0.0f;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < NI; k++)
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const float t = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(term[k]), 4 * q));
                acc = acc + t;
            }
        if (lane == 0) {
            if (a.bias) acc = acc + bv;
            if (a.resid) acc = rv + acc;
            a.out[a.row0 + r] = acc;
        }
    };
    // one row in registers per wave: the waves resident on a SIMD overlap each other's loads
    for (long r = wid; r < n_rows; r += S) {
        body(A, r);
        if (r + S < n_rows) {
            load_row(r + S, A);
            load_br(r + S);
        }
    }
}

// ------------------------------------------------------------------ float-weight matvec (F32/F16/BF16)

template <int WT>
SDY_DEV float welem(const uint8_t *w, size_t i) {
    if constexpr (WT == SDY_F32) return reinterpret_cast<const float *>(w)[i];
    else if constexpr (WT == SDY_F16) return sdy_h2f(reinterpret_cast<const uint16_t *>(w)[i]);
    else return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(w)[i] << 16);
}

// Float-weight matvec in the reference's AVX2 order (csrc/ops_avx2.c:61-134, as op_matmul_rows
// splits the work): rows [row0, row1) in pairs from row0 and, with n_tok >= 4, tokens in groups of
// four take block_2x4's order (one 8-lane FMA chain over 8-element steps per (row, token)); the other
// (row, token) pairs take dot's order (four 8-lane chains over 32-element steps, then 8-element steps
// into the first chain, the lane-wise (a0 + a1) + (a2 + a3)). Both then sum the 8 lanes as hsum does,
// ((v0 + v4) + (v2 + v6)) + ((v1 + v5) + (v3 + v7)), and add the n_in % 8 tail one rounded product
// at a time. The results are the reference's bits.

// hsum of the 8 lanes of a group (lane l of the group holds v_l; the result is in every lane)
SDY_DEV float hsum8_group(float v, int base) {
    const float s0 = __shfl(v, base + 0), s1 = __shfl(v, base + 1), s2 = __shfl(v, base + 2), s3 = __shfl(v, base + 3);
    const float s4 = __shfl(v, base + 4), s5 = __shfl(v, base + 5), s6 = __shfl(v, base + 6), s7 = __shfl(v, base + 7);
    return ((s0 + s4) + (s2 + s6)) + ((s1 + s5) + (s3 + s7));
}

template <int WT>
SDY_DEV float float_tail(const uint8_t *wr, const float *xr, int n_in, float sum) {
    for (int i = n_in & ~7; i < n_in; i++) {
        const float p = xr[i] * welem<WT>(wr, i);
        sum = sum + p;
    }
    return sum;
}

template <int WT>
SDY_DEV void float_store(float acc, long row, int t, float *out, long out_stride, const float *bias,
                         const float *resid) {
    if (bias) acc = acc + bias[row];
    if (resid) acc = resid[(size_t)t * out_stride + row] + acc;
    out[(size_t)t * out_stride + row] = acc;
}

// RMSNorm of a one-token row fused into the float matvec that reads it (NORM): the activation is
// (x[i] * scale) * nw[i], scale = 1 / sqrt(mean(x^2) + eps) with k_norm_quant's sum order, and workgroup
// b also writes super-block b of the normalised row's Q8_K bytes (when xq is set) — the bytes
// k_norm_quant writes.
struct FloatNorm {
    const float *nw;
    float eps;
    uint8_t *xq;
};

// dot's order: one (row, token) per 32-lane half-wave. Items: with n_tok >= 4 the paired rows times
// the tokens past the last group of four, then the unpaired last row times every token; with fewer
// tokens every (row, token).
template <int WT, bool NORM = false>
__global__ __launch_bounds__(THREADS) void k_matvec_float_dot(const uint8_t *__restrict__ w, int n_in,
                                                              const float *__restrict__ x, int n_tok, float *out,
                                                              long out_stride, const float *bias, const float *resid,
                                                              long row0, long row1, FloatNorm fn = {}) {
    const int lane = threadIdx.x & 63, L = lane & 31, base = lane & 32;
    constexpr int B = 32;  // steps whose loads go out together before their chain runs in order
    // NORM (one token): the half-wave's first B steps of weights are requested right after the
    // prologue's own loads, before its computation (they do not depend on it); half-waves past the
    // rows read row0's
    float wv0[NORM ? B : 1];
    const bool pre = NORM && (n_in & ~31) >= 32 * 2 * B;
    // NORM: the normalised row in LDS, built by every thread (one token, n_in <= 4096, a multiple of 256)
    __shared__ __align__(16) float xn[NORM ? 4096 : 4];
    if constexpr (NORM) {
        __shared__ double sh[4];
        const int tid = threadIdx.x, wave = tid >> 6, n4 = n_in >> 2;
        float4 keep[4], wk[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int c = tid + 256 * k < n4 ? tid + 256 * k : n4 - 1;
            keep[k] = *reinterpret_cast<const float4 *>(x + 4 * c);
            wk[k] = *reinterpret_cast<const float4 *>(fn.nw + 4 * c);
        }
        __builtin_amdgcn_sched_barrier(0);  // (the prologue's loads stay ahead of the weights')
        {
            const long it = ((long)blockIdx.x * THREADS + threadIdx.x) >> 5;
            const long rr = it < row1 - row0 ? row0 + it : row0;
            const uint8_t *wr0 = w + (size_t)rr * n_in * (WT == SDY_F32 ? 4 : 2);
            // (unconditional, indices clamped to the row, so that the compiler's wait counts stay
            // exact; used only when pre)
#pragma unroll
            for (int j = 0; j < B; j++) wv0[j] = welem<WT>(wr0, min(L + 32 * j, n_in - 1));
        }
        // sdy_row_sumsq's order (x is 16-byte aligned and n_in <= 4096: the four chunks tid + 256 k)
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (tid + 256 * k < n4) {
                const float4 v = keep[k];
                ss += (double)v.x * (double)v.x;
                ss += (double)v.y * (double)v.y;
                ss += (double)v.z * (double)v.z;
                ss += (double)v.w * (double)v.w;
            }
        ss = sdy_block_sum256(ss, sh);
        const float scale = (float)(1.0 / sqrt(ss / (double)n_in + (double)fn.eps));
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (tid + 256 * k < n4)
                *reinterpret_cast<float4 *>(&xn[4 * (tid + 256 * k)]) =
                    make_float4((keep[k].x * scale) * wk[k].x, (keep[k].y * scale) * wk[k].y,
                                (keep[k].z * scale) * wk[k].z, (keep[k].w * scale) * wk[k].w);
        __syncthreads();
        for (int sb = blockIdx.x + wave * gridDim.x; fn.xq && sb < (n_in >> 8); sb += 4 * gridDim.x) {
            const float4 v = *reinterpret_cast<const float4 *>(&xn[256 * sb + 4 * lane]);
            const float xs[4] = {v.x, v.y, v.z, v.w};
            sdy_q8k_block(xs, lane, fn.xq + (size_t)sb * 292);
        }
    }
    // the activation element i (from the normalised row in LDS when NORM)
    auto xe = [&](const float *xr, int i) {
        if constexpr (NORM) return xn[i];
        else return xr[i];
    };
    const long n_rows = row1 - row0, n_pr = n_tok >= 4 ? (n_rows & ~1L) : 0;
    const int n_gt = n_tok >= 4 ? (n_tok & ~3) : 0;
    const long n_a = n_pr * (n_tok - n_gt), n_items = n_a + (n_rows - n_pr) * n_tok;
    const long item = ((long)blockIdx.x * THREADS + threadIdx.x) >> 5;
    if (item >= n_items) return;  // (uniform per half-wave)
    long r;
    int t;
    if (item < n_a) {
        r = item / (n_tok - n_gt);
        t = n_gt + (int)(item - r * (n_tok - n_gt));
    } else {
        const long k = item - n_a;
        r = n_pr + k / n_tok;
        t = (int)(k % n_tok);
    }
    const long row = row0 + r;
    const uint8_t *wr = w + (size_t)row * n_in * (WT == SDY_F32 ? 4 : 2);
    const float *xr = x + (size_t)t * n_in;
    float acc = 0.0f;
    const int n32 = n_in & ~31, n8 = n_in & ~7;
    int i = L;
    if constexpr (NORM) {
        if (pre) {
            // the first B steps, whose weights are in wv0; the next B steps' weights are requested
            // before their chain runs, so that their loads are in flight during it (n_in = 2048:
            // the whole row)
            float wv1[B];
#pragma unroll
            for (int j = 0; j < B; j++) wv1[j] = welem<WT>(wr, i + 32 * (B + j));
#pragma unroll
            for (int j = 0; j < B; j++) acc = fmaf(wv0[j], xe(xr, i + 32 * j), acc);
#pragma unroll
            for (int j = 0; j < B; j++) acc = fmaf(wv1[j], xe(xr, i + 32 * (B + j)), acc);
            i += 32 * 2 * B;
        }
    }
    for (; i + 32 * (B - 1) < n32; i += 32 * B) {
        float wv[B], xv[B];
#pragma unroll
        for (int j = 0; j < B; j++) {
            wv[j] = welem<WT>(wr, i + 32 * j);
            xv[j] = xe(xr, i + 32 * j);
        }
#pragma unroll
        for (int j = 0; j < B; j++) acc = fmaf(wv[j], xv[j], acc);
    }
    for (; i + 32 * 7 < n32; i += 32 * 8) {
        float wv[8], xv[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            wv[j] = welem<WT>(wr, i + 32 * j);
            xv[j] = xe(xr, i + 32 * j);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) acc = fmaf(wv[j], xv[j], acc);
    }
    for (; i < n32; i += 32) acc = fmaf(welem<WT>(wr, i), xe(xr, i), acc);
    if (L < 8)
        for (int i = n32 + L; i < n8; i += 8) acc = fmaf(welem<WT>(wr, i), xe(xr, i), acc);
    // lanes 0..7 of the half: v_l = (a0_l + a1_l) + (a2_l + a3_l)
    const float a1 = __shfl(acc, base + ((L + 8) & 31)), a2 = __shfl(acc, base + ((L + 16) & 31)),
                a3 = __shfl(acc, base + ((L + 24) & 31));
    const float v = (acc + a1) + (a2 + a3);
    float sum = hsum8_group(v, base);
    if (L == 0) float_store<WT>(float_tail<WT>(wr, xr, n_in, sum), row, t, out, out_stride, bias, resid);
}

// block_2x4's order: one (row, token) per 8-lane group, for the paired rows times the tokens of the
// groups of four (n_tok >= 4).
template <int WT>
__global__ __launch_bounds__(THREADS) void k_matvec_float_block(const uint8_t *__restrict__ w, int n_in,
                                                                const float *__restrict__ x, int n_tok, float *out,
                                                                long out_stride, const float *bias,
                                                                const float *resid, long row0, long row1) {
    const int lane = threadIdx.x & 63, l = lane & 7, base = lane & 56;
    const long n_pr = (row1 - row0) & ~1L;
    const int n_gt = n_tok & ~3;
    const long item = ((long)blockIdx.x * THREADS + threadIdx.x) >> 3;
    if (item >= n_pr * n_gt) return;  // (uniform per group)
    const long r = item / n_gt;
    const int t = (int)(item - r * n_gt);
    const long row = row0 + r;
    const uint8_t *wr = w + (size_t)row * n_in * (WT == SDY_F32 ? 4 : 2);
    const float *xr = x + (size_t)t * n_in;
    float acc = 0.0f;
    const int n8 = n_in & ~7;
    int i = l;
    for (; i + 8 * 7 < n8; i += 8 * 8) {  // 8 steps' loads first, then their chain in order
        float wv[8], xv[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            wv[j] = welem<WT>(wr, i + 8 * j);
            xv[j] = xr[i + 8 * j];
        }
#pragma unroll
        for (int j = 0; j < 8; j++) acc = fmaf(wv[j], xv[j], acc);
    }
    for (; i < n8; i += 8) acc = fmaf(welem<WT>(wr, i), xr[i], acc);
    const float sum = hsum8_group(acc, base);
    if (l == 0) float_store<WT>(float_tail<WT>(wr, xr, n_in, sum), row, t, out, out_stride, bias, resid);
}

// block_2x4's order for many rows and tokens (the MoE router over a prompt's tokens): a workgroup of
// 32 groups of 8 lanes owns 16 rows x 16 tokens; group g computes the 2 x 4 (row, token) pairs of
// rows 2 (g / 4) + {0, 1}, tokens 4 (g % 4) + {0..3}, lane l carrying chain l (elements l, l + 8, ...
// in order) of all eight, from row and token tiles of FT_K elements staged in LDS (as f32) that the
// whole workgroup shares, the next tile's loads in flight while the current one is multiplied. In
// LDS a row's chain l is contiguous (element 8 s + l at [row][l][s]), so a lane reads four steps of
// a row with one 16-byte read. The chains, the hsum tree and the tail are k_matvec_float_block's,
// so the bits are the same; an element is read from memory once per workgroup instead of once per
// pair.
typedef float ft_f32x4 __attribute__((ext_vector_type(4)));
constexpr int FT_ROWS = 16, FT_TOKS = 16, FT_K = 256;
constexpr int FT_SP = FT_K / 8 + 4;  // floats per (row, chain) in LDS: the 8 chains' 16-byte reads in distinct banks

template <int WT>
__global__ __launch_bounds__(256) void k_matvec_float_tile(const uint8_t *__restrict__ w, int n_in,
                                                          const float *__restrict__ x, int n_tok, float *out,
                                                          long out_stride, const float *bias, const float *resid,
                                                          long row0, long row1) {
    constexpr int NTH = 256, NW = FT_ROWS * FT_K / NTH / 4, NX = FT_TOKS * FT_K / NTH / 4;  // 4-element loads
    __shared__ __align__(16) float ws[FT_ROWS * 8 * FT_SP], xs[FT_TOKS * 8 * FT_SP];
    const int tid = threadIdx.x, l = tid & 7, g = tid >> 3, rb = g >> 2, tb = g & 3;
    const int base = (tid & 63) & 56;
    const long n_pr = (row1 - row0) & ~1L;
    const int n_gt = n_tok & ~3;
    const long r_tile = row0 + (long)blockIdx.y * FT_ROWS;
    const int t_tile = blockIdx.x * FT_TOKS;
    const int n8 = n_in & ~7;
    float acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;
    // a chunk's elements in 4-element loads, all requested before any is used (elements i .. i + 3,
    // i = 4 (tid + u NTH): row i / FT_K of the tile, columns i % FT_K ...; clamped rows and columns
    // past the chunk read in bounds; kn is a multiple of 8, so a load is wholly in or out)
    ft_f32x4 wv[NW], xv[NX];
    auto fetch = [&](int k0, int kn) {
#pragma unroll
        for (int u = 0; u < NW; u++) {
            const int i = 4 * (tid + u * NTH), r = i / FT_K, e = i - r * FT_K;
            const long row = r_tile + r < row0 + n_pr ? r_tile + r : row0;
            const size_t o = (size_t)row * n_in + k0 + (e < kn ? e : 0);
            if constexpr (WT == SDY_F32) {
                wv[u] = *reinterpret_cast<const ft_f32x4 *>(reinterpret_cast<const float *>(w) + o);
            } else {
                const uint2 h = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(w) + o);
                const uint16_t hv[4] = {(uint16_t)(h.x & 0xFFFFu), (uint16_t)(h.x >> 16), (uint16_t)(h.y & 0xFFFFu),
                                        (uint16_t)(h.y >> 16)};
#pragma unroll
                for (int c = 0; c < 4; c++)
                    wv[u][c] = WT == SDY_F16 ? sdy_h2f(hv[c]) : __uint_as_float((uint32_t)hv[c] << 16);
            }
        }
#pragma unroll
        for (int u = 0; u < NX; u++) {
            const int i = 4 * (tid + u * NTH), t = i / FT_K, e = i - t * FT_K;
            const int tk = t_tile + t < n_gt ? t_tile + t : 0;
            xv[u] = *reinterpret_cast<const ft_f32x4 *>(x + (size_t)tk * n_in + k0 + (e < kn ? e : 0));
        }
    };
    const float *wr = ws + (2 * rb * 8 + l) * FT_SP, *xr = xs + (4 * tb * 8 + l) * FT_SP;
    // steps 4 q .. 4 q + 3 of the lane's chain (elements 8 (4q + c) + l)
    auto step4 = [&](int q) {
        ft_f32x4 a[2], b[4];
#pragma unroll
        for (int i = 0; i < 2; i++) a[i] = *reinterpret_cast<const ft_f32x4 *>(wr + i * 8 * FT_SP + 4 * q);
#pragma unroll
        for (int j = 0; j < 4; j++) b[j] = *reinterpret_cast<const ft_f32x4 *>(xr + j * 8 * FT_SP + 4 * q);
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = fmaf(a[i][c], b[j][c], acc[i][j]);
    };
    auto step1 = [&](int st) {  // one step (a chunk's last steps, when they are not a multiple of 4)
        float a[2], b[4];
#pragma unroll
        for (int i = 0; i < 2; i++) a[i] = wr[i * 8 * FT_SP + st];
#pragma unroll
        for (int j = 0; j < 4; j++) b[j] = xr[j * 8 * FT_SP + st];
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    };
    if (n8 > 0) fetch(0, n8 < FT_K ? n8 : FT_K);
    for (int k0 = 0; k0 < n8; k0 += FT_K) {
        const int kn = n8 - k0 < FT_K ? n8 - k0 : FT_K;  // a multiple of 8
        __syncthreads();  // the previous chunk's reads are done
#pragma unroll
        for (int u = 0; u < NW; u++) {
            const int i = 4 * (tid + u * NTH), r = i / FT_K, e = i - r * FT_K;
#pragma unroll
            for (int c = 0; c < 4; c++) ws[(r * 8 + ((e + c) & 7)) * FT_SP + (e >> 3)] = wv[u][c];
        }
#pragma unroll
        for (int u = 0; u < NX; u++) {
            const int i = 4 * (tid + u * NTH), t = i / FT_K, e = i - t * FT_K;
#pragma unroll
            for (int c = 0; c < 4; c++) xs[(t * 8 + ((e + c) & 7)) * FT_SP + (e >> 3)] = xv[u][c];
        }
        __syncthreads();
        if (k0 + FT_K < n8) fetch(k0 + FT_K, n8 - k0 - FT_K < FT_K ? n8 - k0 - FT_K : FT_K);
        const int ns = kn >> 3;  // steps of the chunk
        if (ns == FT_K / 8) {
#pragma unroll
            for (int q = 0; q < FT_K / 32; q++) step4(q);
        } else {
            int st = 0;
            for (; st + 4 <= ns; st += 4) step4(st >> 2);
            for (; st < ns; st++) step1(st);
        }
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float sum = hsum8_group(acc[i][j], base);
            const long row = r_tile + 2 * rb + i;
            const int t = t_tile + 4 * tb + j;
            if (l == 0 && row < row0 + n_pr && t < n_gt) {
                const uint8_t *wrow = w + (size_t)row * n_in * (WT == SDY_F32 ? 4 : 2);
                float_store<WT>(float_tail<WT>(wrow, x + (size_t)t * n_in, n_in, sum), row, t, out, out_stride, bias,
                                resid);
            }
        }
}

}  // namespace

// =============================================================================== host launchers

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }



static int n_units(int type, int n_in) {
    if (type == SDY_Q4_K || type == SDY_Q6_K) return n_in / 64;
    return (n_in + 63) / 64;
}

static int n_blocks(int type, int n_in) {
    if (type == SDY_Q4_K || type == SDY_Q6_K) return n_in / 256;
    return n_in / 32;
}

// per-row bytes of each plane
static void plane_row_bytes(int type, int n_in, size_t pb[5]) {
    int T = n_units(type, n_in), nb = n_blocks(type, n_in);
    for (int i = 0; i < 5; i++) pb[i] = 0;
    switch (type) {
    case SDY_Q4_K: pb[0] = pb[1] = 16u * T; pb[2] = 16u * nb; break;
    case SDY_Q6_K: pb[0] = pb[1] = pb[2] = 16u * T; pb[3] = 16u * nb; pb[4] = 2u * nb; break;
    case SDY_Q8_0: pb[0] = pb[1] = pb[2] = pb[3] = 16u * T; pb[4] = 4u * T; break;
    case SDY_Q4_0: pb[0] = pb[1] = 16u * T; pb[4] = 4u * T; break;
    case SDY_Q5_0: pb[0] = pb[1] = 16u * T; pb[2] = 8u * T; pb[4] = 4u * T; break;
    case SDY_F32: pb[0] = 4u * n_in; break;
    case SDY_F16: case SDY_BF16: pb[0] = 2u * n_in; break;
    default: break;
    }
}

static bool type_ok(int type) {
    switch (type) {
    case SDY_F32: case SDY_F16: case SDY_BF16: case SDY_Q8_0: case SDY_Q4_0: case SDY_Q5_0: case SDY_Q4_K:
    case SDY_Q6_K: return true;
    default: return false;
    }
}

static bool is_float_type(int type) { return type == SDY_F32 || type == SDY_F16 || type == SDY_BF16; }

size_t sdy_raw_row_bytes(int type, int n_in) {
    switch (type) {
    case SDY_F32: return 4u * n_in;
    case SDY_F16: case SDY_BF16: return 2u * n_in;
    case SDY_Q8_0: return (size_t)(n_in / 32) * 34;
    case SDY_Q4_0: return (size_t)(n_in / 32) * 18;
    case SDY_Q5_0: return (size_t)(n_in / 32) * 22;
    case SDY_Q4_K: return (size_t)(n_in / 256) * 144;
    case SDY_Q6_K: return (size_t)(n_in / 256) * 210;
    case SDY_Q8_K: return (size_t)(n_in / 256) * 292;
    default: return 0;
    }
}

extern "C" size_t sdy_mat_bytes(int type, int n_in, long n_rows) {
    size_t pb[5], tot = 0;
    plane_row_bytes(type, n_in, pb);
    for (int i = 0; i < 5; i++)
        if (pb[i]) tot += align256(pb[i] * (size_t)n_rows);
    return tot;
}

static Planes planes_of(const sdy_mat *m) {
    Planes P;
    for (int i = 0; i < 5; i++) P.p[i] = (const uint8_t *)m->base + m->plane_off[i];
    P.n_in = m->n_in;
    P.T = m->n_units;
    P.nb = n_blocks(m->type, m->n_in);
    return P;
}

static int check_shape(int type, int n_in, long n_rows) {
    if (!type_ok(type)) return sdy_fail(-1, "weight type %d not supported on the GPU path", type);
    if (n_in <= 0 || n_rows <= 0) return sdy_fail(-1, "empty matrix (%d x %ld)", n_in, n_rows);
    if ((type == SDY_Q4_K || type == SDY_Q6_K) && n_in % 256)
        return sdy_fail(-1, "K-quant rows must be a multiple of 256 (got %d)", n_in);
    if ((type == SDY_Q8_0 || type == SDY_Q4_0 || type == SDY_Q5_0) && n_in % 32)
        return sdy_fail(-1, "32-element block rows must be a multiple of 32 (got %d)", n_in);
    return 0;
}

static int mat_alloc(sdy_mat *m, int type, int n_in, long n_rows, bool host) {
    int rc = check_shape(type, n_in, n_rows);
    if (rc) return rc;
    memset(m, 0, sizeof(*m));
    m->type = type;
    m->n_in = n_in;
    m->n_rows = n_rows;
    m->n_units = n_units(type, n_in);
    m->bytes = sdy_mat_bytes(type, n_in, n_rows);
    if ((rc = host ? sdy_host_alloc_mapped(&m->hbase, &m->base, m->bytes) : sdy_malloc(&m->base, m->bytes))) return rc;
    size_t pb[5], off = 0;
    plane_row_bytes(type, n_in, pb);
    for (int i = 0; i < 5; i++) {
        m->plane_off[i] = off;
        if (pb[i]) off += align256(pb[i] * (size_t)n_rows);
    }
    // zero rows pass the GEMM check, so a matrix filled in several uploads is checked piecewise. A
    // matrix in host memory is not checked (the check's reads would cross the host link) and takes
    // the GEMM's wide variant, exact for every block
    m->gemm_ok = type == SDY_Q4_K || type == SDY_Q6_K ? (host ? 2 : 1) : 0;
    // (zeroed by the GPU for host memory too: its pages are mapped to the device at allocation, and the
    // CPU's first touch of each would fault. Completed before returning: the uploads run on other,
    // non-blocking streams)
    if (m->gemm_ok && ((rc = sdy_memset(m->base, 0, m->bytes, nullptr)) || (rc = sdy_sync(nullptr)))) return rc;
    return 0;
}

extern "C" int sdy_mat_alloc(sdy_mat *m, int type, int n_in, long n_rows) {
    return mat_alloc(m, type, n_in, n_rows, false);
}

extern "C" int sdy_mat_alloc_host(sdy_mat *m, int type, int n_in, long n_rows) {
    return mat_alloc(m, type, n_in, n_rows, true);
}

// The GEMM's copy of m, stale once rows change: freed (the GEMM then reads the planes).
static int drop_gemm_layout(sdy_mat *m) {
    if (!m->gbase) return 0;
    const int rc = sdy_free(m->gbase);
    m->gbase = nullptr;
    m->gbytes = 0;
    return rc;
}

// Repacks n raw GGUF-layout rows (device memory) into rows r0 + map(i) of m (RowMap above),
// queued on s (no allocation, no synchronisation).
static int repack_rows_async(sdy_mat *m, long r0, RowMap map, long n, const void *dev_raw, sdy_stream s) {
    hipStream_t st = (hipStream_t)s;
    if (int rc = drop_gemm_layout(m)) return rc;
    const int type = m->type;
    const size_t src_row = sdy_raw_row_bytes(type, m->n_in);
    if (is_float_type(type)) {
        if (map.step != 1 || map.gstride != 0)
            return sdy_fail(-1, "interleaved layouts are for quantized types");
        return sdy_d2d((uint8_t *)m->base + m->plane_off[0] + src_row * r0, dev_raw, src_row * n, s);
    }
    size_t pb[5];
    plane_row_bytes(type, m->n_in, pb);
    DstPlanes dst;
    for (int i = 0; i < 5; i++) dst.p[i] = (uint8_t *)m->base + m->plane_off[i] + pb[i] * (size_t)r0;
    Planes P = planes_of(m);
    long total = n * (long)m->n_units;
    dim3 grid((unsigned)((total + 255) / 256)), block(256);
    const uint8_t *src = (const uint8_t *)dev_raw;
    switch (type) {
    case SDY_Q4_K: hipLaunchKernelGGL(k_repack<SDY_Q4_K>, grid, block, 0, st, src, src_row, P, dst, n, map); break;
    case SDY_Q6_K: hipLaunchKernelGGL(k_repack<SDY_Q6_K>, grid, block, 0, st, src, src_row, P, dst, n, map); break;
    case SDY_Q8_0: hipLaunchKernelGGL(k_repack<SDY_Q8_0>, grid, block, 0, st, src, src_row, P, dst, n, map); break;
    case SDY_Q4_0: hipLaunchKernelGGL(k_repack<SDY_Q4_0>, grid, block, 0, st, src, src_row, P, dst, n, map); break;
    case SDY_Q5_0: hipLaunchKernelGGL(k_repack<SDY_Q5_0>, grid, block, 0, st, src, src_row, P, dst, n, map); break;
    }
    return sdy_check_launch("repack");
}

static int repack_rows(sdy_mat *m, long r0, RowMap map, long n, const void *dev_raw, sdy_stream s) {
    int rc = repack_rows_async(m, r0, map, n, dev_raw, s);
    return rc ? rc : sdy_sync(s);
}

// The last destination row and the end of the first group's span of an n-row map from r0 (or -1
// with an error when they fall outside m).
static int map_bounds(const sdy_mat *m, long r0, long n, long step, long grp, long gstride, long *span) {
    if (n < 0 || r0 < 0 || step < 1 || grp < 1 || gstride < 0) return sdy_fail(-1, "upload: bad row map");
    if (n == 0) return 0;
    const long last = r0 + ((n - 1) / grp) * gstride + ((n - 1) % grp) * step;
    *span = r0 + ((n - 1) / grp) * gstride + (grp - 1 < n - 1 ? grp - 1 : n - 1) * step;
    if (last >= m->n_rows || *span >= m->n_rows)
        return sdy_fail(-1, "upload of %ld rows from row %ld (step %ld) outside %ld rows", n, r0, step, m->n_rows);
    return 0;
}

extern "C" int sdy_mat_repack_async(sdy_mat *m, long r0, long n, long step, long grp, long gstride,
                                    const void *dev_raw, sdy_stream s) {
    long span = 0;
    const int rc = map_bounds(m, r0, n, step, grp, gstride, &span);
    if (rc || n == 0) return rc;
    return repack_rows_async(m, r0, RowMap{step, grp, gstride}, n, dev_raw, s);
}

extern "C" int sdy_mat_from_device(sdy_mat *m, int type, int n_in, long n_rows, const void *dev_raw, sdy_stream s) {
    int rc = sdy_mat_alloc(m, type, n_in, n_rows);
    if (rc) return rc;
    if ((rc = repack_rows(m, 0, RowMap{1, n_rows, 0}, n_rows, dev_raw, s))) {
        sdy_mat_free(m);
        return rc;
    }
    if (m->gemm_ok) {
        int bad = 1;
        if ((rc = sdy_gemm_check_rows(m, 0, n_rows, &bad, s))) return rc;
        if (bad) m->gemm_ok = 2;
    }
    return 0;
}

extern "C" int sdy_mat_upload_map(sdy_mat *m, long r0, long n, long step, long grp, long gstride,
                                  const void *host_raw, sdy_stream s) {
    long span = 0;
    int rc = map_bounds(m, r0, n, step, grp, gstride, &span);
    if (rc || n == 0) return rc;
    size_t raw = sdy_raw_row_bytes(m->type, m->n_in) * (size_t)n;
    void *tmp = nullptr;
    if ((rc = sdy_malloc(&tmp, raw))) return rc;
    if (!(rc = sdy_h2d(tmp, host_raw, raw, s))) rc = repack_rows(m, r0, RowMap{step, grp, gstride}, n, tmp, s);
    if (!rc) rc = sdy_sync(s);
    sdy_free(tmp);
    if (!rc && m->gemm_ok) {
        int bad = 1;
        rc = sdy_gemm_check_rows(m, r0, span - r0 + 1, &bad, s);
        if (!rc && bad) m->gemm_ok = 2;
    }
    return rc;
}

extern "C" int sdy_mat_upload_rows(sdy_mat *m, long r0, long step, long n, const void *host_raw, sdy_stream s) {
    return sdy_mat_upload_map(m, r0, n, step, n > 0 ? n : 1, 0, host_raw, s);
}

extern "C" int sdy_mat_upload(sdy_mat *m, int type, int n_in, long n_rows, const void *host_raw, sdy_stream s) {
    int rc = sdy_mat_alloc(m, type, n_in, n_rows);
    if (rc) return rc;
    if ((rc = sdy_mat_upload_rows(m, 0, 1, n_rows, host_raw, s))) sdy_mat_free(m);
    return rc;
}

extern "C" int sdy_mat_free(sdy_mat *m) {
    if (!m || !m->base) return 0;
    int rc = drop_gemm_layout(m);
    const int rc2 = m->hbase ? sdy_host_free(m->hbase) : sdy_free(m->base);
    m->base = m->hbase = nullptr;
    return rc ? rc : rc2;
}

extern "C" sdy_mat sdy_mat_rows(const sdy_mat *m, long r0, long n) {
    // A view: plane pointers advanced by r0 rows. Planes are per-row arrays, so the view keeps the
    // same base with shifted offsets.
    sdy_mat v = *m;
    size_t pb[5];
    plane_row_bytes(m->type, m->n_in, pb);
    for (int i = 0; i < 5; i++) v.plane_off[i] = m->plane_off[i] + pb[i] * (size_t)r0;
    v.grow0 = m->grow0 + r0;  // the GEMM's copy (shared) is addressed by rows of the whole matrix
    v.n_rows = n;
    return v;
}

static int dequant_impl(const sdy_mat *m, const int32_t *idx, long r0, long n, float *out, sdy_stream s) {
    hipStream_t st = (hipStream_t)s;
    if (n <= 0) return 0;
    if (is_float_type(m->type)) {
        long total = n * (long)m->n_in;
        dim3 grid((unsigned)((total + 255) / 256));
        const uint8_t *w = (const uint8_t *)m->base + m->plane_off[0];
        switch (m->type) {
        case SDY_F32: hipLaunchKernelGGL(k_dequant_float<SDY_F32>, grid, dim3(256), 0, st, w, m->n_in, idx, r0, n, out); break;
        case SDY_F16: hipLaunchKernelGGL(k_dequant_float<SDY_F16>, grid, dim3(256), 0, st, w, m->n_in, idx, r0, n, out); break;
        default: hipLaunchKernelGGL(k_dequant_float<SDY_BF16>, grid, dim3(256), 0, st, w, m->n_in, idx, r0, n, out); break;
        }
        return sdy_check_launch("dequant_float");
    }
    Planes P = planes_of(m);
    long total = n * (long)P.T;
    dim3 grid((unsigned)((total + 127) / 128)), block(128);
    switch (m->type) {
    case SDY_Q4_K: hipLaunchKernelGGL(k_dequant<SDY_Q4_K>, grid, block, 0, st, P, idx, r0, n, out); break;
    case SDY_Q6_K: hipLaunchKernelGGL(k_dequant<SDY_Q6_K>, grid, block, 0, st, P, idx, r0, n, out); break;
    case SDY_Q8_0: hipLaunchKernelGGL(k_dequant<SDY_Q8_0>, grid, block, 0, st, P, idx, r0, n, out); break;
    case SDY_Q4_0: hipLaunchKernelGGL(k_dequant<SDY_Q4_0>, grid, block, 0, st, P, idx, r0, n, out); break;
    case SDY_Q5_0: hipLaunchKernelGGL(k_dequant<SDY_Q5_0>, grid, block, 0, st, P, idx, r0, n, out); break;
    default: return sdy_fail(-1, "dequant: type %d", m->type);
    }
    return sdy_check_launch("dequant");
}

extern "C" int sdy_dequant_rows(const sdy_mat *m, long r0, long n, float *out, sdy_stream s) {
    if (r0 < 0 || r0 + n > m->n_rows) return sdy_fail(-1, "dequant rows [%ld, %ld) outside %ld rows", r0, r0 + n, m->n_rows);
    return dequant_impl(m, nullptr, r0, n, out, s);
}

extern "C" int sdy_dequant_gather(const sdy_mat *m, const int32_t *idx, int n, float *out, sdy_stream s) {
    return dequant_impl(m, idx, 0, n, out, s);
}

extern "C" int sdy_quantize(int vtype, const float *x, void *xq, int n_in, int n_tok, sdy_stream s) {
    hipStream_t st = (hipStream_t)s;
    if (n_tok <= 0) return 0;
    if (vtype == SDY_Q8_K) {
        if (n_in % 256) return sdy_fail(-1, "Q8_K rows must be a multiple of 256 (got %d)", n_in);
        hipLaunchKernelGGL(k_quant_q8k, dim3((n_in / 256 + 3) / 4, n_tok), dim3(256), 0, st, x, (uint8_t *)xq, n_in,
                           SdyGemmExp{nullptr, nullptr, nullptr});
        return sdy_check_launch("quant_q8k");
    }
    if (vtype == SDY_Q8_0) {
        if (n_in % 32) return sdy_fail(-1, "Q8_0 rows must be a multiple of 32 (got %d)", n_in);
        int nblk = n_in / 32;
        hipLaunchKernelGGL(k_quant_q8_0, dim3((nblk + 1) / 2, n_tok), dim3(64), 0, st, x, (uint8_t *)xq, n_in);
        return sdy_check_launch("quant_q8_0");
    }
    return sdy_fail(-1, "activation type %d", vtype);
}

// Q8_K rows plus the GEMM's expansion of them in ws (the layout sdy_gemm reads)
extern "C" int sdy_quantize_gemm(const float *x, void *xq, int n_in, int n_tok, void *ws, sdy_stream s) {
    if (n_tok <= 0) return 0;
    if (n_in % 256) return sdy_fail(-1, "Q8_K rows must be a multiple of 256 (got %d)", n_in);
    hipLaunchKernelGGL(k_quant_q8k, dim3((n_in / 256 + 3) / 4, n_tok), dim3(256), 0, (hipStream_t)s, x, (uint8_t *)xq,
                       n_in, sdy_gemm_exp(ws, n_tok, n_in));
    return sdy_check_launch("quant_q8k");
}

static int g_n_cu = 0;

// Rows per batch: the smallest count giving at least 64 (row, unit) tasks with little idle-lane
// waste, so that small matrices spread over many waves; long rows (T >= 64) take one row per batch.
// With the SwiGLU epilogue the count is rounded up to even, so that a (gate, up) pair of rows
// never straddles two batches.
static int rows_per_batch(int T, bool swiglu) {
    int rb = 64;
    if (T >= 64) rb = 1;
    else if (64 % T == 0) rb = 64 / T;
    else
        for (int r = (64 + T - 1) / T; r < 64; r++) {
            int tasks = r * T, its = (tasks + 63) / 64;
            if (its * 64 - tasks <= its * 8) {  // at most 1/8 of the lanes idle
                rb = r;
                break;
            }
        }
    return swiglu ? (rb + 1) & ~1 : rb;
}

// LDS bytes of k_matvec: staged activations of MT tokens plus the per-wave term buffers.
static size_t mv_lds_bytes(int wt, int T, int nb, int MT, int rb) {
    int nterm = is_k(wt) ? nb : T;
    return (size_t)MT * 4 * T * 16 + (size_t)MT * T * 16 + (size_t)WAVES * rb * MT * nterm * 4;
}

constexpr size_t LDS_MAX = 160 * 1024;

template <int WT, int MT, bool YREG>
static int launch_mv_k(MvArgs &A, size_t lds, hipStream_t st) {
    static int per_cu = 0;  // resident workgroups per CU for this instantiation (at this LDS size)
    static size_t per_cu_lds = 0, granted = 0;
    const void *fn = (const void *)k_matvec<WT, MT, YREG>;
    int rc = sdy_lds_limit(fn, lds, &granted);
    if (rc) return rc;
    if (per_cu == 0 || per_cu_lds != lds) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, THREADS, lds) != hipSuccess || n < 1) n = 1;
        per_cu = n;
        per_cu_lds = lds;
    }
    long n_rows = A.row1 - A.row0;
    long n_batches = (n_rows + A.rb - 1) / A.rb;
    long wgs = (n_batches + WAVES - 1) / WAVES;
    long cap = (long)(g_n_cu ? g_n_cu : 256) * per_cu;
    if (wgs > cap) wgs = cap;
    SDY_NOTE_KERNEL((k_matvec<WT, MT, YREG>));
    hipLaunchKernelGGL((k_matvec<WT, MT, YREG>), dim3((unsigned)wgs), dim3(THREADS), lds, st, A);
    return sdy_check_launch("matvec");
}

static size_t mv_lds_bytes_rl(int T, int MT) { return (size_t)MT * 4 * T * 16 + (size_t)MT * T * 16; }

// Workgroups of a THREADS-thread kernel with `lds` bytes of dynamic LDS that the GPU holds at once
// (the occupancy is cached per kernel and LDS size).
static long resident_wgs(const void *fn, size_t lds, int &per_cu, size_t &per_cu_lds, int threads = THREADS) {
    if (per_cu == 0 || per_cu_lds != lds) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, lds) != hipSuccess || n < 1) n = 1;
        per_cu = n;
        per_cu_lds = lds;
    }
    return (long)(g_n_cu ? g_n_cu : 256) * per_cu;
}

// LDS of the workgroup-quantised activation row (q8k_row_lds): 0 when the kernel reads a.xq
static size_t pro_lds(const MvArgs &A) { return A.px ? (size_t)A.P.nb * 292 : 0; }
static int pro_kind(const MvArgs &A) { return A.px ? (A.pnw ? 2 : 1) : A.route_logits ? 3 : 0; }

template <int WT, int NIT, int NSB, int PRO, int WV>
static long cap_1t(size_t lds) {
    static int per_cu = 0;
    static size_t per_cu_lds = 0;
    return resident_wgs((const void *)k_matvec_1t<WT, NIT, NSB, PRO, WV>, lds, per_cu, per_cu_lds, 64 * WV);
}


static void prep_1t(MvArgs &A) {
    A.rpi = 64 / A.P.T;
    A.tmag = (65536 + A.P.T - 1) / A.P.T;
    A.n_it = (int)((A.row1 - A.row0 + A.rpi - 1) / A.rpi);
}

// One token on k_matvec_1t with the smallest NIT (iterations per wave, at most 4) whose grid the GPU
// holds at once, so that every wave's loads go out at the start; 1 when no NIT fits (the caller
// then runs the persistent k_matvec_rl).
// (dry: report whether some NIT fits, launch nothing)
template <int WT, int NSB, int PRO, int WV = WAVES>
static int launch_mv_1t_nsb(MvArgs &A, hipStream_t st, int n_slot, bool dry) {
    const long n_it = A.n_it;
    const size_t lds = pro_lds(A);
    auto wgs = [&](int nit) { return (n_it + (long)WV * nit - 1) / ((long)WV * nit); };
#define SDY_1T(NIT)                                                                                                  \
    if (wgs(NIT) * n_slot <= cap_1t<WT, NIT, NSB, PRO, WV>(lds)) {                                                   \
        if (dry) return 0;                                                                                           \
        SDY_NOTE_KERNEL((k_matvec_1t<WT, NIT, NSB, PRO, WV>));                                                        \
        hipLaunchKernelGGL((k_matvec_1t<WT, NIT, NSB, PRO, WV>), dim3((unsigned)wgs(NIT), (unsigned)n_slot),           \
                           dim3(64 * WV), lds, st, A);                                                               \
        return sdy_check_launch("matvec");                                                                           \
    }
    if (PRO || n_slot > 1) {
        // the workgroup-quantised row is built once per workgroup: fewer, fuller workgroups while
        // every CU still gets three (measured on the 22016 x 2048 gate|up: NIT 3); the same for the
        // grouped launches, counting every slot's workgroups
        const long want = 3L * (g_n_cu ? g_n_cu : 256) * WAVES / WV;
        if (wgs(4) * n_slot >= want) { SDY_1T(4) }
        if (wgs(3) * n_slot >= want) { SDY_1T(3) }
        if (wgs(2) * n_slot >= want) { SDY_1T(2) }
    }
    SDY_1T(1)
    SDY_1T(2)
    SDY_1T(3)
    SDY_1T(4)
#undef SDY_1T
    return 1;
}

template <int WT, int PRO, int WV = WAVES>
static int launch_mv_1t_wv(MvArgs &A, hipStream_t st, int n_slot, bool dry) {
    switch (A.P.T) {  // NSB: the row's super-block count when it is a common one (n_in 768, 2048, 4096)
    case 12: return launch_mv_1t_nsb<WT, 3, PRO, WV>(A, st, n_slot, dry);
    case 32: return launch_mv_1t_nsb<WT, 8, PRO, WV>(A, st, n_slot, dry);
    case 64: return launch_mv_1t_nsb<WT, 16, PRO, WV>(A, st, n_slot, dry);
    default: return launch_mv_1t_nsb<WT, 0, PRO, WV>(A, st, n_slot, dry);
    }
}

// The RMS-normalised row (PRO 2) on 8-wave workgroups that build it while the weights stream: 3B
// decode 682-685 against 674-676 tok/s with 4-wave workgroups building it before requesting them
// (30B-A3B: 453 against 452). The quantiser alone (PRO 1) stays on 4 waves (8: 682-688 against
// 687-690).
template <int WT, int PRO>
static int launch_mv_1t_pro(MvArgs &A, hipStream_t st, int n_slot, bool dry) {
    if constexpr (PRO == 2) return launch_mv_1t_wv<WT, PRO, 8>(A, st, n_slot, dry);
    return launch_mv_1t_wv<WT, PRO>(A, st, n_slot, dry);
}

template <int WT>
static int launch_mv_1t(MvArgs &A, hipStream_t st, int n_slot, bool dry = false) {
    prep_1t(A);
    switch (pro_kind(A)) {
    case 1: return launch_mv_1t_pro<WT, 1>(A, st, n_slot, dry);
    case 2: return launch_mv_1t_pro<WT, 2>(A, st, n_slot, dry);
    case 3: return launch_mv_1t_pro<WT, 3>(A, st, n_slot, dry);
    default: return launch_mv_1t_pro<WT, 0>(A, st, n_slot, dry);
    }
}

template <int WT, int NB, int NSB, int PRO = 0>
static int launch_mv_ring_nsb(MvArgs &A, hipStream_t st, bool dry = false) {
    static int per_cu = 0;
    static size_t per_cu_lds = 0;
    const size_t lds = PRO ? pro_lds(A) : is_k(WT) ? 0 : mv_lds_bytes_rl(A.P.T, 1);
    long wgs = ((long)A.n_it + WAVES - 1) / WAVES;
    const long cap = resident_wgs((const void *)k_matvec_ring<WT, NB, NSB, PRO>, lds, per_cu, per_cu_lds);
    if (wgs > cap) wgs = cap;
    if (wgs > 8) wgs &= ~7L;  // a multiple of 8: the XCD-aware numbering applies
    if (dry) return 0;
    SDY_NOTE_KERNEL((k_matvec_ring<WT, NB, NSB, PRO>));
    hipLaunchKernelGGL((k_matvec_ring<WT, NB, NSB, PRO>), dim3((unsigned)wgs), dim3(THREADS), lds, st, A);
    return sdy_check_launch("matvec");
}

// one token, one slot: the persistent ring kernel (ring depth measured on the 151936 x 2048 output
// head: Q6_K 3, Q4_K 2); PRO 1 / 2 (K-quants): the workgroups quantise the f32 row a.px themselves
template <int WT, int PRO = 0>
static int launch_mv_ring(MvArgs &A, hipStream_t st, bool dry = false) {
    constexpr int NB = WT == SDY_Q6_K || WT == SDY_Q8_0 ? 3 : 2;
    prep_1t(A);
    switch (A.P.T) {
    case 32: return launch_mv_ring_nsb<WT, NB, 8, PRO>(A, st, dry);
    case 64: return launch_mv_ring_nsb<WT, NB, 16, PRO>(A, st, dry);
    default: return launch_mv_ring_nsb<WT, NB, 0, PRO>(A, st, dry);
    }
}

template <int WT, int MT, bool YREG>
static int launch_mv_rl(MvArgs &A, size_t lds, hipStream_t st, int n_slot = 1) {
    if constexpr (MT == 1 && YREG && is_k(WT)) {
        const int rc = launch_mv_1t<WT>(A, st, n_slot);
        if (rc <= 0) return rc;
        if (n_slot == 1 && !A.px && !A.swiglu) return launch_mv_ring<WT>(A, st);
    } else if constexpr (MT == 1 && YREG) {
        if (n_slot == 1 && !A.swiglu && 64 % A.P.T == 0) return launch_mv_ring<WT>(A, st);
    }
    static int per_cu = 0;
    static size_t per_cu_lds = 0;
    const void *fn = (const void *)k_matvec_rl<WT, MT, YREG>;
    if (per_cu == 0 || per_cu_lds != lds) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, THREADS, lds) != hipSuccess || n < 1) n = 1;
        per_cu = n;
        per_cu_lds = lds;
    }
    const int rpi = 64 / A.P.T;
    long n_it = (A.row1 - A.row0 + rpi - 1) / rpi;
    long wgs = (n_it + WAVES - 1) / WAVES;
    long cap = (long)(g_n_cu ? g_n_cu : 256) * per_cu / n_slot;
    if (cap < 8) cap = 8;
    if (wgs > cap) wgs = cap;
    SDY_NOTE_KERNEL((k_matvec_rl<WT, MT, YREG>));
    hipLaunchKernelGGL((k_matvec_rl<WT, MT, YREG>), dim3((unsigned)wgs, (unsigned)n_slot), dim3(THREADS), lds, st, A);
    return sdy_check_launch("matvec");
}

// one-token K-quant matvecs of rows that fit k_matvec_rl's lanes: T <= 64, an even rows-per-iteration
// count with the SwiGLU epilogue
static bool rl_one_token_ok(const sdy_mat *m, int epilogue) {
    const int T = m->n_units;
    return (m->type == SDY_Q4_K || m->type == SDY_Q6_K) && T <= 64 &&
           (epilogue != SDY_EPI_SWIGLU || (64 / T) % 2 == 0);
}

static long rl_wgs(const MvArgs &A, int per_cu) {
    const int rpi = 64 / A.P.T;
    const long n_it = (A.row1 - A.row0 + rpi - 1) / rpi;
    long wgs = (n_it + WAVES - 1) / WAVES;
    long cap = (long)(g_n_cu ? g_n_cu : 256) * per_cu;
    if (cap < 8) cap = 8;
    return wgs > cap ? cap : wgs;
}

template <int WT1, int WT2, int NSB, int PRO, int WV = WAVES>
static int launch_mv_pair_1t(MvArgs &A, MvArgs &B, hipStream_t st, bool dry) {
    static int per_cu = 0;
    static size_t per_cu_lds = 0;
    const size_t lds = pro_lds(A);
    const long cap =
        resident_wgs((const void *)k_matvec_1t_pair<WT1, WT2, NSB, PRO, WV>, lds, per_cu, per_cu_lds, 64 * WV);
    auto wgs1 = [](const MvArgs &M) { return ((long)M.n_it + WV - 1) / WV; };
    const long g1 = (wgs1(A) + 7) / 8 * 8, g2 = wgs1(B);
    if (g1 + g2 > cap) return 1;
    if (dry) return 0;
    SDY_NOTE_KERNEL((k_matvec_1t_pair<WT1, WT2, NSB, PRO, WV>));
    hipLaunchKernelGGL((k_matvec_1t_pair<WT1, WT2, NSB, PRO, WV>), dim3((unsigned)(g1 + g2)), dim3(64 * WV), lds, st, A,
                       B, (int)g1);
    return sdy_check_launch("matvec_pair");
}

// the pair on k_matvec_1t_pair when its grid fits the GPU at once (1 when not)
template <int WT1, int WT2, int PRO>
static int launch_mv_pair_pro(MvArgs &A, MvArgs &B, hipStream_t st, bool dry = false) {
    prep_1t(A);
    prep_1t(B);
    constexpr int WV = PRO == 2 ? 8 : WAVES;  // (as launch_mv_1t_pro)
    if (A.P.T == 32 && B.P.T == 32) return launch_mv_pair_1t<WT1, WT2, 8, PRO, WV>(A, B, st, dry);  // 2048-element rows
    return launch_mv_pair_1t<WT1, WT2, 0, PRO, WV>(A, B, st, dry);
}

template <int WT1, int WT2>
static int launch_mv_pair(MvArgs &A, MvArgs &B, hipStream_t st) {
    {
        int rc;
        switch (pro_kind(A)) {
        case 1: return launch_mv_pair_pro<WT1, WT2, 1>(A, B, st);  // no other kernel for these
        case 2: return launch_mv_pair_pro<WT1, WT2, 2>(A, B, st);
        default: rc = launch_mv_pair_pro<WT1, WT2, 0>(A, B, st);
        }
        if (rc <= 0) return rc;
    }
    static int per_cu = 0;
    if (per_cu == 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void *)k_matvec_rl_pair<WT1, WT2>, THREADS, 0) !=
                hipSuccess || n < 1)
            n = 1;
        per_cu = n;
    }
    const long g1 = (rl_wgs(A, per_cu) + 7) / 8 * 8, g2 = rl_wgs(B, per_cu);
    SDY_NOTE_KERNEL((k_matvec_rl_pair<WT1, WT2>));
    hipLaunchKernelGGL((k_matvec_rl_pair<WT1, WT2>), dim3((unsigned)(g1 + g2)), dim3(THREADS), 0, st, A, B, (int)g1);
    return sdy_check_launch("matvec_pair");
}

template <int WT, int NI, int PRO>
static int launch_mv_lr_ni(MvArgs &A, size_t lds, hipStream_t st, bool dry) {
    // the workgroup-quantised row: 8-wave workgroups, the row built while the weights stream
    constexpr int WV = PRO ? 8 : WAVES;
    static int per_cu = 0;
    static size_t per_cu_lds = 0, granted = 0;
    const void *fn = (const void *)k_matvec_lr<WT, NI, PRO, WV>;
    int rc = sdy_lds_limit(fn, lds, &granted);
    if (rc) return rc;
    if (per_cu == 0 || per_cu_lds != lds) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, 64 * WV, lds) != hipSuccess || n < 1) n = 1;
        per_cu = n;
        per_cu_lds = lds;
    }
    long wgs = (A.row1 - A.row0 + WV - 1) / WV;
    long cap = (long)(g_n_cu ? g_n_cu : 256) * per_cu;
    if (wgs > cap) {
        // the workgroup-quantised row needs every workgroup's waves at once (each quantises once)
        if (PRO) return 1;
        wgs = cap;
    }
    if (dry) return 0;
    SDY_NOTE_KERNEL((k_matvec_lr<WT, NI, PRO, WV>));
    hipLaunchKernelGGL((k_matvec_lr<WT, NI, PRO, WV>), dim3((unsigned)wgs), dim3(64 * WV), lds, st, A);
    return sdy_check_launch("matvec");
}

// one token, long rows: NI = ceil(T / 64) passes per row
template <int WT, int PRO = 0>
static int launch_mv_lr(MvArgs &A, size_t lds, hipStream_t st, bool dry = false) {
    if (PRO) lds = pro_lds(A);
    switch ((A.P.T + 63) / 64) {
    case 1: return launch_mv_lr_ni<WT, 1, PRO>(A, lds, st, dry);
    case 2: return launch_mv_lr_ni<WT, 2, PRO>(A, lds, st, dry);
    case 3: return launch_mv_lr_ni<WT, 3, PRO>(A, lds, st, dry);
    case 4: return launch_mv_lr_ni<WT, 4, PRO>(A, lds, st, dry);
    case 5: return launch_mv_lr_ni<WT, 5, PRO>(A, lds, st, dry);
    case 6: return launch_mv_lr_ni<WT, 6, PRO>(A, lds, st, dry);
    default: return sdy_fail(-1, "matvec: rows of %d elements are above the one-token kernel's 24576", A.P.n_in);
    }
}

template <int WT, int MT>
static int launch_mv(const sdy_mat *m, const sdy_mv_args *a, int n_tok, const uint8_t *xq, float *out,
                     const float *resid, hipStream_t st) {
    MvArgs A = {};
    A.P = planes_of(m);
    A.xq = xq;
    A.n_tok = n_tok;
    A.out = out;
    A.out_stride = a->out_stride;
    A.bias = a->bias;
    A.resid = resid;
    A.row0 = a->row0;
    A.row1 = a->row1;
    const int T = A.P.T;
    A.swiglu = a->epilogue == SDY_EPI_SWIGLU;
    A.rb = rows_per_batch(T, A.swiglu);
    A.ipb = (A.rb * T + 63) / 64;
    A.q64 = 64 / T;
    A.r64 = 64 % T;
    A.nterm = is_k(WT) ? A.P.nb : T;
    size_t lds = mv_lds_bytes(WT, T, A.P.nb, MT, A.rb);
    if (lds > LDS_MAX) return sdy_fail(-1, "matvec: %zu bytes of LDS needed (n_in %d, %d tokens)", lds, m->n_in, MT);
    if (T <= 64 && 64 % T == 0 && (!A.swiglu || (64 / T) % 2 == 0)) {
        lds = (MT == 1 && is_k(WT)) ? 0 : mv_lds_bytes_rl(T, MT);  // one K-quant token: no staging
        if (MT == 1) return launch_mv_rl<WT, MT, true>(A, lds, st);
        return launch_mv_rl<WT, MT, false>(A, lds, st);
    }
    // one K-quant token, T < 64 not dividing 64 (e.g. 768-element rows, T = 12): floor(64/T) rows per
    // wave iteration
    if constexpr (MT == 1 && is_k(WT))
        if (T < 64 && (!A.swiglu || (64 / T) % 2 == 0)) return launch_mv_rl<WT, 1, true>(A, 0, st);
    if constexpr (MT == 1 && is_k(WT))
        if (!A.swiglu) return launch_mv_lr<WT>(A, 0, st);
    return launch_mv_k<WT, MT, false>(A, lds, st);
}

template <int WT>
static int mv_type(const sdy_mat *m, const sdy_mv_args *a, hipStream_t st) {
    size_t xrow = sdy_raw_row_bytes(is_k(WT) ? SDY_Q8_K : SDY_Q8_0, m->n_in);
    const int T = m->n_units, nb = n_blocks(WT, m->n_in);
    // largest token capacity (8, 4, 2, 1) whose LDS fits; tokens are processed in chunks of it
    const int rb = rows_per_batch(T, a->epilogue == SDY_EPI_SWIGLU);
    int cap = 8;
    while (cap > 1 && mv_lds_bytes(WT, T, nb, cap, rb) > LDS_MAX) cap /= 2;
    for (int t0 = 0; t0 < a->n_tok;) {
        int n = a->n_tok - t0 < cap ? a->n_tok - t0 : cap;
        const uint8_t *xq = (const uint8_t *)a->xq + xrow * t0;
        float *out = a->out + a->out_stride * t0;
        const float *resid = a->resid ? a->resid + a->out_stride * t0 : nullptr;
        int rc;  // the smallest token capacity that holds n
        if (n > 4) rc = launch_mv<WT, 8>(m, a, n, xq, out, resid, st);
        else if (n > 2) rc = launch_mv<WT, 4>(m, a, n, xq, out, resid, st);
        else if (n == 2) rc = launch_mv<WT, 2>(m, a, n, xq, out, resid, st);
        else rc = launch_mv<WT, 1>(m, a, 1, xq, out, resid, st);
        if (rc) return rc;
        t0 += n;
    }
    return 0;
}

static int check_mv_rows(const sdy_mat *m, const sdy_mv_args *a) {
    if (a->row0 < 0 || a->row1 > m->n_rows || a->row0 > a->row1)
        return sdy_fail(-1, "matvec rows [%ld, %ld) outside %ld", a->row0, a->row1, m->n_rows);
    if (a->epilogue == SDY_EPI_SWIGLU && (((a->row1 - a->row0) | a->row0) & 1 || a->bias || a->resid))
        return sdy_fail(-1, "matvec: the SwiGLU epilogue needs an even row range starting at an even row, no bias "
                            "and no residual");
    return 0;
}

static MvArgs rl_args(const sdy_mat *m, const sdy_mv_args *a) {
    MvArgs A = {};
    A.P = planes_of(m);
    A.xq = (const uint8_t *)a->xq;
    A.n_tok = 1;
    A.out = a->out;
    A.out_stride = a->out_stride;
    A.bias = a->bias;
    A.resid = a->resid;
    A.row0 = a->row0;
    A.row1 = a->row1;
    A.swiglu = a->epilogue == SDY_EPI_SWIGLU;
    A.nterm = A.P.nb;
    if (!a->xq && a->x) {  // the workgroup quantises the f32 row
        A.px = a->x;
        A.pnw = a->nw;
        A.peps = a->eps;
    }
    return A;
}

static void ensure_n_cu() {
    if (!g_n_cu) {
        int n_cu = 0;
        size_t mem = 0;
        sdy_device_info(&n_cu, &mem);
        g_n_cu = n_cu;
    }
}

// The argument checks of a workgroup-quantised (xq = NULL, x set) one-token matvec; 0 when fine.
static int fused_args_check(const sdy_mat *m, const sdy_mv_args *a) {
    if (m->type != SDY_Q4_K && m->type != SDY_Q6_K) return sdy_fail(-1, "matvec: in-kernel quantisation needs Q4_K / Q6_K");
    if (a->n_tok != 1) return sdy_fail(-1, "matvec: in-kernel quantisation of one token only");
    if (m->n_in % 256 || ((uintptr_t)a->x & 15) || (a->nw && ((uintptr_t)a->nw & 15)))
        return sdy_fail(-1, "matvec: in-kernel quantisation needs 256-element blocks and 16-byte aligned rows");
    if (a->nw && m->n_in > 4096) return sdy_fail(-1, "matvec: in-kernel RMSNorm of rows above 4096 elements");
    if (a->row0 < 0 || a->row1 > m->n_rows || a->row0 > a->row1)
        return sdy_fail(-1, "matvec rows [%ld, %ld) outside %ld", a->row0, a->row1, m->n_rows);
    if (m->n_units <= 64) {
        if (!rl_one_token_ok(m, a->epilogue)) return sdy_fail(-1, "matvec: SwiGLU rows per iteration must be even");
    } else if (a->nw || a->epilogue == SDY_EPI_SWIGLU) {
        return sdy_fail(-1, "matvec: rows above 4096 elements are quantised in-kernel without RMSNorm or SwiGLU");
    }
    return 0;
}

// launch (or, dry, test) one workgroup-quantised matvec: 0 done, 1 no grid fits, < 0 error
static int fused_launch(const sdy_mat *m, const sdy_mv_args *a, hipStream_t st, bool dry) {
    int rc = fused_args_check(m, a);
    if (rc) return rc;
    ensure_n_cu();
    MvArgs A = rl_args(m, a);
    const bool q4 = m->type == SDY_Q4_K;
    if (m->n_units <= 64) {
        const int rc = q4 ? launch_mv_1t<SDY_Q4_K>(A, st, 1, dry) : launch_mv_1t<SDY_Q6_K>(A, st, 1, dry);
        if (rc != 1 || A.swiglu) return rc;
        // too many rows for a grid the GPU holds at once (the output head): the persistent ring
        // kernel, its workgroups quantising the row themselves
        if (A.pnw) return q4 ? launch_mv_ring<SDY_Q4_K, 2>(A, st, dry) : launch_mv_ring<SDY_Q6_K, 2>(A, st, dry);
        return q4 ? launch_mv_ring<SDY_Q4_K, 1>(A, st, dry) : launch_mv_ring<SDY_Q6_K, 1>(A, st, dry);
    }
    return q4 ? launch_mv_lr<SDY_Q4_K, 1>(A, 0, st, dry) : launch_mv_lr<SDY_Q6_K, 1>(A, 0, st, dry);
}

template <int WT1, int WT2>
static int pair_fused_launch(MvArgs &A, MvArgs &B, hipStream_t st, bool dry) {
    return A.pnw ? launch_mv_pair_pro<WT1, WT2, 2>(A, B, st, dry) : launch_mv_pair_pro<WT1, WT2, 1>(A, B, st, dry);
}

static int pair_fused(const sdy_mat *m1, const sdy_mv_args *a1, const sdy_mat *m2, const sdy_mv_args *a2, hipStream_t st,
                      bool dry) {
    int rc;
    if ((rc = fused_args_check(m1, a1)) || (rc = fused_args_check(m2, a2))) return rc;
    if (m1->n_units > 64 || m2->n_units > 64 || a1->x != a2->x || a1->nw != a2->nw || a1->eps != a2->eps)
        return sdy_fail(-1, "matvec_pair: in-kernel quantisation needs rows of at most 4096 elements and one shared row");
    ensure_n_cu();
    MvArgs A = rl_args(m1, a1), B = rl_args(m2, a2);
    const bool q4a = m1->type == SDY_Q4_K, q4b = m2->type == SDY_Q4_K;
    if (q4a && q4b) return pair_fused_launch<SDY_Q4_K, SDY_Q4_K>(A, B, st, dry);
    if (q4a) return pair_fused_launch<SDY_Q4_K, SDY_Q6_K>(A, B, st, dry);
    if (q4b) return pair_fused_launch<SDY_Q6_K, SDY_Q4_K>(A, B, st, dry);
    return pair_fused_launch<SDY_Q6_K, SDY_Q6_K>(A, B, st, dry);
}

extern "C" int sdy_matvec_fused_ok(const sdy_mat *m, const sdy_mv_args *a, const sdy_mat *m2, const sdy_mv_args *a2) {
    if (!a || a->xq || !a->x || (m2 && (!a2 || a2->xq))) return 0;
    const int rc = m2 ? pair_fused(m, a, m2, a2, nullptr, true) : fused_launch(m, a, nullptr, true);
    return rc == 0;
}

extern "C" int sdy_matvec_pair_ok(const sdy_mat *m1, int epilogue1, const sdy_mat *m2, int epilogue2) {
    return rl_one_token_ok(m1, epilogue1) && rl_one_token_ok(m2, epilogue2);
}

extern "C" int sdy_matvec_pair(const sdy_mat *m1, const sdy_mv_args *a1, const sdy_mat *m2, const sdy_mv_args *a2,
                               sdy_stream s) {
    if (!sdy_matvec_pair_ok(m1, a1->epilogue, m2, a2->epilogue))
        return sdy_fail(-1, "matvec_pair: two Q4_K / Q6_K matrices of at most 4096-element rows (64 units) needed");
    if (a1->n_tok != 1 || a2->n_tok != 1) return sdy_fail(-1, "matvec_pair: one token only");
    int rc;
    if ((rc = check_mv_rows(m1, a1)) || (rc = check_mv_rows(m2, a2))) return rc;
    if (!g_n_cu) {
        int n_cu = 0;
        size_t mem = 0;
        sdy_device_info(&n_cu, &mem);
        g_n_cu = n_cu;
    }
    if (a1->row0 == a1->row1) return sdy_matvec(m2, a2, s);
    if (a2->row0 == a2->row1) return sdy_matvec(m1, a1, s);
    if (!a1->xq || !a2->xq) {
        if (a1->xq || a2->xq) return sdy_fail(-1, "matvec_pair: both quantised rows or neither");
        const int frc = pair_fused(m1, a1, m2, a2, (hipStream_t)s, false);
        return frc > 0 ? sdy_fail(-1, "matvec_pair: no grid of the in-kernel quantisation fits these matrices") : frc;
    }
    MvArgs A = rl_args(m1, a1), B = rl_args(m2, a2);
    hipStream_t st = (hipStream_t)s;
    const bool q4a = m1->type == SDY_Q4_K, q4b = m2->type == SDY_Q4_K;
    if (q4a && q4b) return launch_mv_pair<SDY_Q4_K, SDY_Q4_K>(A, B, st);
    if (q4a) return launch_mv_pair<SDY_Q4_K, SDY_Q6_K>(A, B, st);
    if (q4b) return launch_mv_pair<SDY_Q6_K, SDY_Q4_K>(A, B, st);
    return launch_mv_pair<SDY_Q6_K, SDY_Q6_K>(A, B, st);
}

extern "C" int sdy_matvec(const sdy_mat *m, const sdy_mv_args *a, sdy_stream s) {
    hipStream_t st = (hipStream_t)s;
    if (a->row0 < 0 || a->row1 > m->n_rows || a->row0 > a->row1)
        return sdy_fail(-1, "matvec rows [%ld, %ld) outside %ld", a->row0, a->row1, m->n_rows);
    if (a->row0 == a->row1 || a->n_tok <= 0) return 0;
    if (!a->xq && m->type != SDY_F32 && m->type != SDY_F16 && m->type != SDY_BF16) {
        if (!a->x) return sdy_fail(-1, "matvec: no activations (xq and x both null)");
        if (a->epilogue == SDY_EPI_SWIGLU && (((a->row1 - a->row0) | a->row0) & 1 || a->bias || a->resid))
            return sdy_fail(-1, "matvec: the SwiGLU epilogue needs an even row range starting at an even row, no "
                                "bias and no residual");
        const int rc = fused_launch(m, a, st, false);
        return rc > 0 ? sdy_fail(-1, "matvec: no grid of the in-kernel quantisation fits %ld rows", a->row1 - a->row0)
                      : rc;
    }
    if (a->epilogue == SDY_EPI_SWIGLU && (((a->row1 - a->row0) | a->row0) & 1 || a->bias || a->resid))
        return sdy_fail(-1, "matvec: the SwiGLU epilogue needs an even row range starting at an even row, no bias "
                            "and no residual");
    if (a->epilogue == SDY_EPI_SWIGLU && (m->type == SDY_F32 || m->type == SDY_F16 || m->type == SDY_BF16))
        return sdy_fail(-1, "matvec: the SwiGLU epilogue is for quantized weights");
    if (!g_n_cu) {
        int n_cu = 0;
        size_t mem = 0;
        sdy_device_info(&n_cu, &mem);
        g_n_cu = n_cu;
    }
    switch (m->type) {
    case SDY_Q4_K: return mv_type<SDY_Q4_K>(m, a, st);
    case SDY_Q6_K: return mv_type<SDY_Q6_K>(m, a, st);
    case SDY_Q8_0: return mv_type<SDY_Q8_0>(m, a, st);
    case SDY_Q4_0: return mv_type<SDY_Q4_0>(m, a, st);
    case SDY_Q5_0: return mv_type<SDY_Q5_0>(m, a, st);
    case SDY_F32: case SDY_F16: case SDY_BF16:
        return sdy_matvec_float(m->type, (const uint8_t *)m->base + m->plane_off[0], m->n_in, a, s);
    default: return sdy_fail(-1, "matvec: type %d", m->type);
    }
}

static MvArgs grouped_args(const sdy_mat *m, const sdy_mv_args *a, const int32_t *slot_expert, long slot_rows,
                           long xq_slot, long out_slot) {
    MvArgs A = {};
    A.P = planes_of(m);
    A.xq = (const uint8_t *)a->xq;
    A.n_tok = 1;
    A.out = a->out;
    A.out_stride = a->out_stride;
    A.row0 = a->row0;
    A.row1 = a->row1;
    A.swiglu = a->epilogue == SDY_EPI_SWIGLU;
    A.slot_expert = slot_expert;
    A.slot_rows = slot_rows;
    A.n_slot_exp = (int)(m->n_rows / slot_rows);
    A.xq_slot = xq_slot;
    A.out_slot = out_slot;
    return A;
}

template <int WT>
static int mv_grouped(const sdy_mat *m, const sdy_mv_args *a, const int32_t *slot_expert, int n_slot, long slot_rows,
                      long xq_slot, long out_slot, hipStream_t st, bool dry = false) {
    MvArgs A = grouped_args(m, a, slot_expert, slot_rows, xq_slot, out_slot);
    if (!a->xq) {  // the workgroups quantise their slot's f32 row (a->x + slot * xq_slot floats)
        A.xq_slot = 0;
        A.px = a->x;
        A.pnw = a->nw;
        A.peps = a->eps;
        A.px_slot = xq_slot;
        const int rc = launch_mv_1t<WT>(A, st, n_slot, dry);
        return rc > 0 ? sdy_fail(-1, "grouped matvec: no grid of the in-kernel quantisation fits") : rc;
    }
    return launch_mv_rl<WT, 1, true>(A, 0, st, n_slot);
}

// The argument checks of sdy_matvec_grouped; 0 when fine.
static int grouped_check(const sdy_mat *m, const sdy_mv_args *a, int n_slot, long slot_rows, long xq_slot) {
    if (m->type != SDY_Q4_K && m->type != SDY_Q6_K)
        return sdy_fail(-1, "grouped matvec: K-quant weights only (type %d)", m->type);
    if (a->n_tok != 1 || a->bias || a->resid) return sdy_fail(-1, "grouped matvec: one token, no bias or residual");
    if (slot_rows <= 0 || m->n_rows % slot_rows)
        return sdy_fail(-1, "grouped matvec: %ld rows are not a stack of %ld-row experts", m->n_rows, slot_rows);
    if (a->row0 < 0 || a->row1 > slot_rows || a->row0 > a->row1)
        return sdy_fail(-1, "grouped matvec rows [%ld, %ld) outside an expert's %ld", a->row0, a->row1, slot_rows);
    if (n_slot < 1 || n_slot > 65535) return sdy_fail(-1, "grouped matvec: %d slots", n_slot);
    const int T = m->n_units;
    if (T > 64) return sdy_fail(-1, "grouped matvec: rows of %d elements above 4096", m->n_in);
    if (a->epilogue == SDY_EPI_SWIGLU && ((64 / T) % 2 || ((a->row1 - a->row0) | a->row0) & 1))
        return sdy_fail(-1, "grouped matvec: SwiGLU needs an even number of rows per iteration and an even row range");
    if (!a->xq) {
        if (!a->x) return sdy_fail(-1, "grouped matvec: no activations");
        if (m->n_in % 256 || ((uintptr_t)a->x & 15) || (xq_slot * 4) % 16 || (a->nw && ((uintptr_t)a->nw & 15)))
            return sdy_fail(-1, "grouped matvec: in-kernel quantisation needs 256-element blocks and 16-byte aligned rows");
    }
    return 0;
}

extern "C" int sdy_matvec_grouped_fused_ok(const sdy_mat *m, const sdy_mv_args *a, int n_slot, long slot_rows,
                                           long x_slot) {
    if (!a || a->xq || !a->x || grouped_check(m, a, n_slot, slot_rows, x_slot)) return 0;
    ensure_n_cu();
    const int rc = m->type == SDY_Q4_K ? mv_grouped<SDY_Q4_K>(m, a, nullptr, n_slot, slot_rows, x_slot, 0, nullptr, true)
                                       : mv_grouped<SDY_Q6_K>(m, a, nullptr, n_slot, slot_rows, x_slot, 0, nullptr, true);
    return rc == 0;
}

extern "C" int sdy_matvec_grouped(const sdy_mat *m, const sdy_mv_args *a, const int32_t *slot_expert, int n_slot,
                                  long slot_rows, long xq_slot, long out_slot, sdy_stream s) {
    hipStream_t st = (hipStream_t)s;
    int rc = grouped_check(m, a, n_slot, slot_rows, xq_slot);
    if (rc) return rc;
    if (a->row0 == a->row1) return 0;
    if (!g_n_cu) {
        int n_cu = 0;
        size_t mem = 0;
        sdy_device_info(&n_cu, &mem);
        g_n_cu = n_cu;
    }
    if (m->type == SDY_Q4_K) return mv_grouped<SDY_Q4_K>(m, a, slot_expert, n_slot, slot_rows, xq_slot, out_slot, st);
    return mv_grouped<SDY_Q6_K>(m, a, slot_expert, n_slot, slot_rows, xq_slot, out_slot, st);
}

// sdy_matvec_grouped over the k slots of one token whose experts the kernel selects itself from
// the router's n_expert logits (softmax, top k, renormalised weights: the bits of sdy_moe_route,
// which it also writes to top and wts), saving the route launch. The Q8_K row in memory (a->xq),
// n_expert <= 128, k <= 64. Returns 1, launching nothing, when no one-token grid fits: the caller
// then runs sdy_moe_route and sdy_matvec_grouped.
extern "C" int sdy_matvec_grouped_route(const sdy_mat *m, const sdy_mv_args *a, const float *logits, int n_expert,
                                        int k, int32_t *top, float *wts, long slot_rows, long xq_slot, long out_slot,
                                        sdy_stream s) {
    int rc = grouped_check(m, a, k, slot_rows, xq_slot);
    if (rc) return rc;
    if (!a->xq) return sdy_fail(-1, "routed grouped matvec: needs the Q8_K row (xq)");
    if (!logits || !top || !wts || n_expert < 1 || n_expert > 128 || k < 1 || k > 64 || k > n_expert)
        return sdy_fail(-1, "routed grouped matvec: %d of %d experts (at most 64 of 128), logits and outputs set", k,
                        n_expert);
    if (m->n_rows / slot_rows < n_expert)
        return sdy_fail(-1, "routed grouped matvec: a stack of %ld experts for %d logits", m->n_rows / slot_rows,
                        n_expert);
    if (a->row0 == a->row1) return 1;  // no workgroup would write the choices
    ensure_n_cu();
    MvArgs A = grouped_args(m, a, top, slot_rows, xq_slot, out_slot);
    A.route_logits = logits;
    A.route_ne = n_expert;
    A.route_k = k;
    A.route_top = top;
    A.route_wts = wts;
    hipStream_t st = (hipStream_t)s;
    return m->type == SDY_Q4_K ? launch_mv_1t<SDY_Q4_K>(A, st, k) : launch_mv_1t<SDY_Q6_K>(A, st, k);
}

// The routed experts' down projections of one token (the k slots' f32 rows x, n_in apart, through
// expert slot_expert[s] of the stack m, dim rows each) and their combine: out = resid + sum over the
// slots in ascending expert id of wts[s] * y_s. The bits of sdy_matvec_grouped (quantising the
// rows in the kernel) then sdy_moe_combine.
extern "C" int sdy_moe_down_combine(const sdy_mat *m, const float *x, const int32_t *slot_expert, const float *wts,
                                    int k, long dim, float *out, const float *resid, sdy_stream s) {
    if (m->type != SDY_Q4_K && m->type != SDY_Q6_K) return sdy_fail(-1, "moe_down_combine: K-quant weights only");
    if (k < 1 || k > 8 || dim < 1 || m->n_rows % dim || m->n_units > 64 || m->n_in % 256 || ((uintptr_t)x & 15))
        return sdy_fail(-1, "moe_down_combine: 1..8 slots, a stack of %ld-row experts, rows of 256..4096 elements, "
                            "16-byte aligned activations", dim);
    MvArgs A = {};
    A.P = planes_of(m);
    A.n_tok = 1;
    A.row0 = 0;
    A.row1 = dim;
    A.slot_expert = slot_expert;
    A.slot_rows = dim;
    A.n_slot_exp = (int)(m->n_rows / dim);
    A.px = x;
    prep_1t(A);
    const size_t lds = (size_t)k * (m->n_in / 256) * 292 + 8 * 64 * sizeof(float);
    // a multiple of 8 workgroups: the kernel's XCD-aware renumbering then keeps neighbouring rows
    // (whose plane segments share cache lines) on one XCD (the extra workgroups store nothing)
    const unsigned wgs = (unsigned)((A.n_it + 7) & ~7L);
    hipStream_t st = (hipStream_t)s;
#define SDY_MDC(WT, NSB)                                                                                             \
    {                                                                                                                \
        SDY_NOTE_KERNEL((k_moe_down_combine<WT, NSB, 8>));                                                           \
        hipLaunchKernelGGL((k_moe_down_combine<WT, NSB, 8>), dim3(wgs), dim3(512), lds, st, A, wts, k, out,           \
                           resid);                                                                                   \
        return sdy_check_launch("moe_down_combine");                                                                 \
    }
    const int nsb = m->n_in / 256;
    if (m->type == SDY_Q6_K) {
        if (nsb == 3) SDY_MDC(SDY_Q6_K, 3)
        if (nsb == 8) SDY_MDC(SDY_Q6_K, 8)
        SDY_MDC(SDY_Q6_K, 0)
    }
    if (nsb == 3) SDY_MDC(SDY_Q4_K, 3)
    if (nsb == 8) SDY_MDC(SDY_Q4_K, 8)
    SDY_MDC(SDY_Q4_K, 0)
#undef SDY_MDC
}

extern "C" int sdy_matvec_float_norm(int wtype, const void *w, int n_in, const sdy_mv_args *a, void *xq_out,
                                     sdy_stream s) {
    hipStream_t st = (hipStream_t)s;
    const long n_rows = a->row1 - a->row0;
    if (wtype != SDY_F32 && wtype != SDY_F16 && wtype != SDY_BF16) return sdy_fail(-1, "float matvec: type %d", wtype);
    if (a->n_tok != 1 || !a->x || !a->nw || n_in % 256 || n_in > 4096 || ((uintptr_t)a->x & 15) ||
        ((uintptr_t)a->nw & 15))
        return sdy_fail(-1, "float matvec with RMSNorm: one token, rows of 256..4096 elements (multiples of 256), "
                            "16-byte aligned x and norm weights");
    if (n_rows <= 0) return 0;
    const dim3 grid((unsigned)((n_rows + 2 * WAVES - 1) / (2 * WAVES)));
    const FloatNorm fn = {a->nw, a->eps, (uint8_t *)xq_out};
    const uint8_t *wp = (const uint8_t *)w;
    if (wtype == SDY_F32)
        hipLaunchKernelGGL((k_matvec_float_dot<SDY_F32, true>), grid, dim3(THREADS), 0, st, wp, n_in, a->x, 1, a->out,
                           a->out_stride, a->bias, a->resid, a->row0, a->row1, fn);
    else if (wtype == SDY_F16)
        hipLaunchKernelGGL((k_matvec_float_dot<SDY_F16, true>), grid, dim3(THREADS), 0, st, wp, n_in, a->x, 1, a->out,
                           a->out_stride, a->bias, a->resid, a->row0, a->row1, fn);
    else
        hipLaunchKernelGGL((k_matvec_float_dot<SDY_BF16, true>), grid, dim3(THREADS), 0, st, wp, n_in, a->x, 1, a->out,
                           a->out_stride, a->bias, a->resid, a->row0, a->row1, fn);
    return sdy_check_launch("matvec_float_norm");
}

extern "C" int sdy_matvec_float(int wtype, const void *w, int n_in, const sdy_mv_args *a, sdy_stream s) {
    hipStream_t st = (hipStream_t)s;
    const long n_rows = a->row1 - a->row0;
    if (n_rows <= 0 || a->n_tok <= 0) return 0;
    const int n_tok = a->n_tok;
    const long n_pr = n_tok >= 4 ? (n_rows & ~1L) : 0;
    const int n_gt = n_tok >= 4 ? (n_tok & ~3) : 0;
    const long n_block = n_pr * n_gt, n_dot = n_rows * n_tok - n_block;
    const uint8_t *wp = (const uint8_t *)w;
    if (wtype != SDY_F32 && wtype != SDY_F16 && wtype != SDY_BF16) return sdy_fail(-1, "float matvec: type %d", wtype);
#define SDY_FLOAT_LAUNCH(KERNEL, N_ITEMS, PER_WAVE)                                                                  \
    if ((N_ITEMS) > 0) {                                                                                             \
        const dim3 grid((unsigned)(((N_ITEMS) + (PER_WAVE) * WAVES - 1) / ((PER_WAVE) * WAVES)));                    \
        if (wtype == SDY_F32)                                                                                        \
            hipLaunchKernelGGL(KERNEL<SDY_F32>, grid, dim3(THREADS), 0, st, wp, n_in, a->x, n_tok, a->out,            \
                               a->out_stride, a->bias, a->resid, a->row0, a->row1);                                  \
        else if (wtype == SDY_F16)                                                                                   \
            hipLaunchKernelGGL(KERNEL<SDY_F16>, grid, dim3(THREADS), 0, st, wp, n_in, a->x, n_tok, a->out,            \
                               a->out_stride, a->bias, a->resid, a->row0, a->row1);                                  \
        else                                                                                                         \
            hipLaunchKernelGGL(KERNEL<SDY_BF16>, grid, dim3(THREADS), 0, st, wp, n_in, a->x, n_tok, a->out,           \
                               a->out_stride, a->bias, a->resid, a->row0, a->row1);                                  \
    }
    if (n_pr >= FT_ROWS && n_gt >= FT_TOKS && n_in % 4 == 0 && ((uintptr_t)wp & 15) == 0 &&
        ((uintptr_t)a->x & 15) == 0) {
        // many rows and tokens: the block-order pairs from tiles staged in LDS (4-element loads)
        const dim3 grid((unsigned)((n_gt + FT_TOKS - 1) / FT_TOKS), (unsigned)((n_pr + FT_ROWS - 1) / FT_ROWS));
        const dim3 block(256);
        if (wtype == SDY_F32)
            hipLaunchKernelGGL(k_matvec_float_tile<SDY_F32>, grid, block, 0, st, wp, n_in, a->x, n_tok, a->out,
                               a->out_stride, a->bias, a->resid, a->row0, a->row1);
        else if (wtype == SDY_F16)
            hipLaunchKernelGGL(k_matvec_float_tile<SDY_F16>, grid, block, 0, st, wp, n_in, a->x, n_tok, a->out,
                               a->out_stride, a->bias, a->resid, a->row0, a->row1);
        else
            hipLaunchKernelGGL(k_matvec_float_tile<SDY_BF16>, grid, block, 0, st, wp, n_in, a->x, n_tok, a->out,
                               a->out_stride, a->bias, a->resid, a->row0, a->row1);
    } else {
        SDY_FLOAT_LAUNCH(k_matvec_float_block, n_block, 8)
    }
    SDY_FLOAT_LAUNCH(k_matvec_float_dot, n_dot, 2)
#undef SDY_FLOAT_LAUNCH
    return sdy_check_launch("matvec_float");
}

// gfx950 attention (the reference's op_attention_head over attention_worker's (token, head) pairs,
// csrc/ops.c:405-414 and csrc/model_llama.c:619-634) over the KV cache [n_kv_head][max_seq][head_dim]
// of a layer (f32, or f16 rounded at the write: sdy_attn_dev.h), with the reference's arithmetic step
// by step on the cache's f32 values:
//   score_j = dot(q, k_j) * (1 / sqrtf(head_dim)), dot in the AVX2 order of csrc/ops_avx2.c:61-74
//     (four 8-lane FMA chains over 32-element steps, 8-element steps into the first chain, the
//     lane-wise (a0 + a1) + (a2 + a3), the 8-lane tree ((v0 + v4) + (v2 + v6)) + ((v1 + v5) +
//     (v3 + v7)), a scalar tail);
//   op_softmax over every position of the token: the maximum, e_j = expf(score_j - max) (the host
//     libm's expf, sdy_expf.h), their sum in double, the float reciprocal, p_j = e_j * inv;
//   out = sum over the positions in order of axpy(p_j, v_j): one FMA chain per output element
//     (head_dim % 8 == 0: AVX2 axpy fuses every element).
// Only the double sum is taken in a different order (a tree): its rounding can move the float
// reciprocal only when two double roundings straddle a float rounding boundary.
//
//   k_attn_scores<HD, DECODE>     scores of a 64-position chunk for a block of (token, head) pairs
//                                 into scores [n_tok][n_head][max_kv]; the decode variant first
//                                 normalises and rotates q and the new k and writes the new K/V
//   k_attn_softmax_pv<HD, DECODE> softmax and weighted V of 256 / HD heads of one token (the decode
//                                 variant also quantises the 256 outputs to a Q8_K block)
//   k_attn_prefill_pv<HD, TB>     the same for TB tokens at a time (prefill: each V element read once
//                                 for the TB tokens' chains)
//   k_attn_*_any                  the same for other head dims (runtime loops, scalar LDS reads)
#include "sdy_attn_dev.h"
#include "sdy_device.h"
#include "sdy_expf.h"
#include "sdy_internal.h"
#include "sdy_ops.h"
#include "sdy_quant_dev.h"
#include "sdy_shim.h"

namespace {

constexpr int CH = 64;       // positions per scores workgroup (one per lane)
constexpr int PAIRS = 64;    // (token, head) pairs per prefill scores workgroup
constexpr int PW = 8192;     // weights held in LDS at a time by k_attn_softmax_pv (all its heads)

// register arrays of 16-byte loads (an ext vector type: arrays of it stay in registers)
typedef sdy_f32x4 f32x4;

// One wave: optional per-head RMSNorm (qwen3 q/k norm: double sum, one rounding of the scale) then
// RoPE (pairs (i, i + hd/2), or (2i, 2i+1) when interleaved) of the hd-vector in buf (LDS).
SDY_DEV void norm_rope_wave(float *buf, const float *nw, float eps, const float *cs, const float *sn, int hd,
                            int interleaved, int lane) {
    if (nw) {
        double ss = 0.0;
        for (int i = lane; i < hd; i += 64) ss += (double)buf[i] * (double)buf[i];
        for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
        const float sc = (float)(1.0 / sqrt(ss / (double)hd + (double)eps));
        for (int i = lane; i < hd; i += 64) {
            const float tt = buf[i] * sc;
            buf[i] = tt * nw[i];
        }
        sdy_wave_sync();
    }
    const int half = hd / 2;
    for (int i = lane; i < half; i += 64) {
        const int ia = interleaved ? 2 * i : i, ib = interleaved ? 2 * i + 1 : i + half;
        const float a = buf[ia], b = buf[ib];
        const float ac = a * cs[i], bs = b * sn[i], as = a * sn[i], bc = b * cs[i];
        buf[ia] = ac - bs;
        buf[ib] = as + bc;
    }
    sdy_wave_sync();
}

// q/k norm + RoPE of the vectors of n_tok tokens and the KV-cache write at positions pos0 + t; token
// t's q, k and v rows start at t * qs, t * ks, t * vs floats. Grid (n_tok, n_head + n_kv_head), 64 threads.
template <class KT>
__global__ __launch_bounds__(64) void k_qk_rope_kv(float *q, float *k, const float *v, long qs, long ks, long vs,
                                                   const float *qn, const float *kn, float eps, const float *rope_cos,
                                                   const float *rope_sin, int pos0, int n_head, int n_kv_head, int hd,
                                                   int interleaved, KT *k_cache, KT *v_cache, long head_stride) {
    __shared__ float buf[512];
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const bool is_q = h < n_head;
    const int hh = is_q ? h : h - n_head;
    float *vec = is_q ? q + (size_t)t * qs + (size_t)hh * hd : k + (size_t)t * ks + (size_t)hh * hd;
    for (int i = lane; i < hd; i += 64) buf[i] = vec[i];
    sdy_wave_sync();
    const int pos = pos0 + t;
    norm_rope_wave(buf, is_q ? qn : kn, eps, rope_cos + (size_t)pos * (hd / 2), rope_sin + (size_t)pos * (hd / 2), hd,
                   interleaved, lane);
    for (int i = lane; i < hd; i += 64) vec[i] = buf[i];
    if (!is_q && k_cache) {
        KT *kc = k_cache + hh * head_stride + (size_t)pos * hd;
        KT *vc = v_cache + hh * head_stride + (size_t)pos * hd;
        const float *vv = v + (size_t)t * vs + (size_t)hh * hd;
        for (int i = lane; i < hd; i += 64) {
            KvElt<KT>::st(kc, i, buf[i]);
            KvElt<KT>::st(vc, i, vv[i]);
        }
    }
}

struct AttnArgs {
    const float *q;                   // prefill: rotated queries [n_tok][q_stride]; decode: raw [n_head][HD]
    const float *k, *v;               // decode: the token's raw k and v [n_kv_head][HD]
    const float *q_norm, *k_norm;     // decode: per-head norm weights or null
    float eps;
    const float *rope_cos, *rope_sin;
    const int32_t *step;              // decode: step[1] = position of the token
    int n_head, n_kv_head, n_kv0, n_tok, interleaved;
    long q_stride;
    void *k_cache, *v_cache;          // [n_kv_head][max_seq][HD] of the kernel's element type KT
    long head_stride;                 // max_seq * HD
    float *scores;                    // [n_tok][n_head][max_kv]
    int max_kv;
    float scale;
    float *out;                       // [n_tok][out_stride]
    long out_stride;
    uint8_t *xq;                      // decode: Q8_K row of out (or null)
};

// Maximum, and sum in double of expf(row[j] - m), over j = i0, i0 + stride, ... < n, eight loads in
// flight at a time (clamped indices).
SDY_DEV float row_max(const float *row, int i0, int stride, int n) {
    float m = -INFINITY;
    for (int j0 = i0; j0 < n; j0 += 8 * stride) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = j0 + u * stride;
            v[u] = row[j < n ? j : n - 1];
        }
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (j0 + u * stride < n) m = fmaxf(m, v[u]);
    }
    return m;
}

SDY_DEV double row_expsum(const float *row, int i0, int stride, int n, float m) {
    double sum = 0.0;
    for (int j0 = i0; j0 < n; j0 += 8 * stride) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = j0 + u * stride;
            v[u] = row[j < n ? j : n - 1];
        }
        float e[8];  // every exponential first (clamped indices), so the table reads overlap
#pragma unroll
        for (int u = 0; u < 8; u++) e[u] = sdy_expf(v[u] - m);
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (j0 + u * stride < n) sum += (double)e[u];
    }
    return sum;
}

// dst[(j - j_base) * dst_stride] = expf(row[j] - m) * inv for j = i0, i0 + stride, ... < n
SDY_DEV void row_weights(const float *row, int i0, int stride, int n, float m, float inv, float *dst, int j_base,
                         int dst_stride) {
    for (int j0 = i0; j0 < n; j0 += 8 * stride) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = j0 + u * stride;
            v[u] = row[j < n ? j : n - 1];
        }
        float e[8];
#pragma unroll
        for (int u = 0; u < 8; u++) e[u] = sdy_expf(v[u] - m) * inv;
        // all eight computed here, not sunk into the guarded stores one by one
        asm volatile("" : "+v"(e[0]), "+v"(e[1]), "+v"(e[2]), "+v"(e[3]), "+v"(e[4]), "+v"(e[5]), "+v"(e[6]),
                     "+v"(e[7]));
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = j0 + u * stride;
            if (j < n) dst[(j - j_base) * dst_stride] = e[u];
        }
    }
}

// K operands of dot_avx2_order: a row in LDS (16-byte aligned), or a row held in registers
struct KRowLds {
    const float *p;
    SDY_DEV float4 v4(int i) const { return *reinterpret_cast<const float4 *>(p + i); }
    SDY_DEV float v1(int i) const { return p[i]; }
};
template <int HD>
struct KRowReg {
    f32x4 r[HD / 4];
    SDY_DEV float4 v4(int i) const { return make_float4(r[i / 4][0], r[i / 4][1], r[i / 4][2], r[i / 4][3]); }
    SDY_DEV float v1(int i) const { return r[i / 4][i % 4]; }
};

// dot(q, k) in csrc/ops_avx2.c:61-74's order (x = q, w = k), q in LDS (16-byte aligned).
template <int HD, class K>
SDY_DEV float dot_avx2_order(const float *q, const K &k) {
    constexpr int N32 = HD / 32 * 32, N8 = HD / 8 * 8;
    float a[4][8];
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int l = 0; l < 8; l++) a[c][l] = 0.0f;
#pragma unroll
    for (int i = 0; i < N32; i += 32)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float4 q0 = *reinterpret_cast<const float4 *>(q + i + 8 * c);
            const float4 q1 = *reinterpret_cast<const float4 *>(q + i + 8 * c + 4);
            const float4 k0 = k.v4(i + 8 * c);
            const float4 k1 = k.v4(i + 8 * c + 4);
            a[c][0] = fmaf(k0.x, q0.x, a[c][0]);
            a[c][1] = fmaf(k0.y, q0.y, a[c][1]);
            a[c][2] = fmaf(k0.z, q0.z, a[c][2]);
            a[c][3] = fmaf(k0.w, q0.w, a[c][3]);
            a[c][4] = fmaf(k1.x, q1.x, a[c][4]);
            a[c][5] = fmaf(k1.y, q1.y, a[c][5]);
            a[c][6] = fmaf(k1.z, q1.z, a[c][6]);
            a[c][7] = fmaf(k1.w, q1.w, a[c][7]);
        }
#pragma unroll
    for (int i = N32; i < N8; i += 8)
#pragma unroll
        for (int l = 0; l < 8; l++) a[0][l] = fmaf(k.v1(i + l), q[i + l], a[0][l]);
    float v[8];
#pragma unroll
    for (int l = 0; l < 8; l++) {
        const float p = a[0][l] + a[1][l], r = a[2][l] + a[3][l];
        v[l] = p + r;
    }
    float s = ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
#pragma unroll
    for (int i = N8; i < HD; i++) {
        const float p = q[i] * k.v1(i);
        s = s + p;
    }
    return s;
}

// Decode q/k preparation with every input loaded at once (HD a multiple of 128, pairs (i, i + HD/2)):
// lane l of a wave holds elements l + 64 e of a vector, so a RoPE pair sits in one lane and the
// norm's sum has norm_rope_wave's per-lane order (elements l, l + 64, ...) and tree; the results go
// to LDS (qs, kp) and, for the new k, to the KV cache. Returns false (nothing done) for other
// shapes, which take norm_rope_wave.
template <int HD, class KT>
SDY_DEV bool decode_prep_regs(const AttnArgs &a, int g, int n_rep, int pos, bool has_pos, const float *cs,
                              const float *sn, float *qs, float *kp, int wave, int lane) {
    constexpr int E = HD / 64, EH = E / 2, RM = 4;  // elements per lane; vectors per wave
    if constexpr (HD % 128 != 0) {
        return false;
    } else {
        if (a.interleaved || n_rep + 1 > 4 * RM) return false;
        float x[RM][E], qn[E], kn[E], vv[E], c[EH], sv[EH];
        // every load first: the wave's vectors, the norm weights, cos/sin, the new v
#pragma unroll
        for (int i = 0; i < RM; i++) {
            const int r = wave + 4 * i;
            if (r <= n_rep) {
                const float *src = r == n_rep ? a.k + (size_t)g * HD : a.q + (size_t)(g * n_rep + r) * HD;
#pragma unroll
                for (int e = 0; e < E; e++) x[i][e] = src[lane + 64 * e];
            }
        }
#pragma unroll
        for (int e = 0; e < E; e++) {
            qn[e] = a.q_norm ? a.q_norm[lane + 64 * e] : 1.0f;
            kn[e] = a.k_norm ? a.k_norm[lane + 64 * e] : 1.0f;
            vv[e] = a.v[(size_t)g * HD + lane + 64 * e];
        }
#pragma unroll
        for (int e = 0; e < EH; e++) {
            c[e] = cs[lane + 64 * e];
            sv[e] = sn[lane + 64 * e];
        }
#pragma unroll
        for (int i = 0; i < RM; i++) {
            const int r = wave + 4 * i;
            if (r > n_rep) break;
            const bool is_k = r == n_rep;
            float y[E];
#pragma unroll
            for (int e = 0; e < E; e++) y[e] = x[i][e];
            if (is_k ? a.k_norm != nullptr : a.q_norm != nullptr) {
                double ss = 0.0;
#pragma unroll
                for (int e = 0; e < E; e++) ss += (double)y[e] * (double)y[e];
                for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
                const float sc = (float)(1.0 / sqrt(ss / (double)HD + (double)a.eps));
#pragma unroll
                for (int e = 0; e < E; e++) {
                    const float tt = y[e] * sc;
                    y[e] = tt * (is_k ? kn[e] : qn[e]);
                }
            }
#pragma unroll
            for (int e = 0; e < EH; e++) {  // the pair (l + 64 e, l + 64 e + HD/2)
                const float av = y[e], bv = y[e + EH];
                const float ac = av * c[e], bs = bv * sv[e], as = av * sv[e], bc = bv * c[e];
                y[e] = ac - bs;
                y[e + EH] = as + bc;
            }
            float *buf = is_k ? kp : qs + r * HD;
#pragma unroll
            for (int e = 0; e < E; e++) buf[lane + 64 * e] = y[e];
            if (is_k && has_pos) {  // KV-cache write of the new position
                KT *kc = (KT *)a.k_cache + g * a.head_stride + (size_t)pos * HD;
                KT *vc = (KT *)a.v_cache + g * a.head_stride + (size_t)pos * HD;
#pragma unroll
                for (int e = 0; e < E; e++) {
                    KvElt<KT>::st(kc, lane + 64 * e, y[e]);
                    KvElt<KT>::st(vc, lane + 64 * e, vv[e]);
                }
            }
        }
        return true;
    }
}

// Grid (n_chunk, n_kv_head, token blocks), 256 threads. Prefill: the block's tokens are
// PAIRS / n_rep consecutive tokens (queries already rotated, K/V already in the cache). Decode: one
// token at position step[1]; every workgroup normalises and rotates the group's queries and the
// new k in LDS, the workgroup of the last chunk writes the new K/V to the cache, and the new
// position's K comes from LDS. Lane p of a wave computes the score of position p0 + p for one
// (token, head) pair; the waves share the staged K chunk ([CH][HD + 4]: 16-byte rows, 8
// consecutive rows in distinct banks).
template <int HD, bool DECODE, class KT>
__global__ __launch_bounds__(256) void k_attn_scores(AttnArgs a) {
    constexpr int KS = HD + 4;
    constexpr int NV = CH * HD / 4 / 256 > 0 ? CH * HD / 4 / 256 : 1;  // float4 of K per thread
    extern __shared__ __align__(16) float sm[];
    float *ks = sm;            // [CH][KS]
    float *kp = ks + CH * KS;  // [HD]: the new position's rotated k (decode)
    float *qs = kp + HD;       // [pairs][HD]
    const int c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n_rep = a.n_head / a.n_kv_head;
    int t0, t1, n_kv_last, pos = 0;
    if constexpr (DECODE) {
        pos = a.step[1];
        t0 = 0;
        t1 = 1;
        n_kv_last = pos + 1;
    } else {
        const int tbs = PAIRS / n_rep > 0 ? PAIRS / n_rep : 1;
        t0 = blockIdx.z * tbs;
        t1 = t0 + tbs < a.n_tok ? t0 + tbs : a.n_tok;
        n_kv_last = a.n_kv0 + t1 - 1;
    }
    const int p0 = c * CH;
    if (p0 >= n_kv_last) return;
    const int np_max = n_kv_last - p0 < CH ? n_kv_last - p0 : CH;
    // K chunk loads first (clamped indices, unconditional)
    const KT *kg = (const KT *)a.k_cache + g * a.head_stride + (size_t)p0 * HD;
    const int n4 = np_max * HD / 4;
    f32x4 kv[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = tid + 256 * j < n4 ? tid + 256 * j : 0;
        kv[j] = KvElt<KT>::ld4(kg, (size_t)4 * i);
    }
    const int n_pairs = (t1 - t0) * n_rep;
    bool has_pos = false;
    if constexpr (DECODE) {
        // q heads of the group and the new k: norm + RoPE (one wave per vector)
        has_pos = p0 + np_max == pos + 1;
        const float *cs = a.rope_cos + (size_t)pos * (HD / 2), *sn = a.rope_sin + (size_t)pos * (HD / 2);
        const bool done = decode_prep_regs<HD, KT>(a, g, n_rep, pos, has_pos, cs, sn, qs, kp, wave, lane);
        for (int r = wave; !done && r <= n_rep; r += 4) {
            const bool is_k = r == n_rep;
            float *buf = is_k ? kp : qs + r * HD;
            const float *src = is_k ? a.k + (size_t)g * HD : a.q + (size_t)(g * n_rep + r) * HD;
            for (int i = lane; i < HD; i += 64) buf[i] = src[i];
            sdy_wave_sync();
            norm_rope_wave(buf, is_k ? a.k_norm : a.q_norm, a.eps, cs, sn, HD, a.interleaved, lane);
            if (is_k && has_pos) {  // KV-cache write of the new position
                KT *kc = (KT *)a.k_cache + g * a.head_stride + (size_t)pos * HD;
                KT *vc = (KT *)a.v_cache + g * a.head_stride + (size_t)pos * HD;
                const float *vn = a.v + (size_t)g * HD;
                for (int i = lane; i < HD; i += 64) {
                    KvElt<KT>::st(kc, i, buf[i]);
                    KvElt<KT>::st(vc, i, vn[i]);
                }
            }
        }
    } else {
        for (int i = tid; i < n_pairs * HD / 4; i += 256) {
            const int pr = (4 * i) / HD, d = 4 * i - pr * HD;
            const int tl = pr / n_rep, r = pr - tl * n_rep;
            *reinterpret_cast<float4 *>(qs + pr * HD + d) = *reinterpret_cast<const float4 *>(
                a.q + (size_t)(t0 + tl) * a.q_stride + (size_t)(g * n_rep + r) * HD + d);
        }
    }
    const int special = DECODE && has_pos ? pos - p0 : -1;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = tid + 256 * j;
        if (i >= n4) break;
        const int p = (4 * i) / HD, d = 4 * i - p * HD;
        if (p == special) continue;
        *reinterpret_cast<f32x4 *>(ks + p * KS + d) = kv[j];
    }
    __syncthreads();
    if constexpr (DECODE) {  // the new position's K as the cache holds it
        if (special >= 0)
            for (int d = tid; d < HD; d += 256) ks[special * KS + d] = KvElt<KT>::round(kp[d]);
        __syncthreads();
    }
    // the scores of the wave's pairs; with K from kr (the lane's row) or from LDS
    auto pairs = [&](const auto &kr) {
        for (int pr = wave; pr < n_pairs; pr += 4) {
            const int tl = pr / n_rep, r = pr - tl * n_rep, t = t0 + tl;
            const int n_kv = DECODE ? pos + 1 : a.n_kv0 + t;
            const int np = n_kv - p0 < CH ? n_kv - p0 : CH;
            if (lane < np) {
                const float s = dot_avx2_order<HD>(qs + pr * HD, kr) * a.scale;
                a.scores[((size_t)t * a.n_head + g * n_rep + r) * a.max_kv + p0 + lane] = s;
            }
        }
    };
    if constexpr (!DECODE && HD % 32 == 0 && HD <= 128) {
        // prefill: the wave's many pairs share the lane's K row, read out of LDS into registers once
        // (the LDS then serves only the pairs' q, a broadcast)
        KRowReg<HD> kr;
#pragma unroll
        for (int i = 0; i < HD / 4; i++) kr.r[i] = *reinterpret_cast<const f32x4 *>(ks + lane * KS + 4 * i);
        pairs(kr);
    } else {
        pairs(KRowLds{ks + lane * KS});
    }
}

// Grid (n_head * HD / 256, n_tok), 256 threads: thread (head h = h0 + tid / HD, element d = tid % HD).
// Per head: max and the double sum of e_j over the token's positions (reductions across the head's
// threads), then the weights in LDS (PW / HPB positions per head at a time) and out[d] = one FMA
// chain over the positions in order. Decode: the 256 outputs (one Q8_K block) are also quantised to xq.
template <int HD, bool DECODE, class KT>
__global__ __launch_bounds__(256) void k_attn_softmax_pv(AttnArgs a) {
    constexpr int HPB = 256 / HD, GW = HD < 64 ? HD : 64;  // heads per block, lanes per head in a wave
    constexpr int PB = PW / HPB;                           // weights per head per pass
    static_assert(HD * HPB == 256, "head_dim divides 256");
    __shared__ float pw[HPB][PB];
    __shared__ float redf[4];
    __shared__ double redd[4];
    __shared__ float obuf[256];
    const int tid = threadIdx.x, hl = tid / HD, d = tid - hl * HD, wave = tid >> 6;
    const int t = blockIdx.y;
    // (a last, partial group of heads repeats the last head in its spare threads, which store nothing)
    const int h_raw = blockIdx.x * HPB + hl, h = h_raw < a.n_head ? h_raw : a.n_head - 1;
    const int n_rep = a.n_head / a.n_kv_head, g = h / n_rep;
    const int n = DECODE ? a.step[1] + 1 : a.n_kv0 + t;
    const float *row = a.scores + ((size_t)t * a.n_head + h) * a.max_kv;
    // maximum over the head's positions
    float m = row_max(row, d, HD, n);
    for (int off = GW / 2; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if constexpr (HD > 64) {
        if ((tid & 63) == 0) redf[wave] = m;
        __syncthreads();
        m = -INFINITY;
        for (int w = 0; w < HD / 64; w++) m = fmaxf(m, redf[hl * (HD / 64) + w]);
    }
    // sum of expf(score - max) in double
    double sum = row_expsum(row, d, HD, n, m);
    for (int off = GW / 2; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
    if constexpr (HD > 64) {
        if ((tid & 63) == 0) redd[wave] = sum;
        __syncthreads();
        sum = 0.0;
        for (int w = 0; w < HD / 64; w++) sum += redd[hl * (HD / 64) + w];
    }
    const float inv = (float)(1.0 / sum);
    // weighted V, PB positions at a time
    const KT *vg = (const KT *)a.v_cache + g * a.head_stride + d;
    float acc = 0.0f;
    for (int jb = 0; jb < n; jb += PB) {
        const int je = jb + PB < n ? jb + PB : n;
        __syncthreads();
        row_weights(row, jb + d, HD, je, m, inv, pw[hl], jb, 1);
        __syncthreads();
        int j = jb;
        for (; j + 8 <= je; j += 8) {
            float vv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) vv[u] = KvElt<KT>::ld(vg, (size_t)(j + u) * HD);
#pragma unroll
            for (int u = 0; u < 8; u++) acc = fmaf(pw[hl][j + u - jb], vv[u], acc);
        }
        for (; j < je; j++) acc = fmaf(pw[hl][j - jb], KvElt<KT>::ld(vg, (size_t)j * HD), acc);
    }
    if (h_raw < a.n_head) a.out[(size_t)t * a.out_stride + (size_t)h * HD + d] = acc;
    if constexpr (DECODE) {
        if (a.xq) {  // (n_head * HD is a multiple of 256 here: whole blocks)
            obuf[tid] = acc;
            __syncthreads();
            if (wave == 0) {
                const int lane = tid;
                const float xs[4] = {obuf[4 * lane], obuf[4 * lane + 1], obuf[4 * lane + 2], obuf[4 * lane + 3]};
                sdy_q8k_block(xs, lane, a.xq + (size_t)blockIdx.x * 292);
            }
        }
    }
}

// Prefill softmax and weighted V of 256 / HD heads for TB consecutive tokens per workgroup: the
// arithmetic of k_attn_softmax_pv for each (token, head) (same maxima, double sums, weights and one
// in-order FMA chain per output), but each V element is read once for the TB tokens, whose chains
// advance together position by position (TB independent chains per thread). Tokens past n_tok
// repeat the last one and store nothing.
template <int HD, int TB, class KT>
__global__ __launch_bounds__(256) void k_attn_prefill_pv(AttnArgs a) {
    constexpr int HPB = 256 / HD, GW = HD < 64 ? HD : 64, NW = HD > 64 ? HD / 64 : 1;
    constexpr int PB = PW / (HPB * TB);  // weights per (token, head) per pass
    static_assert(HD * HPB == 256 && PB % 4 == 0, "head_dim divides 256");
    __shared__ __align__(16) float pw[TB][HPB][PB];
    __shared__ float redf[4][TB];
    __shared__ double redd[4][TB];
    const int tid = threadIdx.x, hl = tid / HD, d = tid - hl * HD, wave = tid >> 6;
    const int t0 = blockIdx.y * TB;
    const int h_raw = blockIdx.x * HPB + hl, h = h_raw < a.n_head ? h_raw : a.n_head - 1;
    const int n_rep = a.n_head / a.n_kv_head, g = h / n_rep;
    int nt[TB];
    const float *rows[TB];
#pragma unroll
    for (int ti = 0; ti < TB; ti++) {
        const int t = t0 + ti < a.n_tok ? t0 + ti : a.n_tok - 1;
        nt[ti] = a.n_kv0 + t;
        rows[ti] = a.scores + ((size_t)t * a.n_head + h) * a.max_kv;
    }
    float m[TB], inv[TB];
#pragma unroll
    for (int ti = 0; ti < TB; ti++) {
        float mm = row_max(rows[ti], d, HD, nt[ti]);
        for (int off = GW / 2; off >= 1; off >>= 1) mm = fmaxf(mm, __shfl_xor(mm, off));
        m[ti] = mm;
        if (HD > 64 && (tid & 63) == 0) redf[wave][ti] = mm;
    }
    if constexpr (HD > 64) {
        __syncthreads();
#pragma unroll
        for (int ti = 0; ti < TB; ti++) {
            float mm = -INFINITY;
            for (int w = 0; w < NW; w++) mm = fmaxf(mm, redf[hl * NW + w][ti]);
            m[ti] = mm;
        }
    }
#pragma unroll
    for (int ti = 0; ti < TB; ti++) {
        double sum = row_expsum(rows[ti], d, HD, nt[ti], m[ti]);
        for (int off = GW / 2; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
        if (HD > 64 && (tid & 63) == 0) redd[wave][ti] = sum;
        inv[ti] = (float)(1.0 / sum);
    }
    if constexpr (HD > 64) {
        __syncthreads();
#pragma unroll
        for (int ti = 0; ti < TB; ti++) {
            double sum = 0.0;
            for (int w = 0; w < NW; w++) sum += redd[hl * NW + w][ti];
            inv[ti] = (float)(1.0 / sum);
        }
    }
    const KT *vg = (const KT *)a.v_cache + g * a.head_stride + d;
    float acc[TB];
#pragma unroll
    for (int ti = 0; ti < TB; ti++) acc[ti] = 0.0f;
    const int n_lo = nt[0], n_hi = nt[TB - 1];  // positions of the first and the last token
    for (int jb = 0; jb < n_hi; jb += PB) {
        __syncthreads();
#pragma unroll
        for (int ti = 0; ti < TB; ti++) {
            const int je = jb + PB < nt[ti] ? jb + PB : nt[ti];
            row_weights(rows[ti], jb + d, HD, je, m[ti], inv[ti], pw[ti][hl], jb, 1);
        }
        __syncthreads();
        const int je_all = jb + PB < n_lo ? jb + PB : n_lo, je_any = jb + PB < n_hi ? jb + PB : n_hi;
        int j = jb;
        for (; j + 8 <= je_all; j += 8) {  // positions every token of the block sees
            float vv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) vv[u] = KvElt<KT>::ld(vg, (size_t)(j + u) * HD);
#pragma unroll
            for (int u = 0; u < 8; u++)
#pragma unroll
                for (int ti = 0; ti < TB; ti++) acc[ti] = fmaf(pw[ti][hl][j + u - jb], vv[u], acc[ti]);
        }
        for (; j < je_any; j++) {
            const float v = KvElt<KT>::ld(vg, (size_t)j * HD);
#pragma unroll
            for (int ti = 0; ti < TB; ti++)
                if (j < nt[ti]) acc[ti] = fmaf(pw[ti][hl][j - jb], v, acc[ti]);
        }
    }
#pragma unroll
    for (int ti = 0; ti < TB; ti++)
        if (h_raw < a.n_head && t0 + ti < a.n_tok) a.out[(size_t)(t0 + ti) * a.out_stride + (size_t)h * HD + d] = acc[ti];
}

// Decode softmax in place: one workgroup of 256 threads per query head turns the head's scores s_j
// (j = 0..pos) into p_j = expf(s_j - m) * inv, m the maximum and inv = (float)(1 / sum expf(s_j - m))
// with the sum in double. Each thread reads and rewrites only its own entries (j = tid mod 256).
__global__ __launch_bounds__(256) void k_attn_decode_softmax(AttnArgs a) {
    __shared__ float red_m[4];
    __shared__ double red_s[4];
    const int tid = threadIdx.x, wave = tid >> 6, n = a.step[1] + 1;
    float *row = a.scores + (size_t)blockIdx.x * a.max_kv;
    constexpr int KR = 8;  // up to 256 KR positions: each thread's scores stay in registers
    if (n <= 256 * KR) {
        // one read of the row, one exponential per score, one write: the same values and order as
        // the three passes below
        const uint32_t etab = sdy_expf_tab_lane(tid & 63);
        float v[KR];
#pragma unroll
        for (int k = 0; k < KR; k++) {
            const int j = tid + 256 * k;
            v[k] = row[j < n ? j : n - 1];
        }
        float m = -INFINITY;
#pragma unroll
        for (int k = 0; k < KR; k++)
            if (tid + 256 * k < n) m = fmaxf(m, v[k]);
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        if ((tid & 63) == 0) red_m[wave] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
        double sum = 0.0;
#pragma unroll
        for (int k = 0; k < KR; k++) {
            v[k] = sdy_expf_reg(v[k] - m, etab);  // every lane (the table lookup reads other lanes)
            if (tid + 256 * k < n) sum += (double)v[k];
        }
        for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
        if ((tid & 63) == 0) red_s[wave] = sum;
        __syncthreads();
        sum = (red_s[0] + red_s[1]) + (red_s[2] + red_s[3]);
        const float inv = (float)(1.0 / sum);
#pragma unroll
        for (int k = 0; k < KR; k++) {
            const int j = tid + 256 * k;
            if (j < n) row[j] = v[k] * inv;
        }
        return;
    }
    float m = row_max(row, tid, 256, n);
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((tid & 63) == 0) red_m[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
    double sum = row_expsum(row, tid, 256, n, m);
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
    if ((tid & 63) == 0) red_s[wave] = sum;
    __syncthreads();
    sum = (red_s[0] + red_s[1]) + (red_s[2] + red_s[3]);
    row_weights(row, tid, 256, n, m, (float)(1.0 / sum), row, 0, 1);
}

// Decode weighted V: lane (r, d) of a wave owns dim d of query head r of HPW heads that share a KV
// head and runs its FMA chain out = fma(p_j, v_j[d], out) over j = 0..pos in order (the reference's
// in-order axpy). A wave covers DS = 64 / HPW consecutive dims; its loads of V row j read those DS
// floats (each by HPW lanes) and its weight loads read four positions of each head at once. The
// chains are latency-bound, so the grid is n_kv_head * (n_rep / HPW) * (HD / DS) one-wave workgroups
// (one per CU), each with PF positions in flight in registers.
template <int HD, int HPW, int PF, class KT>
__global__ __launch_bounds__(64) void k_attn_decode_wv(AttnArgs a) {
    constexpr int DS = 64 / HPW, NS = HD / DS, G = PF / 4, B = KvElt<KT>::BYTES;
    static_assert(DS * HPW == 64 && NS * DS == HD && PF % 4 == 0 && 3 * HD * 4 < 4096, "shape");
    const int lane = threadIdx.x, r = lane / DS, dd = lane - r * DS;
    const int n_rep = a.n_head / a.n_kv_head, n_hg = n_rep / HPW;
    const int s = blockIdx.x % NS, hg = (blockIdx.x / NS) % n_hg, g = blockIdx.x / (NS * n_hg);
    const int h0 = g * n_rep + hg * HPW, d = s * DS + dd;
    const int n = a.step[1] + 1;
    // Buffer reads, range-checked on the lane offset (plus the instruction's constant offset): V rows
    // at or past n and weights past the last head's row read as 0 and are never used.
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((KT *)a.v_cache + g * a.head_stride, (short)0,
                                                                        n * HD * B, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(a.scores + (size_t)h0 * a.max_kv, (short)0,
                                                                        HPW * a.max_kv * 4, 0x00020000);
    // position j of the group at lane offset o: V row j + k at o + k * HD * B (constant offsets)
    auto ldv = [&](uint32_t o, int k) { return KvElt<KT>::ld_buf(rv, o + k * HD * B); };
    auto ldw = [&](uint32_t o) { return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, o, 0, 0)); };
    uint32_t ov = d * B, ow = r * a.max_kv * 4;  // the next refill's group 0 (V row, weight)
    float vr[PF];
    f32x4 wr[G];  // wr[q][k] and vr[4q + k] hold position j + 4q + k
#pragma unroll
    for (int q = 0; q < G; q++) {
        wr[q] = ldw(ow + q * 16);
#pragma unroll
        for (int k = 0; k < 4; k++) vr[4 * q + k] = ldv(ov + q * 4 * HD * B, k);
        __builtin_amdgcn_sched_barrier(0);  // issued in position order
    }
    ov += PF * HD * B;
    ow += PF * 4;
    float acc = 0.0f;
    int j = 0;
    for (; j + PF <= n; j += PF) {
#pragma unroll
        for (int q = 0; q < G; q++) {
            const f32x4 w = wr[q];
#pragma unroll
            for (int k = 0; k < 4; k++) acc = fmaf(w[k], vr[4 * q + k], acc);
            // an opaque zero that depends on acc: the group's refill cannot be issued before its
            // slots are read, so each refill reuses its slot's registers
            uint32_t z;
            asm volatile("s_mov_b32 %0, 0" : "=s"(z) : "v"(acc));
            const uint32_t oq = ov + q * 4 * HD * B + z;
            wr[q] = ldw(ow + q * 16 + z);
#pragma unroll
            for (int k = 0; k < 4; k++) vr[4 * q + k] = ldv(oq, k);
        }
        ov += PF * HD * B;
        ow += PF * 4;
    }
#pragma unroll
    for (int u = 0; u < PF; u++)  // the last n - j < PF positions, already in the ring
        if (j + u < n) acc = fmaf(wr[u / 4][u % 4], vr[u], acc);
    a.out[(size_t)(h0 + r) * HD + d] = acc;
}

// Decode weighted V, four heads of a KV group per wave (n_rep % 4 == 0): lane (r, c) owns dim
// s*16 + c of head h0 + r and runs its FMA chain out = fma(p_j, v_j[d], out) over j = 0..pos in order
// (the reference's in-order axpy), exactly as k_attn_decode_wv, with fewer instructions per
// position. Per block of 16 positions the wave issues four V loads, lane (r, c) reading V[j + r][d]
// (four positions x 16 dims per instruction), and one weight load, lane (r, c) reading p[h0 + r][j + c].
// Both go through wave-private LDS buffers ([c][position] and [r][position]), so one 16-byte read
// gives a lane four positions of its dim, and one (a broadcast within the head's 16 lanes) four
// of its weights. R blocks of loads stay in flight in registers; LDS is double-buffered by block
// parity (block b + 1 is staged while block b is consumed).
template <int HD, int R, class KT>
__global__ __launch_bounds__(64) void k_attn_decode_wv4(AttnArgs a) {
    constexpr int NS = HD / 16, B = KvElt<KT>::BYTES;
    static_assert(NS * 16 == HD && R % 2 == 0, "shape");
    __shared__ __align__(16) float tv[2][4][64];  // [block parity][group][c * 4 + position in group]
    __shared__ __align__(16) float tw[2][64];     // [block parity][r * 16 + position in block]
    const int lane = threadIdx.x, r = lane >> 4, c = lane & 15;
    const int n_rep = a.n_head / a.n_kv_head, n_hg = n_rep / 4;
    const int s = blockIdx.x % NS, hg = (blockIdx.x / NS) % n_hg, g = blockIdx.x / (NS * n_hg);
    const int h0 = g * n_rep + hg * 4, d = s * 16 + c;
    const int n = a.step[1] + 1, nbk = (n + 15) / 16;
    // Buffer reads, range-checked on the lane offset: V rows at or past n, and weights past the
    // last head's row, read as 0; positions past n are never used.
    const __amdgpu_buffer_rsrc_t rsv = __builtin_amdgcn_make_buffer_rsrc((KT *)a.v_cache + g * a.head_stride, (short)0,
                                                                         n * HD * B, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc(a.scores + (size_t)h0 * a.max_kv, (short)0,
                                                                         4 * a.max_kv * 4, 0x00020000);
    const uint32_t ov = (uint32_t)(r * HD + d) * B, ow = (uint32_t)(r * a.max_kv + c) * 4;
    float rv[R][4], rw[R];  // ring slot t holds the loads of a block b with b % R == t
    auto issue = [&](int t, uint32_t b) {
        const uint32_t vb = ov + b * 16u * HD * B;
#pragma unroll
        for (int q = 0; q < 4; q++) rv[t][q] = KvElt<KT>::ld_buf(rsv, vb + q * 4 * HD * B);
        rw[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsw, ow + b * 64u, 0, 0));
    };
    auto stage = [&](int t, int par) {
#pragma unroll
        for (int q = 0; q < 4; q++) tv[par][q][c * 4 + r] = rv[t][q];
        tw[par][lane] = rw[t];
    };
    float acc = 0.0f;
    // a block's operands out of LDS buffer par into registers set e (read one block ahead of use)
    f32x4 vv[2][4], ww[2][4];
    auto fetch = [&](int e, int par) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            vv[e][q] = *reinterpret_cast<const f32x4 *>(&tv[par][q][c * 4]);
            ww[e][q] = *reinterpret_cast<const f32x4 *>(&tw[par][r * 16 + 4 * q]);
        }
    };
    // the chain over the block at position jb in registers set e; full: all 16 positions below n
    auto consume = [&](int e, int jb, bool full) {
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int k = 0; k < 4; k++)
                if (full || jb + 4 * q + k < n) acc = fmaf(ww[e][q][k], vv[e][q][k], acc);
    };
#pragma unroll
    for (int t = 0; t < R; t++) {
        issue(t, t);
        __builtin_amdgcn_sched_barrier(0);  // issued in block order
    }
    stage(0, 0);
    fetch(0, 0);
    // rounds of R blocks that lie wholly below n: straight-line code, so the loads in flight are the
    // same on every path (a block staged past n reads zeros and is never consumed). Iteration t
    // stages block t + 1 and reads it back (a wave's LDS operations run in order), then runs the
    // chain over block t, whose operands were read in the previous iteration.
    int b0 = 0;
    for (; 16 * (b0 + R) <= n; b0 += R) {
#pragma unroll
        for (int t = 0; t < R; t++) {
            stage((t + 1) % R, (t + 1) & 1);
            fetch((t + 1) & 1, (t + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);  // the reads of block t + 1 go out before block t's chain
            consume(t & 1, 16 * (b0 + t), true);
            // an opaque zero that depends on acc: the refill of slot t cannot be issued before the
            // slot's weights are read, so it reuses the slot's registers
            uint32_t z;
            asm volatile("s_mov_b32 %0, 0" : "=s"(z) : "v"(acc));
            issue(t, (uint32_t)(b0 + t + R) + z);
        }
    }
    // the last (fewer than R) blocks, already in flight
#pragma unroll
    for (int t = 0; t < R; t++) {
        const int b = b0 + t;
        if (b >= nbk) break;
        if (b + 1 < nbk) {
            stage((t + 1) % R, (t + 1) & 1);
            fetch((t + 1) & 1, (t + 1) & 1);
        }
        consume(t & 1, 16 * b, false);
    }
    a.out[(size_t)(h0 + r) * HD + d] = acc;
}

// Any head_dim (hd % 4 == 0 is not required): the same arithmetic with runtime loops and scalar LDS
// reads. Scores: as k_attn_scores (prefill or decode), K rows at an odd stride (hd | 1).
SDY_DEV float dot_avx2_order_any(const float *q, const float *k, int hd) {
    float a[4][8];
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int l = 0; l < 8; l++) a[c][l] = 0.0f;
    int i = 0;
    for (; i + 32 <= hd; i += 32)
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int l = 0; l < 8; l++) a[c][l] = fmaf(k[i + 8 * c + l], q[i + 8 * c + l], a[c][l]);
    for (; i + 8 <= hd; i += 8)
#pragma unroll
        for (int l = 0; l < 8; l++) a[0][l] = fmaf(k[i + l], q[i + l], a[0][l]);
    float v[8];
#pragma unroll
    for (int l = 0; l < 8; l++) {
        const float p = a[0][l] + a[1][l], r = a[2][l] + a[3][l];
        v[l] = p + r;
    }
    float s = ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
    for (; i < hd; i++) {
        const float p = q[i] * k[i];
        s = s + p;
    }
    return s;
}

template <bool DECODE, class KT>
__global__ __launch_bounds__(256) void k_attn_scores_any(AttnArgs a, int hd) {
    extern __shared__ __align__(16) float sm[];
    const int KS = hd | 1;
    float *ks = sm;            // [CH][KS]
    float *kp = ks + CH * KS;  // [hd]
    float *qs = kp + hd;       // [pairs][hd]
    const int c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n_rep = a.n_head / a.n_kv_head;
    int t0, t1, n_kv_last, pos = 0;
    if constexpr (DECODE) {
        pos = a.step[1];
        t0 = 0;
        t1 = 1;
        n_kv_last = pos + 1;
    } else {
        const int tbs = PAIRS / n_rep > 0 ? PAIRS / n_rep : 1;
        t0 = blockIdx.z * tbs;
        t1 = t0 + tbs < a.n_tok ? t0 + tbs : a.n_tok;
        n_kv_last = a.n_kv0 + t1 - 1;
    }
    const int p0 = c * CH;
    if (p0 >= n_kv_last) return;
    const int np_max = n_kv_last - p0 < CH ? n_kv_last - p0 : CH;
    const int n_pairs = (t1 - t0) * n_rep;
    bool has_pos = false;
    if constexpr (DECODE) {
        has_pos = p0 + np_max == pos + 1;
        const float *cs = a.rope_cos + (size_t)pos * (hd / 2), *sn = a.rope_sin + (size_t)pos * (hd / 2);
        for (int r = wave; r <= n_rep; r += 4) {
            const bool is_k = r == n_rep;
            float *buf = is_k ? kp : qs + r * hd;
            const float *src = is_k ? a.k + (size_t)g * hd : a.q + (size_t)(g * n_rep + r) * hd;
            for (int i = lane; i < hd; i += 64) buf[i] = src[i];
            sdy_wave_sync();
            norm_rope_wave(buf, is_k ? a.k_norm : a.q_norm, a.eps, cs, sn, hd, a.interleaved, lane);
            if (is_k && has_pos) {
                KT *kc = (KT *)a.k_cache + g * a.head_stride + (size_t)pos * hd;
                KT *vc = (KT *)a.v_cache + g * a.head_stride + (size_t)pos * hd;
                for (int i = lane; i < hd; i += 64) {
                    KvElt<KT>::st(kc, i, buf[i]);
                    KvElt<KT>::st(vc, i, a.v[(size_t)g * hd + i]);
                }
            }
        }
    } else {
        for (int i = tid; i < n_pairs * hd; i += 256) {
            const int pr = i / hd, d = i - pr * hd, tl = pr / n_rep, r = pr - tl * n_rep;
            qs[pr * hd + d] = a.q[(size_t)(t0 + tl) * a.q_stride + (size_t)(g * n_rep + r) * hd + d];
        }
    }
    const int special = DECODE && has_pos ? pos - p0 : -1;
    const KT *kg = (const KT *)a.k_cache + g * a.head_stride + (size_t)p0 * hd;
    for (int i = tid; i < np_max * hd; i += 256) {
        const int p = i / hd, d = i - p * hd;
        if (p != special) ks[p * KS + d] = KvElt<KT>::ld(kg, i);
    }
    __syncthreads();
    if constexpr (DECODE) {  // the new position's K as the cache holds it
        if (special >= 0)
            for (int d = tid; d < hd; d += 256) ks[special * KS + d] = KvElt<KT>::round(kp[d]);
        __syncthreads();
    }
    for (int pr = wave; pr < n_pairs; pr += 4) {
        const int tl = pr / n_rep, r = pr - tl * n_rep, t = t0 + tl;
        const int n_kv = DECODE ? pos + 1 : a.n_kv0 + t;
        const int np = n_kv - p0 < CH ? n_kv - p0 : CH;
        if (lane < np)
            a.scores[((size_t)t * a.n_head + g * n_rep + r) * a.max_kv + p0 + lane] =
                dot_avx2_order_any(qs + pr * hd, ks + lane * KS, hd) * a.scale;
    }
}

// Softmax and weighted V of one head of one token per workgroup (256 threads; output elements
// tid, tid + 256, ...), any head_dim. Decode: no Q8_K output (the caller quantises).
template <bool DECODE, class KT>
__global__ __launch_bounds__(256) void k_attn_softmax_pv_any(AttnArgs a, int hd) {
    __shared__ float pw[PW];
    __shared__ float redf[4];
    __shared__ double redd[4];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int h = blockIdx.x, t = blockIdx.y;
    const int n_rep = a.n_head / a.n_kv_head, g = h / n_rep;
    const int n = DECODE ? a.step[1] + 1 : a.n_kv0 + t;
    const float *row = a.scores + ((size_t)t * a.n_head + h) * a.max_kv;
    float m = row_max(row, tid, 256, n);
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (lane == 0) redf[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
    double sum = row_expsum(row, tid, 256, n, m);
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
    if (lane == 0) redd[wave] = sum;
    __syncthreads();
    sum = (redd[0] + redd[1]) + (redd[2] + redd[3]);
    const float inv = (float)(1.0 / sum);
    const KT *vg = (const KT *)a.v_cache + g * a.head_stride;
    for (int d0 = 0; d0 < hd; d0 += 256) {
        const int d = d0 + tid;
        float acc = 0.0f;
        for (int jb = 0; jb < n; jb += PW) {
            const int je = jb + PW < n ? jb + PW : n;
            __syncthreads();
            row_weights(row, jb + tid, 256, je, m, inv, pw, jb, 1);
            __syncthreads();
            if (d < hd)
                for (int j = jb; j < je; j++) acc = fmaf(pw[j - jb], KvElt<KT>::ld(vg, (size_t)j * hd + d), acc);
        }
        if (d < hd) a.out[(size_t)t * a.out_stride + (size_t)h * hd + d] = acc;
    }
}

}  // namespace

// =============================================================================== launchers

extern "C" size_t sdy_attn_scores_floats(int n_tok, int n_head, int max_kv) {
    return (size_t)n_tok * n_head * ((max_kv + 3) & ~3);
}

static int head_dim_ok(int n_head, int n_kv_head, int hd) {
    return hd >= 1 && hd <= 1024 && n_kv_head >= 1 && n_head % n_kv_head == 0 && n_head / n_kv_head <= PAIRS;
}

static int shape_fail(int n_head, int n_kv_head, int hd) {
    return sdy_fail(-1, "attention: head_dim %d with %d heads / %d kv heads not supported (head_dim up to 1024, at "
                        "most %d query heads per kv head)", hd, n_head, n_kv_head, PAIRS);
}

static size_t scores_lds(int hd, int n_pairs) {
    return sizeof(float) * ((size_t)CH * (hd + 4) + hd + (size_t)n_pairs * hd);
}

template <int HD, bool DECODE, class KT>
static int launch_attn(AttnArgs &A, int nc, int n_tblk, hipStream_t st) {
    const int n_rep = A.n_head / A.n_kv_head;
    const int n_pairs = DECODE ? n_rep : (PAIRS / n_rep > 0 ? PAIRS / n_rep : 1) * n_rep;
    const size_t lds = scores_lds(HD, n_pairs);
    static size_t granted = 0;
    int rc = sdy_lds_limit((const void *)k_attn_scores<HD, DECODE, KT>, lds, &granted);
    if (rc) return rc;
    SDY_NOTE_KERNEL((k_attn_scores<HD, DECODE, KT>));
    hipLaunchKernelGGL((k_attn_scores<HD, DECODE, KT>), dim3(nc, A.n_kv_head, n_tblk), dim3(256), lds, st, A);
    if ((rc = sdy_check_launch("attention_scores"))) return rc;
    if constexpr (DECODE) {
        SDY_NOTE_KERNEL((k_attn_softmax_pv<HD, DECODE, KT>));
        hipLaunchKernelGGL((k_attn_softmax_pv<HD, DECODE, KT>), dim3((A.n_head * HD + 255) / 256, 1), dim3(256), 0, st,
                           A);
    } else {  // four tokens per workgroup
        constexpr int TB = 4;
        SDY_NOTE_KERNEL((k_attn_prefill_pv<HD, TB, KT>));
        hipLaunchKernelGGL((k_attn_prefill_pv<HD, TB, KT>), dim3((A.n_head * HD + 255) / 256, (A.n_tok + TB - 1) / TB),
                           dim3(256), 0, st, A);
    }
    return sdy_check_launch("attention_softmax_pv");
}

template <bool DECODE, class KT>
static int launch_attn_any(AttnArgs &A, int hd, int nc, int n_tblk, hipStream_t st) {
    const int n_rep = A.n_head / A.n_kv_head;
    const int n_pairs = DECODE ? n_rep : (PAIRS / n_rep > 0 ? PAIRS / n_rep : 1) * n_rep;
    const size_t lds = sizeof(float) * ((size_t)CH * (hd | 1) + hd + (size_t)n_pairs * hd);
    if (lds > 160 * 1024) return sdy_fail(-1, "attention: head_dim %d needs %zu bytes of LDS", hd, lds);
    static size_t granted = 0;
    int rc = sdy_lds_limit((const void *)k_attn_scores_any<DECODE, KT>, lds, &granted);
    if (rc) return rc;
    SDY_NOTE_KERNEL((k_attn_scores_any<DECODE, KT>));
    hipLaunchKernelGGL((k_attn_scores_any<DECODE, KT>), dim3(nc, A.n_kv_head, n_tblk), dim3(256), lds, st, A, hd);
    if ((rc = sdy_check_launch("attention_scores"))) return rc;
    SDY_NOTE_KERNEL((k_attn_softmax_pv_any<DECODE, KT>));
    hipLaunchKernelGGL((k_attn_softmax_pv_any<DECODE, KT>), dim3(A.n_head, DECODE ? 1 : A.n_tok), dim3(256), 0, st, A,
                       hd);
    if ((rc = sdy_check_launch("attention_softmax_pv"))) return rc;
    if (DECODE && A.xq) return sdy_quantize(SDY_Q8_K, A.out, A.xq, A.n_head * hd, 1, (sdy_stream)st);
    return 0;
}

// decode: k_attn_scores, k_attn_decode_softmax, k_attn_decode_wv4 (four heads of a KV group per wave)
// or, when 4 does not divide n_rep, k_attn_decode_wv (one head per wave), then the Q8_K row of the
// output when asked for.
template <int HD, class KT>
static int launch_attn_decode(AttnArgs &A, int nc, hipStream_t st) {
    const int n_rep = A.n_head / A.n_kv_head;
    const size_t lds = scores_lds(HD, n_rep);
    static size_t granted = 0;
    int rc = sdy_lds_limit((const void *)k_attn_scores<HD, true, KT>, lds, &granted);
    if (rc) return rc;
    SDY_NOTE_KERNEL((k_attn_scores<HD, true, KT>));
    hipLaunchKernelGGL((k_attn_scores<HD, true, KT>), dim3(nc, A.n_kv_head, 1), dim3(256), lds, st, A);
    if ((rc = sdy_check_launch("attention_scores"))) return rc;
    SDY_NOTE_KERNEL(k_attn_decode_softmax);
    hipLaunchKernelGGL(k_attn_decode_softmax, dim3(A.n_head), dim3(256), 0, st, A);
    if ((rc = sdy_check_launch("attention_decode_softmax"))) return rc;
    if (n_rep % 4) {
        SDY_NOTE_KERNEL((k_attn_decode_wv<HD, 1, 32, KT>));
        hipLaunchKernelGGL((k_attn_decode_wv<HD, 1, 32, KT>), dim3(A.n_head * (HD / 64)), dim3(64), 0, st, A);
    } else {
        SDY_NOTE_KERNEL((k_attn_decode_wv4<HD, 8, KT>));
        hipLaunchKernelGGL((k_attn_decode_wv4<HD, 8, KT>), dim3(A.n_head * HD / 64), dim3(64), 0, st, A);
    }
    if ((rc = sdy_check_launch("attention_decode_wv"))) return rc;
    if (A.xq) return sdy_quantize(SDY_Q8_K, A.out, A.xq, A.n_head * HD, 1, (sdy_stream)st);
    return 0;
}

template <bool DECODE, class KT>
static int attn_dispatch(AttnArgs &A, int hd, int nc, int n_tblk, hipStream_t st) {
    if constexpr (DECODE) {
        switch (hd) {
        case 64: return launch_attn_decode<64, KT>(A, nc, st);
        case 128: return launch_attn_decode<128, KT>(A, nc, st);
        case 256: return launch_attn_decode<256, KT>(A, nc, st);
        default: break;
        }
    }
    switch (hd) {
    case 32: return launch_attn<32, DECODE, KT>(A, nc, n_tblk, st);
    case 64: return launch_attn<64, DECODE, KT>(A, nc, n_tblk, st);
    case 128: return launch_attn<128, DECODE, KT>(A, nc, n_tblk, st);
    case 256: return launch_attn<256, DECODE, KT>(A, nc, n_tblk, st);
    default: return launch_attn_any<DECODE, KT>(A, hd, nc, n_tblk, st);
    }
}

template <bool DECODE>
static int attn_dispatch_kv(AttnArgs &A, int kv_type, int hd, int nc, int n_tblk, hipStream_t st) {
    return kv_type == SDY_KV_F16 ? attn_dispatch<DECODE, uint16_t>(A, hd, nc, n_tblk, st)
                                 : attn_dispatch<DECODE, float>(A, hd, nc, n_tblk, st);
}

extern "C" size_t sdy_kv_elt_bytes(int kv_type) {
    return kv_type == SDY_KV_F32 ? 4 : kv_type == SDY_KV_F16 ? 2 : 0;
}

static int kv_type_fail(int kv_type) { return sdy_fail(-1, "KV cache element type %d not supported", kv_type); }

extern "C" int sdy_qk_rope_kv(float *q, float *k, const float *v, const float *qn, const float *kn, float eps,
                              const float *rope_cos, const float *rope_sin, int pos0, int n_tok, int n_head,
                              int n_kv_head, int hd, int interleaved, void *k_cache, void *v_cache, int kv_type,
                              long head_stride, sdy_stream s) {
    return sdy_qk_rope_kv_strided(q, k, v, (long)n_head * hd, (long)n_kv_head * hd, (long)n_kv_head * hd, qn, kn, eps,
                                  rope_cos, rope_sin, pos0, n_tok, n_head, n_kv_head, hd, interleaved, k_cache, v_cache,
                                  kv_type, head_stride, s);
}

extern "C" int sdy_qk_rope_kv_strided(float *q, float *k, const float *v, long q_stride, long k_stride, long v_stride,
                                      const float *qn, const float *kn, float eps, const float *rope_cos,
                                      const float *rope_sin, int pos0, int n_tok, int n_head, int n_kv_head, int hd,
                                      int interleaved, void *k_cache, void *v_cache, int kv_type, long head_stride,
                                      sdy_stream s) {
    if (hd > 512) return sdy_fail(-1, "head_dim %d above 512", hd);
    if (!sdy_kv_elt_bytes(kv_type)) return kv_type_fail(kv_type);
    if (n_tok <= 0) return 0;
    if (kv_type == SDY_KV_F16)
        hipLaunchKernelGGL(k_qk_rope_kv<uint16_t>, dim3(n_tok, n_head + n_kv_head), dim3(64), 0, (hipStream_t)s, q, k, v,
                           q_stride, k_stride, v_stride, qn, kn, eps, rope_cos, rope_sin, pos0, n_head, n_kv_head, hd,
                           interleaved, (uint16_t *)k_cache, (uint16_t *)v_cache, head_stride);
    else
        hipLaunchKernelGGL(k_qk_rope_kv<float>, dim3(n_tok, n_head + n_kv_head), dim3(64), 0, (hipStream_t)s, q, k, v,
                           q_stride, k_stride, v_stride, qn, kn, eps, rope_cos, rope_sin, pos0, n_head, n_kv_head, hd,
                           interleaved, (float *)k_cache, (float *)v_cache, head_stride);
    return sdy_check_launch("qk_rope_kv");
}

extern "C" int sdy_attention(const float *q, const void *k_cache, const void *v_cache, int kv_type, int n_tok,
                             int n_head, int n_kv_head, int hd, int n_kv0, long head_stride, long q_stride,
                             float *scores, float *out, long out_stride, sdy_stream s) {
    if (n_tok <= 0) return 0;
    if (!head_dim_ok(n_head, n_kv_head, hd)) return shape_fail(n_head, n_kv_head, hd);
    if (!sdy_kv_elt_bytes(kv_type)) return kv_type_fail(kv_type);
    AttnArgs A = {};
    A.q = q;
    A.n_head = n_head;
    A.n_kv_head = n_kv_head;
    A.n_kv0 = n_kv0;
    A.n_tok = n_tok;
    A.q_stride = q_stride;
    A.k_cache = (void *)k_cache;
    A.v_cache = (void *)v_cache;
    A.head_stride = head_stride;
    A.scores = scores;
    A.max_kv = n_kv0 + n_tok - 1;
    A.scale = 1.0f / sqrtf((float)hd);
    A.out = out;
    A.out_stride = out_stride;
    const int n_rep = n_head / n_kv_head, tbs = PAIRS / n_rep > 0 ? PAIRS / n_rep : 1;
    const int nc = (A.max_kv + CH - 1) / CH;
    return attn_dispatch_kv<false>(A, kv_type, hd, nc, (n_tok + tbs - 1) / tbs, (hipStream_t)s);
}

extern "C" int sdy_attn_decode_ok(int n_head, int n_kv_head, int hd, int max_seq) {
    (void)max_seq;
    return head_dim_ok(n_head, n_kv_head, hd) && scores_lds(hd | 1, n_head / n_kv_head) <= 160 * 1024;
}

extern "C" int sdy_attn_decode(const float *q, const float *k, const float *v, const float *q_norm,
                               const float *k_norm, float eps, const float *rope_cos, const float *rope_sin,
                               const int32_t *step_dev, int n_head, int n_kv_head, int hd, int interleaved,
                               void *k_cache, void *v_cache, int kv_type, long head_stride, int max_seq,
                               float *scores, float *out, void *xq_q8k, sdy_stream s) {
    if (!sdy_attn_decode_ok(n_head, n_kv_head, hd, max_seq)) return shape_fail(n_head, n_kv_head, hd);
    if (!sdy_kv_elt_bytes(kv_type)) return kv_type_fail(kv_type);
    if (xq_q8k && (n_head * hd) % 256) return sdy_fail(-1, "attn_decode: %d outputs are not whole Q8_K blocks", n_head * hd);
    AttnArgs A = {};
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
    A.n_tok = 1;
    A.interleaved = interleaved;
    A.k_cache = k_cache;
    A.v_cache = v_cache;
    A.head_stride = head_stride;
    A.scores = scores;
    A.max_kv = (max_seq + 3) & ~3;  // score rows padded to whole 16-byte groups
    A.scale = 1.0f / sqrtf((float)hd);
    A.out = out;
    A.out_stride = (long)n_head * hd;
    A.xq = (uint8_t *)xq_q8k;
    return attn_dispatch_kv<true>(A, kv_type, hd, (max_seq + CH - 1) / CH, 1, (hipStream_t)s);
}

// Decode attention of one token in two launches, split over spans of positions (within tolerance
// of the reference, not its bits).
//
// The reference's op_attention_head (csrc/ops.c:405-414) computes, per query head, the scores
// s_j = q.k_j / sqrt(head_dim) over every cached position j, one softmax over all of them and the
// weighted sum of the V rows. Here the positions are cut into spans of `span` (a multiple of 64):
//
//   k_attn_chunk<HD, HW, KT>  256 threads, one workgroup per (span, kv head, share of the group's
//                          query heads; the shares of one span and head on one XCD):
//     - q/k RMSNorm (qwen3) and RoPE of the group's queries, and of the new k when the span holds
//       the token's own position (that workgroup writes the new K/V row to the cache);
//     - the span's positions in sub-chunks of 64: K and V rows staged in LDS (the next sub-chunk's
//       loads in flight meanwhile), the scores (lane = position), the running maximum m, e = exp(s - m)
//       and the sums l = sum e, o = sum e * v, rescaled by exp(m_old - m_new) when m grows;
//     - (m, l, o) stored as the span's partial;
//   k_attn_merge<HD>       grid n_head * HD / 256, 256 threads: per (head, dim), over the spans in
//                          ascending order, M = max m_s, L = sum l_s exp(m_s - M),
//                          out = sum o_s exp(m_s - M) / L; and the Q8_K block of the workgroup's 256
//                          outputs when asked for.
//
// Each sum has a fixed order (no float atomics): the results are deterministic. They differ from
// the reference's in rounding only (exponentials of span-relative scores, f32 partial sums). The
// kernel boundary between the two launches publishes the partials to every XCD.
#include "sdy_attn_dev.h"
#include "sdy_device.h"
#include "sdy_internal.h"
#include "sdy_norm_dev.h"
#include "sdy_ops.h"
#include "sdy_quant_dev.h"
#include "sdy_shim.h"

namespace {

constexpr int SUB = 64;      // positions per sub-chunk: one per lane in the scores
constexpr int MAX_REP = 16;  // query heads per kv head
constexpr int MAX_SPANS = 128;  // spans per kv head at most (the span grows with max_seq beyond that)
constexpr int MERGE_ROUND = 16;  // spans whose partials the merge loads at a time

struct ChunkArgs {
    const float *q, *k, *v;          // the token's raw q [n_head][HD], k and v [n_kv_head][HD]
    const float *q_norm, *k_norm;    // per-head RMSNorm weights (qwen3) or null
    float eps;
    const float *rope_cos, *rope_sin;
    const int32_t *step;             // step[1] = the token's position
    int n_head, n_kv_head, interleaved;
    int span, n_span_max;            // positions per workgroup (a multiple of SUB), spans per kv head
    int hsplit;                      // workgroups sharing a kv group's heads (each takes n_rep / hsplit)
    void *k_cache, *v_cache;         // [n_kv_head][max_seq][HD] of KT
    long head_stride;                // max_seq * HD elements
    float scale;                     // 1 / sqrtf(HD)
    float *part;                     // [n_head][n_span_max][HD + 4]: m, l, -, -, o[HD]
    float *out;                      // [n_head][HD]
    uint8_t *xq;                     // Q8_K blocks of out (or null)
};

template <int HD>
constexpr size_t chunk_lds_floats() {
    return (size_t)SUB * (HD + 4) + (size_t)SUB * HD + (size_t)MAX_REP * HD + 2 * HD + (size_t)MAX_REP * SUB +
           MAX_REP;
}

// Wave-wide maximum and sum: DPP within each row of 16 lanes, then the four rows by readlane (the
// result is uniform over the wave).
template <int CTRL>
SDY_DEV float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
SDY_DEV float lane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
SDY_DEV float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));   // quad_perm [1, 0, 3, 2]
    v = fmaxf(v, dpp_f<0x4E>(v));   // quad_perm [2, 3, 0, 1]
    v = fmaxf(v, dpp_f<0x124>(v));  // row_ror 4
    v = fmaxf(v, dpp_f<0x128>(v));  // row_ror 8
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
SDY_DEV float wave_sum(float v) {
    v = v + dpp_f<0xB1>(v);
    v = v + dpp_f<0x4E>(v);
    v = v + dpp_f<0x124>(v);
    v = v + dpp_f<0x128>(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

// HW: query heads per wave in the scores (n_rep / hsplit <= 4 HW); wave w takes heads w, w + 4, ...
template <int HD, int HW, class KT>
__global__ __launch_bounds__(256) void k_attn_chunk(ChunkArgs a) {
    constexpr int KS = HD + 4;           // K rows in LDS: 16-byte aligned, consecutive rows on other banks
    constexpr int L4 = HD / 4;           // float4 per row
    constexpr int PER = SUB * L4 / 256;  // float4 of K (and of V) per thread per sub-chunk
    constexpr int HPS = 256 / HD;        // head slots of the weighted sum (thread = head slot, dim)
    constexpr int NP = 4 * HW / HPS;     // the thread's heads in the weighted sum: slot + HPS * k
    constexpr int E = HD / 64, EH = E / 2;  // vector elements per lane (lane + 64 e)
    constexpr int RV = HW + 1;           // vectors a wave prepares: its queries and, maybe, the new k
    static_assert(PER * 256 == SUB * L4 && HPS * HD == 256 && NP >= 1 && 4 * HW <= MAX_REP, "shape");
    extern __shared__ __align__(16) float sm[];
    float *ks = sm;                    // [SUB][KS]
    float *vs = ks + SUB * KS;         // [SUB][HD]
    float *qs = vs + SUB * HD;         // [MAX_REP][HD] rotated queries
    float *kn = qs + MAX_REP * HD;     // [HD] the new k, rotated
    float *vn = kn + HD;               // [HD] the new v
    float *es = vn + HD;               // [MAX_REP][SUB] exp(s - m) of the sub-chunk
    float *cs_l = es + MAX_REP * SUB;  // [MAX_REP] rescale of a head's old sums at this sub-chunk

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // workgroup -> (span, kv group, share of its heads). With two shares, the two workgroups of one
    // (span, group) are 8 apart in the launch order: workgroups are dealt to the 8 XCDs in turn, so
    // they run on one XCD and the span's K/V rows are fetched from HBM into its L2 once (apart, on
    // two XCDs, every row came from HBM twice: 2.2x the K/V bytes, PMC)
    const int wg = blockIdx.x;
    const int j = a.hsplit == 2 ? ((wg >> 4) << 3) | (wg & 7) : wg, hs = a.hsplit == 2 ? (wg >> 3) & 1 : 0;
    if (j >= a.n_span_max * a.n_kv_head) return;  // (padding of the launch to whole groups of 16)
    const int g = j / a.n_span_max, sp = j - g * a.n_span_max;
    const int n_rep = a.n_head / a.n_kv_head;
    const int nh = n_rep / a.hsplit;   // the workgroup's query heads: h0 .. h0 + nh - 1
    const int h0 = g * n_rep + hs * nh;
    const int pos = a.step[1], n_kv = pos + 1;
    const int p_begin = sp * a.span;
    if (p_begin >= n_kv) return;  // beyond the token's position: no partial
    const int p_end = min(p_begin + a.span, n_kv);
    const bool own = p_end == n_kv;           // the span holds the token's own position
    const int cached_end = own ? pos : p_end;  // rows below come from the cache
    const KT *kc = (const KT *)a.k_cache + g * a.head_stride;
    const KT *vc = (const KT *)a.v_cache + g * a.head_stride;

    sdy_f32x4 kr[PER], vr[PER];
    // every load unconditional (rows past the cached ones read row 0, never stored to LDS), so that
    // the compiler's wait counts stay exact
    auto issue = [&](int p0) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int f = tid + 256 * i, row = f / L4, col = f - row * L4, p = p0 + row;
            const int pl = p < cached_end ? p : 0;
            kr[i] = KvElt<KT>::ld4(kc, (size_t)pl * HD + 4 * col);
            vr[i] = KvElt<KT>::ld4(vc, (size_t)pl * HD + 4 * col);
        }
    };

    // The group's queries and, in the span of the token's position, the new k: vector r = wave + 4 i
    // by wave `wave`, lane l holding elements l + 64 e. Every input is loaded first, then the span's
    // first K/V rows are requested (loads complete in order: the rotation below waits only for its
    // own inputs, not for the K/V tile), then the reference's per-head RMSNorm (qwen3) and rotation.
    {
        const int n_vec = nh + (own ? 1 : 0);
        const float *cs = a.rope_cos + (size_t)pos * (HD / 2), *sn = a.rope_sin + (size_t)pos * (HD / 2);
        float x[RV][E], nq[E], nk[E], vnew[E], c[E], s[E];
#pragma unroll
        for (int i = 0; i < RV; i++) {
            const int r = min(wave + 4 * i, n_vec - 1);
            const float *src = r == nh ? a.k + (size_t)g * HD : a.q + (size_t)(h0 + r) * HD;
#pragma unroll
            for (int e = 0; e < E; e++) x[i][e] = src[lane + 64 * e];
        }
#pragma unroll
        for (int e = 0; e < E; e++) {
            const int j = lane + 64 * e, ci = a.interleaved ? j >> 1 : j & (HD / 2 - 1);
            nq[e] = a.q_norm ? a.q_norm[j] : 1.0f;
            nk[e] = a.k_norm ? a.k_norm[j] : 1.0f;
            vnew[e] = a.v[(size_t)g * HD + j];
            c[e] = cs[ci];
            s[e] = sn[ci];
        }
        __builtin_amdgcn_sched_barrier(0);
        issue(p_begin);
#pragma unroll
        for (int i = 0; i < RV; i++) {
            const int r = wave + 4 * i;
            if (r >= n_vec) break;
            const bool is_k = r == nh;
            float y[E];
#pragma unroll
            for (int e = 0; e < E; e++) y[e] = x[i][e];
            if (is_k ? a.k_norm != nullptr : a.q_norm != nullptr) {
                double ss = 0.0;
#pragma unroll
                for (int e = 0; e < E; e++) ss += (double)y[e] * (double)y[e];
                ss = sdy_wave_sum_f64(ss);  // (the butterfly over lane ^ 32, ..., 1; the branch is uniform)
                const float sc = (float)(1.0 / sqrt(ss / (double)HD + (double)a.eps));
#pragma unroll
                for (int e = 0; e < E; e++) {
                    const float t = y[e] * sc;
                    y[e] = t * (is_k ? nk[e] : nq[e]);
                }
            }
            // RoPE: the pair partner (adjacent lane when interleaved, else element j +- HD/2)
            float pr[E];
            bool first[E];
#pragma unroll
            for (int e = 0; e < E; e++) {
                if (a.interleaved) {
                    pr[e] = dpp_f<0xB1>(y[e]);
                    first[e] = (lane & 1) == 0;
                } else if constexpr (E == 1) {
                    pr[e] = __shfl_xor(y[e], 32);
                    first[e] = lane < 32;
                } else {
                    pr[e] = y[(e + EH) % E];
                    first[e] = e < EH;
                }
            }
            float o[E];
#pragma unroll
            for (int e = 0; e < E; e++) {
                if (first[e]) {
                    const float ac = y[e] * c[e], bs = pr[e] * s[e];
                    o[e] = ac - bs;
                } else {
                    const float as = pr[e] * s[e], bc = y[e] * c[e];
                    o[e] = as + bc;
                }
            }
            float *buf = is_k ? kn : qs + r * HD;
#pragma unroll
            for (int e = 0; e < E; e++) buf[lane + 64 * e] = o[e];
            if (is_k) {  // the new K/V row (written to the cache by the group's first workgroup)
                KT *kw = (KT *)a.k_cache + g * a.head_stride + (size_t)pos * HD;
                KT *vw = (KT *)a.v_cache + g * a.head_stride + (size_t)pos * HD;
#pragma unroll
                for (int e = 0; e < E; e++) {
                    vn[lane + 64 * e] = vnew[e];
                    if (hs == 0) {
                        KvElt<KT>::st(kw, lane + 64 * e, o[e]);
                        KvElt<KT>::st(vw, lane + 64 * e, vnew[e]);
                    }
                }
            }
        }
    }

    // running maximum and sum of the wave's heads (uniform over the wave)
    float m_run[HW], l_run[HW];
#pragma unroll
    for (int h = 0; h < HW; h++) {
        m_run[h] = -INFINITY;
        l_run[h] = 0.0f;
    }
    const int slot = __builtin_amdgcn_readfirstlane(tid / HD), d = tid - slot * HD;
    int rc[NP];  // the weighted sum's heads, clamped to the group (extra ones are computed, not stored)
#pragma unroll
    for (int k = 0; k < NP; k++) rc[k] = min(slot + HPS * k, nh - 1);
    float acc[NP];
#pragma unroll
    for (int k = 0; k < NP; k++) acc[k] = 0.0f;

    for (int p0 = p_begin; p0 < p_end; p0 += SUB) {
        const int np = min(SUB, p_end - p0);
        __syncthreads();  // the previous sub-chunk's readers are done (and, first, the queries are ready)
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int f = tid + 256 * i, row = f / L4, col = f - row * L4;
            if (p0 + row < cached_end) {
                *reinterpret_cast<sdy_f32x4 *>(ks + row * KS + 4 * col) = kr[i];
                *reinterpret_cast<sdy_f32x4 *>(vs + row * HD + 4 * col) = vr[i];
            }
        }
        if (own && pos - p0 < SUB && tid < HD) {  // the token's own row, as the cache holds it
            ks[(pos - p0) * KS + tid] = KvElt<KT>::round(kn[tid]);
            vs[(pos - p0) * HD + tid] = KvElt<KT>::round(vn[tid]);
        }
        __syncthreads();
        if (p0 + SUB < p_end) issue(p0 + SUB);  // the next sub-chunk's loads, in flight during this one

        // scores of the wave's heads at position lane (each K row read once for all of them)
        float sc[HW];
        {
            // blocks of IB float4 steps whose LDS reads (K row, HW query rows) are all issued before
            // their FMAs, at most 12 in flight
            constexpr int IB = HW <= 2 ? 4 : 2;
            float dd[HW][4];
#pragma unroll
            for (int h = 0; h < HW; h++) dd[h][0] = dd[h][1] = dd[h][2] = dd[h][3] = 0.0f;
            const sdy_f32x4 *kp = reinterpret_cast<const sdy_f32x4 *>(ks + lane * KS);
            const sdy_f32x4 *qp = reinterpret_cast<const sdy_f32x4 *>(qs + wave * HD);
            for (int i0 = 0; i0 < L4; i0 += IB) {
                sdy_f32x4 kk[IB], qq[HW][IB];
#pragma unroll
                for (int u = 0; u < IB; u++) kk[u] = kp[i0 + u];
#pragma unroll
                for (int h = 0; h < HW; h++)
#pragma unroll
                    for (int u = 0; u < IB; u++) qq[h][u] = qp[h * L4 * 4 + i0 + u];
#pragma unroll
                for (int u = 0; u < IB; u++)
#pragma unroll
                    for (int h = 0; h < HW; h++) {
                        dd[h][0] = fmaf(qq[h][u][0], kk[u][0], dd[h][0]);
                        dd[h][1] = fmaf(qq[h][u][1], kk[u][1], dd[h][1]);
                        dd[h][2] = fmaf(qq[h][u][2], kk[u][2], dd[h][2]);
                        dd[h][3] = fmaf(qq[h][u][3], kk[u][3], dd[h][3]);
                    }
            }
#pragma unroll
            for (int h = 0; h < HW; h++)
                sc[h] = lane < np ? ((dd[h][0] + dd[h][1]) + (dd[h][2] + dd[h][3])) * a.scale : -INFINITY;
        }
        // the sub-chunk's maximum, exponentials and sum per head; the old sums' rescale for the
        // weighted sum
#pragma unroll
        for (int h = 0; h < HW; h++) {
            const int r = wave + 4 * h;
            if (r >= nh) break;
            const float m_new = fmaxf(m_run[h], wave_max(sc[h]));
            const float e = lane < np ? __expf(sc[h] - m_new) : 0.0f;
            const float cr = __expf(m_run[h] - m_new);  // 0 on the first sub-chunk (m_run = -inf)
            l_run[h] = fmaf(l_run[h], cr, wave_sum(e));
            m_run[h] = m_new;
            es[r * SUB + lane] = e;
            if (lane == 0) cs_l[r] = cr;
        }
        __syncthreads();

        // weighted V: thread (slot, dim d) for heads slot + HPS * k; V[j][d] read once for all of them
#pragma unroll
        for (int k = 0; k < NP; k++) acc[k] *= cs_l[rc[k]];
        int j = 0;
#pragma unroll 2
        for (; j + 4 <= np; j += 4) {
            float v4[4];
#pragma unroll
            for (int u = 0; u < 4; u++) v4[u] = vs[(j + u) * HD + d];
#pragma unroll
            for (int k = 0; k < NP; k++) {
                const sdy_f32x4 e4 = *reinterpret_cast<const sdy_f32x4 *>(es + rc[k] * SUB + j);
#pragma unroll
                for (int u = 0; u < 4; u++) acc[k] = fmaf(e4[u], v4[u], acc[k]);
            }
        }
        for (; j < np; j++) {
            const float vv = vs[j * HD + d];
#pragma unroll
            for (int k = 0; k < NP; k++) acc[k] = fmaf(es[rc[k] * SUB + j], vv, acc[k]);
        }
    }

    // the span's partials (published to the merge launch by the kernel boundary)
#pragma unroll
    for (int k = 0; k < NP; k++) {
        const int r = slot + HPS * k;
        if (r < nh) a.part[((size_t)(h0 + r) * a.n_span_max + sp) * (HD + 4) + 4 + d] = acc[k];
    }
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < HW; h++) {
            const int r = wave + 4 * h;
            if (r < nh) {
                float *pp = a.part + ((size_t)(h0 + r) * a.n_span_max + sp) * (HD + 4);
                pp[0] = m_run[h];
                pp[1] = l_run[h];
            }
        }
    }
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_merge(ChunkArgs a) {
    constexpr int HPS = 256 / HD;
    __shared__ __align__(16) float obuf[256];
    const int tid = threadIdx.x, slot = tid / HD, d = tid - slot * HD;
    const int h_raw = blockIdx.x * HPS + slot, h = h_raw < a.n_head ? h_raw : a.n_head - 1;
    const int n_span = a.step[1] / a.span + 1;
    const float *pb = a.part + (size_t)h * a.n_span_max * (HD + 4);
    // rounds of MERGE_ROUND spans whose loads are issued before use, folded with the running maximum.
    // The head is uniform over a wave (HD >= 64): lane u loads span s0 + u's m and l and computes its
    // weight, which the fold reads by lane; a thread loads only its own dimension of each span's o.
    const int lane = tid & 63;
    float M = -INFINITY, L = 0.0f, o = 0.0f;
    for (int s0 = 0; s0 < n_span; s0 += MERGE_ROUND) {
        const int lu = lane < MERGE_ROUND ? lane : 0;
        const bool lu_ok = lane < MERGE_ROUND && s0 + lu < n_span;
        const float *pl = pb + (size_t)(lu_ok ? s0 + lu : s0) * (HD + 4);
        const float m_l = pl[0], l_l = pl[1];
        float ov[MERGE_ROUND];
#pragma unroll
        for (int u = 0; u < MERGE_ROUND; u++) {
            const int s = s0 + u < n_span ? s0 + u : s0;
            ov[u] = pb[(size_t)s * (HD + 4) + 4 + d];
        }
        const float Mr = fmaxf(M, wave_max(lu_ok ? m_l : -INFINITY));
        const float sc = __expf(M - Mr);  // 0 on the first round (M = -inf)
        L *= sc;
        o *= sc;
        const float w_l = __expf(m_l - Mr);
#pragma unroll
        for (int u = 0; u < MERGE_ROUND; u++) {
            if (s0 + u < n_span) {
                const float w = lane_f(w_l, u);
                L = fmaf(lane_f(l_l, u), w, L);
                o = fmaf(ov[u], w, o);
            }
        }
        M = Mr;
    }
    const float r = o * (1.0f / L);
    if (h_raw < a.n_head) a.out[(size_t)h * HD + d] = r;
    if (a.xq) {  // (n_head * HD is a multiple of 256 here: the workgroup's outputs are one block)
        obuf[tid] = r;
        __syncthreads();
        if (tid < 64) {
            const sdy_f32x4 x4 = *reinterpret_cast<const sdy_f32x4 *>(obuf + 4 * tid);
            const float xs[4] = {x4[0], x4[1], x4[2], x4[3]};
            sdy_q8k_block(xs, tid, a.xq + (size_t)blockIdx.x * 292);
        }
    }
}

template <int HD, int HW, class KT>
int launch_chunked(const ChunkArgs &A, hipStream_t st) {
    static size_t granted = 0;
    const size_t lds = sizeof(float) * chunk_lds_floats<HD>();
    int rc = sdy_lds_limit((const void *)k_attn_chunk<HD, HW, KT>, lds, &granted);
    if (rc) return rc;
    SDY_NOTE_KERNEL((k_attn_chunk<HD, HW, KT>));
    const int pairs = A.n_span_max * A.n_kv_head;
    const int n_wg = A.hsplit == 2 ? (pairs + 7) / 8 * 16 : pairs;
    hipLaunchKernelGGL((k_attn_chunk<HD, HW, KT>), dim3(n_wg), dim3(256), lds, st, A);
    if ((rc = sdy_check_launch("attn_chunk"))) return rc;
    hipLaunchKernelGGL((k_attn_merge<HD>), dim3((A.n_head * HD + 255) / 256), dim3(256), 0, st, A);
    return sdy_check_launch("attn_merge");
}

template <int HD, int HW>
int launch_chunked_kv(const ChunkArgs &A, int kv_type, hipStream_t st) {
    return kv_type == SDY_KV_F16 ? launch_chunked<HD, HW, uint16_t>(A, st) : launch_chunked<HD, HW, float>(A, st);
}

template <int HD>
int launch_chunked_hw(const ChunkArgs &A, int kv_type, hipStream_t st) {
    const int nh = A.n_head / A.n_kv_head / A.hsplit;
    return nh <= 4 ? launch_chunked_kv<HD, 1>(A, kv_type, st)
           : nh <= 8 ? launch_chunked_kv<HD, 2>(A, kv_type, st)
                     : launch_chunked_kv<HD, 4>(A, kv_type, st);
}

// positions per span for a cache of max_seq positions: SUB, or a multiple of SUB that keeps the
// spans per kv head at MAX_SPANS or fewer
int span_for(int max_seq) {
    const int subs = (max_seq + SUB * MAX_SPANS - 1) / (SUB * MAX_SPANS);
    return SUB * (subs > 1 ? subs : 1);
}

}  // namespace

extern "C" int sdy_attn_chunked_ok(int n_head, int n_kv_head, int hd) {
    return (hd == 64 || hd == 128 || hd == 256) && n_kv_head >= 1 && n_head % n_kv_head == 0 &&
           n_head / n_kv_head <= MAX_REP;
}

extern "C" size_t sdy_attn_chunked_floats(int n_head, int hd, int max_seq) {
    const int span = span_for(max_seq);
    return (size_t)n_head * ((max_seq + span - 1) / span) * (hd + 4);
}

extern "C" int sdy_attn_decode_chunked(const float *q, const float *k, const float *v, const float *q_norm,
                                       const float *k_norm, float eps, const float *rope_cos, const float *rope_sin,
                                       const int32_t *step_dev, int n_head, int n_kv_head, int hd, int interleaved,
                                       void *k_cache, void *v_cache, int kv_type, long head_stride, int max_seq,
                                       float *part, float *out, void *xq_q8k, sdy_stream s) {
    if (!sdy_attn_chunked_ok(n_head, n_kv_head, hd))
        return sdy_fail(-1, "attn_decode_chunked: head_dim %d with %d heads / %d kv heads not supported", hd, n_head,
                        n_kv_head);
    if (!sdy_kv_elt_bytes(kv_type)) return sdy_fail(-1, "attn_decode_chunked: KV element type %d", kv_type);
    if (max_seq < 1) return sdy_fail(-1, "attn_decode_chunked: max_seq %d", max_seq);
    if (xq_q8k && (n_head * hd) % 256)
        return sdy_fail(-1, "attn_decode_chunked: %d outputs are not whole Q8_K blocks", n_head * hd);
    ChunkArgs A = {};
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
    A.span = span_for(max_seq);
    // two workgroups per (span, kv group), each with half the group's heads, when the group has four
    // or more: twice the workgroups (the K/V rows are read by both), half the serial work in each
    const int n_rep = n_head / n_kv_head;
    A.hsplit = n_rep >= 4 && n_rep % 2 == 0 ? 2 : 1;
    A.n_span_max = (max_seq + A.span - 1) / A.span;
    A.k_cache = k_cache;
    A.v_cache = v_cache;
    A.head_stride = head_stride;
    A.scale = 1.0f / sqrtf((float)hd);
    A.part = part;
    A.out = out;
    A.xq = (uint8_t *)xq_q8k;
    switch (hd) {
    case 64: return launch_chunked_hw<64>(A, kv_type, (hipStream_t)s);
    case 128: return launch_chunked_hw<128>(A, kv_type, (hipStream_t)s);
    default: return launch_chunked_hw<256>(A, kv_type, (hipStream_t)s);
    }
}

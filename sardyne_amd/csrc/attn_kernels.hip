// gfx950 attention kernels (the reference's op_attention / attention_worker, csrc/ops.c:405-423 and
// csrc/model_llama.c:619-640), over the f32 KV cache [n_kv_head][max_seq][head_dim] of a layer.
//
// Positions are cut into chunks of CH = 64. A workgroup stages a chunk's K and V in LDS with 16-byte
// loads and, for each of its tokens, computes the scores of the n_rep query heads that share the KV
// head and writes per head the chunk maximum m, the sum l of exp(score - m) and the exp-weighted
// sum o of V. A merge then combines the chunks of each (token, head) in chunk order:
// M = max m_c, e_c = exp(m_c - M), L = sum l_c e_c, out = (sum o_c e_c) / L. Every path (prefill,
// the fused decode step, the host-pointer op_attention) uses these same functions, so they agree
// bit for bit; the result differs from the reference's single softmax only by f32 rounding.
//
//   k_attn_partial + k_attn_combine   n tokens at positions n_kv0 - 1 + t (causal), two launches
//   k_attn_decode                     one token at the position held in device memory: q/k norm,
//                                     RoPE and the KV-cache write of that position, the chunks, and
//                                     the merge (plus the quantisation for the next matvec) in the
//                                     last workgroup to arrive
//
// Partial records: o [n_tok][n_head][n_chunk][hd] then (m, l) [n_tok][n_head][n_chunk][2].
#include "sdy_device.h"
#include "sdy_internal.h"
#include "sdy_ops.h"
#include "sdy_quant_dev.h"
#include "sdy_attn_dev.h"
#include "sdy_shim.h"

namespace {

constexpr int CH = 64;

struct ChunkLds {
    float *ks, *vs, *qs, *ps;  // K [CH][hd+1] (odd stride: conflict-free score reads), V [CH][hd],
                               // q [n_rep][hd], scores / weights [n_rep][CH]
};

SDY_DEV ChunkLds chunk_lds(float *sm, int hd, int n_rep) {
    ChunkLds L;
    L.ks = sm;
    L.vs = L.ks + CH * (hd + 1);
    L.qs = L.vs + CH * hd;
    L.ps = L.qs + n_rep * hd;
    return L;
}

__host__ __device__ inline size_t chunk_lds_floats(int hd, int n_rep) {
    return (size_t)CH * (hd + 1) + (size_t)CH * hd + (size_t)n_rep * hd + (size_t)n_rep * CH;
}

// K/V of positions [p0, p0 + np) into LDS, 16 bytes per load (hd % 4 == 0). Position `special`
// (if in range) takes its K from kspec and its V from vspec instead of the cache.
template <int NT>
SDY_DEV void stage_kv(const ChunkLds &L, const float *kg, const float *vg, int np, int hd, int special,
                      const float *kspec, const float *vspec) {
    const int n4 = np * hd / 4, tid = threadIdx.x;
    // batches of B loads per thread (a chunk of 64 x 128 floats is 2048 float4 of K and of V) go out
    // before their LDS stores (clamped indices, no conditional load), so that their latencies overlap
    constexpr int B = NT >= 1024 ? 2 : 4;
    for (int i0 = tid; i0 < n4; i0 += B * NT) {
        float4 kv[B], vv[B];
#pragma unroll
        for (int j = 0; j < B; j++) {
            const int i = i0 + j * NT < n4 ? i0 + j * NT : i0;
            kv[j] = reinterpret_cast<const float4 *>(kg)[i];
            vv[j] = reinterpret_cast<const float4 *>(vg)[i];
        }
#pragma unroll
        for (int j = 0; j < B; j++) {
            const int i = i0 + j * NT;
            if (i >= n4) break;
            const int p = (4 * i) / hd, d = 4 * i - p * hd;
            if (p == special) continue;
            float *kr = L.ks + p * (hd + 1) + d;
            kr[0] = kv[j].x;
            kr[1] = kv[j].y;
            kr[2] = kv[j].z;
            kr[3] = kv[j].w;
            *reinterpret_cast<float4 *>(L.vs + 4 * i) = vv[j];
        }
    }
    if (special >= 0 && special < np)
        for (int d = tid; d < hd; d += NT) {
            L.ks[special * (hd + 1) + d] = kspec[d];
            L.vs[special * hd + d] = vspec[d];
        }
}

// Scores, chunk max / exp-sum and exp-weighted V of n_rep heads over np staged positions (LDS
// staged and synchronised by the caller). Head r's records: o at o_base + (rec0 + r * rstride) * hd,
// (m, l) at ml_base + (rec0 + r * rstride) * 2.
template <int NT>
SDY_DEV void chunk_attend(const ChunkLds &L, int n_rep, int hd, int np, float scale, float *o_base, float *ml_base,
                          size_t rec0, int rstride) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, kstride = hd + 1;
    for (int i = tid; i < n_rep * CH; i += NT) {
        const int r = i / CH, p = i - r * CH;
        float sc = -INFINITY;
        if (p < np) {
            const float *qq = L.qs + r * hd, *kk = L.ks + p * kstride;
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
            for (int d = 0; d < hd; d += 4) {
                a0 = fmaf(qq[d], kk[d], a0);
                a1 = fmaf(qq[d + 1], kk[d + 1], a1);
                a2 = fmaf(qq[d + 2], kk[d + 2], a2);
                a3 = fmaf(qq[d + 3], kk[d + 3], a3);
            }
            sc = ((a0 + a1) + (a2 + a3)) * scale;
        }
        L.ps[i] = sc;
    }
    __syncthreads();
    for (int r = wave; r < n_rep; r += NT / 64) {  // CH == 64: one position per lane
        float m = L.ps[r * CH + lane];
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        const float e = lane < np ? expf(L.ps[r * CH + lane] - m) : 0.0f;
        L.ps[r * CH + lane] = e;
        float l = e;
        for (int off = 32; off >= 1; off >>= 1) l += __shfl_xor(l, off);
        if (lane == 0) {
            float *ml = ml_base + (rec0 + (size_t)r * rstride) * 2;
            ml[0] = m;
            ml[1] = l;
        }
    }
    __syncthreads();
    for (int i = tid; i < n_rep * hd / 4; i += NT) {
        const int r = (4 * i) / hd, d = 4 * i - r * hd;
        const float *pr = L.ps + r * CH;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int p = 0; p < np; p++) {
            const float w = pr[p];
            const float4 v = *reinterpret_cast<const float4 *>(L.vs + p * hd + d);
            acc.x = fmaf(w, v.x, acc.x);
            acc.y = fmaf(w, v.y, acc.y);
            acc.z = fmaf(w, v.z, acc.z);
            acc.w = fmaf(w, v.w, acc.w);
        }
        *reinterpret_cast<float4 *>(o_base + (rec0 + (size_t)r * rstride) * hd + d) = acc;
    }
}

// ------------------------------------------------------------------ prefill: n tokens, two launches

// Grid (n_chunk, n_kv_head, ceil(n_tok / TB)): tokens tb*TB .. tb*TB + TB - 1, token t attending to
// positions 0..n_kv0-1+t. The chunk's K and V are staged once for the workgroup's tokens (for the
// last of them that reaches the chunk); each token then stages its queries and runs chunk_attend
// over its own np positions, so every record has the bits of a workgroup for that token alone.
constexpr int TB = 16;
__global__ __launch_bounds__(256) void k_attn_partial(const float *__restrict__ q, const float *__restrict__ k_cache,
                                                      const float *__restrict__ v_cache, int n_head, int n_kv_head,
                                                      int hd, int n_kv0, long head_stride, long q_stride,
                                                      float *__restrict__ part, int n_tok, int n_chunk_max,
                                                      float scale) {
    extern __shared__ float sm[];
    const int c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    const int t0 = blockIdx.z * TB, t1 = t0 + TB < n_tok ? t0 + TB : n_tok;
    const int p0 = c * CH;
    const int n_kv_last = n_kv0 + t1 - 1;
    if (p0 >= n_kv_last) return;  // no token of the block reaches this chunk
    const int np_max = n_kv_last - p0 < CH ? n_kv_last - p0 : CH;
    const int n_rep = n_head / n_kv_head;
    const ChunkLds L = chunk_lds(sm, hd, n_rep);
    stage_kv<256>(L, k_cache + g * head_stride + (size_t)p0 * hd, v_cache + g * head_stride + (size_t)p0 * hd, np_max,
                  hd, -1, nullptr, nullptr);
    for (int t = t0 < (p0 + 1 - n_kv0) ? (p0 + 1 - n_kv0) : t0; t < t1; t++) {  // tokens that reach the chunk
        const int n_kv = n_kv0 + t;
        const int np = n_kv - p0 < CH ? n_kv - p0 : CH;
        for (int i = tid; i < n_rep * hd; i += 256) L.qs[i] = q[(size_t)t * q_stride + (size_t)g * n_rep * hd + i];
        __syncthreads();
        chunk_attend<256>(L, n_rep, hd, np, scale, part, part + (size_t)n_tok * n_head * n_chunk_max * hd,
                          ((size_t)t * n_head + g * n_rep) * n_chunk_max + c, n_chunk_max);
    }
}

// Register-blocked prefill chunk: a workgroup takes R = 64 query rows (TBR = 64 / n_rep tokens x
// the n_rep heads of KV head g) against the CH = 64 positions of chunk c. K is staged transposed
// ([HD][64]), V as [64][HD], the scores / weights as [64][64]; the queries are read from global
// memory (L1). Thread
// (row group rg, column group cg) computes the scores of rows 4rg..4rg+3 x positions 4cg..4cg+3 and
// then the weighted V of rows 4rg..4rg+3 x dims (HD/16)cg.. . Every sum has chunk_attend's order
// (scores: four partial sums by d mod 4, then (a0 + a1) + (a2 + a3); weighted V: one chain over
// the positions; weights past a row's own positions are exact zeros and leave the chain unchanged),
// so the records are bit-identical to those of k_attn_partial. 80 KB of LDS: two workgroups, two
// waves per SIMD, per CU (the register budget is set for that occupancy, so that the next operands
// can be read while the current ones are multiplied). Token blocks are launched last first.
template <int HD>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_attn_prefill(const float *__restrict__ q, const float *__restrict__ k_cache,
                                                      const float *__restrict__ v_cache, int n_head, int n_kv_head,
                                                      int n_kv0, long head_stride, long q_stride,
                                                      float *__restrict__ part, int n_tok, int n_chunk_max,
                                                      float scale) {
    constexpr int R = 64, DG = HD / 16;  // rows per workgroup, dims per thread in the weighted sum
    extern __shared__ __align__(16) float sm[];
    float *kT = sm;                // [HD][64]
    float *vs = kT + HD * CH;      // [64][HD]
    float *ps = vs + CH * HD;      // [R][64]
    const int c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n_rep = n_head / n_kv_head, tbr = R / n_rep;
    // the last token blocks reach the most chunks: they are launched first
    const int blk = (int)gridDim.z - 1 - (int)blockIdx.z;
    const int t0 = blk * tbr, t1 = t0 + tbr < n_tok ? t0 + tbr : n_tok;
    const int p0 = c * CH;
    const int n_kv_last = n_kv0 + t1 - 1;
    if (p0 >= n_kv_last) return;
    const int np_max = n_kv_last - p0 < CH ? n_kv_last - p0 : CH;
    // stage K transposed and V (positions past np_max as zeros), and the queries (rows past the
    // last token repeat it)
    // (each batch of 8 loads goes out before its LDS stores: unconditional, clamped addresses, so
    // that their latencies overlap)
    const float *kg = k_cache + g * head_stride + (size_t)p0 * HD, *vg = v_cache + g * head_stride + (size_t)p0 * HD;
    constexpr int NV = CH * HD / 4 / 256;  // float4 of K (and of V) per thread
    constexpr int NBT = NV < 8 ? NV : 8;   // per batch
    static_assert(NV % NBT == 0, "batches");
    for (int b0 = 0; b0 < NV; b0 += NBT) {
        float4 kv[NBT], vv[NBT];
#pragma unroll
        for (int j = 0; j < NBT; j++) {
            const int i = tid + 256 * (b0 + j);
            const int pp = i % CH, d4 = i / CH;  // position fastest: conflict-free transposed writes
            kv[j] = *reinterpret_cast<const float4 *>(kg + (size_t)(pp < np_max ? pp : 0) * HD + 4 * d4);
            const int pv = (4 * i) / HD;
            vv[j] = reinterpret_cast<const float4 *>(vg)[pv < np_max ? i : 0];
        }
#pragma unroll
        for (int j = 0; j < NBT; j++) {
            const int i = tid + 256 * (b0 + j);
            const int pp = i % CH, d4 = i / CH, pv = (4 * i) / HD;
            const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 k4 = pp < np_max ? kv[j] : z;
            kT[(4 * d4 + 0) * CH + pp] = k4.x;
            kT[(4 * d4 + 1) * CH + pp] = k4.y;
            kT[(4 * d4 + 2) * CH + pp] = k4.z;
            kT[(4 * d4 + 3) * CH + pp] = k4.w;
            reinterpret_cast<float4 *>(vs)[i] = pv < np_max ? vv[j] : z;
        }
    }
    __syncthreads();
    const int rg = tid >> 4, cg = tid & 15;
    // the thread's 4 query rows, read from global memory (the 16 threads of a row group share them)
    const float *qrow[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 4 * rg + i, tl = r / n_rep, jj = r - tl * n_rep;
        const int t = t0 + tl < t1 ? t0 + tl : t1 - 1;
        qrow[i] = q + (size_t)t * q_stride + (size_t)(g * n_rep + jj) * HD;
    }
    {
        float a[4][4][4];  // [row][position][d mod 4]
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int k = 0; k < 4; k++)
#pragma unroll
                for (int m = 0; m < 4; m++) a[i][k][m] = 0.0f;
        // the next 4 dims' operands are read while the current ones are multiplied
        float4 qn[4], kn[4];
#pragma unroll
        for (int i = 0; i < 4; i++) qn[i] = *reinterpret_cast<const float4 *>(qrow[i]);
#pragma unroll
        for (int m = 0; m < 4; m++) kn[m] = *reinterpret_cast<const float4 *>(kT + m * CH + 4 * cg);
        for (int d = 0; d < HD; d += 4) {
            float4 qv[4], kv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) qv[i] = qn[i];
#pragma unroll
            for (int m = 0; m < 4; m++) kv[m] = kn[m];
            const int dn = d + 4 < HD ? d + 4 : d;
#pragma unroll
            for (int i = 0; i < 4; i++) qn[i] = *reinterpret_cast<const float4 *>(qrow[i] + dn);
#pragma unroll
            for (int m = 0; m < 4; m++) kn[m] = *reinterpret_cast<const float4 *>(kT + (dn + m) * CH + 4 * cg);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float qd[4] = {qv[i].x, qv[i].y, qv[i].z, qv[i].w};
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    const float kk[4] = {kv[m].x, kv[m].y, kv[m].z, kv[m].w};
#pragma unroll
                    for (int k = 0; k < 4; k++) a[i][k][m] = fmaf(qd[m], kk[k], a[i][k][m]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float4 sc;
            sc.x = ((a[i][0][0] + a[i][0][1]) + (a[i][0][2] + a[i][0][3])) * scale;
            sc.y = ((a[i][1][0] + a[i][1][1]) + (a[i][1][2] + a[i][1][3])) * scale;
            sc.z = ((a[i][2][0] + a[i][2][1]) + (a[i][2][2] + a[i][2][3])) * scale;
            sc.w = ((a[i][3][0] + a[i][3][1]) + (a[i][3][2] + a[i][3][3])) * scale;
            *reinterpret_cast<float4 *>(ps + (4 * rg + i) * CH + 4 * cg) = sc;
        }
    }
    __syncthreads();
    // softmax pieces per row (one wave per row, lane = position), as in chunk_attend
    float *ml_base = part + (size_t)n_tok * n_head * n_chunk_max * HD;
    for (int r = wave; r < R; r += 4) {
        const int tl = r / n_rep, j = r - tl * n_rep, t = t0 + tl;
        const int np = t < t1 ? (n_kv0 + t - p0 < CH ? n_kv0 + t - p0 : CH) : 0;
        float e = 0.0f;
        if (np > 0) {
            const float sv = lane < np ? ps[r * CH + lane] : -INFINITY;
            float m = sv;
            for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
            e = lane < np ? expf(sv - m) : 0.0f;
            float l = e;
            for (int off = 32; off >= 1; off >>= 1) l += __shfl_xor(l, off);
            if (lane == 0) {
                float *ml = ml_base + (((size_t)t * n_head + g * n_rep + j) * n_chunk_max + c) * 2;
                ml[0] = m;
                ml[1] = l;
            }
        }
        ps[r * CH + lane] = e;
    }
    __syncthreads();
    // weighted V: rows 4rg..4rg+3, dims DG*cg .. DG*cg + DG - 1, one chain over the positions
    {
        float o[4][DG];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int k = 0; k < DG; k++) o[i][k] = 0.0f;
        // (the next position's weights and V are read while the current ones are multiplied)
        float wn[4];
        float4 vn[DG / 4];
#pragma unroll
        for (int i = 0; i < 4; i++) wn[i] = ps[(4 * rg + i) * CH];
#pragma unroll
        for (int k = 0; k < DG / 4; k++) vn[k] = *reinterpret_cast<const float4 *>(vs + DG * cg + 4 * k);
        for (int pp = 0; pp < np_max; pp++) {
            float w[4];
            float vv[DG];
#pragma unroll
            for (int i = 0; i < 4; i++) w[i] = wn[i];
#pragma unroll
            for (int k = 0; k < DG / 4; k++) {
                vv[4 * k] = vn[k].x;
                vv[4 * k + 1] = vn[k].y;
                vv[4 * k + 2] = vn[k].z;
                vv[4 * k + 3] = vn[k].w;
            }
            const int pn = pp + 1 < CH ? pp + 1 : pp;
#pragma unroll
            for (int i = 0; i < 4; i++) wn[i] = ps[(4 * rg + i) * CH + pn];
#pragma unroll
            for (int k = 0; k < DG / 4; k++) vn[k] = *reinterpret_cast<const float4 *>(vs + pn * HD + DG * cg + 4 * k);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int k = 0; k < DG; k++) o[i][k] = fmaf(w[i], vv[k], o[i][k]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 4 * rg + i, tl = r / n_rep, j = r - tl * n_rep, t = t0 + tl;
            if (t >= t1 || n_kv0 + t - p0 <= 0) continue;
            float *ob = part + (((size_t)t * n_head + g * n_rep + j) * n_chunk_max + c) * HD + DG * cg;
#pragma unroll
            for (int k = 0; k < DG; k += 4) *reinterpret_cast<float4 *>(ob + k) = make_float4(o[i][k], o[i][k + 1], o[i][k + 2], o[i][k + 3]);
        }
    }
}

// Grid (n_head, n_tok), 128 threads.
__global__ __launch_bounds__(128) void k_attn_combine(const float *__restrict__ part, int n_head, int hd, int n_kv0,
                                                      int n_tok, int n_chunk_max, float *__restrict__ out,
                                                      long out_stride) {
    extern __shared__ float e[];  // [n_chunk_max] weights, then [n_chunk_max] scratch
    __shared__ float sL;
    const int h = blockIdx.x, t = blockIdx.y;
    const int n_kv = n_kv0 + t, nc = (n_kv + CH - 1) / CH;
    const size_t rec0 = ((size_t)t * n_head + h) * n_chunk_max;
    const float *o = part + rec0 * hd;
    const float *ml = part + (size_t)n_tok * n_head * n_chunk_max * hd + rec0 * 2;
    if (threadIdx.x < 64) {
        const float L = merge_weights_wave(ml, nc, e, e + n_chunk_max, threadIdx.x);
        if (threadIdx.x == 0) sL = L;
    }
    __syncthreads();
    for (int d = 4 * threadIdx.x; d < hd; d += 4 * blockDim.x)
        *reinterpret_cast<float4 *>(out + (size_t)t * out_stride + (size_t)h * hd + d) =
            merge4(o, n_chunk_max, nc, hd, d, e, sL);
}

// ------------------------------------------------------------------ one-token decode, one launch

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

// q/k norm + RoPE of the vectors of n_tok tokens and the KV-cache write at positions pos0 + t.
// Grid (n_tok, n_head + n_kv_head), 64 threads.
__global__ __launch_bounds__(64) void k_qk_rope_kv(float *q, float *k, const float *v, const float *qn, const float *kn,
                                                   float eps, const float *rope_cos, const float *rope_sin, int pos0,
                                                   int n_head, int n_kv_head, int hd, int interleaved, float *k_cache,
                                                   float *v_cache, long head_stride) {
    __shared__ float buf[512];
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const bool is_q = h < n_head;
    const int hh = is_q ? h : h - n_head;
    float *vec = is_q ? q + ((size_t)t * n_head + hh) * hd : k + ((size_t)t * n_kv_head + hh) * hd;
    for (int i = lane; i < hd; i += 64) buf[i] = vec[i];
    sdy_wave_sync();
    const int pos = pos0 + t;
    norm_rope_wave(buf, is_q ? qn : kn, eps, rope_cos + (size_t)pos * (hd / 2), rope_sin + (size_t)pos * (hd / 2), hd,
                   interleaved, lane);
    for (int i = lane; i < hd; i += 64) vec[i] = buf[i];
    if (!is_q && k_cache) {
        float *kc = k_cache + hh * head_stride + (size_t)pos * hd;
        float *vc = v_cache + hh * head_stride + (size_t)pos * hd;
        const float *vv = v + ((size_t)t * n_kv_head + hh) * hd;
        for (int i = lane; i < hd; i += 64) {
            kc[i] = buf[i];
            vc[i] = vv[i];
        }
    }
}

struct AttnDecodeArgs {
    const float *q, *k, *v;          // this token's projections: [n_head][hd], [n_kv_head][hd] x 2
    const float *q_norm, *k_norm;    // per-head norm weights or null
    float eps;
    const float *rope_cos, *rope_sin;
    const int32_t *step;             // step[1] = position of the token
    int n_head, n_kv_head, hd, interleaved;
    float *k_cache, *v_cache;        // this layer: [n_kv_head][max_seq][hd]
    long head_stride;                // max_seq * hd
    float *part;                     // partial records of one token
    int n_chunk_max;
    float scale;
};

// Grid (n_chunk_max, n_kv_head), DEC_NT threads (8 waves); chunks past the position exit at once.
// Writes the partial records of every chunk; the merge is a separate launch (k_attn_merge1*).
// The chunk's K and V loads go out first; meanwhile each wave normalises and rotates its query
// heads (and one wave the new position's k, which it also writes to the cache). After one barrier
// wave w takes heads w, w + 8, ...: lane p computes the score of position p with chunk_attend's
// four partial sums (d mod 4), the wave forms m, l and the weights as chunk_attend does, and lane l
// accumulates dims l, l + 64, ... of the weighted V over the positions in order (the weight of
// position p read from lane p). The records are therefore those of chunk_attend, bit for bit.
constexpr int DEC_NT = 512, DEC_W = DEC_NT / 64;

template <int HD>
__global__ __launch_bounds__(DEC_NT) void k_attn_decode(AttnDecodeArgs a) {
    constexpr int KS = HD + 1;            // K row stride (odd: conflict-free reads by position)
    constexpr int NV = CH * HD / 4 / DEC_NT;  // float4 of K (and of V) per thread
    static_assert(NV >= 1 && NV * DEC_NT * 4 == CH * HD, "chunk");
    extern __shared__ float sm[];
    float *ks = sm;                       // [CH][HD + 1]
    float *vs = ks + CH * KS;             // [CH][HD]
    float *kp = vs + CH * HD;             // [HD]: normalised, rotated k of the new position
    float *qs = kp + HD;                  // [n_rep][HD]
    const int c = blockIdx.x, g = blockIdx.y, wave = threadIdx.x >> 6, lane = threadIdx.x & 63, tid = threadIdx.x;
    const int pos = a.step[1], n_kv = pos + 1;
    const int nch = (n_kv + CH - 1) / CH;
    if (c >= nch) return;
    const int n_rep = a.n_head / a.n_kv_head;
    const int p0 = c * CH, np = n_kv - p0 < CH ? n_kv - p0 : CH;
    const bool has_pos = c == nch - 1;  // this chunk holds the new position
    // 0. the chunk's K and V from the cache (clamped indices: every load is unconditional)
    const float *kg = a.k_cache + g * a.head_stride + (size_t)p0 * HD, *vg = a.v_cache + g * a.head_stride + (size_t)p0 * HD;
    const int n4 = np * HD / 4;
    float4 kv[NV], vv[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = tid + j * DEC_NT < n4 ? tid + j * DEC_NT : 0;
        kv[j] = reinterpret_cast<const float4 *>(kg)[i];
        vv[j] = reinterpret_cast<const float4 *>(vg)[i];
    }
    // 1. q heads of this group (and k of the new position): norm + RoPE in LDS
    const float *cs = a.rope_cos + (size_t)pos * (HD / 2), *sn = a.rope_sin + (size_t)pos * (HD / 2);
    const int tasks = n_rep + (has_pos ? 1 : 0);
    for (int r = wave; r < tasks; r += DEC_W) {
        const bool is_k = r == n_rep;
        float *buf = is_k ? kp : qs + r * HD;
        const float *src = is_k ? a.k + (size_t)g * HD : a.q + (size_t)(g * n_rep + r) * HD;
        for (int i = lane; i < HD; i += 64) buf[i] = src[i];
        sdy_wave_sync();
        norm_rope_wave(buf, is_k ? a.k_norm : a.q_norm, a.eps, cs, sn, HD, a.interleaved, lane);
        if (is_k) {  // KV-cache write of the new position
            float *kc = a.k_cache + g * a.head_stride + (size_t)pos * HD;
            float *vc = a.v_cache + g * a.head_stride + (size_t)pos * HD;
            const float *vn = a.v + (size_t)g * HD;
            for (int i = lane; i < HD; i += 64) {
                kc[i] = buf[i];
                vc[i] = vn[i];
            }
        }
    }
    // 2. the chunk into LDS (the new position from LDS / the raw v: its cache entry is written above)
    const int special = has_pos ? pos - p0 : -1;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = tid + j * DEC_NT;
        if (i >= n4) break;
        const int p = (4 * i) / HD, d = 4 * i - p * HD;
        if (p == special) continue;
        float *kr = ks + p * KS + d;
        kr[0] = kv[j].x;
        kr[1] = kv[j].y;
        kr[2] = kv[j].z;
        kr[3] = kv[j].w;
        *reinterpret_cast<float4 *>(vs + 4 * i) = vv[j];
    }
    __syncthreads();  // (also orders the k of the new position in kp before its use below)
    if (special >= 0)
        for (int d = tid; d < HD; d += DEC_NT) {
            ks[special * KS + d] = kp[d];
            vs[special * HD + d] = a.v[(size_t)g * HD + d];
        }
    __syncthreads();
    // 3. per head: scores (lane = position), weights, weighted V (lane = dims)
    float *o_base = a.part, *ml_base = a.part + (size_t)a.n_head * a.n_chunk_max * HD;
    for (int r = wave; r < n_rep; r += DEC_W) {
        const float *qq = qs + r * HD;
        float sc = -INFINITY;
        if (lane < np) {
            const float *kk = ks + lane * KS;
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll 8
            for (int d = 0; d < HD; d += 4) {
                const float4 q4 = *reinterpret_cast<const float4 *>(qq + d);
                a0 = fmaf(q4.x, kk[d], a0);
                a1 = fmaf(q4.y, kk[d + 1], a1);
                a2 = fmaf(q4.z, kk[d + 2], a2);
                a3 = fmaf(q4.w, kk[d + 3], a3);
            }
            sc = ((a0 + a1) + (a2 + a3)) * a.scale;
        }
        float m = sc;
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        const float e = lane < np ? expf(sc - m) : 0.0f;
        float l = e;
        for (int off = 32; off >= 1; off >>= 1) l += __shfl_xor(l, off);
        const size_t rec = (size_t)(g * n_rep + r) * a.n_chunk_max + c;
        if (lane == 0) {
            ml_base[rec * 2] = m;
            ml_base[rec * 2 + 1] = l;
        }
        float acc[HD / 64];
#pragma unroll
        for (int k = 0; k < HD / 64; k++) acc[k] = 0.0f;
        for (int p = 0; p < np; p++) {
            const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), p));
#pragma unroll
            for (int k = 0; k < HD / 64; k++) acc[k] = fmaf(w, vs[p * HD + lane + 64 * k], acc[k]);
        }
#pragma unroll
        for (int k = 0; k < HD / 64; k++) o_base[rec * HD + lane + 64 * k] = acc[k];
    }
}

// Merge of one token's partial records (position in step[1]) into out [n_head * hd], for output
// projections without an activation prologue. Grid n_head, one wave each.
__global__ __launch_bounds__(64) void k_attn_merge1(const float *__restrict__ part, const int32_t *__restrict__ step,
                                                    int n_head, int hd, int n_chunk_max, float *__restrict__ out) {
    extern __shared__ float e[];  // [n_chunk_max] weights, [n_chunk_max] scratch
    const int h = blockIdx.x, lane = threadIdx.x;
    const int nch = (step[1] + 1 + CH - 1) / CH;
    const float *ml = part + (size_t)n_head * n_chunk_max * hd + (size_t)h * n_chunk_max * 2;
    const float L = merge_weights_wave(ml, nch, e, e + n_chunk_max, lane);
    for (int d = 4 * lane; d < hd; d += 256)
        *reinterpret_cast<float4 *>(out + (size_t)h * hd + d) =
            merge4(part + (size_t)h * n_chunk_max * hd, n_chunk_max, nch, hd, d, e, L);
}

// Merge of one token's records into the Q8_K row of the output projection: one wave per 256-element
// super-block (lane l: elements 4l..4l+3), the merge weights of the super-block's heads in LDS, the
// merged values also written to out (f32).
__global__ __launch_bounds__(64) void k_attn_merge1_q8k(const float *__restrict__ part,
                                                        const int32_t *__restrict__ step, int n_head, int hd,
                                                        int n_chunk_max, float *__restrict__ out,
                                                        uint8_t *__restrict__ xq) {
    extern __shared__ float sm[];  // per head of the super-block: [n_chunk_max] weights, [n_chunk_max] scratch
    __shared__ float sL[64];
    const int sb = blockIdx.x, lane = threadIdx.x;
    const int nch = (step[1] + 1 + CH - 1) / CH;
    const int h0 = 256 * sb / hd, h1 = (256 * sb + 255) / hd;
    const float *ml = part + (size_t)n_head * n_chunk_max * hd;
    for (int h = h0; h <= h1; h++) {
        const float L = merge_weights_wave(ml + (size_t)h * n_chunk_max * 2, nch, sm + (h - h0) * 2 * n_chunk_max,
                                           sm + (h - h0) * 2 * n_chunk_max + n_chunk_max, lane);
        if (lane == 0) sL[h - h0] = L;
    }
    sdy_wave_sync();
    const int e0 = 256 * sb + 4 * lane, h = e0 / hd, d = e0 - h * hd;
    const float4 v =
        merge4(part + (size_t)h * n_chunk_max * hd, n_chunk_max, nch, hd, d, sm + (h - h0) * 2 * n_chunk_max, sL[h - h0]);
    *reinterpret_cast<float4 *>(out + e0) = v;
    const float xs[4] = {v.x, v.y, v.z, v.w};
    sdy_q8k_block(xs, lane, xq + (size_t)sb * 292);
}

}  // namespace

// =============================================================================== launchers

extern "C" size_t sdy_attn_part_floats(int n_tok, int n_head, int hd, int max_kv) {
    int nc = (max_kv + CH - 1) / CH;
    return (size_t)n_tok * n_head * nc * (hd + 2);
}

static int shape_ok(int n_head, int n_kv_head, int hd) {
    if (hd > 512 || hd % 4 || n_kv_head < 1 || n_head % n_kv_head)
        return sdy_fail(-1, "attention: head_dim %d / %d heads / %d kv heads not supported", hd, n_head, n_kv_head);
    return 0;
}

extern "C" int sdy_qk_rope_kv(float *q, float *k, const float *v, const float *qn, const float *kn, float eps,
                              const float *rope_cos, const float *rope_sin, int pos0, int n_tok, int n_head,
                              int n_kv_head, int hd, int interleaved, float *k_cache, float *v_cache,
                              long head_stride, sdy_stream s) {
    if (hd > 512) return sdy_fail(-1, "head_dim %d above 512", hd);
    hipLaunchKernelGGL(k_qk_rope_kv, dim3(n_tok, n_head + n_kv_head), dim3(64), 0, (hipStream_t)s, q, k, v, qn, kn, eps,
                       rope_cos, rope_sin, pos0, n_head, n_kv_head, hd, interleaved, k_cache, v_cache, head_stride);
    return sdy_check_launch("qk_rope_kv");
}

extern "C" int sdy_attention(const float *q, const float *k_cache, const float *v_cache, int n_tok, int n_head,
                             int n_kv_head, int hd, int n_kv0, long head_stride, long q_stride, float *part,
                             float *out, long out_stride, sdy_stream s) {
    hipStream_t st = (hipStream_t)s;
    if (n_tok <= 0) return 0;
    int rc = shape_ok(n_head, n_kv_head, hd);
    if (rc) return rc;
    const int n_rep = n_head / n_kv_head;
    const int n_kv_max = n_kv0 + n_tok - 1;
    const int nc = (n_kv_max + CH - 1) / CH;
    const size_t lds = sizeof(float) * chunk_lds_floats(hd, n_rep);
    if (lds > 160 * 1024) return sdy_fail(-1, "attention: %zu bytes of LDS (head_dim %d, %d heads per KV head)", lds, hd, n_rep);
    static size_t granted = 0;
    if ((rc = sdy_lds_limit((const void *)k_attn_partial, lds, &granted))) return rc;
    float scale = 1.0f / sqrtf((float)hd);
    if (n_tok >= 16 && 64 % n_rep == 0 && (hd == 64 || hd == 128)) {
        // many tokens: the register-blocked chunk kernel (the same records, bit for bit)
        const int tbr = 64 / n_rep;
        const size_t lds2 = sizeof(float) * ((size_t)hd * CH * 2 + 64 * CH);
        static size_t granted2[2] = {0, 0};
        const void *fn = hd == 128 ? (const void *)k_attn_prefill<128> : (const void *)k_attn_prefill<64>;
        if ((rc = sdy_lds_limit(fn, lds2, &granted2[hd == 128]))) return rc;
        const dim3 grid(nc, n_kv_head, (n_tok + tbr - 1) / tbr);
        if (hd == 128)
            hipLaunchKernelGGL(k_attn_prefill<128>, grid, dim3(256), lds2, st, q, k_cache, v_cache, n_head, n_kv_head,
                               n_kv0, head_stride, q_stride, part, n_tok, nc, scale);
        else
            hipLaunchKernelGGL(k_attn_prefill<64>, grid, dim3(256), lds2, st, q, k_cache, v_cache, n_head, n_kv_head,
                               n_kv0, head_stride, q_stride, part, n_tok, nc, scale);
    } else {
        hipLaunchKernelGGL(k_attn_partial, dim3(nc, n_kv_head, (n_tok + TB - 1) / TB), dim3(256), lds, st, q, k_cache,
                           v_cache, n_head, n_kv_head, hd, n_kv0, head_stride, q_stride, part, n_tok, nc, scale);
    }
    if ((rc = sdy_check_launch("attention"))) return rc;
    hipLaunchKernelGGL(k_attn_combine, dim3(n_head, n_tok), dim3(128), 2 * nc * sizeof(float), st, part, n_head, hd,
                       n_kv0, n_tok, nc, out, out_stride);
    return sdy_check_launch("attention_combine");
}

static size_t attn_decode_lds(int n_head, int n_kv_head, int hd) {
    return sizeof(float) * ((size_t)CH * (hd + 1) + (size_t)CH * hd + hd + (size_t)(n_head / n_kv_head) * hd);
}

extern "C" int sdy_attn_decode_ok(int n_head, int n_kv_head, int hd, int max_seq) {
    (void)max_seq;
    // the decode kernel is built for head_dim 64 and 128
    if ((hd != 64 && hd != 128) || n_kv_head < 1 || n_head % n_kv_head || n_head > 64) return 0;
    return attn_decode_lds(n_head, n_kv_head, hd) <= 160 * 1024;
}

extern "C" size_t sdy_attn_decode_chunks(int max_seq) { return (size_t)((max_seq + CH - 1) / CH); }

extern "C" int sdy_attn_decode(const float *q, const float *k, const float *v, const float *q_norm,
                               const float *k_norm, float eps, const float *rope_cos, const float *rope_sin,
                               const int32_t *step_dev, int n_head, int n_kv_head, int hd, int interleaved,
                               float *k_cache, float *v_cache, long head_stride, int max_seq, float *part,
                               sdy_stream s) {
    if (!sdy_attn_decode_ok(n_head, n_kv_head, hd, max_seq))
        return sdy_fail(-1, "attn_decode: unsupported shape (%d heads, %d kv heads, head_dim %d)", n_head, n_kv_head,
                        hd);
    const size_t lds = attn_decode_lds(n_head, n_kv_head, hd);
    static size_t granted[2] = {0, 0};
    const void *fn = hd == 128 ? (const void *)k_attn_decode<128> : (const void *)k_attn_decode<64>;
    int rc = sdy_lds_limit(fn, lds, &granted[hd == 128]);
    if (rc) return rc;
    AttnDecodeArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.eps = eps;
    a.rope_cos = rope_cos;
    a.rope_sin = rope_sin;
    a.step = step_dev;
    a.n_head = n_head;
    a.n_kv_head = n_kv_head;
    a.hd = hd;
    a.interleaved = interleaved;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.head_stride = head_stride;
    a.part = part;
    a.n_chunk_max = (max_seq + CH - 1) / CH;
    a.scale = 1.0f / sqrtf((float)hd);
    if (hd == 128)
        hipLaunchKernelGGL(k_attn_decode<128>, dim3(a.n_chunk_max, n_kv_head), dim3(DEC_NT), lds, (hipStream_t)s, a);
    else
        hipLaunchKernelGGL(k_attn_decode<64>, dim3(a.n_chunk_max, n_kv_head), dim3(DEC_NT), lds, (hipStream_t)s, a);
    return sdy_check_launch("attn_decode");
}

extern "C" int sdy_attn_merge1(const float *part, const int32_t *step_dev, int n_head, int hd, int max_seq, float *out,
                               void *xq_q8k, sdy_stream s) {
    const int nchm = (max_seq + CH - 1) / CH;
    const int n_out = n_head * hd, hps = (255 + hd - 1) / hd + 1;  // heads a super-block can touch
    const size_t lds = (size_t)hps * 2 * nchm * sizeof(float);
    if (xq_q8k && n_out % 256 == 0 && hps <= 64 && lds <= 64 * 1024) {
        hipLaunchKernelGGL(k_attn_merge1_q8k, dim3(n_out / 256), dim3(64), lds, (hipStream_t)s, part, step_dev, n_head,
                           hd, nchm, out, (uint8_t *)xq_q8k);
        return sdy_check_launch("attn_merge1_q8k");
    }
    if (xq_q8k) return sdy_fail(-1, "attn_merge1: no Q8_K merge for %d heads of %d", n_head, hd);
    hipLaunchKernelGGL(k_attn_merge1, dim3(n_head), dim3(64), 2 * nchm * sizeof(float), (hipStream_t)s, part, step_dev,
                       n_head, hd, nchm, out);
    return sdy_check_launch("attn_merge1");
}

extern "C" int sdy_attn_merge1_q8k_ok(int n_head, int hd, int max_seq) {
    const int nchm = (max_seq + CH - 1) / CH, hps = (255 + hd - 1) / hd + 1;
    return (n_head * hd) % 256 == 0 && (size_t)hps * 2 * nchm * sizeof(float) <= 64 * 1024;
}

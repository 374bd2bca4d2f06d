// Prefill attention in flash form on the f32 matrix cores (within tolerance of the reference, not
// its bits; the reference's own arithmetic is sdy_attention in attn_kernels.hip).
//
// For each prompt token t and query head, the reference (csrc/ops.c:405-414, called per token from
// csrc/model_llama.c:619-647) takes the scores s_j = q.k_j / sqrt(head_dim) over the positions
// j < n_kv0 + t, one softmax over them and the weighted sum of the V rows. Here:
//
//   k_attn_flash<HD, KT>  grid (ceil(n_tok / 32), n_head), 512 threads: one workgroup per 32
//   consecutive queries of one head (the blocks with the most keys first), its eight waves sharing
//   the key tiles of 32 positions (wave w: tiles w, w + 8, ...). Per tile a wave computes
//   S^T = K Q^T on v_mfma_f32_32x32x2_f32 (keys as rows, so a lane holds its own query's 16 scores
//   of the tile), masks the positions at or past each query's causal limit, and keeps the running
//   maximum m, the sum l of exp(s - m) and O^T = V^T P (HD / 32 tiles of 32 dims), rescaled by
//   exp(m_old - m_new) when m grows. The queries' Q^T rows sit in LDS, read by all eight waves.
//   The waves' (m, l, O) are then merged through LDS in wave order:
//   out = sum_w O_w exp(m_w - M) / sum_w l_w exp(m_w - M), M = max_w m_w.
//
// Each sum has a fixed order (no float atomics), so the results are deterministic. They differ
// from the reference's in rounding: f32 products summed in the matrix core's order, tile-relative
// exponentials.
#include "sdy_attn_dev.h"
#include "sdy_device.h"
#include "sdy_internal.h"
#include "sdy_ops.h"
#include "sdy_shim.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int QB = 32;  // queries per workgroup (the MFMA's 32 columns)
constexpr int KB = 32;  // positions per key tile (the MFMA's 32 rows)
constexpr int FW = 8;   // waves per workgroup

struct FlashArgs {
    const float *q;          // rotated queries [n_tok][q_stride], head h at h * HD
    long q_stride;
    const void *k_cache, *v_cache;  // [n_kv_head][max_seq][HD] of the element type KT
    long head_stride;        // max_seq * HD
    int n_head, n_kv_head, n_tok, n_kv0;  // token t attends to positions < n_kv0 + t
    float scale;             // 1 / sqrt(HD)
    float *out;              // [n_tok][out_stride], head h at h * HD
    long out_stride;
};

// LDS: Q^T of the block as [2][32][QS] (element (query q, dim half * HD/2 + s) at [half][q][s]),
// then, after the key tiles, the merge area: the waves' O dims, 1/MS of them at a time, as
// [FW][32][OS] and their m, l as [2][FW][32] (HD 128: 134 KB for MS 1, one workgroup per CU;
// 68 KB for MS 2, two).
template <int HD, int MS>
struct FlashLds {
    static constexpr int HH = HD / 2, QS = HH + 4, OS = HD / MS + 1;
    static constexpr size_t q_floats = 2 * 32 * QS;
    static constexpr size_t merge_floats = (size_t)FW * 32 * OS + 2 * FW * 32;
    static constexpr size_t bytes = 4 * (q_floats > merge_floats ? q_floats : merge_floats);
};

// ND consecutive elements of a V row (the lane's dims ND * (lane % 32) + dt, dt < ND)
template <int ND, class KT>
struct VLoad;
template <class KT>
struct VLoad<4, KT> {
    using T = sdy_f32x4;
    SDY_DEV static T ld(const KT *p, size_t i) { return KvElt<KT>::ld4(p, i); }
    SDY_DEV static float at(const T &v, int j) { return v[j]; }
};
template <class KT>
struct VLoad<2, KT> {
    using T = float2;
    SDY_DEV static T ld(const KT *p, size_t i) { return KvElt<KT>::ld2(p, i); }
    SDY_DEV static float at(const T &v, int j) { return j ? v.y : v.x; }
};

template <int HD, class KT, int MS>
__global__ __launch_bounds__(64 * FW) void k_attn_flash(FlashArgs a) {
    using LY = FlashLds<HD, MS>;
    constexpr int HH = HD / 2, ND = HD / 32;
    using VL = VLoad<ND, KT>;
    extern __shared__ __align__(16) float lds[];
    const int tid = threadIdx.x, lane = tid & 63, hh = lane >> 5, ql = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qb = (int)gridDim.x - 1 - (int)blockIdx.x;  // the blocks with the most keys first
    const int h = blockIdx.y, g = h / (a.n_head / a.n_kv_head);
    const int q0 = qb * QB;
    const int t_last = q0 + QB < a.n_tok ? q0 + QB - 1 : a.n_tok - 1;
    const int n_kv_max = a.n_kv0 + t_last;  // positions of the block's last query
    const int n_kt = (n_kv_max + KB - 1) / KB;

    for (int i = tid; i < QB * HD / 4; i += 64 * FW) {
        const int q = i / (HD / 4), d = 4 * (i - q * (HD / 4));
        const int t = q0 + q < a.n_tok ? q0 + q : a.n_tok - 1;
        const float4 v = *reinterpret_cast<const float4 *>(a.q + (size_t)t * a.q_stride + (size_t)h * HD + d);
        const int part = d / HH, s = d - part * HH;
        *reinterpret_cast<float4 *>(lds + (part * 32 + q) * LY::QS + s) = v;
    }
    __syncthreads();

    const int t = q0 + ql;
    const int lim = t < a.n_tok ? a.n_kv0 + t : 0;  // this lane's query sees positions < lim
    const KT *kb = (const KT *)a.k_cache + (size_t)g * a.head_stride;
    const KT *vb = (const KT *)a.v_cache + (size_t)g * a.head_stride;
    const float *qs = lds + (hh * 32 + ql) * LY::QS;
    f32x16 o[ND];
#pragma unroll
    for (int dt = 0; dt < ND; dt++) o[dt] = f32x16{};
    float m_run = -INFINITY, l_run = 0.0f;
    for (int kt = wave; kt < n_kt; kt += FW) {
        const int k0 = kt * KB;
        // K: lane (key ql of the tile, dims hh * HH ...); V of the PV step r: key
        // 8 (r / 4) + 4 hh + r % 4 of the tile (the key of the lane's score register r), dims
        // ND * ql ... (positions past the block's last one read its row: masked below)
        const int kr = k0 + ql < n_kv_max ? k0 + ql : n_kv_max - 1;
        sdy_f32x4 kv[HH / 4];
#pragma unroll
        for (int i = 0; i < HH / 4; i++) kv[i] = KvElt<KT>::ld4(kb, (size_t)kr * HD + hh * HH + 4 * i);
        typename VL::T vv[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = k0 + 8 * (r >> 2) + 4 * hh + (r & 3);
            vv[r] = VL::ld(vb, (size_t)(key < n_kv_max ? key : n_kv_max - 1) * HD + ND * ql);
        }
        // S^T[key][query] = sum over dims of K[key][d] Q[query][d]: step (i, j) pairs dim 4i + j
        // (lanes 0-31) with dim HH + 4i + j (lanes 32-63)
        f32x16 s = f32x16{};
#pragma unroll
        for (int i = 0; i < HH / 4; i++) {
            const sdy_f32x4 qv = *reinterpret_cast<const sdy_f32x4 *>(qs + 4 * i);
#pragma unroll
            for (int j = 0; j < 4; j++) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[i][j], qv[j], s, 0, 0, 0);
        }
        // scores of the lane's query (register r: key 8 (r / 4) + 4 hh + r % 4), running maximum
        // and sum; the other half of the tile's keys is in lane ^ 32
        float p[16];
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = k0 + 8 * (r >> 2) + 4 * hh + (r & 3);
            p[r] = key < lim ? s[r] * a.scale : -INFINITY;
            mt = fmaxf(mt, p[r]);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float m_new = fmaxf(m_run, mt);
        const float mu = m_new == -INFINITY ? 0.0f : m_new;  // no key yet: every term is 0
        float ls = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            p[r] = __expf(p[r] - mu);
            ls += p[r];
        }
        ls += __shfl_xor(ls, 32);
        const float corr = __expf(m_run - mu);
        l_run = l_run * corr + ls;
        m_run = m_new;
#pragma unroll
        for (int dt = 0; dt < ND; dt++)
#pragma unroll
            for (int e = 0; e < 16; e++) o[dt][e] = o[dt][e] * corr;
        // O^T[dim][query] += V^T[dim][key] P[key][query] over the tile's keys, two per step
#pragma unroll
        for (int r = 0; r < 16; r++)
#pragma unroll
            for (int dt = 0; dt < ND; dt++)
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(VL::at(vv[r], dt), p[r], o[dt], 0, 0, 0);
    }

    // merge of the waves' partials in wave order (the Q^T area is reused), in MS parts of the dims:
    // part x holds the O columns dt in [x NDH, (x + 1) NDH), dims ND * row + dt, at NDH * row + dt - x NDH
    constexpr int NDH = ND / MS;
    float *ml = lds + (size_t)FW * 32 * LY::OS;  // m [FW][32], then l [FW][32]
#pragma unroll
    for (int x = 0; x < MS; x++) {
        __syncthreads();
        float *om = lds + (size_t)wave * 32 * LY::OS;
#pragma unroll
        for (int dt = x * NDH; dt < (x + 1) * NDH; dt++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = 8 * (r >> 2) + 4 * hh + (r & 3);  // D row: dim ND * row + dt
                om[ql * LY::OS + NDH * row + dt - x * NDH] = o[dt][r];
            }
        if (x == 0 && hh == 0) {
            ml[wave * 32 + ql] = m_run;
            ml[FW * 32 + wave * 32 + ql] = l_run;
        }
        __syncthreads();
        for (int i = tid; i < QB * (HD / MS); i += 64 * FW) {
            const int q = i / (HD / MS), dl = i - q * (HD / MS);
            if (q0 + q >= a.n_tok) continue;
            const int d = ND * (dl / NDH) + x * NDH + dl % NDH;
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < FW; w++) M = fmaxf(M, ml[w * 32 + q]);
            float ls = 0.0f, os = 0.0f;
#pragma unroll
            for (int w = 0; w < FW; w++) {
                const float e = __expf(ml[w * 32 + q] - M);  // a wave without keys: m = -inf, e = 0
                ls += ml[FW * 32 + w * 32 + q] * e;
                os += lds[((size_t)w * 32 + q) * LY::OS + dl] * e;
            }
            a.out[(size_t)(q0 + q) * a.out_stride + (size_t)h * HD + d] = os / ls;
        }
    }
}

template <int HD, class KT, int MS>
int launch_flash(const FlashArgs &A, hipStream_t st) {
    static size_t granted = 0;
    const void *fn = (const void *)k_attn_flash<HD, KT, MS>;
    int rc = sdy_lds_limit(fn, FlashLds<HD, MS>::bytes, &granted);
    if (rc) return rc;
    SDY_NOTE_KERNEL((k_attn_flash<HD, KT, MS>));
    hipLaunchKernelGGL((k_attn_flash<HD, KT, MS>), dim3((unsigned)((A.n_tok + QB - 1) / QB), (unsigned)A.n_head),
                       dim3(64 * FW), (FlashLds<HD, MS>::bytes), st, A);
    return sdy_check_launch("attn_flash");
}

// The merge in two parts (two workgroups per CU) when the grid has more workgroups than the GPU
// has CUs: the 30B-A3B's 32 heads x 16 blocks, 36.0 -> 34.2 ms for its 1024-token prefill; the 3B's
// 16 x 16 fill the CUs once, and a second merge round only costs (53.8k against 53.4k tok/s).
template <int HD, class KT>
int launch_flash_ms(const FlashArgs &A, hipStream_t st) {
    int n_cu = 0;
    size_t mem = 0;
    if (sdy_device_info(&n_cu, &mem) || n_cu <= 0) n_cu = 256;
    const long wgs = (long)((A.n_tok + QB - 1) / QB) * A.n_head;
    return wgs > n_cu ? launch_flash<HD, KT, 2>(A, st) : launch_flash<HD, KT, 1>(A, st);
}

template <int HD>
int launch_flash_kv(const FlashArgs &A, int kv_type, hipStream_t st) {
    return kv_type == SDY_KV_F16 ? launch_flash_ms<HD, uint16_t>(A, st) : launch_flash_ms<HD, float>(A, st);
}

}  // namespace

extern "C" int sdy_attention_flash_ok(int n_head, int n_kv_head, int hd) {
    return (hd == 64 || hd == 128) && n_head > 0 && n_kv_head > 0 && n_head % n_kv_head == 0;
}

extern "C" int sdy_attention_flash(const float *q, const void *k_cache, const void *v_cache, int kv_type, int n_tok,
                                   int n_head, int n_kv_head, int hd, int n_kv0, long head_stride, long q_stride,
                                   float *out, long out_stride, sdy_stream s) {
    if (n_tok <= 0) return 0;
    if (!sdy_attention_flash_ok(n_head, n_kv_head, hd))
        return sdy_fail(-1, "attention_flash: head_dim 64 or 128 and n_head a multiple of n_kv_head (got %d, %d, %d)",
                        hd, n_head, n_kv_head);
    if (kv_type != SDY_KV_F32 && kv_type != SDY_KV_F16) return sdy_fail(-1, "attention_flash: KV type %d", kv_type);
    if (n_kv0 < 1) return sdy_fail(-1, "attention_flash: the first token needs a position (n_kv0 %d)", n_kv0);
    if ((q_stride | out_stride) & 3 || (uintptr_t)q & 15)
        return sdy_fail(-1, "attention_flash: q rows (and strides) aligned to 16 bytes");
    FlashArgs A;
    A.q = q;
    A.q_stride = q_stride;
    A.k_cache = k_cache;
    A.v_cache = v_cache;
    A.head_stride = head_stride;
    A.n_head = n_head;
    A.n_kv_head = n_kv_head;
    A.n_tok = n_tok;
    A.n_kv0 = n_kv0;
    A.scale = 1.0f / sqrtf((float)hd);
    A.out = out;
    A.out_stride = out_stride;
    hipStream_t st = (hipStream_t)s;
    return hd == 64 ? launch_flash_kv<64>(A, kv_type, st) : launch_flash_kv<128>(A, kv_type, st);
}

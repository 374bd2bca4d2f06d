// gfx950 kernels for the float side of the forward pass: RMSNorm, softmax, SiLU·mul, RoPE table
// and rotation, MoE router (softmax + top-k) and the small elementwise ops of the kernel-level ABI
// (attention: attn_kernels.hip).
//
// Numerics follow the reference (csrc/ops.c:346-423, csrc/model_llama.c:653-666) where it matters
// for parity: RMSNorm and softmax sum in double and round the scale once, RoPE angles are computed
// in double, top-k keeps the lower expert index on ties and renormalises with a sequential float
// sum. Reductions use fixed trees, so every result is reproducible run to run.
#include "sdy_device.h"
#include "sdy_expf.h"
#include "sdy_internal.h"
#include "sdy_norm_dev.h"
#include "sdy_ops.h"
#include "sdy_route_dev.h"
#include "sdy_shim.h"

namespace {

template <typename T>
SDY_DEV T block_reduce_sum(T v, T *sh) {  // blockDim.x == 256, fixed tree
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    T r = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    __syncthreads();
    return r;
}

SDY_DEV float block_reduce_max(float v, float *sh) {
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    float r = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
    __syncthreads();
    return r;
}

// out[r] = x[r] * (1/sqrt(mean(x[r]^2) + eps)) * w, one 256-thread block per row
// (csrc/ops.c:346-351: sum of squares in double, scale rounded to float once).
__global__ __launch_bounds__(256) void k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w, float *out,
                                                 int n, float eps, long x_stride, long out_stride) {
    __shared__ double sh[4];
    const float *xr = x + blockIdx.x * x_stride;
    float *o = out + blockIdx.x * out_stride;
    const double ss = sdy_row_sumsq<0>(xr, n, nullptr, sh);
    const float scale = (float)(1.0 / sqrt(ss / (double)n + (double)eps));
    for (int i = threadIdx.x; i < n; i += 256) {
        float t = xr[i] * scale;
        o[i] = t * w[i];
    }
}

// ------------------------------------------------------------------------------ elementwise

// gate = silu(gate) * up   (csrc/ops.c:366-371)
__global__ void k_silu_mul(float *gate, const float *up, long n) {
    long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (i >= n) return;
    float g = gate[i];
    float s = g / (1.0f + sdy_expf(-g));
    gate[i] = s * up[i];
}

__global__ void k_add(const float *a, const float *b, float *out, long n) {
    long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

__global__ void k_axpy(float *y, float a, const float *x, long n) {
    long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (i < n) y[i] = fmaf(a, x[i], y[i]);
}

__global__ void k_f16_to_f32(const uint16_t *x, float *out, long n) {
    long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (i < n) out[i] = sdy_h2f(x[i]);
}

__global__ void k_f32_to_f16(const float *x, uint16_t *out, long n) {
    long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (i < n) out[i] = sdy_f2h(x[i]);
}

// dot product of two vectors: one block, fixed tree (4 chains per thread, then the block tree)
__global__ __launch_bounds__(256) void k_dot(const float *a, const float *b, int n, float *out) {
    __shared__ float sh[4];
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) s = fmaf(a[i], b[i], s);
    s = block_reduce_sum(s, sh);
    if (threadIdx.x == 0) *out = s;
}

// softmax over n values of each row (csrc/ops.c:353-364): max, expf, double sum, float reciprocal
__global__ __launch_bounds__(256) void k_softmax(float *x, int n, long stride) {
    __shared__ float shf[4];
    __shared__ double shd[4];
    float *r = x + blockIdx.x * stride;
    float m = -INFINITY;
    for (int i = threadIdx.x; i < n; i += 256) m = fmaxf(m, r[i]);
    m = block_reduce_max(m, shf);
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) {
        float e = sdy_expf(r[i] - m);
        r[i] = e;
        s += (double)e;
    }
    s = block_reduce_sum(s, shd);
    float inv = (float)(1.0 / s);
    for (int i = threadIdx.x; i < n; i += 256) r[i] *= inv;
}

// rotate n_heads vectors by one row of the tables (csrc/ops.c:388-401)
__global__ void k_rope(float *x, int n_heads, int hd, const float *cs, const float *sn, int interleaved) {
    long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    const int half = hd / 2;
    if (i >= (long)n_heads * half) return;
    int h = (int)(i / half), j = (int)(i - (long)h * half);
    float *v = x + (size_t)h * hd;
    int ia = interleaved ? 2 * j : j, ib = interleaved ? 2 * j + 1 : j + half;
    float a = v[ia], b = v[ib];
    float ac = a * cs[j], bs = b * sn[j], as = a * sn[j], bc = b * cs[j];
    v[ia] = ac - bs;
    v[ib] = as + bc;
}

// ---------------------------------------------------------------------------------- MoE router
// One wave per token: softmax over the expert logits (max, expf, double sum, float reciprocal),
// then top-k by repeated arg-max with ties to the lower index (the order moe_select produces,
// csrc/model_llama.c:653-666) and weights renormalised by their sequential float sum
// (sdy_moe_route_wave).
template <int NPL>  // experts held per lane: n_expert <= 64 * NPL
__global__ __launch_bounds__(64) void k_moe_route(const float *logits, int n_expert, int k, int32_t *top,
                                                  float *wts) {
    const int t = blockIdx.x, lane = threadIdx.x;
    const uint32_t etab = sdy_expf_tab_lane(lane);  // the exponential's table, loaded with the logits
    int my_e;
    float my_p, chosen_sum;
    sdy_moe_route_wave<NPL>(logits + (size_t)t * n_expert, n_expert, k, lane, etab, my_e, my_p, chosen_sum);
    if (lane < k) {
        top[(size_t)t * k + lane] = my_e;
        wts[(size_t)t * k + lane] = my_p / chosen_sum;
    }
}

// One step of the reference's AVX2 axpy (csrc/ops_avx2.c:142-147) at element d of a dim-element
// row: fused in the 8-lane body, a rounded product then a sum in the tail.
SDY_DEV float axpy1(float acc, float w, float y, int d, int dim) {
    return d < (dim & ~7) ? fmaf(w, y, acc) : acc + w * y;
}

// out[t] = sum over the k chosen experts, in ascending expert id, of w * y   (moe_ffn's axpy order
// over experts, csrc/model_llama.c:734-750), plus resid. y is [n_tok][k][dim] in top-k slot order.
// The k (id, weight, value) triples of a token are sorted by id in registers (k <= KMAX).
template <int KMAX>
__global__ void k_moe_combine(const float *y, const int32_t *top, const float *wts, int k, int dim, float *out,
                              const float *resid) {
    const int t = blockIdx.y;
    const int d0 = blockIdx.x * blockDim.x + threadIdx.x;
    const int d = d0 < dim ? d0 : dim - 1;
    const int32_t *tt = top + (size_t)t * k;
    int id[KMAX];
    float w[KMAX], yv[KMAX];
#pragma unroll
    for (int i = 0; i < KMAX; i++) {
        const int ii = i < k ? i : 0;
        id[i] = i < k ? tt[ii] : 0x7fffffff;
        w[i] = wts[(size_t)t * k + ii];
        yv[i] = y[((size_t)t * k + ii) * dim + d];
    }
#pragma unroll
    for (int a = 0; a < KMAX; a++)
#pragma unroll
        for (int b = 0; b + 1 < KMAX - a; b++)
            if (id[b] > id[b + 1]) {
                const int ti = id[b];
                id[b] = id[b + 1];
                id[b + 1] = ti;
                const float tw = w[b];
                w[b] = w[b + 1];
                w[b + 1] = tw;
                const float ty = yv[b];
                yv[b] = yv[b + 1];
                yv[b + 1] = ty;
            }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < KMAX; i++)
        if (i < k) acc = axpy1(acc, w[i], yv[i], d, dim);
    if (d0 < dim) out[(size_t)t * dim + d] = resid ? resid[(size_t)t * dim + d] + acc : acc;
}

// dst[r] = src[idx[r]] (rows of dim floats)
__global__ void k_gather_rows(const float *src, const int32_t *idx, int dim, float *dst) {
    const int r = blockIdx.y;
    int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d < dim) dst[(size_t)r * dim + d] = src[(size_t)idx[r] * dim + d];
}

// dst[idx[r]] += w[r] * src[r]  (rows of dim floats; the idx of one launch are distinct)
__global__ void k_scatter_axpy(float *dst, const int32_t *idx, const float *w, const float *src, int dim) {
    const int r = blockIdx.y;
    int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d < dim) {
        float *o = dst + (size_t)idx[r] * dim + d;
        *o = axpy1(*o, w[r], src[(size_t)r * dim + d], d, dim);
    }
}

}  // namespace

// =============================================================================== launchers

#define GRID1(n, b) dim3((unsigned)(((n) + (b)-1) / (b)))

extern "C" int sdy_rmsnorm(const float *x, const float *w, float *out, int n, float eps, int n_rows, long x_stride,
                           long out_stride, sdy_stream s) {
    if (n_rows <= 0) return 0;
    hipLaunchKernelGGL(k_rmsnorm, dim3(n_rows), dim3(256), 0, (hipStream_t)s, x, w, out, n, eps, x_stride, out_stride);
    return sdy_check_launch("rmsnorm");
}

extern "C" int sdy_silu_mul(float *gate, const float *up, long n, sdy_stream s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_silu_mul, GRID1(n, 256), dim3(256), 0, (hipStream_t)s, gate, up, n);
    return sdy_check_launch("silu_mul");
}

extern "C" int sdy_add(const float *a, const float *b, float *out, long n, sdy_stream s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_add, GRID1(n, 256), dim3(256), 0, (hipStream_t)s, a, b, out, n);
    return sdy_check_launch("add");
}

extern "C" int sdy_axpy(float *y, float a, const float *x, long n, sdy_stream s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_axpy, GRID1(n, 256), dim3(256), 0, (hipStream_t)s, y, a, x, n);
    return sdy_check_launch("axpy");
}

extern "C" int sdy_dot(const float *a, const float *b, int n, float *out, sdy_stream s) {
    hipLaunchKernelGGL(k_dot, dim3(1), dim3(256), 0, (hipStream_t)s, a, b, n, out);
    return sdy_check_launch("dot");
}

extern "C" int sdy_f16_to_f32(const uint16_t *x, float *out, long n, sdy_stream s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_f16_to_f32, GRID1(n, 256), dim3(256), 0, (hipStream_t)s, x, out, n);
    return sdy_check_launch("f16_to_f32");
}

extern "C" int sdy_f32_to_f16(const float *x, uint16_t *out, long n, sdy_stream s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_f32_to_f16, GRID1(n, 256), dim3(256), 0, (hipStream_t)s, x, out, n);
    return sdy_check_launch("f32_to_f16");
}

extern "C" int sdy_softmax(float *x, int n, int n_rows, long stride, sdy_stream s) {
    if (n_rows <= 0 || n <= 0) return 0;
    hipLaunchKernelGGL(k_softmax, dim3(n_rows), dim3(256), 0, (hipStream_t)s, x, n, stride);
    return sdy_check_launch("softmax");
}

extern "C" int sdy_rope(float *x, int n_heads, int hd, const float *cs, const float *sn, int interleaved, sdy_stream s) {
    long n = (long)n_heads * (hd / 2);
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_rope, GRID1(n, 256), dim3(256), 0, (hipStream_t)s, x, n_heads, hd, cs, sn, interleaved);
    return sdy_check_launch("rope");
}

extern "C" int sdy_moe_route(float *probs, int n_tok, int n_expert, int k, int32_t *top, float *wts, sdy_stream s) {
    if (n_expert > 512) return sdy_fail(-1, "n_expert %d above 512", n_expert);
    if (k < 1 || k > n_expert || k > 64) return sdy_fail(-1, "n_expert_used %d (of %d experts)", k, n_expert);
    hipStream_t st = (hipStream_t)s;
    if (n_expert <= 64) hipLaunchKernelGGL(k_moe_route<1>, dim3(n_tok), dim3(64), 0, st, probs, n_expert, k, top, wts);
    else if (n_expert <= 128) hipLaunchKernelGGL(k_moe_route<2>, dim3(n_tok), dim3(64), 0, st, probs, n_expert, k, top, wts);
    else if (n_expert <= 256) hipLaunchKernelGGL(k_moe_route<4>, dim3(n_tok), dim3(64), 0, st, probs, n_expert, k, top, wts);
    else hipLaunchKernelGGL(k_moe_route<8>, dim3(n_tok), dim3(64), 0, st, probs, n_expert, k, top, wts);
    return sdy_check_launch("moe_route");
}

extern "C" int sdy_moe_combine(const float *y, const int32_t *top, const float *wts, int n_tok, int k, int dim,
                               float *out, const float *resid, sdy_stream s) {
    hipStream_t st = (hipStream_t)s;
    const dim3 grid((dim + 63) / 64, n_tok);
    if (k < 1 || k > 16) return sdy_fail(-1, "moe_combine: %d experts per token (1..16)", k);
    if (k <= 8) hipLaunchKernelGGL(k_moe_combine<8>, grid, dim3(64), 0, st, y, top, wts, k, dim, out, resid);
    else hipLaunchKernelGGL(k_moe_combine<16>, grid, dim3(64), 0, st, y, top, wts, k, dim, out, resid);
    return sdy_check_launch("moe_combine");
}

// The routed (token, slot) pairs grouped by expert for the grouped GEMM: a stable sort of the
// n = n_tok * k expert ids in top (the reference groups a batch's tokens per expert the same way,
// csrc/model_llama.c:676-700). Sorted row r holds pair out_row[r] = t * k + s, of token
// src_tok[r] = t; rows grp_tok[e] .. grp_tok[e + 1] - 1 are expert e's, in (t, s) order;
// grp_tile[e] is the number of bn-row tiles of the experts before e.
//
// k_moe_sort_rank (when its per-chunk counts fit in LDS): one workgroup of 16 waves. The list is cut
// into chunks of 64 pairs (one per lane); in a chunk, the lanes holding the same expert are found
// with one ballot per bit of the expert id, so a pair's rank among them is a popcount of the lower
// lanes. Each chunk's count per expert goes to LDS; one thread per expert turns its column into
// offsets over the chunks (in chunk order), the experts' first rows and tile offsets are exclusive
// scans, and each pair lands at its expert's first row + its chunk's offset + its rank.
// k_moe_sort (lists whose chunk counts do not fit): SORT_SEG threads count, then place, the pairs of
// their segment of the list; per (segment, expert) counts in LDS make the placement stable.
constexpr int SORT_SEG = 64;
constexpr int SORT_RANK_LDS = 128 * 1024;  // bytes of per-chunk counts k_moe_sort_rank may use

__global__ __launch_bounds__(1024) void k_moe_sort_rank(const int32_t *top, int n, int k, int ne, int bn,
                                                        int *grp_tok, int *grp_tile, int32_t *src_tok,
                                                        int32_t *out_row) {
    extern __shared__ uint16_t ccnt[];  // [n_chunk][ne]: counts, then offsets within the expert
    __shared__ int first[513];          // each expert's first row, [ne] = n
    __shared__ int wsum[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n_chunk = (n + 63) >> 6;
    for (int i = tid; i < n_chunk * ne; i += 1024) ccnt[i] = 0;
    __syncthreads();
    // lanes of the wave holding the same expert (ids up to 511; past the list: the id ne)
    auto peers = [&](int e) {
        uint64_t m = ~0ull;
#pragma unroll
        for (int b = 0; b < 10; b++) {
            const uint64_t v = __ballot((e >> b) & 1);
            m &= ((e >> b) & 1) ? v : ~v;
        }
        return m;
    };
    auto expert_of = [&](int i) {
        if (i >= n) return ne;
        const int e = top[i];
        return e < 0 ? 0 : e >= ne ? ne - 1 : e;
    };
    const uint64_t below = (1ull << lane) - 1;  // lanes under this one
    for (int c = wave; c < n_chunk; c += 16) {
        const int i = 64 * c + lane, e = expert_of(i);
        const uint64_t m = peers(e);
        if (e < ne && (m & below) == 0) ccnt[c * ne + e] = (uint16_t)__popcll(m);
    }
    __syncthreads();
    for (int e = tid; e < ne; e += 1024) {  // chunk offsets within the expert, in chunk order
        int run = 0;
        for (int c = 0; c < n_chunk; c++) {
            const int v = ccnt[c * ne + e];
            ccnt[c * ne + e] = (uint16_t)run;
            run += v;
        }
        first[e] = run;  // the expert's total, for now
    }
    __syncthreads();
    // experts' first rows and tile offsets: exclusive scans over the experts (ne <= 512: waves 0-7)
    const int cnt_e = tid < ne ? first[tid] : 0, tiles = (cnt_e + bn - 1) / bn;
    int inc_r = cnt_e, inc_t = tiles;
    for (int off = 1; off < 64; off <<= 1) {
        const int vr = __shfl_up(inc_r, off), vt = __shfl_up(inc_t, off);
        if (lane >= off) {
            inc_r += vr;
            inc_t += vt;
        }
    }
    if (lane == 63) wsum[wave] = inc_r;
    __syncthreads();
    int before_r = 0;
    for (int w = 0; w < wave; w++) before_r += wsum[w];
    __syncthreads();
    if (lane == 63) wsum[wave] = inc_t;
    __syncthreads();
    int before_t = 0;
    for (int w = 0; w < wave; w++) before_t += wsum[w];
    __syncthreads();  // every thread has read the totals of the experts' counts
    if (tid <= ne) {
        const int row = before_r + inc_r - cnt_e;  // (tid == ne: cnt_e = 0, the total n)
        first[tid] = row;
        grp_tok[tid] = row;
        grp_tile[tid] = before_t + inc_t - tiles;
    }
    __syncthreads();
    for (int c = wave; c < n_chunk; c += 16) {
        const int i = 64 * c + lane, e = expert_of(i);
        const uint64_t m = peers(e);
        if (e < ne) {
            const int r = first[e] + ccnt[c * ne + e] + __popcll(m & below);
            src_tok[r] = i / k;
            out_row[r] = i;
        }
    }
}

__global__ __launch_bounds__(256) void k_moe_sort(const int32_t *top, int n, int k, int ne, int bn, int *grp_tok,
                                                  int *grp_tile, int32_t *src_tok, int32_t *out_row) {
    extern __shared__ int sort_lds[];
    int *cnt = sort_lds;              // [SORT_SEG][ne]: counts, then running offsets
    int *base = cnt + SORT_SEG * ne;  // [ne + 1] first row of each expert
    const int tid = threadIdx.x, seg_len = (n + SORT_SEG - 1) / SORT_SEG;
    for (int i = tid; i < SORT_SEG * ne; i += 256) cnt[i] = 0;
    __syncthreads();
    auto expert_of = [&](int i) {
        const int e = top[i];
        return e < 0 ? 0 : e >= ne ? ne - 1 : e;
    };
    if (tid < SORT_SEG) {
        const int b = tid * seg_len, end = b + seg_len < n ? b + seg_len : n;
        for (int i = b; i < end; i++) cnt[tid * ne + expert_of(i)]++;
    }
    __syncthreads();
    for (int e = tid; e < ne; e += 256) {  // offsets of each segment within its expert
        int run = 0;
        for (int sg = 0; sg < SORT_SEG; sg++) {
            const int c = cnt[sg * ne + e];
            cnt[sg * ne + e] = run;
            run += c;
        }
        base[e] = run;  // the expert's total, for now
    }
    __syncthreads();
    if (tid == 0) {
        int rows = 0, tiles = 0;
        for (int e = 0; e < ne; e++) {
            const int c = base[e];
            base[e] = rows;
            grp_tok[e] = rows;
            grp_tile[e] = tiles;
            rows += c;
            tiles += (c + bn - 1) / bn;
        }
        base[ne] = rows;
        grp_tok[ne] = rows;
        grp_tile[ne] = tiles;
    }
    __syncthreads();
    if (tid < SORT_SEG) {
        const int b = tid * seg_len, end = b + seg_len < n ? b + seg_len : n;
        for (int i = b; i < end; i++) {
            const int e = expert_of(i), r = base[e] + cnt[tid * ne + e]++;
            src_tok[r] = i / k;
            out_row[r] = i;
        }
    }
}

extern "C" int sdy_moe_sort(const int32_t *top, int n_tok, int k, int n_expert, int bn, int *grp_tok, int *grp_tile,
                            int32_t *src_tok, int32_t *out_row, sdy_stream s) {
    if (n_expert < 1 || n_expert > 512 || k < 1 || n_tok < 1 || bn < 1)
        return sdy_fail(-1, "moe_sort: %d tokens x %d of %d experts (at most 512), tiles of %d", n_tok, k, n_expert, bn);
    const int n = n_tok * k;
    int rc;
    const size_t rank_lds = sizeof(uint16_t) * (size_t)((n + 63) / 64) * n_expert;
    if (rank_lds <= SORT_RANK_LDS && n <= 65535) {
        static size_t granted_rank = 0;
        if ((rc = sdy_lds_limit((const void *)k_moe_sort_rank, rank_lds, &granted_rank))) return rc;
        SDY_NOTE_KERNEL(k_moe_sort_rank);
        hipLaunchKernelGGL(k_moe_sort_rank, dim3(1), dim3(1024), rank_lds, (hipStream_t)s, top, n, k, n_expert, bn,
                           grp_tok, grp_tile, src_tok, out_row);
        return sdy_check_launch("moe_sort");
    }
    const size_t lds = sizeof(int) * ((size_t)SORT_SEG * n_expert + n_expert + 1);
    static size_t granted = 0;
    if ((rc = sdy_lds_limit((const void *)k_moe_sort, lds, &granted))) return rc;
    SDY_NOTE_KERNEL(k_moe_sort);
    hipLaunchKernelGGL(k_moe_sort, dim3(1), dim3(256), lds, (hipStream_t)s, top, n, k, n_expert, bn, grp_tok,
                       grp_tile, src_tok, out_row);
    return sdy_check_launch("moe_sort");
}

extern "C" int sdy_gather_rows(const float *src, const int32_t *idx, int n, int dim, float *dst, sdy_stream s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_gather_rows, dim3((dim + 255) / 256, n), dim3(256), 0, (hipStream_t)s, src, idx, dim, dst);
    return sdy_check_launch("gather_rows");
}

extern "C" int sdy_scatter_axpy(float *dst, const int32_t *idx, const float *w, const float *src, int n, int dim,
                                sdy_stream s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_scatter_axpy, dim3((dim + 255) / 256, n), dim3(256), 0, (hipStream_t)s, dst, idx, w, src, dim);
    return sdy_check_launch("scatter_axpy");
}

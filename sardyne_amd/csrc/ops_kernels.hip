// gfx950 kernels for the float side of the forward pass: RMSNorm, softmax, SiLU·mul, RoPE table
// and rotation, GQA attention (split over positions, deterministic two-pass combine), MoE router
// (softmax + top-k) and the small elementwise ops of the kernel-level ABI.
//
// Numerics follow the reference (csrc/ops.c:456-533, csrc/model_llama.c:653-666) where it matters
// for parity: RMSNorm and softmax sum in double and round the scale once, RoPE angles are computed
// in double, top-k keeps the lower expert index on ties and renormalises with a sequential float
// sum. Reductions use fixed trees, so every result is reproducible run to run.
#include "sdy_device.h"
#include "sdy_internal.h"
#include "sdy_ops.h"
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
// (csrc/ops.c:456-461: sum of squares in double, scale rounded to float once).
__global__ __launch_bounds__(256) void k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w, float *out,
                                                 int n, float eps, long x_stride, long out_stride) {
    __shared__ double sh[4];
    const float *xr = x + blockIdx.x * x_stride;
    float *o = out + blockIdx.x * out_stride;
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) ss += (double)xr[i] * (double)xr[i];
    ss = block_reduce_sum(ss, sh);
    float scale = (float)(1.0 / sqrt(ss / (double)n + (double)eps));
    for (int i = threadIdx.x; i < n; i += 256) {
        float t = xr[i] * scale;
        o[i] = t * w[i];
    }
}

// Per-head RMSNorm of q and k (qwen3 q/k norm), then RoPE, then K and V written into the cache.
// Grid: (n_tok, n_head + n_kv_head), block 64 threads (head_dim <= 512).
__global__ __launch_bounds__(64) void k_qk_rope_kv(float *q, float *k, const float *v, const float *qn, const float *kn,
                                                   float eps, const float *rope_cos, const float *rope_sin, int pos0,
                                                   int n_head, int n_kv_head, int hd, int interleaved, float *k_cache,
                                                   float *v_cache, long head_stride) {
    __shared__ float buf[512];
    __shared__ double shd[1];
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const bool is_q = h < n_head;
    const int hh = is_q ? h : h - n_head;
    float *vec = is_q ? q + ((size_t)t * n_head + hh) * hd : k + ((size_t)t * n_kv_head + hh) * hd;
    const float *nw = is_q ? qn : kn;
    for (int i = lane; i < hd; i += 64) buf[i] = vec[i];
    __syncthreads();
    if (nw) {
        double ss = 0.0;
        for (int i = lane; i < hd; i += 64) ss += (double)buf[i] * (double)buf[i];
        for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
        float scale = (float)(1.0 / sqrt(ss / (double)hd + (double)eps));
        for (int i = lane; i < hd; i += 64) {
            float tt = buf[i] * scale;
            buf[i] = tt * nw[i];
        }
        __syncthreads();
    }
    (void)shd;
    const int half = hd / 2, pos = pos0 + t;
    const float *cs = rope_cos + (size_t)pos * half, *sn = rope_sin + (size_t)pos * half;
    for (int i = lane; i < half; i += 64) {
        int ia = interleaved ? 2 * i : i, ib = interleaved ? 2 * i + 1 : i + half;
        float a = buf[ia], b = buf[ib];
        float ac = a * cs[i], bs = b * sn[i], as = a * sn[i], bc = b * cs[i];
        buf[ia] = ac - bs;
        buf[ib] = as + bc;
    }
    __syncthreads();
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

// ---------------------------------------------------------------------------------- attention
// Pass 1: block (chunk c, kv head g, token t) scores positions [c*CH, min((c+1)*CH, n_kv(t))) for
// the n_rep query heads of g: K/V chunk staged in LDS once, then per head the chunk max, the sum
// of exp, and the exp-weighted sum of V. Pass 2 merges the chunks of each (token, head) in chunk
// order. n_kv(t) = n_kv0 + t (causal mask: token t sees positions 0..pos0+t).
constexpr int ATT_CH = 64;

__global__ __launch_bounds__(256) void k_attn_partial(const float *__restrict__ q, const float *__restrict__ k_cache,
                                                      const float *__restrict__ v_cache, int n_head, int n_kv_head,
                                                      int hd, int n_kv0, long head_stride, long q_stride,
                                                      float *__restrict__ part, int n_chunk_max, float scale) {
    extern __shared__ float sm[];
    const int c = blockIdx.x, g = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
    const int n_kv = n_kv0 + t, p0 = c * ATT_CH;
    if (p0 >= n_kv) return;
    const int np = n_kv - p0 < ATT_CH ? n_kv - p0 : ATT_CH;
    const int n_rep = n_head / n_kv_head, kstride = hd + 1;
    float *ks = sm;                        // [ATT_CH][hd+1]
    float *vs = ks + ATT_CH * kstride;     // [ATT_CH][hd]
    float *qs = vs + ATT_CH * hd;          // [n_rep][hd]
    float *ps = qs + n_rep * hd;           // [n_rep][ATT_CH]
    const float *kg = k_cache + g * head_stride + (size_t)p0 * hd;
    const float *vg = v_cache + g * head_stride + (size_t)p0 * hd;
    for (int i = tid; i < np * hd; i += 256) {
        int p = i / hd, d = i - p * hd;
        ks[p * kstride + d] = kg[i];
        vs[i] = vg[i];
    }
    for (int i = tid; i < n_rep * hd; i += 256) qs[i] = q[(size_t)t * q_stride + (size_t)g * n_rep * hd + i];
    __syncthreads();
    // scores: one (head, position) pair per thread and step
    for (int i = tid; i < n_rep * ATT_CH; i += 256) {
        int r = i / ATT_CH, p = i - r * ATT_CH;
        float s = -INFINITY;
        if (p < np) {
            const float *qq = qs + r * hd, *kk = ks + p * kstride;
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
            int d = 0;
            for (; d + 4 <= hd; d += 4) {
                a0 = fmaf(qq[d], kk[d], a0);
                a1 = fmaf(qq[d + 1], kk[d + 1], a1);
                a2 = fmaf(qq[d + 2], kk[d + 2], a2);
                a3 = fmaf(qq[d + 3], kk[d + 3], a3);
            }
            for (; d < hd; d++) a0 = fmaf(qq[d], kk[d], a0);
            s = ((a0 + a1) + (a2 + a3)) * scale;
        }
        ps[i] = s;
    }
    __syncthreads();
    // per head: chunk max, exp, sum (one wave per head in turn)
    const int wave = tid >> 6, lane = tid & 63;
    for (int r = wave; r < n_rep; r += 4) {
        float m = ps[r * ATT_CH + lane];  // ATT_CH == 64: one position per lane
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        float e = lane < np ? expf(ps[r * ATT_CH + lane] - m) : 0.0f;
        ps[r * ATT_CH + lane] = e;
        float l = e;
        for (int off = 32; off >= 1; off >>= 1) l += __shfl_xor(l, off);
        if (lane == 0) {
            float *pp = part + (((size_t)t * n_head + g * n_rep + r) * n_chunk_max + c) * (hd + 2);
            pp[0] = m;
            pp[1] = l;
        }
    }
    __syncthreads();
    // o[r][d] = sum_p e[r][p] * v[p][d]
    for (int i = tid; i < n_rep * hd; i += 256) {
        int r = i / hd, d = i - r * hd;
        const float *pr = ps + r * ATT_CH;
        float a = 0.0f;
        for (int p = 0; p < np; p++) a = fmaf(pr[p], vs[p * hd + d], a);
        part[(((size_t)t * n_head + g * n_rep + r) * n_chunk_max + c) * (hd + 2) + 2 + d] = a;
    }
}

// Pass 2: one block per (head, token); merges the chunks in order.
__global__ __launch_bounds__(128) void k_attn_combine(const float *__restrict__ part, int n_head, int hd, int n_kv0,
                                                      int n_chunk_max, float *__restrict__ out, long out_stride) {
    const int h = blockIdx.x, t = blockIdx.y;
    const int n_kv = n_kv0 + t, nc = (n_kv + ATT_CH - 1) / ATT_CH;
    const float *pp = part + ((size_t)t * n_head + h) * n_chunk_max * (hd + 2);
    float M = -INFINITY;
    for (int c = 0; c < nc; c++) M = fmaxf(M, pp[c * (hd + 2)]);
    float L = 0.0f;
    for (int c = 0; c < nc; c++) L = L + pp[c * (hd + 2) + 1] * expf(pp[c * (hd + 2)] - M);
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float a = 0.0f;
        for (int c = 0; c < nc; c++) a = fmaf(pp[c * (hd + 2) + 2 + d], expf(pp[c * (hd + 2)] - M), a);
        out[(size_t)t * out_stride + (size_t)h * hd + d] = a / L;
    }
}

// ------------------------------------------------------------------------------ elementwise

// gate = silu(gate) * up   (csrc/ops.c:476-481)
__global__ void k_silu_mul(float *gate, const float *up, long n) {
    long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (i >= n) return;
    float g = gate[i];
    float s = g / (1.0f + expf(-g));
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

// softmax over n values of each row (csrc/ops.c:463-474): max, expf, double sum, float reciprocal
__global__ __launch_bounds__(256) void k_softmax(float *x, int n, long stride) {
    __shared__ float shf[4];
    __shared__ double shd[4];
    float *r = x + blockIdx.x * stride;
    float m = -INFINITY;
    for (int i = threadIdx.x; i < n; i += 256) m = fmaxf(m, r[i]);
    m = block_reduce_max(m, shf);
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) {
        float e = expf(r[i] - m);
        r[i] = e;
        s += (double)e;
    }
    s = block_reduce_sum(s, shd);
    float inv = (float)(1.0 / s);
    for (int i = threadIdx.x; i < n; i += 256) r[i] *= inv;
}

// RoPE tables in double (csrc/ops.c:485-496)
__global__ void k_rope_table(float *cos_out, float *sin_out, int n_pos, int hd, float theta) {
    long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    const int half = hd / 2;
    if (i >= (long)n_pos * half) return;
    int p = (int)(i / half), j = (int)(i - (long)p * half);
    double inv_freq = 1.0 / pow((double)theta, (double)(2 * j) / (double)hd);
    double ang = (double)p * inv_freq;
    cos_out[i] = (float)cos(ang);
    sin_out[i] = (float)sin(ang);
}

// rotate n_heads vectors by one row of the tables (csrc/ops.c:498-511)
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
// csrc/model_llama.c:653-666) and weights renormalised by their sequential float sum.
__global__ __launch_bounds__(64) void k_moe_route(float *probs, int n_expert, int k, int32_t *top, float *wts) {
    const int t = blockIdx.x, lane = threadIdx.x;
    float *p = probs + (size_t)t * n_expert;
    float m = -INFINITY;
    for (int e = lane; e < n_expert; e += 64) m = fmaxf(m, p[e]);
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    double s = 0.0;
    for (int e = lane; e < n_expert; e += 64) {
        float v = expf(p[e] - m);
        p[e] = v;
        s += (double)v;
    }
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
    float inv = (float)(1.0 / s);
    for (int e = lane; e < n_expert; e += 64) p[e] *= inv;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    // top-k
    float chosen_sum = 0.0f;
    int32_t *tt = top + (size_t)t * k;
    uint32_t taken[4] = {0u, 0u, 0u, 0u};  // bitmask of taken experts per lane slot (n_expert <= 256)
    for (int i = 0; i < k; i++) {
        float best = -1.0f;
        int bi = 0x7fffffff;
        for (int e = lane, slot = 0; e < n_expert; e += 64, slot++) {
            if (taken[slot >> 5] >> (slot & 31) & 1u) continue;
            float v = p[e];
            if (v > best || (v == best && e < bi)) {
                best = v;
                bi = e;
            }
        }
        for (int off = 32; off >= 1; off >>= 1) {
            float ob = __shfl_xor(best, off);
            int oi = __shfl_xor(bi, off);
            if (ob > best || (ob == best && oi < bi)) {
                best = ob;
                bi = oi;
            }
        }
        if ((bi & 63) == lane) {
            int slot = bi >> 6;
            taken[slot >> 5] |= 1u << (slot & 31);
        }
        if (lane == 0) tt[i] = bi;
        chosen_sum = chosen_sum + best;
    }
    if (lane < k) {
        int e = tt[lane];
        wts[(size_t)t * k + lane] = p[e] / chosen_sum;
    }
}

// out[t] = sum over the k chosen experts, in ascending expert id, of w * y   (moe_ffn's axpy order
// over experts, csrc/model_llama.c:734-750). y is [n_tok][k][dim] in top-k slot order.
__global__ void k_moe_combine(const float *y, const int32_t *top, const float *wts, int k, int dim, float *out,
                              const float *resid) {
    const int t = blockIdx.y;
    int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= dim) return;
    const int32_t *tt = top + (size_t)t * k;
    float acc = 0.0f;
    int last = -1;
    for (int i = 0; i < k; i++) {  // visit slots in ascending expert id
        int best = -1, bid = 0x7fffffff;
        for (int j = 0; j < k; j++)
            if (tt[j] > last && tt[j] < bid) {
                bid = tt[j];
                best = j;
            }
        last = bid;
        acc = fmaf(wts[(size_t)t * k + best], y[((size_t)t * k + best) * dim + d], acc);
    }
    out[(size_t)t * dim + d] = resid ? resid[(size_t)t * dim + d] + acc : acc;
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
        *o = fmaf(w[r], src[(size_t)r * dim + d], *o);
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

extern "C" int sdy_qk_rope_kv(float *q, float *k, const float *v, const float *qn, const float *kn, float eps,
                              const float *rope_cos, const float *rope_sin, int pos0, int n_tok, int n_head,
                              int n_kv_head, int hd, int interleaved, float *k_cache, float *v_cache,
                              long head_stride, sdy_stream s) {
    if (hd > 512) return sdy_fail(-1, "head_dim %d above 512", hd);
    hipLaunchKernelGGL(k_qk_rope_kv, dim3(n_tok, n_head + n_kv_head), dim3(64), 0, (hipStream_t)s, q, k, v, qn, kn, eps,
                       rope_cos, rope_sin, pos0, n_head, n_kv_head, hd, interleaved, k_cache, v_cache, head_stride);
    return sdy_check_launch("qk_rope_kv");
}

extern "C" size_t sdy_attn_part_floats(int n_tok, int n_head, int hd, int max_kv) {
    int nc = (max_kv + ATT_CH - 1) / ATT_CH;
    return (size_t)n_tok * n_head * nc * (hd + 2);
}

extern "C" int sdy_attention(const float *q, const float *k_cache, const float *v_cache, int n_tok, int n_head,
                             int n_kv_head, int hd, int n_kv0, long head_stride, long q_stride, float *part,
                             float *out, long out_stride, sdy_stream s) {
    hipStream_t st = (hipStream_t)s;
    if (n_tok <= 0) return 0;
    const int n_rep = n_head / n_kv_head;
    const int n_kv_max = n_kv0 + n_tok - 1;
    const int nc = (n_kv_max + ATT_CH - 1) / ATT_CH;
    size_t lds = sizeof(float) * ((size_t)ATT_CH * (hd + 1) + (size_t)ATT_CH * hd + (size_t)n_rep * hd +
                                  (size_t)n_rep * ATT_CH);
    if (lds > 160 * 1024) return sdy_fail(-1, "attention: %zu bytes of LDS (head_dim %d, %d heads per KV head)", lds, hd, n_rep);
    static int attr_set = 0;
    if (lds > 64 * 1024 && !attr_set) {
        (void)hipFuncSetAttribute((const void *)k_attn_partial, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        attr_set = 1;
    }
    float scale = 1.0f / sqrtf((float)hd);
    hipLaunchKernelGGL(k_attn_partial, dim3(nc, n_kv_head, n_tok), dim3(256), lds, st, q, k_cache, v_cache, n_head,
                       n_kv_head, hd, n_kv0, head_stride, q_stride, part, nc, scale);
    int rc = sdy_check_launch("attention");
    if (rc) return rc;
    hipLaunchKernelGGL(k_attn_combine, dim3(n_head, n_tok), dim3(128), 0, st, part, n_head, hd, n_kv0, nc, out, out_stride);
    return sdy_check_launch("attention_combine");
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

extern "C" int sdy_rope_table(float *cos_out, float *sin_out, int n_pos, int hd, float theta, sdy_stream s) {
    long n = (long)n_pos * (hd / 2);
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_rope_table, GRID1(n, 256), dim3(256), 0, (hipStream_t)s, cos_out, sin_out, n_pos, hd, theta);
    return sdy_check_launch("rope_table");
}

extern "C" int sdy_rope(float *x, int n_heads, int hd, const float *cs, const float *sn, int interleaved, sdy_stream s) {
    long n = (long)n_heads * (hd / 2);
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_rope, GRID1(n, 256), dim3(256), 0, (hipStream_t)s, x, n_heads, hd, cs, sn, interleaved);
    return sdy_check_launch("rope");
}

extern "C" int sdy_moe_route(float *probs, int n_tok, int n_expert, int k, int32_t *top, float *wts, sdy_stream s) {
    if (n_expert > 8192) return sdy_fail(-1, "n_expert %d above 8192", n_expert);
    if (k > 64) return sdy_fail(-1, "n_expert_used %d above 64", k);
    hipLaunchKernelGGL(k_moe_route, dim3(n_tok), dim3(64), 0, (hipStream_t)s, probs, n_expert, k, top, wts);
    return sdy_check_launch("moe_route");
}

extern "C" int sdy_moe_combine(const float *y, const int32_t *top, const float *wts, int n_tok, int k, int dim,
                               float *out, const float *resid, sdy_stream s) {
    hipLaunchKernelGGL(k_moe_combine, dim3((dim + 255) / 256, n_tok), dim3(256), 0, (hipStream_t)s, y, top, wts, k, dim,
                       out, resid);
    return sdy_check_launch("moe_combine");
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

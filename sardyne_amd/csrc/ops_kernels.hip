// gfx950 kernels for the float side of the forward pass: RMSNorm, softmax, SiLU·mul, RoPE table
// and rotation, MoE router (softmax + top-k) and the small elementwise ops of the kernel-level ABI
// (attention: attn_kernels.hip).
//
// Numerics follow the reference (csrc/ops.c:456-533, csrc/model_llama.c:653-666) where it matters
// for parity: RMSNorm and softmax sum in double and round the scale once, RoPE angles are computed
// in double, top-k keeps the lower expert index on ties and renormalises with a sequential float
// sum. Reductions use fixed trees, so every result is reproducible run to run.
#include "sdy_device.h"
#include "sdy_internal.h"
#include "sdy_norm_dev.h"
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

// One step of the reference's AVX2 axpy (csrc/ops_avx2.c:142-147) at element d of a dim-element
// row: fused in the 8-lane body, a rounded product then a sum in the tail.
SDY_DEV float axpy1(float acc, float w, float y, int d, int dim) {
    return d < (dim & ~7) ? fmaf(w, y, acc) : acc + w * y;
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
        acc = axpy1(acc, wts[(size_t)t * k + best], y[((size_t)t * k + best) * dim + d], d, dim);
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

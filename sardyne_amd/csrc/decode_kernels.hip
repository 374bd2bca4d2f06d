// RMSNorm fused with the activation quantiser of the next matvec: k_norm_quant writes the bytes of
// k_rmsnorm followed by k_quant_q8k / k_quant_q8_0 (same sum order, same wave quantisers) in one
// launch. (The fused decode attention is in attn_kernels.hip.)
#include "sdy_device.h"
#include "sdy_internal.h"
#include "sdy_norm_dev.h"
#include "sdy_ops.h"
#include "sdy_quant_dev.h"
#include "sdy_shim.h"

namespace {

// VT = SDY_Q8_K, SDY_Q8_0 or SDY_F32 (normalise only). xb (f32 result) may be null for the
// quantising variants; with e.y16 set, Q8_K also writes the GEMM's expansion of its blocks. Grid: one 256-thread block per row. For Q8_K rows of up to 4096 elements
// the row is read once: the float4 chunks of the sum of squares are the elements each lane
// quantises (superblock wave + 4k, elements 4 lane .. 4 lane + 3).
template <int VT>
__global__ __launch_bounds__(256) void k_norm_quant(const float *__restrict__ x, const float *__restrict__ w,
                                                    float eps, int n, float *__restrict__ xb,
                                                    uint8_t *__restrict__ xq, SdyGemmExp e) {
    constexpr int NREG = 4;
    __shared__ double sh[4];
    const int t = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const float *xr = x + (size_t)t * n;
    float4 keep[NREG];
    // the norm weights of the lane's first NREG super-blocks, requested before the row's reduction
    float4 wk[NREG];
    if constexpr (VT == SDY_Q8_K) {
        const int nb = n / 256;
#pragma unroll
        for (int k = 0; k < NREG; k++) {
            const int s = wave + 4 * k < nb ? wave + 4 * k : nb - 1;
            wk[k] = s >= 0 ? *reinterpret_cast<const float4 *>(w + 256 * s + 4 * lane) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    const double ss = sdy_row_sumsq<VT == SDY_Q8_K ? NREG : 0>(xr, n, keep, sh);
    const float scale = (float)(1.0 / sqrt(ss / (double)n + (double)eps));
    if constexpr (VT == SDY_Q8_K) {
        const int nb = n / 256;
        const bool in_regs = sdy_rows_vec4(xr, n);
        auto values = [&](int s, const float4 &v, const float4 &wv) {
            float4 o;
            o.x = (v.x * scale) * wv.x;
            o.y = (v.y * scale) * wv.y;
            o.z = (v.z * scale) * wv.z;
            o.w = (v.w * scale) * wv.w;
            return o;
        };
        auto store_xb = [&](int s, const float *v4) {
            if (xb) *reinterpret_cast<float4 *>(xb + (size_t)t * n + 256 * s + 4 * lane) = make_float4(v4[0], v4[1], v4[2], v4[3]);
        };
        auto from_mem = [&](int s) {
            const int e0 = 256 * s + 4 * lane;
            return make_float4(xr[e0], xr[e0 + 1], xr[e0 + 2], xr[e0 + 3]);
        };
        // the first NREG super-blocks of the wave (wave + 4k) quantised together: their
        // cross-lane reductions overlap
        float xs[NREG][4];
#pragma unroll
        for (int k = 0; k < NREG; k++) {
            const int s = wave + 4 * k < nb ? wave + 4 * k : nb - 1;
            const float4 o = values(s, in_regs ? keep[k] : from_mem(s), wk[k]);
            xs[k][0] = o.x;
            xs[k][1] = o.y;
            xs[k][2] = o.z;
            xs[k][3] = o.w;
        }
        SdyQ8kLane r[NREG];
        sdy_q8k_lanes<NREG>(xs, lane, r);
#pragma unroll
        for (int k = 0; k < NREG; k++)
            if (wave + 4 * k < nb) {  // (slots past the row repeat its last super-block: skipped)
                store_xb(wave + 4 * k, xs[k]);
                uint8_t *ob = xq + ((size_t)t * nb + wave + 4 * k) * 292;
                *reinterpret_cast<uint32_t *>(ob + 4 + 4 * lane) = r[k].packed;
                if ((lane & 3) == 0) *reinterpret_cast<int16_t *>(ob + 260 + 2 * (lane >> 2)) = (int16_t)r[k].gsum;
                if (lane == 0) *reinterpret_cast<float *>(ob) = r[k].d;
                if (e.y16) e.put(r[k], lane, (size_t)t * nb + wave + 4 * k);
            }
        for (int s = wave + 4 * NREG; s < nb; s += 4) {
            const float4 o = values(s, from_mem(s), *reinterpret_cast<const float4 *>(w + 256 * s + 4 * lane));
            const float x1[4] = {o.x, o.y, o.z, o.w};
            store_xb(s, x1);
            const SdyQ8kLane r1 = sdy_q8k_lane(x1, lane);
            uint8_t *ob = xq + ((size_t)t * nb + s) * 292;
            *reinterpret_cast<uint32_t *>(ob + 4 + 4 * lane) = r1.packed;
            if ((lane & 3) == 0) *reinterpret_cast<int16_t *>(ob + 260 + 2 * (lane >> 2)) = (int16_t)r1.gsum;
            if (lane == 0) *reinterpret_cast<float *>(ob) = r1.d;
            if (e.y16) e.put(r1, lane, (size_t)t * nb + s);
        }
    } else if constexpr (VT == SDY_Q8_0) {
        const int nblk = n / 32, l = lane & 31;
        for (int b = 2 * wave + (lane >> 5); b < nblk; b += 8) {  // uniform per half-wave
            const float tt = xr[32 * b + l] * scale;
            const float v = tt * w[32 * b + l];
            if (xb) xb[(size_t)t * n + 32 * b + l] = v;
            sdy_q8_0_block(v, l, xq + ((size_t)t * nblk + b) * 34);
        }
    } else {
        for (int i = tid; i < n; i += 256) {
            const float tt = xr[i] * scale;
            xb[(size_t)t * n + i] = tt * w[i];
        }
    }
}

}  // namespace

// =============================================================================== launchers

extern "C" int sdy_norm_quant(const float *x, const float *w, float eps, int n, int n_rows, float *xb, int vtype,
                              void *xq, sdy_stream s) {
    hipStream_t st = (hipStream_t)s;
    if (n_rows <= 0) return 0;
    uint8_t *q = (uint8_t *)xq;
    switch (vtype) {
    case SDY_Q8_K:
        if (n % 256) return sdy_fail(-1, "norm_quant: Q8_K rows must be a multiple of 256 (got %d)", n);
        hipLaunchKernelGGL(k_norm_quant<SDY_Q8_K>, dim3(n_rows), dim3(256), 0, st, x, w, eps, n, xb, q, SdyGemmExp{});
        break;
    case SDY_Q8_0:
        if (n % 32) return sdy_fail(-1, "norm_quant: Q8_0 rows must be a multiple of 32 (got %d)", n);
        hipLaunchKernelGGL(k_norm_quant<SDY_Q8_0>, dim3(n_rows), dim3(256), 0, st, x, w, eps, n, xb, q, SdyGemmExp{});
        break;
    case SDY_F32:
        if (!xb) return sdy_fail(-1, "norm_quant: no output");
        hipLaunchKernelGGL(k_norm_quant<SDY_F32>, dim3(n_rows), dim3(256), 0, st, x, w, eps, n, xb, q, SdyGemmExp{});
        break;
    default: return sdy_fail(-1, "norm_quant: activation type %d", vtype);
    }
    return sdy_check_launch("norm_quant");
}

// sdy_norm_quant to Q8_K plus the GEMM's expansion of the rows in ws (the layout sdy_gemm reads)
extern "C" int sdy_norm_quant_gemm(const float *x, const float *w, float eps, int n, int n_rows, float *xb, void *xq,
                                   void *ws, sdy_stream s) {
    if (n_rows <= 0) return 0;
    if (n % 256) return sdy_fail(-1, "norm_quant: Q8_K rows must be a multiple of 256 (got %d)", n);
    hipLaunchKernelGGL(k_norm_quant<SDY_Q8_K>, dim3(n_rows), dim3(256), 0, (hipStream_t)s, x, w, eps, n, xb,
                       (uint8_t *)xq, sdy_gemm_exp(ws, n_rows, n));
    return sdy_check_launch("norm_quant");
}


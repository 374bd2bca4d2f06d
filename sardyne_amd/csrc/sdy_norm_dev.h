// Sum of squares of a row as every RMSNorm kernel computes it (csrc/ops.c:346-351 sums in double):
// thread t of a 256-thread block adds, in order, the squares of its float4 chunks t, t + 256, ...
// (its scalar elements t, t + 256, ... when the row is not a whole number of aligned float4s), then
// the fixed block tree. Sharing the order keeps the fused and unfused kernels bit-identical.
#pragma once
#include "sdy_device.h"

SDY_DEV double sdy_block_sum256(double v, double *sh) {
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    const double r = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    __syncthreads();
    return r;
}

SDY_DEV bool sdy_rows_vec4(const float *xr, int n) {
    return (n & 3) == 0 && (reinterpret_cast<uintptr_t>(xr) & 15) == 0;
}

// The chunks of the first NREG rounds are kept in keep[] for the caller (vec4 rows only).
template <int NREG>
SDY_DEV double sdy_row_sumsq(const float *xr, int n, float4 *keep, double *sh) {
    const int tid = threadIdx.x;
    double ss = 0.0;
    if (sdy_rows_vec4(xr, n)) {
        const float4 *x4 = reinterpret_cast<const float4 *>(xr);
        const int n4 = n / 4;
        auto add = [&](const float4 &v) {
            ss += (double)v.x * (double)v.x;
            ss += (double)v.y * (double)v.y;
            ss += (double)v.z * (double)v.z;
            ss += (double)v.w * (double)v.w;
        };
        // all loads first (clamped indices, so none is conditional), then the adds in order
#pragma unroll
        for (int k = 0; k < NREG; k++) {
            const int i = tid + 256 * k;
            keep[k] = x4[i < n4 ? i : n4 - 1];
        }
#pragma unroll
        for (int k = 0; k < NREG; k++)
            if (tid + 256 * k < n4) add(keep[k]);
        for (int i = tid + 256 * NREG; i < n4; i += 256) add(x4[i]);
    } else {
        for (int i = tid; i < n; i += 256) ss += (double)xr[i] * (double)xr[i];
    }
    return sdy_block_sum256(ss, sh);
}

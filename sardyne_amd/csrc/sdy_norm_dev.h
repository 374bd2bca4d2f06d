// Sum of squares of a row as every RMSNorm kernel computes it (csrc/ops.c:346-351 sums in double):
// thread t of a 256-thread block adds, in order, the squares of its float4 chunks t, t + 256, ...
// (its scalar elements t, t + 256, ... when the row is not a whole number of aligned float4s), then
// the fixed block tree. Sharing the order keeps the fused and unfused kernels bit-identical.
#pragma once
#include "sdy_device.h"

// lane l's double from the DPP source of control CTRL within its row of 16 lanes (both words)
template <int CTRL>
SDY_DEV double sdy_dpp_f64(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)b, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// The wave's sum by the butterfly over lane ^ 32, 16, 8, 4, 2, 1 (each lane adds its partner's
// value; every lane ends with the same sum): the last four steps by DPP (row_ror 8; row_shl or
// row_shr 4 by the lane's bit 2; quad perms), the same pairs in the same order as __shfl_xor.
SDY_DEV double sdy_wave_sum_f64(double v) {
    const int lane = threadIdx.x & 63;
    v += __shfl_xor(v, 32);
    v += __shfl_xor(v, 16);
    v += sdy_dpp_f64<0x128>(v);
    const double up = sdy_dpp_f64<0x104>(v), down = sdy_dpp_f64<0x114>(v);
    v += (lane & 4) ? down : up;
    v += sdy_dpp_f64<0x4E>(v);
    v += sdy_dpp_f64<0xB1>(v);
    return v;
}

SDY_DEV double sdy_block_sum256(double v, double *sh) {
    v = sdy_wave_sum_f64(v);
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

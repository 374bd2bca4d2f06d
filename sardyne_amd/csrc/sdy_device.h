// Device-side helpers shared by the gfx950 kernels: f16 conversions with the reference's exact
// semantics, packed int8 dots, quad reductions and wavefront-level LDS ordering.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SDY_DEV __device__ __forceinline__

// f16 -> f32, exact for every value (subnormals included; the kernels are built with f16
// denormals enabled, which is gfx950's default mode).
SDY_DEV float sdy_h2f(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

// f32 -> f16 with the reference's rules (csrc/ops.c:43-62): round to nearest even, values at or
// above 65520 become infinity, NaN becomes a quiet NaN with its sign. Integer arithmetic only, so
// the result does not depend on the hardware rounding or denormal modes.
SDY_DEV uint16_t sdy_f2h(float f) {
    uint32_t x = __float_as_uint(f);
    uint32_t sign = (x >> 16) & 0x8000u, a = x & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (a < 0x38800000u) {  // result is a subnormal half (or zero): quantum 2^-24
        int e = (int)(a >> 23);
        if (e < 102) return (uint16_t)sign;  // below 2^-25: rounds to zero
        uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
        int shift = 126 - e;  // value = mant * 2^(e-150); in units of 2^-24: mant >> (126 - e)
        uint32_t q = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = ((a >> 23) - 112u) << 10 | ((a >> 13) & 0x3FFu);
    uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

// Σ of four int8 products plus acc (v_dot4c_i32_i8): exact.
SDY_DEV int sdy_dot4(int a, int b, int acc) { return __builtin_amdgcn_sdot4(a, b, acc, false); }

// The maximum of a 32-bit unsigned value over the wave, in every lane (all lanes active): DPP
// within rows of 16 lanes (quad perms, row rotations), then the four rows' maxima by readlane.
SDY_DEV uint32_t wave_max_u32(uint32_t v) {
    uint32_t o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
    v = o > v ? o : v;
    o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);  // quad_perm [2, 3, 0, 1]
    v = o > v ? o : v;
    o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xF, 0xF, false);  // row_ror 4
    v = o > v ? o : v;
    o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false);  // row_ror 8
    v = o > v ? o : v;
    uint32_t r = 0;
#pragma unroll
    for (int row = 0; row < 4; row++) {
        const uint32_t x = (uint32_t)__builtin_amdgcn_readlane((int)v, 16 * row);
        r = x > r ? x : r;
    }
    return r;
}

// Sum over the 4 lanes of a quad (lanes 4k..4k+3), result in every lane of the quad: exact for ints.
SDY_DEV int sdy_quad_sum(int v) {
    v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    return v;
}

// Orders this wavefront's LDS writes before its later LDS reads by other lanes of the same wave.
SDY_DEV void sdy_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Bit-exact round-half-even of the reference's nearest_int (csrc/quant.c:111-116), including its
// behaviour on non-finite inputs.
SDY_DEV int sdy_nearest_int(float v) {
    float f = v + 12582912.0f;
    return (int)(__float_as_uint(f) & 0x007FFFFFu) - 0x00400000;
}

// Spread the 4 low bits of v to bit 4 of each byte (Q5_0 fifth bits).
SDY_DEV uint32_t sdy_spread4(uint32_t v) { return ((v & 15u) * 0x00204081u & 0x01010101u) << 4; }

// Wave-level activation quantisers shared by the standalone quantiser kernels and the fused
// decode kernels, so that every producer of a Q8_K / Q8_0 row writes the same bytes.
#pragma once
#include "sdy_device.h"
#include "sdy_expf.h"

// One 256-element Q8_K block (csrc/quant.c:118-144) held by a wave64, lane l holding elements
// 4l..4l+3 in xs. The signed maximum is the first element of largest magnitude (strict '>' in
// index order); iscale = -127/max; q = min(127, nearest_int(iscale*x)) with the reference's
// round-half-even; d = 1/iscale; bsums[g] = sum of the 16 quants of group g. An all-zero block is
// all zero bytes. Result per lane: its 4 quants packed, the sum of its group (lanes 4g..4g+3 all
// hold bsums[g]) and d.
struct SdyQ8kLane {
    uint32_t packed;
    int gsum;
    float d;
};

// NB blocks at once (each the same result as one block alone). The signed maximum: the magnitude is
// reduced over the wave in any order (a maximum is order-free), then the first lane holding it (a
// ballot) and that lane's first element of that magnitude give the element: the first one in index
// order, as the reference's strict '>' picks. NaN never wins (fmaxf drops it within the lane, and a
// lane whose four elements are all NaN enters the wave maximum as 0); a block with no finite nonzero
// element is all zero bytes, as in the reference. The wave maximum runs on the magnitudes' bits
// (non-negative floats order as their bits) through DPP and readlane, and the element is read with
// readlane from the uniform first holder: no LDS permutes. With NB > 1 the blocks' two divisions
// (-127/max and 1/iscale, correctly rounded) run once for all blocks, block b's operand in lane b.
template <int NB>
SDY_DEV void sdy_q8k_lanes(const float (&xs)[NB][4], int lane, SdyQ8kLane (&r)[NB]) {
    float lm[NB], bval[NB];
    uint32_t mb[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        lm[b] = fmaxf(fmaxf(fabsf(xs[b][0]), fabsf(xs[b][1])), fmaxf(fabsf(xs[b][2]), fabsf(xs[b][3])));
        const uint32_t u = __float_as_uint(lm[b]);
        mb[b] = u > 0x7F800000u ? 0u : u;
    }
#pragma unroll
    for (int b = 0; b < NB; b++) mb[b] = wave_max_u32(mb[b]);
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const float amax = __uint_as_float(mb[b]);
        const unsigned long long holders = __ballot(lm[b] == amax);
        const int first = holders ? __builtin_ctzll(holders) : 0;
        const float mine = fabsf(xs[b][0]) == amax   ? xs[b][0]
                           : fabsf(xs[b][1]) == amax ? xs[b][1]
                           : fabsf(xs[b][2]) == amax ? xs[b][2]
                                                     : xs[b][3];
        bval[b] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), first));
    }
    float iscale[NB], dinv[NB];
    if constexpr (NB == 1) {
        iscale[0] = -127.0f / bval[0];
        dinv[0] = 1.0f / iscale[0];
    } else {
        float bv = bval[0];
#pragma unroll
        for (int b = 1; b < NB; b++) bv = lane == b ? bval[b] : bv;
        const float is = -127.0f / bv;
        const float dv = 1.0f / is;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            iscale[b] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, is), b));
            dinv[b] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, dv), b));
        }
    }
    int lsum[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        lsum[b] = 0;
        r[b].packed = 0u;
        r[b].d = 0.0f;
        if (mb[b] > 0u) {
            uint32_t packed = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                int q = sdy_nearest_int(iscale[b] * xs[b][e]);
                q = q < 127 ? q : 127;
                lsum[b] += (int8_t)q;
                packed |= (uint32_t)(uint8_t)(int8_t)q << (8 * e);
            }
            r[b].packed = packed;
            r[b].d = dinv[b];
        }
    }
#pragma unroll
    for (int b = 0; b < NB; b++) r[b].gsum = sdy_quad_sum(lsum[b]);
}

SDY_DEV SdyQ8kLane sdy_q8k_lane(const float xs[4], int lane) {
    float x1[1][4] = {{xs[0], xs[1], xs[2], xs[3]}};
    SdyQ8kLane r[1];
    sdy_q8k_lanes<1>(x1, lane, r);
    return r[0];
}

// The block in the reference layout (292 bytes at ob: f32 d, int8 qs[256], int16 bsums[16]).
// The prefill GEMM's f16 expansion of a Q8_K row (the workspace of sdy_gemm; y16 null: none).
struct SdyGemmExp {
    _Float16 *y16;  // [super-block][256] the int8 values
    float *yd;      // [super-block] the scales
    _Float16 *bs16; // [super-block][16] the 16-element sums
    // super-block sbg (of the row-major sequence) from the lane's quantiser result: the bits
    // k_gemm_prep makes of the block's bytes (|q| <= 127 and |bsum| <= 2032 are exact in f16)
    SDY_DEV void put(const SdyQ8kLane &r, int lane, size_t sbg) const {
        typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
        f16x4 o;
#pragma unroll
        for (int e = 0; e < 4; e++) o[e] = (_Float16)(float)(int8_t)((r.packed >> (8 * e)) & 255u);
        *reinterpret_cast<f16x4 *>(y16 + sbg * 256 + 4 * lane) = o;
        if ((lane & 3) == 0) bs16[sbg * 16 + (lane >> 2)] = (_Float16)(float)(int16_t)r.gsum;
        if (lane == 0) yd[sbg] = r.d;
    }
};

// sdy_gemm's workspace for n_tok rows of n_in: y16, then yd, then bs16, each 256-byte aligned
inline SdyGemmExp sdy_gemm_exp(void *ws, int n_tok, int n_in) {
    uint8_t *w = (uint8_t *)ws;
    SdyGemmExp e;
    e.y16 = (_Float16 *)w;
    w += ((size_t)n_tok * n_in * 2 + 255) & ~(size_t)255;
    e.yd = (float *)w;
    w += ((size_t)n_tok * (n_in / 256) * 4 + 255) & ~(size_t)255;
    e.bs16 = (_Float16 *)w;
    return e;
}

SDY_DEV void sdy_q8k_block(const float xs[4], int lane, uint8_t *ob) {
    const SdyQ8kLane r = sdy_q8k_lane(xs, lane);
    *reinterpret_cast<uint32_t *>(ob + 4 + 4 * lane) = r.packed;
    if ((lane & 3) == 0) *reinterpret_cast<int16_t *>(ob + 260 + 2 * (lane >> 2)) = (int16_t)r.gsum;
    if (lane == 0) *reinterpret_cast<float *>(ob) = r.d;
}

// One 32-element Q8_0 block (csrc/quant.c:98-108) held by a half-wave, one element per lane l
// (0..31 within the half): d = amax/127 stored as f16, q = roundf(x/d) computed with the unrounded
// reciprocal. The maximum starts from 0 in every lane, as the reference's does, so that NaN never
// enters it (a block of NaN has d = 0). ob points at the 34-byte block.
SDY_DEV void sdy_q8_0_block(float xv, int l, uint8_t *ob) {
    float amax = fmaxf(0.0f, fabsf(xv));
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    ob[2 + l] = (uint8_t)(int8_t)roundf(xv * id);
    if (l == 0) {
        const uint16_t h = sdy_f2h(d);
        ob[0] = (uint8_t)(h & 255);
        ob[1] = (uint8_t)(h >> 8);
    }
}

// SiLU(g) * u as the reference computes it (csrc/ops.c:366-371), with the host libm's expf.
SDY_DEV float sdy_silu_mul1(float g, float u) {
    const float s = g / (1.0f + sdy_expf(-g));
    return s * u;
}

// sdy_silu_mul1 with the exponential's table in a register (sdy_expf_reg; all lanes active)
SDY_DEV float sdy_silu_mul1_reg(float g, float u, uint32_t tab) {
    const float s = g / (1.0f + sdy_expf_reg(-g, tab));
    return s * u;
}

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

SDY_DEV SdyQ8kLane sdy_q8k_lane(const float xs[4], int lane) {
    float best = 0.0f, bval = 0.0f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (fabsf(xs[e]) > best) {
            best = fabsf(xs[e]);
            bval = xs[e];
            bi = 4 * lane + e;
        }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        float ob_ = __shfl_xor(best, off), ov = __shfl_xor(bval, off);
        int oi = __shfl_xor(bi, off);
        if (ob_ > best || (ob_ == best && oi < bi)) {
            best = ob_;
            bval = ov;
            bi = oi;
        }
    }
    SdyQ8kLane r;
    if (best == 0.0f) {
        r.packed = 0u;
        r.gsum = 0;
        r.d = 0.0f;
        return r;
    }
    const float iscale = -127.0f / bval;
    uint32_t packed = 0;
    int lsum = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        int q = sdy_nearest_int(iscale * xs[e]);
        q = q < 127 ? q : 127;
        lsum += (int8_t)q;
        packed |= (uint32_t)(uint8_t)(int8_t)q << (8 * e);
    }
    r.packed = packed;
    r.gsum = sdy_quad_sum(lsum);
    r.d = 1.0f / iscale;
    return r;
}

// NB blocks at once (the same result per block as sdy_q8k_lane); their cross-lane reductions are
// interleaved so that the latencies overlap.
template <int NB>
SDY_DEV void sdy_q8k_lanes(const float (&xs)[NB][4], int lane, SdyQ8kLane (&r)[NB]) {
    float best[NB], bval[NB];
    int bi[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        best[b] = 0.0f;
        bval[b] = 0.0f;
        bi[b] = 0x7fffffff;
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (fabsf(xs[b][e]) > best[b]) {
                best[b] = fabsf(xs[b][e]);
                bval[b] = xs[b][e];
                bi[b] = 4 * lane + e;
            }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        float ob_[NB], ov[NB];
        int oi[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            ob_[b] = __shfl_xor(best[b], off);
            ov[b] = __shfl_xor(bval[b], off);
            oi[b] = __shfl_xor(bi[b], off);
        }
#pragma unroll
        for (int b = 0; b < NB; b++)
            if (ob_[b] > best[b] || (ob_[b] == best[b] && oi[b] < bi[b])) {
                best[b] = ob_[b];
                bval[b] = ov[b];
                bi[b] = oi[b];
            }
    }
    int lsum[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        lsum[b] = 0;
        r[b].packed = 0u;
        r[b].d = 0.0f;
        if (best[b] != 0.0f) {
            const float iscale = -127.0f / bval[b];
            uint32_t packed = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                int q = sdy_nearest_int(iscale * xs[b][e]);
                q = q < 127 ? q : 127;
                lsum[b] += (int8_t)q;
                packed |= (uint32_t)(uint8_t)(int8_t)q << (8 * e);
            }
            r[b].packed = packed;
            r[b].d = 1.0f / iscale;
        }
    }
#pragma unroll
    for (int b = 0; b < NB; b++) r[b].gsum = sdy_quad_sum(lsum[b]);
}

// The block in the reference layout (292 bytes at ob: f32 d, int8 qs[256], int16 bsums[16]).
SDY_DEV void sdy_q8k_block(const float xs[4], int lane, uint8_t *ob) {
    const SdyQ8kLane r = sdy_q8k_lane(xs, lane);
    *reinterpret_cast<uint32_t *>(ob + 4 + 4 * lane) = r.packed;
    if ((lane & 3) == 0) *reinterpret_cast<int16_t *>(ob + 260 + 2 * (lane >> 2)) = (int16_t)r.gsum;
    if (lane == 0) *reinterpret_cast<float *>(ob) = r.d;
}

// One 32-element Q8_0 block (csrc/quant.c:98-108) held by a half-wave, one element per lane l
// (0..31 within the half): d = amax/127 stored as f16, q = roundf(x/d) computed with the unrounded
// reciprocal. ob points at the 34-byte block.
SDY_DEV void sdy_q8_0_block(float xv, int l, uint8_t *ob) {
    float amax = fabsf(xv);
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

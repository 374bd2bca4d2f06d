// Merge of split attention (chunks of 64 positions), shared by the attention kernels and the
// matvec prologue that rebuilds the attention output for the output projection, so that every
// consumer computes the same bits. A chunk c of a (token, head) holds m_c (score maximum), l_c
// (sum of exp(score - m_c)) and o_c (exp-weighted sum of V).
#pragma once
#include "sdy_device.h"

// Merge weights of one (token, head), computed by one wave: M = max m_c, e_c = exp(m_c - M) into
// e[0..nc) (LDS), and L = sum over c in order of l_c * e_c (products in parallel, the sum in chunk
// order from LDS, so the value is that of a sequential loop). pe: LDS scratch of nc floats.
SDY_DEV float merge_weights_wave(const float *ml, int nc, float *e, float *pe, int lane) {
    float M = -INFINITY;
    for (int c = lane; c < nc; c += 64) M = fmaxf(M, ml[2 * c]);
    for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
    for (int c = lane; c < nc; c += 64) {
        const float ec = expf(ml[2 * c] - M);
        e[c] = ec;
        pe[c] = ml[2 * c + 1] * ec;
    }
    sdy_wave_sync();
    // L in chunk order: lane 0 reads the products 4 at a time (reads ahead of the adds)
    float L = 0.0f;
    if (lane == 0) {
        int c = 0;
        for (; c + 4 <= nc; c += 4) {
            const float p0 = pe[c], p1 = pe[c + 1], p2 = pe[c + 2], p3 = pe[c + 3];
            L = L + p0;
            L = L + p1;
            L = L + p2;
            L = L + p3;
        }
        for (; c < nc; c++) L = L + pe[c];
    }
    return __shfl(L, 0);
}

// out[d..d+3] of one (token, head) = (sum over chunks in order of o_c * e_c) / L
// (loads in groups of 8 chunks issued before their FMAs, clamped so that none is conditional)
SDY_DEV float4 merge4(const float *o, int nc_max, int nc, int hd, int d, const float *e, float L) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    (void)nc_max;
    for (int c0 = 0; c0 < nc; c0 += 8) {
        float4 v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int c = c0 + j < nc ? c0 + j : nc - 1;
            v[j] = *reinterpret_cast<const float4 *>(o + (size_t)c * hd + d);
        }
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (c0 + j < nc) {
                const float w = e[c0 + j];
                acc.x = fmaf(v[j].x, w, acc.x);
                acc.y = fmaf(v[j].y, w, acc.y);
                acc.z = fmaf(v[j].z, w, acc.z);
                acc.w = fmaf(v[j].w, w, acc.w);
            }
    }
    return make_float4(acc.x / L, acc.y / L, acc.z / L, acc.w / L);
}


// The MoE router's softmax and top-k for one token on one wave, shared by the route kernel and the
// routed-expert matvec that selects its own expert.
#pragma once
#include "sdy_device.h"
#include "sdy_expf.h"
#include "sdy_norm_dev.h"

// The maximum of a float over the wave, in every lane (wave_max_u32's DPP and readlane pattern)
SDY_DEV float wave_max_f32(float v) {
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false)));
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Softmax over the n_expert logits p (n_expert <= 64 * NPL) and the top k (k <= 64) of one token,
// every lane of the wave active. Afterwards lane i < k holds the i-th choice: its expert in my_e,
// its probability in my_p; chosen_sum (every lane) is the sum of the k chosen probabilities in rank
// order, which the routing weights my_p / chosen_sum divide by.
//  - op_softmax (csrc/ops.c:353-364): expf(x - max) (the host libm's expf, bit for bit), the sum in
//    double, times (float)(1 / sum). The probabilities stay in registers; -1 marks lanes past
//    n_expert (never chosen).
//  - moe_select (csrc/model_llama.c:653-666): k times the largest remaining probability, ties to the
//    lowest expert; chosen ones are marked -2. Each round's arg-max is the wave maximum of a 32-bit
//    key, the probability's bits plus one (probabilities are >= 0, so their bits order as unsigned;
//    the marks map to 0), through DPP and readlane (no LDS round trip); then the lowest expert id
//    holding it from ballots (the lower id wins a tie).
template <int NPL>
SDY_DEV void sdy_moe_route_wave(const float *p, int n_expert, int k, int lane, uint32_t etab, int &my_e,
                                float &my_p, float &chosen_sum) {
    float v[NPL];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NPL; j++) {
        const int e = lane + 64 * j;
        v[j] = e < n_expert ? p[e] : -INFINITY;
        m = fmaxf(m, v[j]);
    }
    m = wave_max_f32(m);  // (a maximum: the same value in any order)
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < NPL; j++) {
        v[j] = sdy_expf_reg(v[j] - m, etab);  // every lane (the table lookup reads other lanes): 0 past n_expert
        if (lane + 64 * j < n_expert) s += (double)v[j];
    }
    s = sdy_wave_sum_f64(s);  // the butterfly over lane ^ 32, 16, ..., 1
    const float inv = (float)(1.0 / s);
#pragma unroll
    for (int j = 0; j < NPL; j++) v[j] = lane + 64 * j < n_expert ? v[j] * inv : -1.0f;
    chosen_sum = 0.0f;
    my_p = 0.0f;
    my_e = 0;
    for (int i = 0; i < k; i++) {
        // the largest key over the wave, then the lowest expert holding it: the first slot j whose
        // ballot has a lane, its lowest lane
        uint32_t hk[NPL], key = 0;
#pragma unroll
        for (int j = 0; j < NPL; j++) {
            hk[j] = v[j] >= 0.0f ? __float_as_uint(fabsf(v[j])) + 1u : 0u;
            key = hk[j] > key ? hk[j] : key;
        }
        key = wave_max_u32(key);
        int bi = -1;
#pragma unroll
        for (int j = NPL - 1; j >= 0; j--) {
            const uint64_t bal = __ballot(hk[j] == key);
            if (bal) bi = 64 * j + (int)__builtin_ctzll(bal);
        }
        const float best = __uint_as_float(key - 1u);
#pragma unroll
        for (int j = 0; j < NPL; j++)
            if (bi == lane + 64 * j) v[j] = -2.0f;
        if (lane == i) {
            my_p = best;
            my_e = bi;
        }
        chosen_sum = chosen_sum + best;
    }
}

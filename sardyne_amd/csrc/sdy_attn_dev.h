// Device helpers shared by the attention kernels: the KV-cache element types.
//
// The cache of a layer is [n_kv_head][max_seq][head_dim] elements of one type:
//   float     f32, the reference's cache (csrc/model_llama.c:428-466);
//   uint16_t  f16 bits: each K/V value is rounded when it is written, with the reference's own
//             f32 -> f16 conversion (round to nearest even, csrc/ops.c:43-62, sdy_f2h), and read
//             back exactly (sdy_h2f), so every kernel computes on the f32 values of the rounded cache.
#pragma once
#include "sdy_device.h"

typedef float sdy_f32x4 __attribute__((ext_vector_type(4)));

template <class T>
struct KvElt;

template <>
struct KvElt<float> {
    static constexpr int BYTES = 4;
    SDY_DEV static float ld(const float *p, size_t i) { return p[i]; }
    // four consecutive elements from i (i a multiple of 4)
    SDY_DEV static sdy_f32x4 ld4(const float *p, size_t i) { return *reinterpret_cast<const sdy_f32x4 *>(p + i); }
    // two consecutive elements from i (i even)
    SDY_DEV static float2 ld2(const float *p, size_t i) { return *reinterpret_cast<const float2 *>(p + i); }
    SDY_DEV static void st(float *p, size_t i, float v) { p[i] = v; }
    // the value a write then a read of v gives
    SDY_DEV static float round(float v) { return v; }
    // one element of a buffer resource at byte offset o
    SDY_DEV static float ld_buf(__amdgpu_buffer_rsrc_t r, uint32_t o) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, o, 0, 0));
    }
};

template <>
struct KvElt<uint16_t> {
    static constexpr int BYTES = 2;
    SDY_DEV static float ld(const uint16_t *p, size_t i) { return sdy_h2f(p[i]); }
    SDY_DEV static sdy_f32x4 ld4(const uint16_t *p, size_t i) {
        const uint2 u = *reinterpret_cast<const uint2 *>(p + i);
        sdy_f32x4 r;
        r[0] = sdy_h2f((uint16_t)(u.x & 0xFFFFu));
        r[1] = sdy_h2f((uint16_t)(u.x >> 16));
        r[2] = sdy_h2f((uint16_t)(u.y & 0xFFFFu));
        r[3] = sdy_h2f((uint16_t)(u.y >> 16));
        return r;
    }
    SDY_DEV static float2 ld2(const uint16_t *p, size_t i) {
        const uint32_t u = *reinterpret_cast<const uint32_t *>(p + i);
        return make_float2(sdy_h2f((uint16_t)(u & 0xFFFFu)), sdy_h2f((uint16_t)(u >> 16)));
    }
    SDY_DEV static void st(uint16_t *p, size_t i, float v) { p[i] = sdy_f2h(v); }
    SDY_DEV static float round(float v) { return sdy_h2f(sdy_f2h(v)); }
    SDY_DEV static float ld_buf(__amdgpu_buffer_rsrc_t r, uint32_t o) {
        return sdy_h2f(__builtin_amdgcn_raw_buffer_load_b16(r, o, 0, 0));
    }
};

// RMSNorm (weights nw, when set) then RoPE at table row (cs, sn) of the HD-vector in LDS buf, by one
// wave: the reference's per-head norm (double sum of squares, scale rounded once) and rotation.
template <int HD>
SDY_DEV void sdy_norm_rope(float *buf, const float *nw, float eps, const float *cs, const float *sn,
                           int interleaved, int lane) {
    if (nw) {
        double ss = 0.0;
        for (int i = lane; i < HD; i += 64) ss += (double)buf[i] * (double)buf[i];
        for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
        const float sc = (float)(1.0 / sqrt(ss / (double)HD + (double)eps));
        for (int i = lane; i < HD; i += 64) {
            const float t = buf[i] * sc;
            buf[i] = t * nw[i];
        }
        sdy_wave_sync();
    }
    constexpr int H = HD / 2;
    for (int i = lane; i < H; i += 64) {
        const int ia = interleaved ? 2 * i : i, ib = interleaved ? 2 * i + 1 : i + H;
        const float a = buf[ia], b = buf[ib];
        const float ac = a * cs[i], bs = b * sn[i], as = a * sn[i], bc = b * cs[i];
        buf[ia] = ac - bs;
        buf[ib] = as + bc;
    }
    sdy_wave_sync();
}

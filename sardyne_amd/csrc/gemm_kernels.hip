// Quantized-weight GEMM for prefill (many tokens) on gfx950 MFMA, bit-exact with the reference's
// integer-dot path (csrc/quant.c:191-235, csrc/quant.h:84-91; the reference's 4-token micro-kernels
// csrc/quant_avx2.c:290-385 give the same bits as its one-token dots).
//
// Per 256-element super-block the reference computes an exact integer isum = sum_k (sc_g q_k) y_k
// (and for Q4_K msum = sum_j m_j bsum_j), then combines acc + (yd*d*isum - yd*dmin*msum) in f32.
// Here every wave dequantises its weight fragments in registers as f16 w' = sc * q (Q4_K) or
// sc * (q - 32) (Q6_K) — exact small integers — and multiplies them with the Q8_K activations as
// f16 (exact int8 values) on v_mfma_f32_32x32x16_f16, accumulating one super-block at a time in
// f32. The products are exact and every partial sum stays below 2^24 when
// 127 * sum_k |w'_k| < 2^24 and |w'| <= 2048 for each row and super-block, so the accumulator
// holds isum exactly. Matrices with a block beyond that (real Q6_K files store int8 scales down to
// -128) take the wide variant, exact for every block the formats can hold: Q6_K splits each scale,
// sc = 16 sh + sl with 0 <= sl < 16, into two fragments with two accumulators, isum = 16 ihi + ilo;
// Q4_K centres its quants, isum = sum sc (q - 8) y + sum_j 8 sc_j bsum_j. Each part's partial sums
// stay below 2^24 and the two are added in f32 with one rounding, that of (float)isum. The check
// runs once per matrix at upload. The Q4_K min term is one more MFMA of the mins against
// the 16-element bsums. The f32 combine then follows the reference's expression and super-block
// order, so each output has the reference's bits.
//
// The activations are expanded to f16 by k_gemm_prep, once per call unless the caller says the
// workspace already holds them (ws_ready: q, k and v of one input).
#include <stdlib.h>

#include "sdy_device.h"
#include "sdy_internal.h"
#include "sdy_quant_dev.h"
#include "sdy_shim.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x32 __attribute__((ext_vector_type(32)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct GemmArgs {
    const uint8_t *p[5];  // weight planes (quant_kernels.hip layout)
    uint32_t psz[5];      // their sizes in bytes (bounds of the buffer resources)
    int n_in, T, nb;      // elements, 64-element units and super-blocks per row
    long row0, n_rows;    // rows row0 .. row0 + n_rows of the planes
    int n_tok;
    const _Float16 *y16;  // [n_tok][n_in] activations (the Q8_K int8 values)
    const float *yd;      // [n_tok][nb] Q8_K scales
    const _Float16 *bs16; // [n_tok][nb][16] Q8_K bsums
    float *out;
    long out_stride;
    const float *bias, *resid;
    int swiglu;
    // grouped launch (k_gemm3 only; grp_tile null: one matrix): group e (a routed expert) multiplies
    // weight rows row0 + e * grp_rows + [0, n_rows) with activation rows grp_tok[e] .. grp_tok[e + 1]
    // - 1; its token tiles are grp_tile[e] .. grp_tile[e + 1] - 1 of the grid. out_row (or null)
    // sends activation row t's outputs to output row out_row[t].
    const int *grp_tile, *grp_tok, *out_row;
    const int *act_row;  // or null: the activation (expansion) row of row t of the tile
    long grp_rows;
    int n_grp;
    int wide;  // host-side: the wide variant is needed (k_gemm3 only)
    // k_gemm3: p holds the GEMM's copy of the planes (sdy_mat_gemm_layout: rows in tiles of 32,
    // records unit- or super-block-major within a tile); row r of the matrix is row grow0 + r there
    int blk;
    long grow0;
    int exp_rows;  // rows of the activations' expansion (y16, yd, bs16)
};

SDY_DEV u32x2 ld8(const uint8_t *p) { return *reinterpret_cast<const u32x2 *>(p); }

// f16 pairs (1024 + b0, 1024 + b1) from byte lanes 0,1 (sel lo) or 2,3 (hi) of v: the magic
// exponent 0x64 put above each byte by v_perm_b32.
SDY_DEV uint32_t magic_lo(uint32_t v) { return __builtin_amdgcn_perm(0x64646464u, v, 0x05010400u); }
SDY_DEV uint32_t magic_hi(uint32_t v) { return __builtin_amdgcn_perm(0x64646464u, v, 0x05030402u); }

SDY_DEV half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }

// 8 Q4_K quants q (one per byte of n.x, n.y) times sc as f16 with one fused multiply-add per
// pair: (1024 + q) * sc - 1024 * sc. The exact result q * sc <= 945 is representable, so the single
// rounding of the fma is exact (1024 * sc <= 64512 is exact too).
SDY_DEV half8 frag_q4(u32x2 n, half2v sc2, half2v nsc2) {
    half8 r;
    const uint32_t w[4] = {magic_lo(n.x), magic_hi(n.x), magic_lo(n.y), magic_hi(n.y)};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const half2v t = __builtin_elementwise_fma(as_h2(w[i]), sc2, nsc2);
        r[2 * i] = t[0];
        r[2 * i + 1] = t[1];
    }
    return r;
}
SDY_DEV uint32_t as_u(half2v v) { return __builtin_bit_cast(uint32_t, v); }

// 8 small unsigned integers (one per byte of n.x, n.y) times sc as f16: ((1024 + q) - 1024) * sc,
// every step exact (q <= 63, |q * sc| <= 2048).
SDY_DEV half8 frag_scaled(u32x2 n, half2v off, half2v sc2) {
    half8 r;
    const uint32_t w[4] = {magic_lo(n.x), magic_hi(n.x), magic_lo(n.y), magic_hi(n.y)};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const half2v t = (as_h2(w[i]) + off) * sc2;
        r[2 * i] = t[0];
        r[2 * i + 1] = t[1];
    }
    return r;
}

template <int WT>
SDY_DEV void load_unit(const GemmArgs &g, long row, int u, int h, u32x2 (&q)[3]) {
    const size_t ou = ((size_t)row * g.T + u) * 16 + 8 * h;
    if constexpr (WT == SDY_Q4_K) {
        q[0] = ld8(g.p[0] + ou);  // QA
        q[1] = ld8(g.p[1] + ou);  // QB
    } else {
        q[0] = ld8(g.p[0] + ou);  // N0
        q[1] = ld8(g.p[1] + ou);  // N1
        q[2] = ld8(g.p[2] + ou);  // HB
    }
}

// The weights of one super-block for one lane: its A row's quants for k-half h of the 4 units, the
// scale record (Q4_K: d, dmin and the 12 packed scale/min bytes; Q6_K: the 16 int8 scales) and
// the Q6_K d.
struct SbRegs {
    u32x2 q[4][3];
    u32x4 hd;
    uint32_t d6;
};

template <int WT>
SDY_DEV void load_sb(const GemmArgs &g, long row, int sb, int h, SbRegs &r) {
#pragma unroll
    for (int un = 0; un < 4; un++) load_unit<WT>(g, row, 4 * sb + un, h, r.q[un]);
    if constexpr (WT == SDY_Q4_K) {
        r.hd = *reinterpret_cast<const u32x4 *>(g.p[2] + ((size_t)row * g.nb + sb) * 16);
        r.d6 = 0;
    } else {
        r.hd = *reinterpret_cast<const u32x4 *>(g.p[3] + ((size_t)row * g.nb + sb) * 16);
        r.d6 = *reinterpret_cast<const uint16_t *>(g.p[4] + ((size_t)row * g.nb + sb) * 2);
    }
}

// k_gemm3's weights of one super-block for one lane: the quants of its units (all 16 bytes of each
// plane's record: both k-halves), the scale record and the Q6_K d.
struct SbRegs3 {
    u32x4 q[2][3];
    u32x4 hd;
    uint32_t d6;
};

typedef __attribute__((address_space(3))) void *lds_ptr_t;
typedef float f32x4 __attribute__((ext_vector_type(4)));

SDY_DEV uint32_t lds_addr(const float *p) {
    return (uint32_t)(size_t)(const __attribute__((address_space(3))) float *)p;
}

// Four 16-byte LDS reads at a, a + 32, a + 64, a + 96 and four at b, b + 32, ... as one asm block
// that waits for them itself. The compiler then does not see LDS loads here: it would otherwise
// make them wait for every activation DMA in flight (it cannot tell that they do not alias).
SDY_DEV void lds_read8(uint32_t a, uint32_t b, f32x4 &a0, f32x4 &a1, f32x4 &a2, f32x4 &a3, f32x4 &b0, f32x4 &b1,
                       f32x4 &b2, f32x4 &b3) {
    __asm__ volatile(
        "ds_read_b128 %0, %8\n"
        "ds_read_b128 %1, %8 offset:32\n"
        "ds_read_b128 %2, %8 offset:64\n"
        "ds_read_b128 %3, %8 offset:96\n"
        "ds_read_b128 %4, %9\n"
        "ds_read_b128 %5, %9 offset:32\n"
        "ds_read_b128 %6, %9 offset:64\n"
        "ds_read_b128 %7, %9 offset:96\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(a0), "=&v"(a1), "=&v"(a2), "=&v"(a3), "=&v"(b0), "=&v"(b1), "=&v"(b2), "=&v"(b3)
        : "v"(a), "v"(b)
        : "memory");
}

// Two 16-byte LDS reads at a, a + 32 and two at b, b + 32, as lds_read8.
SDY_DEV void lds_read4(uint32_t a, uint32_t b, f32x4 &a0, f32x4 &a1, f32x4 &b0, f32x4 &b1) {
    __asm__ volatile(
        "ds_read_b128 %0, %4\n"
        "ds_read_b128 %1, %4 offset:32\n"
        "ds_read_b128 %2, %5\n"
        "ds_read_b128 %3, %5 offset:32\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(a0), "=&v"(a1), "=&v"(b0), "=&v"(b1)
        : "v"(a), "v"(b)
        : "memory");
}

// The s_waitcnt immediate that waits for at most n (< 64) vector memory operations outstanding and
// lgkm (0 or 15: every LDS access, or none) LDS and scalar ones (vmcnt in bits 3:0 and 15:14,
// expcnt at its maximum, lgkmcnt in bits 11:8).
constexpr int sdy_vmcnt_imm(int n, int lgkm = 0) { return (n & 15) | (((n >> 4) & 3) << 14) | (7 << 4) | (lgkm << 8); }

// SIZE bytes per lane from buffer r at vo + so into LDS at dst + SIZE * lane (the host pass of this
// file does not know the builtin: it has no body there)
template <int SIZE>
SDY_DEV void buf_to_lds(__amdgpu_buffer_rsrc_t r, lds_ptr_t dst, uint32_t vo, int so) {
    static_assert(SIZE == 4 || SIZE == 16, "dword or dwordx4");
#if __HIP_DEVICE_COMPILE__
    if constexpr (SIZE == 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, vo, so, 0, 0);
    else __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 4, vo, so, 0, 0);
#endif
}

SDY_DEV __amdgpu_buffer_rsrc_t plane_rsrc(const uint8_t *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, (int)bytes, 0x00020000);
}

// The MFMA GEMM with the activations staged by LDS DMA. A workgroup of WM waves covers 32*MT*WM
// rows x 32*NT tokens; each wave owns 32*MT rows (MT MFMA row tiles, dequantised in registers
// from buffer loads whose per-super-block advance is a scalar offset) and shares the staged
// activations of all the workgroup's tokens. The two lanes of a row split its units, each loading
// whole 16-byte records (lane half h: units 2h, 2h+1), so that a load instruction reads 32 bytes
// of each of its 32 rows (the vector L1 looks up a cache line per row and instruction); a step's
// MFMA k-slots are then the lane halves' own units, and the activation fragments are read to
// match (the integer sums do not depend on the k order). Per super-block and stage the activations are
// copied global -> LDS with global_load_lds (no registers): LDS chunk p (16 bytes) holds token
// p / 32, chunk (p % 32) ^ (token % 8), so that the fragment reads of 8 consecutive lanes hit
// distinct banks. Two stages: super-block s + 1 is in flight while s is multiplied; one
// s_waitcnt + barrier per super-block. The per-row d (and dmin) are converted once per row into a
// per-wave LDS table.
//
// KS = 2 splits each super-block's four 64-element units between the two waves of a pair that own
// the same rows (units 0-1 and 2-3): each wave sums its units' integer products, the pair exchanges
// half of its accumulator through LDS at the super-block's barrier, and each wave completes and
// combines its half of the tile (D registers 0-7 or 8-15). Integer partial sums add exactly, so the
// bits are KS 1's; a grid has twice the waves (for shapes with one wave per SIMD otherwise: the
// 2048-row down and attention projections of a prompt).
//
// PF = 2 keeps two super-blocks in flight (three register sets and three stage buffers): the wave
// waits by count for the loads of the next super-block only, and the workgroup barrier orders LDS
// alone. For grids of one wave per SIMD, whose super-blocks otherwise each wait a full memory round
// trip.
//
// The body below takes the workgroup's place in its grid (bx, by of gx, gy: a pair launch gives
// each matrix a part of one grid) and its LDS: the stages (dynamic), the per-wave d table and the
// KS 2 exchange (static objects of the kernel, sized by gemm3_dtab_floats / gemm3_xch_floats).
template <int MT, int WM>
constexpr int gemm3_dtab_floats() { return WM * 64 * MT; }
template <int WT, int MT, int NT, int WM, bool WIDE, int KS>
constexpr int gemm3_xch_floats() { return KS == 2 ? 2 * WM * (WIDE && WT == SDY_Q6_K ? 2 : 1) * MT * NT * 8 * 64 : 1; }

template <int WT, int MT, int NT, int WM, bool WIDE, int KS, int PF>
SDY_DEV void gemm3_body(const GemmArgs &g, int bx, int by, int gx, int gy, uint8_t *lds, float *dtab_all,
                        float *xch) {
    static_assert(KS == 1 || (KS == 2 && WM % 2 == 0), "unit split");
    static_assert(PF == 1 || PF == 2, "prefetch depth");
    constexpr int UN = 4 / KS, PAIRS = WM / KS;  // units per wave, row tiles per workgroup
    constexpr int BN = 32 * NT, NTH = 64 * WM;
    constexpr int YDN = BN < 64 ? 64 : BN;                  // yd slots (one DMA dword per lane)
    // PF 2: every wave issues the same loads (so that its waits can be counted): each copies the yd
    // row into a slot of its own and a 1/WM share of the bsums, as dwords
    constexpr int YDOFF = BN * 512, BSOFF = YDOFF + (PF == 2 ? WM : 1) * YDN * 4;
    constexpr int BUF = BSOFF + BN * 32;                    // bytes of one stage
    constexpr int NBSW = BN * 8 / (64 * WM);                // PF 2: bsum dword loads per wave
    static_assert(PF == 1 || (BN * 8) % (64 * WM) == 0, "PF 2: the bsums in whole dword loads per wave");
    constexpr int NI = BN * 32 / NTH;                       // activation DMA chunks per lane per stage
    static_assert((BN * 32) % NTH == 0 && NI >= 1, "tile");
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, h = lane >> 5,
              lr = lane & 31;
    // token tiles of a row tile on one XCD (workgroups are dealt round-robin to the 8 XCDs)
    const int n_tt = gx;
    const long n_rt = gy, L = (long)by * n_tt + bx;
    long rti, tti;
    {
        const long grp = 8L * n_tt, full = n_rt / 8 * grp;
        if (L < full) {
            const long gq = L / grp, w = L - gq * grp;
            rti = gq * 8 + (w & 7);
            tti = w >> 3;
        } else {
            const long w = L - full;
            rti = n_rt / 8 * 8 + w / n_tt;
            tti = w - (w / n_tt) * n_tt;
        }
    }
    const int pw = __builtin_amdgcn_readfirstlane(wave / KS);  // the wave's row tile
    const int ks = __builtin_amdgcn_readfirstlane(wave - pw * KS);  // and unit share
    const long rt = rti * (32 * MT * PAIRS) + 32 * MT * pw;
    int t0 = (int)tti * BN, t_end = g.n_tok;
    long row0 = g.row0;
    if (g.grp_tile) {
        // the group of this token tile: the last e with grp_tile[e] <= tti (empty groups share
        // their successor's start, so the last one is the group that owns the tile)
        if (tti >= g.grp_tile[g.n_grp]) return;  // past the routed tokens (uniform over the workgroup)
        int lo = 0, hi = g.n_grp - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (g.grp_tile[mid] <= (int)tti) lo = mid;
            else hi = mid - 1;
        }
        t0 = g.grp_tok[lo] + ((int)tti - g.grp_tile[lo]) * BN;
        t_end = g.grp_tok[lo + 1];
        row0 += (long)lo * g.grp_rows;
    }
    const int nb = g.nb;
    auto tok_of = [&](int t) { return t0 + t < t_end ? t0 + t : t_end - 1; };
    // the expansion rows the stages read: this lane's rows of the tile, looked up once
    auto act_of = [&](int t) { return g.act_row ? g.act_row[tok_of(t)] : tok_of(t); };
    int ar_st[NI], ar_yd[YDN / 64], ar_bs[BN / 32 > 0 ? BN / 32 : 1], ar_b2[PF == 2 && NBSW > 0 ? NBSW : 1];
#pragma unroll
    for (int j = 0; j < NI; j++) ar_st[j] = act_of(((j * WM + wave) * 64 + lane) >> 5);
#pragma unroll
    for (int i = 0; i < YDN / 64; i++) ar_yd[i] = act_of(64 * i + lane);
#pragma unroll
    for (int i = 0; i < BN / 32; i++) ar_bs[i] = act_of(32 * i + (lane >> 1));
    if constexpr (PF == 2 && WT == SDY_Q4_K) {
#pragma unroll
        for (int i = 0; i < NBSW; i++) ar_b2[i] = act_of(((i * WM + wave) * 64 + lane) >> 3);
    }
    // the stage's loads as buffer loads to LDS: the lanes' byte offsets are fixed, the super-block
    // advance is a scalar offset (no per-super-block address arithmetic)
    const __amdgpu_buffer_rsrc_t ry = plane_rsrc(reinterpret_cast<const uint8_t *>(g.y16), (uint32_t)g.exp_rows * g.n_in * 2u),
                                 ryd = plane_rsrc(reinterpret_cast<const uint8_t *>(g.yd), (uint32_t)g.exp_rows * nb * 4u),
                                 rbs = plane_rsrc(reinterpret_cast<const uint8_t *>(g.bs16), (uint32_t)g.exp_rows * nb * 32u);
    uint32_t vst[NI], vyd[YDN / 64], vbs[BN / 32 > 0 ? BN / 32 : 1], vb2[PF == 2 && NBSW > 0 ? NBSW : 1];
#pragma unroll
    for (int j = 0; j < NI; j++) {
        const int p = (j * WM + wave) * 64 + lane, t = p >> 5, c = (p & 31) ^ (t & 7);
        vst[j] = ((uint32_t)ar_st[j] * (uint32_t)g.n_in + 8u * (uint32_t)c) * 2u;
    }
#pragma unroll
    for (int i = 0; i < YDN / 64; i++) vyd[i] = (uint32_t)ar_yd[i] * (uint32_t)nb * 4u;
#pragma unroll
    for (int i = 0; i < BN / 32; i++) vbs[i] = (uint32_t)ar_bs[i] * (uint32_t)nb * 32u + 16u * (uint32_t)(lane & 1);
    if constexpr (PF == 2 && WT == SDY_Q4_K) {
#pragma unroll
        for (int i = 0; i < NBSW; i++) vb2[i] = (uint32_t)ar_b2[i] * (uint32_t)nb * 32u + 4u * (uint32_t)(lane & 7);
    }

    // weight buffer resources and this lane's per-row offsets
    __amdgpu_buffer_rsrc_t rq[3], rh, rd;
#pragma unroll
    for (int i = 0; i < 3; i++) rq[i] = plane_rsrc(g.p[i], g.psz[i]);
    rh = plane_rsrc(g.p[WT == SDY_Q4_K ? 2 : 3], g.psz[WT == SDY_Q4_K ? 2 : 3]);
    rd = plane_rsrc(g.p[4], g.psz[4]);
    // the lane's units of each super-block: ub + uu, uu < UN / 2
    constexpr int UL = UN / 2;
    const int ub = ks * UN + h * UL;
    // the lane's LDS byte offsets in a stage of its activation fragments' chunks k = 2 s + hh of unit ub
    uint32_t rbo[8];
#pragma unroll
    for (int k = 0; k < 8; k++) rbo[k] = 16u * (uint32_t)(lr * 32 + 8 * ub + (k ^ (lr & 7)));
    // per-lane offsets of the row's records, and the scalar strides of a unit and a super-block:
    // planes row-major, or the GEMM copy (tiles of 32 rows, the tile's 32 records of one unit or
    // super-block adjacent: a load instruction reads 512 contiguous bytes per half-wave)
    uint32_t oq[MT], oh[MT], od[MT];
    const uint32_t ust = g.blk ? 512u : 16u, hst = g.blk ? 512u : 16u, dst2 = g.blk ? 64u : 2u;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const long ri = rt + 32 * mt + lr;
        const uint32_t row = (uint32_t)(row0 + (ri < g.n_rows ? ri : g.n_rows - 1));
        if (g.blk) {
            const uint32_t R = (uint32_t)g.grow0 + row, tb = R >> 5, r = R & 31u;
            oq[mt] = (tb * (uint32_t)g.T * 32u + r) * 16u + 512u * (uint32_t)(h * UL);
            oh[mt] = (tb * (uint32_t)nb * 32u + r) * 16u;
            od[mt] = (tb * (uint32_t)nb * 32u + r) * 2u;
        } else {
            oq[mt] = row * (uint32_t)g.T * 16u + 16u * (uint32_t)(h * UL);
            oh[mt] = row * (uint32_t)nb * 16u;
            od[mt] = row * (uint32_t)nb * 2u;
        }
    }
    auto load_sb3 = [&](int sb, SbRegs3 (&R)[MT]) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
#pragma unroll
            for (int uu = 0; uu < UL; uu++) {  // units ub + uu (h UL in the lane's offset)
                const int so = (4 * sb + ks * UN + uu) * (int)ust;
                R[mt].q[uu][0] = __builtin_amdgcn_raw_buffer_load_b128(rq[0], oq[mt], so, 0);
                R[mt].q[uu][1] = __builtin_amdgcn_raw_buffer_load_b128(rq[1], oq[mt], so, 0);
                if constexpr (WT == SDY_Q6_K) R[mt].q[uu][2] = __builtin_amdgcn_raw_buffer_load_b128(rq[2], oq[mt], so, 0);
            }
            R[mt].hd = __builtin_amdgcn_raw_buffer_load_b128(rh, oh[mt], sb * (int)hst, 0);
            R[mt].d6 = WT == SDY_Q6_K ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rd, od[mt], sb * (int)dst2, 0) : 0u;
        }
    };
    // activation stage of super-block sb into buffer buf (asynchronous; completes at s_waitcnt)
    auto stage = [&](int sb, int buf) {
        uint8_t *base = lds + buf * BUF;
#pragma unroll
        for (int j = 0; j < NI; j++) {
            const int blk = j * WM + wave;  // 64-chunk block written by this wave instruction
            buf_to_lds<16>(ry, (lds_ptr_t)(base + blk * 1024), vst[j], sb * 512);
        }
        if constexpr (PF == 2) {
#pragma unroll
            for (int i = 0; i < YDN / 64; i++)
                buf_to_lds<4>(ryd, (lds_ptr_t)(base + YDOFF + wave * (YDN * 4) + 256 * i), vyd[i], sb * 4);
            if constexpr (WT == SDY_Q4_K) {
#pragma unroll
                for (int i = 0; i < NBSW; i++)  // bsum dword p = (i WM + wave) 64 + lane: token p / 8, bytes 4 (p % 8)
                    buf_to_lds<4>(rbs, (lds_ptr_t)(base + BSOFF + 256 * (i * WM + wave)), vb2[i], sb * 32);
            }
        } else {
            if (wave == 0) {
#pragma unroll
                for (int i = 0; i < YDN / 64; i++)
                    buf_to_lds<4>(ryd, (lds_ptr_t)(base + YDOFF + 256 * i), vyd[i], sb * 4);
            }
        }
        if constexpr (WT == SDY_Q4_K && PF == 1) {
            if (wave == (WM > 1 ? 1 : 0)) {
#pragma unroll
                for (int i = 0; i < BN / 32; i++)
                    buf_to_lds<16>(rbs, (lds_ptr_t)(base + BSOFF + 1024 * i), vbs[i], sb * 32);
            }
        }
    };
    // PF 1: the barrier's release fence waits for every load of the wave, the DMA of the stage included.
    // PF 2: the loads of the iteration's super-block sb + 2 stay in flight: wait until at most as
    // many as the wave issued for it are outstanding (loads complete in order), then a barrier that
    // orders the LDS accesses (the activations DMA'd by every wave, the exchange)
    constexpr int NWL = MT * (UL * (WT == SDY_Q6_K ? 3 : 2) + (WT == SDY_Q6_K ? 2 : 1));  // load_sb3's loads
    constexpr int NSL = NI + YDN / 64 + (WT == SDY_Q4_K ? NBSW : 0);                     // PF 2: stage()'s
    static_assert(PF == 1 || NWL + NSL < 64, "wait count");
    auto wait_stage = [&]() {
        if constexpr (PF == 1) {
            __syncthreads();
        } else {
            // s_waitcnt vmcnt(NWL + NSL) lgkmcnt(0) (the compiler's own wait tracking sees it), then the
            // barrier as a compiler memory barrier too (a fence would wait for the DMA in flight: it
            // writes LDS)
            __builtin_amdgcn_s_waitcnt(sdy_vmcnt_imm(NWL + NSL));
            __asm__ volatile("s_barrier" ::: "memory");
        }
    };

    constexpr int RH = 16 / KS;  // D registers (of 16) that a wave completes: RH ks .. RH ks + RH - 1
    float acc[MT][NT][RH];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int i = 0; i < RH; i++) acc[mt][nt][i] = 0.0f;
    const half2v off6 = {(_Float16)-1056.0f, (_Float16)-1056.0f};
    const half2v off4c = {(_Float16)-1032.0f, (_Float16)-1032.0f};  // centred Q4_K quants q - 8
    // per-wave d[32 MT] then dmin[32 MT] as f32 (static LDS: a separate object from the DMA target,
    // so its reads need not wait for the activation loads in flight)
    float *dtab = dtab_all + wave * (64 * MT);
    // KS 2: the half accumulators a wave hands its partner (xch), [parity][wave][sum][mt][nt][8][64]
    constexpr int NXS = WIDE && WT == SDY_Q6_K ? 2 : 1;

    constexpr int NBUF = PF + 1;  // stage buffers
    // one super-block: sb's weights in A, the loads of sb + PF issued into An (clamped to the last
    // super-block, so that every iteration issues the same weight loads)
    auto iter = [&](int sb, SbRegs3(&A)[MT], SbRegs3(&An)[MT]) {
        const int cur = sb & 1;
        // issue priorities over a super-block (the SIMD's other wave is at another point of its own):
        // the next super-block's weight loads and activation DMA first (2), then the fragment reads
        // and MFMA loop (1), the combine (VALU only) last (0). 3B prefill +1.4 % and +4.6 % on two
        // boxes for the MFMA loop's 1, +0.7 % more for the loads' 2; the priority around the MFMA
        // instructions alone changed nothing
        __builtin_amdgcn_s_setprio(2);
        load_sb3(sb + PF < nb ? sb + PF : nb - 1, An);
        // PF 2 stages the last super-block again past the end (into the buffer of sb - 1, which is
        // read no more), so that every iteration issues the same loads
        if constexpr (PF == 2) {
            stage(sb + PF < nb ? sb + PF : nb - 1, (sb + PF) % NBUF);
            // already true (the previous iteration waited for sb's loads): stated so that the
            // compiler's wait tracking, which loses count at the loop head, knows A complete
            __builtin_amdgcn_s_waitcnt(sdy_vmcnt_imm(2 * (NWL + NSL), 15));
        } else if (sb + PF < nb) {
            stage(sb + PF, (sb + PF) % NBUF);
        }
        __builtin_amdgcn_s_setprio(1);
        // d (and dmin) of the lane's row (lr, the same in both lane halves) as f32
        float drow[MT], mrow[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const uint32_t dp = WT == SDY_Q4_K ? A[mt].hd.x : A[mt].d6;
            drow[mt] = sdy_h2f((uint16_t)(dp & 0xFFFFu));
            mrow[mt] = WT == SDY_Q4_K ? sdy_h2f((uint16_t)(dp >> 16)) : 0.0f;
        }
        // KS 1: the combine's scale products from the matrix cores (outer products, below); KS 2 keeps
        // them on the VALU from a per-wave LDS table (the MFMA form's registers cost the unit split's
        // grids an occupancy step)
        constexpr bool OUTER = KS == 1;
        if constexpr (!OUTER) {
            if (h == 0) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    dtab[32 * mt + lr] = drow[mt];
                    if constexpr (WT == SDY_Q4_K) dtab[32 * MT + 32 * mt + lr] = mrow[mt];
                }
            }
        }
        const uint8_t *bbuf = lds + (sb % NBUF) * BUF;
        // WIDE (any block the formats can hold):
        //   Q6_K: each scale sc = 16 sh + sl (sl in [0, 16), sh in [-8, 7]) is applied in two exact
        //         fragments with their own integer sums, isum = 16 ihi + ilo; the partial sums stay
        //         below 2^24 (127 * 256 * 32 * 15 and 127 * 256 * 32 * 8);
        //   Q4_K: the quants are centred, isum = sum sc (q - 8) y + sum_j 8 sc_j bsum_j: the first sum
        //         below 127 * 256 * 63 * 8 < 2^24, the second one more MFMA against the bsums.
        constexpr bool SPLIT6 = WIDE && WT == SDY_Q6_K;
        float16v isum[MT][NT], ihi[SPLIT6 ? MT : 1][SPLIT6 ? NT : 1];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) isum[mt][nt] = float16v{};
        if constexpr (SPLIT6) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++) ihi[mt][nt] = float16v{};
        }
        // the lane's scales for its units, once per super-block. Q4_K: the 6-bit scales of sub-blocks
        // 2 ub .. 2 ub + 2 UL - 1 as bytes (sub-blocks 0-3 from the low bits of the first word, 4-7
        // from the third word and the top bits of the first); Q6_K: the int8 scale words of units ub + uu
        uint32_t scw[MT][UL];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            if constexpr (WT == SDY_Q4_K) {
                const uint32_t Aw = A[mt].hd.y, Cw = A[mt].hd.w;
                const uint32_t f1 = Aw & 0x3F3F3F3Fu, f2 = (Cw & 0x0F0F0F0Fu) | ((Aw >> 2) & 0x30303030u);
                scw[mt][0] = (ub >= 2 ? f2 : f1) >> (16 * (ub & 1));
            } else {
#pragma unroll
                for (int uu = 0; uu < UL; uu++) {
                    const int w = ub + uu;
                    const uint32_t lo = (w & 1) ? A[mt].hd.y : A[mt].hd.x, hi2 = (w & 1) ? A[mt].hd.w : A[mt].hd.z;
                    scw[mt][uu] = (w & 2) ? hi2 : lo;
                }
            }
        }
        // step sl = 8 uu + 4 hh + s of the lane: k-half hh of unit ub + uu, quarter s (its 16-element
        // chunk 8 (ub + uu) + 2 s + hh of each token), read from LDS one step ahead of its MFMAs
        half8 bf[2][NT];
        // chunk 8 (ub + uu) + k of token 32 nt + lr sits at bbuf + rbo[k] + 128 uu + 16384 nt (the swizzle
        // only permutes the low three bits of the chunk index: k ^ (lr & 7))
        const uint8_t *rbp[8];
#pragma unroll
        for (int k = 0; k < 8; k++) rbp[k] = bbuf + rbo[k];
        auto read_b = [&](int sl, half8 (&dst)[NT]) {
            const int k = 2 * (sl & 3) + ((sl >> 2) & 1), uu = sl >> 3;
#pragma unroll
            for (int nt = 0; nt < NT; nt++) dst[nt] = *reinterpret_cast<const half8 *>(rbp[k] + 128 * uu + 16384 * nt);
        };
        read_b(0, bf[0]);
#pragma unroll
        for (int uu = 0; uu < UL; uu++) {
#pragma unroll
            for (int hh = 0; hh < 2; hh++)
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const int sl = 8 * uu + 4 * hh + s;  // the lane's step
                if (sl + 1 < 4 * UN) read_b(sl + 1, bf[(sl + 1) & 1]);
                __builtin_amdgcn_sched_barrier(0);  // the next step's reads go out before this step's work
                half8 a[MT], ah[SPLIT6 ? MT : 1];
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    auto half_of = [&](const u32x4 &v) { return hh ? u32x2{v.z, v.w} : u32x2{v.x, v.y}; };
                    if constexpr (WT == SDY_Q4_K) {
                        // sub-block 2 (ub + uu) + s / 2
                        const int sc = (int)((scw[mt][0] >> (8 * (2 * uu + (s >> 1)))) & 255u);
                        const u32x2 src = half_of((s & 1) ? A[mt].q[uu][1] : A[mt].q[uu][0]);
                        const u32x2 nib = (s & 2) ? ((src >> 4u) & 0x0F0F0F0Fu) : (src & 0x0F0F0F0Fu);
                        if constexpr (WIDE) {
                            const _Float16 f = (_Float16)(float)sc;
                            a[mt] = frag_scaled(nib, off4c, half2v{f, f});
                        } else {
                            const _Float16 f = (_Float16)(float)sc, nf = (_Float16)(float)(-1024 * sc);
                            a[mt] = frag_q4(nib, half2v{f, f}, half2v{nf, nf});
                        }
                    } else {
                        const int sc = (int)(int8_t)((scw[mt][uu] >> (8 * s)) & 255u);
                        const u32x2 src = half_of((s & 1) ? A[mt].q[uu][1] : A[mt].q[uu][0]);
                        const u32x2 lo = (s & 2) ? ((src >> 4u) & 0x0F0F0F0Fu) : (src & 0x0F0F0F0Fu);
                        const u32x2 hi = ((half_of(A[mt].q[uu][2]) >> (unsigned)(2 * s)) & 0x03030303u) << 4u;
                        if constexpr (SPLIT6) {
                            const int sl6 = sc & 15, sh = sc >> 4;
                            const _Float16 fl = (_Float16)(float)sl6, fh = (_Float16)(float)sh;
                            a[mt] = frag_scaled(lo | hi, off6, half2v{fl, fl});
                            ah[mt] = frag_scaled(lo | hi, off6, half2v{fh, fh});
                        } else {
                            const _Float16 f = (_Float16)(float)sc;
                            a[mt] = frag_scaled(lo | hi, off6, half2v{f, f});
                        }
                    }
                }
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        isum[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[mt], bf[sl & 1][nt], isum[mt][nt], 0, 0, 0);
                        if constexpr (SPLIT6)
                            ihi[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[mt], bf[sl & 1][nt], ihi[mt][nt], 0, 0, 0);
                    }
                }
            }
        }
        __builtin_amdgcn_s_setprio(0);
        // combine in the reference's order: acc + (yd*d*isum - yd*dmin*msum)
        float ydn[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
            ydn[nt] = *reinterpret_cast<const float *>(bbuf + YDOFF + (PF == 2 ? wave * (YDN * 4) : 0) + 4 * (32 * nt + lr));
        // Q4_K, row tile mt: msum = sum_j m_j bsum_j and, WIDE, cw = sum_j 8 sc_j bsum_j (below 16 * 504 *
        // 2032 < 2^24), both exact, from the staged bsums
        auto bsum_mfma = [&](int mt, float16v(&msum)[NT], float16v(&cw)[NT]) {
            const uint32_t Aw = A[mt].hd.y, Bw = A[mt].hd.z, Cw = A[mt].hd.w;
            half8 a2, a3;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int j = 4 * h + (e >> 1);  // sub-block of 16-group 8h + e
                const int m = j < 4 ? (int)((Bw >> (8 * j)) & 63)
                                    : (int)(((Cw >> (8 * (j - 4) + 4)) & 15) | (((Bw >> (8 * (j - 4) + 6)) & 3) << 4));
                a2[e] = (_Float16)(float)m;
                if constexpr (WIDE) {
                    const int sc = j < 4 ? (int)((Aw >> (8 * j)) & 63)
                                         : (int)(((Cw >> (8 * (j - 4))) & 15) | (((Aw >> (8 * (j - 4) + 6)) & 3) << 4));
                    a3[e] = (_Float16)(float)(8 * sc);
                }
            }
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const half8 b2 = *reinterpret_cast<const half8 *>(bbuf + BSOFF + 32 * (32 * nt + lr) + 16 * h);
                msum[nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a2, b2, float16v{}, 0, 0, 0);
                if constexpr (WIDE) cw[nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a3, b2, float16v{}, 0, 0, 0);
            }
        };
        // acc += yd d isum - yd dmin msum over the wave's D registers of row tile mt: register RH ks + i
        // holds row 8 q + 4 h + (i & 3) of the tile, q = (RH ks + i) / 4
        auto combine = [&](int mt, const float(&tot)[NT][RH], const float(&ms)[NT][RH]) {
            if constexpr (OUTER) {
                // yd*d and yd*dmin of the tile's (row, token) pairs as the outer products of an f32 MFMA
                // with k = 1: one rounding of a single product, the bits of the VALU's multiply (a zero
                // product may come out +0 where the multiply gives -0; acc starts at +0 and sums of
                // zeros of either sign keep it +0, so the results are the same). Two blocks: token
                // tiles 2p and 2p + 1 from lane halves 0 and 1 (past the last tile, block 1 repeats it
                // and is not read); the D register r of block b holds the row and token that isum's
                // register r holds.
#pragma unroll
                for (int pr = 0; pr < (NT + 1) / 2; pr++) {
                    const float ydb = h && 2 * pr + 1 < NT ? ydn[2 * pr + 1] : ydn[2 * pr];
                    const f32x32 da = __builtin_amdgcn_mfma_f32_32x32x1f32(drow[mt], ydb, f32x32{}, 0, 0, 0);
                    f32x32 dmv = {};
                    if constexpr (WT == SDY_Q4_K)
                        dmv = __builtin_amdgcn_mfma_f32_32x32x1f32(mrow[mt], ydb, f32x32{}, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < RH; i++) {
#pragma unroll
                        for (int b = 0; b < 2; b++) {
                            const int nt = 2 * pr + b;
                            if (nt >= NT) continue;
                            const int r = 16 * b + RH * ks + i;
                            if constexpr (WT == SDY_Q4_K) {
                                const float t1 = da[r] * tot[nt][i], t2 = dmv[r] * ms[nt][i];
                                acc[mt][nt][i] = acc[mt][nt][i] + (t1 - t2);
                            } else {
                                acc[mt][nt][i] = acc[mt][nt][i] + da[r] * tot[nt][i];
                            }
                        }
                    }
                }
                return;
            }
            float dv[RH], dm[RH];
            const uint32_t da = lds_addr(dtab + 32 * mt + 4 * h + 8 * (RH / 4) * ks);
            if constexpr (KS == 1) {
                f32x4 d0, d1, d2, d3, m0, m1, m2, m3;
                lds_read8(da, da + 4 * 32 * MT, d0, d1, d2, d3, m0, m1, m2, m3);
                const f32x4 dq[4] = {d0, d1, d2, d3}, mq[4] = {m0, m1, m2, m3};
#pragma unroll
                for (int q = 0; q < 4; q++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        dv[4 * q + i] = dq[q][i];
                        dm[4 * q + i] = WT == SDY_Q4_K ? mq[q][i] : 0.0f;
                    }
            } else {
                f32x4 d0, d1, m0, m1;
                lds_read4(da, da + 4 * 32 * MT, d0, d1, m0, m1);
                const f32x4 dq[2] = {d0, d1}, mq[2] = {m0, m1};
#pragma unroll
                for (int q = 0; q < 2; q++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        dv[4 * q + i] = dq[q][i];
                        dm[4 * q + i] = WT == SDY_Q4_K ? mq[q][i] : 0.0f;
                    }
            }
#pragma unroll
            for (int i = 0; i < RH; i++) {
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    if constexpr (WT == SDY_Q4_K) {
                        const float dall = ydn[nt] * dv[i], dmn = ydn[nt] * dm[i];
                        const float t1 = dall * tot[nt][i], t2 = dmn * ms[nt][i];
                        acc[mt][nt][i] = acc[mt][nt][i] + (t1 - t2);
                    } else {
                        const float ydd = ydn[nt] * dv[i];
                        acc[mt][nt][i] = acc[mt][nt][i] + ydd * tot[nt][i];
                    }
                }
            }
        };
        if constexpr (KS == 1) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                float16v msum[NT], cw[NT];
                if constexpr (WT == SDY_Q4_K) bsum_mfma(mt, msum, cw);
                float tot[NT][16], ms[NT][16];
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        float v = isum[mt][nt][r];
                        // SPLIT6: isum = 16 ihi + ilo, 16 ihi exact, one rounding of the sum (that of (float)isum)
                        if constexpr (SPLIT6) v = 16.0f * ihi[mt][nt][r] + v;
                        if constexpr (WT == SDY_Q4_K && WIDE) v = v + cw[nt][r];  // one rounding
                        tot[nt][r] = v;
                        ms[nt][r] = WT == SDY_Q4_K ? msum[nt][r] : 0.0f;
                    }
                combine(mt, tot, ms);
            }
            wait_stage();
        } else {
            // before the barrier (after it the stage buffer is refilled): the bsum products, and the half
            // of the integer sums that the partner completes into its slot
            float ms[MT][NT][RH], cws[MT][NT][RH];
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                float16v msum[NT], cw[NT];
                if constexpr (WT == SDY_Q4_K) {
                    bsum_mfma(mt, msum, cw);
#pragma unroll
                    for (int nt = 0; nt < NT; nt++)
#pragma unroll
                        for (int i = 0; i < RH; i++) {
                            ms[mt][nt][i] = ks ? msum[nt][RH + i] : msum[nt][i];
                            if constexpr (WIDE) cws[mt][nt][i] = ks ? cw[nt][RH + i] : cw[nt][i];
                        }
                }
            }
            float *xw = xch + (size_t)(cur * WM + wave) * (NXS * MT * NT * 512);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
#pragma unroll
                    for (int i = 0; i < RH; i++) {
                        const int o = ((mt * NT + nt) * 8 + i) * 64 + lane;
                        xw[o] = ks ? isum[mt][nt][i] : isum[mt][nt][RH + i];
                        if constexpr (SPLIT6) xw[MT * NT * 512 + o] = ks ? ihi[mt][nt][i] : ihi[mt][nt][RH + i];
                    }
            wait_stage();
            const float *xr = xch + (size_t)(cur * WM + (wave ^ 1)) * (NXS * MT * NT * 512);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                float tot[NT][RH], msh[NT][RH];
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
#pragma unroll
                    for (int i = 0; i < RH; i++) {
                        const int o = ((mt * NT + nt) * 8 + i) * 64 + lane;
                        // the unit halves' sums are integers below 2^24: their sum is isum exactly
                        float v = (ks ? isum[mt][nt][RH + i] : isum[mt][nt][i]) + xr[o];
                        if constexpr (SPLIT6) {
                            const float hi = (ks ? ihi[mt][nt][RH + i] : ihi[mt][nt][i]) + xr[MT * NT * 512 + o];
                            v = 16.0f * hi + v;
                        }
                        if constexpr (WT == SDY_Q4_K && WIDE) v = v + cws[mt][nt][i];
                        tot[nt][i] = v;
                        msh[nt][i] = WT == SDY_Q4_K ? ms[mt][nt][i] : 0.0f;
                    }
                combine(mt, tot, msh);
            }
        }
    };
    if constexpr (PF == 1) {
        SbRegs3 A[MT];
        load_sb3(0, A);
        stage(0, 0);
        __syncthreads();
        for (int sb = 0; sb < nb; sb++) {
            SbRegs3 An[MT];
            iter(sb, A, An);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) A[mt] = An[mt];
        }
    } else {
        // a ring of three register sets, rotated by name
        SbRegs3 S0[MT], S1[MT], S2[MT];
        load_sb3(0, S0);
        stage(0, 0);
        load_sb3(nb > 1 ? 1 : 0, S1);
        if (nb > 1) stage(1, 1);
        __syncthreads();
        // whole rounds of three, then the rest (no exit inside a round: the compiler's wait tracking
        // would merge such exits into the loop's back edge, with the next set still pending)
        int sb = 0;
        for (; sb + 3 <= nb; sb += 3) {
            iter(sb, S0, S2);
            iter(sb + 1, S1, S0);
            iter(sb + 2, S2, S1);
        }
        if (sb < nb) {
            iter(sb, S0, S2);
            if (sb + 1 < nb) iter(sb + 1, S1, S0);
        }
    }
    // store (bias, residual, or the SwiGLU pair of rows 2i, 2i+1 held by this lane). The output rows,
    // bias and residual values are all requested before the first store (one memory round trip);
    // tokens and rows past the ends read the last valid ones and store nothing.
    int orow[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int tok = t0 + 32 * nt + lr;
        orow[nt] = tok < t_end ? tok : t_end - 1;
    }
    if (g.out_row) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) orow[nt] = g.out_row[orow[nt]];
    }
    auto row_of = [&](int mt, int i) {  // the matrix row of D register RH ks + i of row tile mt (clamped)
        const int r = RH * ks + i;
        const long ri = rt + 32 * mt + 8 * (r >> 2) + 4 * h + (r & 3);
        return ri < g.n_rows ? ri : g.n_rows - 1;
    };
    // the SwiGLU exponential's table in a register (its lane reads need every lane: the values are
    // computed before the stores' branches)
    const uint32_t etab = sdy_expf_tab_lane(lane);
    float bv[MT][RH], rv[MT][NT][RH];
    if (g.bias) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < RH; i++) bv[mt][i] = g.bias[g.row0 + row_of(mt, i)];
    }
    if (g.resid) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int i = 0; i < RH; i++) rv[mt][nt][i] = g.resid[(size_t)orow[nt] * g.out_stride + g.row0 + row_of(mt, i)];
    }
    if (g.swiglu) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int i = 0; i < RH; i += 2)
                    acc[mt][nt][i] = sdy_silu_mul1_reg(acc[mt][nt][i], acc[mt][nt][i + 1], etab);
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            if (t0 + 32 * nt + lr >= t_end) continue;
            float *orp = g.out + (size_t)orow[nt] * g.out_stride;
#pragma unroll
            for (int i = 0; i < RH; i++) {
                const int r = RH * ks + i;  // the D register
                const long ri = rt + 32 * mt + 8 * (r >> 2) + 4 * h + (r & 3);
                if (ri >= g.n_rows) continue;
                const long row = g.grp_tile ? ri : g.row0 + ri;
                if (g.swiglu) {
                    if ((i & 1) == 0) orp[ri >> 1] = acc[mt][nt][i];
                } else {
                    float v = acc[mt][nt][i];
                    if (g.bias) v = v + bv[mt][i];
                    if (g.resid) v = rv[mt][nt][i] + v;
                    orp[row] = v;
                }
            }
        }
}

template <int WT, int MT, int NT, int WM, bool WIDE, int KS = 1, int PF = 1>
__global__ __launch_bounds__(64 * WM) void k_gemm3(GemmArgs g) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ __align__(16) float dtab_all[gemm3_dtab_floats<MT, WM>()];
    __shared__ float xch[gemm3_xch_floats<WT, MT, NT, WM, WIDE, KS>()];
    gemm3_body<WT, MT, NT, WM, WIDE, KS, PF>(g, (int)blockIdx.x, (int)blockIdx.y, (int)gridDim.x, (int)gridDim.y, lds,
                                             dtab_all, xch);
}

// Two GEMMs on the same activations in one launch (a layer's q|k and a v of another type): row
// tiles [0, gy1) of the grid multiply g1, the rest g2; both take the <MT, NT, WM, KS> tile form.
template <int WT1, bool WIDE1, int WT2, bool WIDE2, int MT, int NT, int WM, int KS>
__global__ __launch_bounds__(64 * WM) void k_gemm3_pair(GemmArgs g1, GemmArgs g2, int gy1) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int X1 = gemm3_xch_floats<WT1, MT, NT, WM, WIDE1, KS>(), X2 = gemm3_xch_floats<WT2, MT, NT, WM, WIDE2, KS>();
    __shared__ __align__(16) float dtab_all[gemm3_dtab_floats<MT, WM>()];
    __shared__ float xch[X1 > X2 ? X1 : X2];
    if ((int)blockIdx.y < gy1)
        gemm3_body<WT1, MT, NT, WM, WIDE1, KS, 1>(g1, (int)blockIdx.x, (int)blockIdx.y, (int)gridDim.x, gy1, lds,
                                                  dtab_all, xch);
    else
        gemm3_body<WT2, MT, NT, WM, WIDE2, KS, 1>(g2, (int)blockIdx.x, (int)blockIdx.y - gy1, (int)gridDim.x,
                                                  (int)gridDim.y - gy1, lds, dtab_all, xch);
}


// Q8_K rows -> f16 values, f32 scales and f16 bsums for the GEMM (all exact: |q| <= 127, |bsum| <=
// 2032). One thread per 16 values of a super-block (n_sb = n_tok * nb super-blocks in a row): four
// 4-byte loads, two 16-byte stores, and the super-block's bsum number `part`; 256 threads.
__global__ __launch_bounds__(256) void k_gemm_prep(const uint8_t *__restrict__ xq, long n_sb,
                                                   _Float16 *__restrict__ y16, float *__restrict__ yd,
                                                   _Float16 *__restrict__ bs16) {
    const long g = blockIdx.x * 256L + threadIdx.x, sbg = g >> 4;
    const int part = (int)(g & 15);
    if (sbg >= n_sb) return;
    const uint8_t *blk = xq + sbg * 292;
    const uint32_t *q4 = reinterpret_cast<const uint32_t *>(blk + 4 + 16 * part);
    typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
    f16x8 o[2];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t v = q4[w];
#pragma unroll
        for (int e = 0; e < 4; e++) o[w >> 1][4 * (w & 1) + e] = (_Float16)(float)(int8_t)((v >> (8 * e)) & 255u);
    }
    f16x8 *dst = reinterpret_cast<f16x8 *>(y16 + sbg * 256 + 16 * part);
    dst[0] = o[0];
    dst[1] = o[1];
    bs16[sbg * 16 + part] = (_Float16)(float)reinterpret_cast<const int16_t *>(blk + 260)[part];
    if (part == 0) yd[sbg] = *reinterpret_cast<const float *>(blk);
}

// Which variant of the GEMM multiplies a K-quant matrix exactly: flags a row super-block whose
// 127 * sum |w'| reaches 2^24 or (Q6_K) whose |sc * (q - 32)| exceeds 2048, which the one-fragment
// scheme would round; the wide variant multiplies every block exactly. One thread per
// (row, super-block) of rows [0, n_rows) of the planes.
template <int WT>
__global__ void k_gemm_check(GemmArgs g, int *bad) {
    const long gid = blockIdx.x * (long)blockDim.x + threadIdx.x;
    const long row = gid / g.nb;
    const int sb = (int)(gid - row * g.nb);
    if (row >= g.n_rows) return;
    long sum = 0;
    int over = 0;
    if constexpr (WT == SDY_Q4_K) {
        const uint8_t *hd = g.p[2] + ((size_t)row * g.nb + sb) * 16 + 4;
        for (int u = 0; u < 4; u++)
            for (int half = 0; half < 2; half++) {
                const uint8_t *qp = g.p[half] + ((size_t)row * g.T + 4 * sb + u) * 16;
                const int j0 = 2 * u, j1 = 2 * u + 1;
                const int s0 = j0 < 4 ? hd[j0] & 63 : (hd[j0 + 4] & 15) | ((hd[j0 - 4] >> 6) << 4);
                const int s1 = j1 < 4 ? hd[j1] & 63 : (hd[j1 + 4] & 15) | ((hd[j1 - 4] >> 6) << 4);
                for (int i = 0; i < 16; i++) sum += (long)s0 * (qp[i] & 15) + (long)s1 * (qp[i] >> 4);
            }
    } else {
        const int8_t *scs = reinterpret_cast<const int8_t *>(g.p[3] + ((size_t)row * g.nb + sb) * 16);
        for (int u = 0; u < 4; u++) {
            const size_t ou = ((size_t)row * g.T + 4 * sb + u) * 16;
            for (int e = 0; e < 64; e++) {
                const int lo = e < 32 ? (g.p[e < 16 ? 0 : 1][ou + (e & 15)] & 15) : (g.p[e < 48 ? 0 : 1][ou + (e & 15)] >> 4);
                const int hi = (g.p[2][ou + (e & 15)] >> (2 * (e >> 4))) & 3;
                const int w = scs[4 * u + (e >> 4)] * ((lo | (hi << 4)) - 32);
                const int aw = w < 0 ? -w : w;
                if (aw > 2048) over = 1;
                sum += aw;
            }
        }
    }
    if (over || 127 * sum >= (1L << 24)) atomicOr(bad, 1);
}

}  // namespace

// =============================================================================== host

// Offsets and sizes of the planes of the GEMM's copy of a matrix of `rows` rows (tiles of 32 rows:
// the 16-byte unit records [tile][unit][32], the per-super-block records [tile][super-block][32]).
static size_t gemm_layout_planes(int type, int n_in, long rows, size_t off[5], size_t sz[5]) {
    const size_t tiles = (size_t)(rows + 31) / 32, T = (size_t)n_in / 64, nb = (size_t)n_in / 256;
    const size_t unit = tiles * T * 512, sbk = tiles * nb * 32;
    const size_t s4[5] = {unit, unit, sbk * 16, 0, 0}, s6[5] = {unit, unit, unit, sbk * 16, sbk * 2};
    size_t o = 0;
    for (int i = 0; i < 5; i++) {
        sz[i] = type == SDY_Q4_K ? s4[i] : s6[i];
        off[i] = o;
        o += (sz[i] + 255) & ~(size_t)255;
    }
    return o;
}

// The kernel arguments of m; with its GEMM copy (k_gemm3) when it has one and `layout` is set.
static GemmArgs gemm_args(const sdy_mat *m, bool layout = false) {
    GemmArgs g;
    memset(&g, 0, sizeof(g));
    for (int i = 0; i < 5; i++) g.p[i] = (const uint8_t *)m->base + m->plane_off[i];
    g.n_in = m->n_in;
    g.T = m->n_units;
    g.nb = m->n_in / 256;
    g.n_rows = m->n_rows;
    const size_t rows = (size_t)m->n_rows, unit = rows * g.T * 16, sbk = rows * g.nb;
    size_t sz[5] = {unit, unit, m->type == SDY_Q4_K ? sbk * 16 : unit, m->type == SDY_Q4_K ? 0 : sbk * 16,
                    m->type == SDY_Q4_K ? 0 : sbk * 2};
    if (layout && m->gbase) {
        size_t off[5];
        gemm_layout_planes(m->type, m->n_in, m->grows, off, sz);
        for (int i = 0; i < 5; i++) g.p[i] = (const uint8_t *)m->gbase + off[i];
        g.blk = 1;
        g.grow0 = m->grow0;
    }
    for (int i = 0; i < 5; i++) g.psz[i] = sz[i] < 0xFFFFFFFFu ? (uint32_t)sz[i] : 0xFFFFFFFFu;
    g.wide = m->gemm_ok == 2;
    return g;
}

// Plane record r = row * n_rec + j (rs bytes, rs 16 or 2) into the tiled copy: [row / 32][j][row % 32].
__global__ __launch_bounds__(256) void k_gemm_layout(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                     long n_rows, int n_rec, int rs) {
    const long i = blockIdx.x * 256L + threadIdx.x;
    if (i >= n_rows * (long)n_rec) return;
    const long row = i / n_rec;
    const int j = (int)(i - row * n_rec);
    const size_t o = (((size_t)(row >> 5) * n_rec + j) * 32 + (row & 31)) * rs;
    if (rs == 16) *reinterpret_cast<uint4 *>(dst + o) = *reinterpret_cast<const uint4 *>(src + (size_t)i * 16);
    else *reinterpret_cast<uint16_t *>(dst + o) = *reinterpret_cast<const uint16_t *>(src + (size_t)i * 2);
}

extern "C" size_t sdy_mat_gemm_layout_bytes(const sdy_mat *m) {
    if (!m || !m->base || m->hbase || (m->type != SDY_Q4_K && m->type != SDY_Q6_K) || !m->gemm_ok || m->gbase)
        return 0;
    size_t off[5], sz[5];
    return gemm_layout_planes(m->type, m->n_in, m->n_rows, off, sz);
}

extern "C" int sdy_mat_gemm_layout(sdy_mat *m, sdy_stream s) {
    // (a matrix in host memory keeps no copy: the GEMM reads its planes in place)
    if (!m || !m->base || m->hbase || (m->type != SDY_Q4_K && m->type != SDY_Q6_K) || !m->gemm_ok) return 0;
    if (m->grow0 != 0 || (m->gbase && m->grows != m->n_rows))
        return sdy_fail(-1, "gemm_layout: made for a whole matrix, not a row view");
    size_t off[5], sz[5];
    const size_t bytes = gemm_layout_planes(m->type, m->n_in, m->n_rows, off, sz);
    int rc;
    if (!m->gbase) {
        if ((rc = sdy_malloc(&m->gbase, bytes))) return rc;
        m->gbytes = bytes;
        m->grows = m->n_rows;
        // the padding rows of the last tile: zero (never read: the GEMM clamps its rows)
        if ((rc = sdy_memset(m->gbase, 0, bytes, s))) return rc;
    }
    const int T = m->n_units, nb = m->n_in / 256;
    const int nrec[5] = {T, T, m->type == SDY_Q4_K ? nb : T, nb, nb};
    const int rsz[5] = {16, 16, 16, 16, 2};
    for (int i = 0; i < 5; i++) {
        if (!sz[i]) continue;
        const long total = m->n_rows * (long)nrec[i];
        SDY_NOTE_KERNEL(k_gemm_layout);
        hipLaunchKernelGGL(k_gemm_layout, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)s,
                           (const uint8_t *)m->base + m->plane_off[i], (uint8_t *)m->gbase + off[i], m->n_rows,
                           nrec[i], rsz[i]);
        if ((rc = sdy_check_launch("gemm_layout"))) return rc;
    }
    return 0;
}

// Flags (bad = 1) rows [r0, r0 + n) of m that the GEMM cannot multiply exactly. Synchronous.
extern "C" int sdy_gemm_check_rows_async(const sdy_mat *m, long r0, long n, int *bad_dev, sdy_stream s) {
    if ((m->type != SDY_Q4_K && m->type != SDY_Q6_K) || m->hbase) return 0;  // (host memory: wide, unchecked)
    sdy_mat v = sdy_mat_rows(m, r0, n);
    GemmArgs g = gemm_args(&v);
    const long total = n * (long)g.nb;
    dim3 grid((unsigned)((total + 255) / 256));
    if (m->type == SDY_Q4_K) hipLaunchKernelGGL(k_gemm_check<SDY_Q4_K>, grid, dim3(256), 0, (hipStream_t)s, g, bad_dev);
    else hipLaunchKernelGGL(k_gemm_check<SDY_Q6_K>, grid, dim3(256), 0, (hipStream_t)s, g, bad_dev);
    return sdy_check_launch("gemm_check");
}

extern "C" int sdy_gemm_check_rows(const sdy_mat *m, long r0, long n, int *bad_host, sdy_stream s) {
    *bad_host = 1;
    if ((m->type != SDY_Q4_K && m->type != SDY_Q6_K) || m->hbase) return 0;
    sdy_mat v = sdy_mat_rows(m, r0, n);
    GemmArgs g = gemm_args(&v);
    int *bad = nullptr, rc;
    if ((rc = sdy_malloc((void **)&bad, sizeof(int)))) return rc;
    if ((rc = sdy_memset(bad, 0, sizeof(int), s))) {
        sdy_free(bad);
        return rc;
    }
    const long total = n * (long)g.nb;
    dim3 grid((unsigned)((total + 255) / 256));
    if (m->type == SDY_Q4_K) hipLaunchKernelGGL(k_gemm_check<SDY_Q4_K>, grid, dim3(256), 0, (hipStream_t)s, g, bad);
    else hipLaunchKernelGGL(k_gemm_check<SDY_Q6_K>, grid, dim3(256), 0, (hipStream_t)s, g, bad);
    if (!(rc = sdy_check_launch("gemm_check")) && !(rc = sdy_d2h(bad_host, bad, sizeof(int), s))) rc = sdy_sync(s);
    sdy_free(bad);
    return rc;
}

extern "C" size_t sdy_gemm_ws_bytes(int n_tok, int n_in) {
    const size_t nb = (size_t)n_in / 256;
    return (size_t)n_tok * n_in * 2 + (size_t)n_tok * nb * 4 + (size_t)n_tok * nb * 32 + 3 * 256;
}

extern "C" int sdy_gemm_ok(const sdy_mat *m, int n_tok) {
    // buffer resources address each plane with 32-bit offsets: planes below 4 GiB
    return (m->type == SDY_Q4_K || m->type == SDY_Q6_K) && m->gemm_ok && n_tok >= 2 &&
           (size_t)m->n_rows * m->n_units * 16 < 0xFFFFFFFFu;
}

template <int WT, int MT, int NT, int WM, bool WIDE, int KS, int PF>
static int launch_gemm3_s(GemmArgs &g, hipStream_t st) {
    constexpr int BN = 32 * NT, BM = 32 * MT * WM / KS, YDN = BN < 64 ? 64 : BN;
    constexpr size_t lds = (PF + 1) * (size_t)(BN * 512 + (PF == 2 ? WM : 1) * YDN * 4 + BN * 32);
    static size_t granted = 0;
    const void *fn = (const void *)k_gemm3<WT, MT, NT, WM, WIDE, KS, PF>;
    int rc = sdy_lds_limit(fn, lds, &granted);
    if (rc) return rc;
    const unsigned tok_tiles = (unsigned)((g.n_tok + BN - 1) / BN), row_tiles = (unsigned)((g.n_rows + BM - 1) / BM);
    SDY_NOTE_KERNEL((k_gemm3<WT, MT, NT, WM, WIDE, KS, PF>));
    hipLaunchKernelGGL((k_gemm3<WT, MT, NT, WM, WIDE, KS, PF>), dim3(tok_tiles, row_tiles), dim3(64 * WM), lds, st, g);
    return sdy_check_launch("gemm");
}

// g.wide: the matrix has blocks that the one-fragment scheme cannot multiply exactly
template <int WT, int MT, int NT, int WM, int KS = 1, int PF = 1>
static int launch_gemm3(GemmArgs &g, hipStream_t st) {
    return g.wide ? launch_gemm3_s<WT, MT, NT, WM, true, KS, PF>(g, st)
                  : launch_gemm3_s<WT, MT, NT, WM, false, KS, PF>(g, st);
}

template <int WT, int MT, int NT, int WM, bool WIDE, int KS>
static int launch_gemm3_grid_s(GemmArgs &g, unsigned tok_tiles, unsigned row_tiles, hipStream_t st) {
    constexpr int BN = 32 * NT, YDN = BN < 64 ? 64 : BN;
    constexpr size_t lds = 2 * (size_t)(BN * 512 + YDN * 4 + BN * 32);
    static size_t granted = 0;
    const void *fn = (const void *)k_gemm3<WT, MT, NT, WM, WIDE, KS>;
    int rc = sdy_lds_limit(fn, lds, &granted);
    if (rc) return rc;
    SDY_NOTE_KERNEL((k_gemm3<WT, MT, NT, WM, WIDE, KS>));
    hipLaunchKernelGGL((k_gemm3<WT, MT, NT, WM, WIDE, KS>), dim3(tok_tiles, row_tiles), dim3(64 * WM), lds, st, g);
    return sdy_check_launch("gemm");
}

template <int WT, int MT, int NT, int WM, int KS>
static int launch_gemm3_grid(GemmArgs &g, unsigned tok_tiles, unsigned row_tiles, hipStream_t st) {
    return g.wide ? launch_gemm3_grid_s<WT, MT, NT, WM, true, KS>(g, tok_tiles, row_tiles, st)
                   : launch_gemm3_grid_s<WT, MT, NT, WM, false, KS>(g, tok_tiles, row_tiles, st);
}

template <int WT>
static int gemm_type(GemmArgs &g, hipStream_t st) {
    // SARDYNE_GEMM_VARIANT picks one tile shape (tests and tuning); default: by shape
    const char *ev = getenv("SARDYNE_GEMM_VARIANT");
    const int variant = ev ? atoi(ev) : 1;
    switch (variant) {
    case 11: return launch_gemm3<WT, 1, 4, 8>(g, st);
    case 12: return launch_gemm3<WT, 1, 2, 4>(g, st);
    case 13: return launch_gemm3<WT, 1, 2, 8>(g, st);
    case 14: return launch_gemm3<WT, 1, 1, 4>(g, st);
    case 15: return launch_gemm3<WT, 1, 4, 4>(g, st);
    case 16: return launch_gemm3<WT, 2, 2, 4>(g, st);
    case 17: return launch_gemm3<WT, 1, 1, 4, 2>(g, st);
    case 18: return launch_gemm3<WT, 1, 1, 8, 2>(g, st);
    case 19: return launch_gemm3<WT, 1, 1, 4, 1, 2>(g, st);
    case 20: return launch_gemm3<WT, 1, 1, 4, 2, 2>(g, st);
    default: break;
    }
    // 128-row workgroup tiles (4 waves of 32 rows) of 64 tokens when there are enough row tiles to
    // fill the GPU twice over with them; else 64-row tiles of 32 tokens, two waves to a row tile
    // splitting each super-block's units (twice the waves for the grids of one wave per SIMD).
    // Measured on the 256- to 22016-row matrices of a 512-token prefill.
    const long r128 = (g.n_rows + 127) / 128, t64 = (g.n_tok + 63) / 64;
    if (r128 * t64 >= 1024) return launch_gemm3<WT, 1, 2, 4>(g, st);
    return launch_gemm3<WT, 1, 1, 4, 2>(g, st);
}

// out[t][row] for rows [a->row0, a->row1) and a->n_tok tokens of Q8_K activations a->xq, through
// the MFMA GEMM; ws: sdy_gemm_ws_bytes(n_tok, n_in) bytes of device scratch.
// The checks and kernel arguments of one sdy_gemm call; the activations' expansion is made first
// unless ws_ready. *empty: an empty row range (nothing to launch).
static int gemm_setup(const sdy_mat *m, const sdy_mv_args *a, void *ws, hipStream_t st, GemmArgs &g, bool *empty) {
    *empty = false;
    if (!sdy_gemm_ok(m, a->n_tok)) return sdy_fail(-1, "gemm: matrix not eligible (type %d)", m->type);
    if (a->row0 < 0 || a->row1 > m->n_rows || a->row0 > a->row1)
        return sdy_fail(-1, "gemm rows [%ld, %ld) outside %ld", a->row0, a->row1, m->n_rows);
    if (a->epilogue == SDY_EPI_SWIGLU && (((a->row1 - a->row0) | a->row0) & 1 || a->bias || a->resid))
        return sdy_fail(-1, "gemm: the SwiGLU epilogue needs an even row range from an even row, no bias, no residual");
    if (a->row0 == a->row1) {
        *empty = true;
        return 0;
    }
    g = gemm_args(m, true);
    const int nb = g.nb, n_tok = a->n_tok;
    const SdyGemmExp e = sdy_gemm_exp(ws, n_tok, g.n_in);
    g.exp_rows = n_tok;
    g.y16 = e.y16;
    g.yd = e.yd;
    g.bs16 = e.bs16;
    if (!a->ws_ready) {
        const long n_sb = (long)n_tok * nb;
        SDY_NOTE_KERNEL(k_gemm_prep);
        hipLaunchKernelGGL(k_gemm_prep, dim3((unsigned)((n_sb * 16 + 255) / 256)), dim3(256), 0, st,
                           (const uint8_t *)a->xq, n_sb, (_Float16 *)g.y16, (float *)g.yd, (_Float16 *)g.bs16);
        if (int rc = sdy_check_launch("gemm_prep")) return rc;
    }
    g.row0 = a->row0;
    g.n_rows = a->row1 - a->row0;
    g.n_tok = n_tok;
    g.out = a->out;
    g.out_stride = a->out_stride;
    g.bias = a->bias;
    g.resid = a->resid;
    g.swiglu = a->epilogue == SDY_EPI_SWIGLU;
    // with a row range the outputs are indexed by row - row0 only for SwiGLU (as in the matvec)
    return 0;
}

extern "C" int sdy_gemm(const sdy_mat *m, const sdy_mv_args *a, void *ws, sdy_stream s) {
    hipStream_t st = (hipStream_t)s;
    GemmArgs g;
    bool empty;
    if (int rc = gemm_setup(m, a, ws, st, g, &empty)) return rc;
    if (empty) return 0;
    return m->type == SDY_Q4_K ? gemm_type<SDY_Q4_K>(g, st) : gemm_type<SDY_Q6_K>(g, st);
}

// the small-grid tile form of gemm_type (64-row tiles of 32 tokens, the unit split)
static bool gemm_small_grid(long n_rows, int n_tok) {
    return ((n_rows + 127) / 128) * (long)((n_tok + 63) / 64) < 1024;
}

template <int WT1, bool WIDE1, int WT2, bool WIDE2>
static int launch_gemm3_pair_s(GemmArgs &g1, GemmArgs &g2, hipStream_t st) {
    constexpr int NT = 1, BN = 32 * NT, YDN = 64, BM = 64;
    constexpr size_t lds = 2 * (size_t)(BN * 512 + YDN * 4 + BN * 32);
    static size_t granted = 0;
    const void *fn = (const void *)k_gemm3_pair<WT1, WIDE1, WT2, WIDE2, 1, NT, 4, 2>;
    int rc = sdy_lds_limit(fn, lds, &granted);
    if (rc) return rc;
    const unsigned tok_tiles = (unsigned)((g1.n_tok + BN - 1) / BN);
    const int gy1 = (int)((g1.n_rows + BM - 1) / BM), gy2 = (int)((g2.n_rows + BM - 1) / BM);
    SDY_NOTE_KERNEL((k_gemm3_pair<WT1, WIDE1, WT2, WIDE2, 1, NT, 4, 2>));
    hipLaunchKernelGGL((k_gemm3_pair<WT1, WIDE1, WT2, WIDE2, 1, NT, 4, 2>), dim3(tok_tiles, (unsigned)(gy1 + gy2)),
                       dim3(256), lds, st, g1, g2, gy1);
    return sdy_check_launch("gemm2");
}

// Two GEMMs over the same activations (a layer's q|k and its v): one launch when the first matrix
// is Q4_K and the second Q6_K, each on the small-grid tile form (the bits of two sdy_gemm calls);
// otherwise, or with SARDYNE_GEMM_VARIANT set, two sdy_gemm calls.
extern "C" int sdy_gemm2(const sdy_mat *m1, const sdy_mv_args *a1, const sdy_mat *m2, const sdy_mv_args *a2, void *ws,
                         sdy_stream s) {
    hipStream_t st = (hipStream_t)s;
    if (a2->xq != a1->xq || a2->n_tok != a1->n_tok || m2->n_in != m1->n_in)
        return sdy_fail(-1, "gemm2: the two GEMMs must read the same activation rows");
    const bool pair = m1->type == SDY_Q4_K && m2->type == SDY_Q6_K && !getenv("SARDYNE_GEMM_VARIANT") &&
                      a1->row1 > a1->row0 && a2->row1 > a2->row0 && gemm_small_grid(a1->row1 - a1->row0, a1->n_tok) &&
                      gemm_small_grid(a2->row1 - a2->row0, a2->n_tok);
    if (!pair) {
        if (int rc = sdy_gemm(m1, a1, ws, s)) return rc;
        sdy_mv_args b = *a2;
        b.ws_ready = 1;  // the expansion the first call made (or found)
        return sdy_gemm(m2, &b, ws, s);
    }
    GemmArgs g1, g2;
    bool e1, e2;
    sdy_mv_args b = *a2;
    b.ws_ready = 1;
    if (int rc = gemm_setup(m1, a1, ws, st, g1, &e1)) return rc;  // (both ranges non-empty here)
    if (int rc = gemm_setup(m2, &b, ws, st, g2, &e2)) return rc;
    if (g1.wide) return g2.wide ? launch_gemm3_pair_s<SDY_Q4_K, true, SDY_Q6_K, true>(g1, g2, st)
                                : launch_gemm3_pair_s<SDY_Q4_K, true, SDY_Q6_K, false>(g1, g2, st);
    return g2.wide ? launch_gemm3_pair_s<SDY_Q4_K, false, SDY_Q6_K, true>(g1, g2, st)
                   : launch_gemm3_pair_s<SDY_Q4_K, false, SDY_Q6_K, false>(g1, g2, st);
}

extern "C" int sdy_gemm_grouped_tile(void) { return 32; }

extern "C" int sdy_gemm_grouped(const sdy_mat *m, long grp_rows, int n_grp, const int *grp_tok, const int *grp_tile,
                                const int *out_row, const int *act_row, int n_act, const sdy_mv_args *a, void *ws,
                                sdy_stream s) {
    hipStream_t st = (hipStream_t)s;
    const int n_tok = a->n_tok;
    if (n_tok <= 0) return 0;
    if (!((m->type == SDY_Q4_K || m->type == SDY_Q6_K) && m->gemm_ok &&
          (size_t)m->n_rows * m->n_units * 16 < 0xFFFFFFFFu))
        return sdy_fail(-1, "gemm_grouped: matrix not eligible (type %d)", m->type);
    if (n_grp < 1 || grp_rows < 1 || (long)n_grp * grp_rows > m->n_rows)
        return sdy_fail(-1, "gemm_grouped: %d groups of %ld rows in %ld rows", n_grp, grp_rows, m->n_rows);
    if (a->bias || a->resid || (a->epilogue == SDY_EPI_SWIGLU && (grp_rows & 1)))
        return sdy_fail(-1, "gemm_grouped: no bias or residual; the SwiGLU epilogue needs an even row count per group");
    if (act_row && (!a->ws_ready || n_act < 1))
        return sdy_fail(-1, "gemm_grouped: activation rows by index read an expansion of n_act >= 1 rows that the "
                            "caller made (ws_ready)");
    GemmArgs g = gemm_args(m, true);
    const SdyGemmExp e = sdy_gemm_exp(ws, act_row ? n_act : n_tok, g.n_in);
    g.exp_rows = act_row ? n_act : n_tok;
    g.y16 = e.y16;
    g.yd = e.yd;
    g.bs16 = e.bs16;
    int rc;
    if (!a->ws_ready) {
        const long n_sb = (long)n_tok * g.nb;
        SDY_NOTE_KERNEL(k_gemm_prep);
        hipLaunchKernelGGL(k_gemm_prep, dim3((unsigned)((n_sb * 16 + 255) / 256)), dim3(256), 0, st,
                           (const uint8_t *)a->xq, n_sb, (_Float16 *)g.y16, (float *)g.yd, (_Float16 *)g.bs16);
        if ((rc = sdy_check_launch("gemm_prep"))) return rc;
    }
    g.row0 = 0;
    g.n_rows = grp_rows;
    g.n_tok = n_tok;
    g.out = a->out;
    g.out_stride = a->out_stride;
    g.bias = a->bias;
    g.resid = a->resid;
    g.swiglu = a->epilogue == SDY_EPI_SWIGLU;
    g.grp_tile = grp_tile;
    g.grp_tok = grp_tok;
    g.out_row = out_row;
    g.act_row = act_row;
    g.grp_rows = grp_rows;
    g.n_grp = n_grp;
    // token tiles: at most one partial tile per group beyond the full ones (the grid's extra
    // workgroups return at once)
    // (128-row tiles, one wave to a row tile: the unit split of the dense GEMM's small grids measured
    // slower here, 38.5 against 36.3 ms for the 30B-A3B-shaped 1024-token prefill)
    constexpr int BN = 32;
    const unsigned tok_tiles = (unsigned)((n_tok + BN - 1) / BN + n_grp - 1);
    const unsigned row_tiles = (unsigned)((grp_rows + 127) / 128);
    return m->type == SDY_Q4_K ? launch_gemm3_grid<SDY_Q4_K, 1, 1, 4, 1>(g, tok_tiles, row_tiles, st)
                               : launch_gemm3_grid<SDY_Q6_K, 1, 1, 4, 1>(g, tok_tiles, row_tiles, st);
}

/* Oracle restatement of the reference's block formats, conversions, dequantisation, activation
 * quantisers and quantized dots. Test infrastructure only (see oracle.h).
 *
 * Reference files restated here: csrc/quant.h, csrc/quant.c, csrc/quant_avx2.c, csrc/ops.c:15-62
 * and csrc/ops.c:211-327.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* ------------------------------------------------------------------ block formats
 * csrc/quant.h:16-56. Field order and sizes are the on-disk GGUF layout. */
typedef struct { uint16_t d; int8_t qs[32]; } orc_q8_0;
typedef struct { uint16_t d; uint8_t qs[16]; } orc_q4_0;
typedef struct { uint16_t d; uint8_t qh[4]; uint8_t qs[16]; } orc_q5_0;
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } orc_q4_K;
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } orc_q6_K;
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } orc_q8_K;

_Static_assert(sizeof(orc_q8_0) == 34, "q8_0");
_Static_assert(sizeof(orc_q4_0) == 18, "q4_0");
_Static_assert(sizeof(orc_q5_0) == 22, "q5_0");
_Static_assert(sizeof(orc_q4_K) == 144, "q4_K");
_Static_assert(sizeof(orc_q6_K) == 210, "q6_K");
_Static_assert(sizeof(orc_q8_K) == 292, "q8_K");

/* ------------------------------------------------------------------ f16 <-> f32
 * csrc/ops.c:15-41: exact widening, subnormals included. Restated arithmetically: a subnormal
 * half is mant * 2^-24, which float represents exactly. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15), e = (h >> 10) & 31u, m = h & 1023u;
    float v;
    if (e == 0) {
        v = (float)m * 0x1p-24f;
        return sign ? -v : v;
    }
    uint32_t bits;
    if (e == 31) bits = 0x7F800000u | (m << 13);
    else bits = ((e + 112u) << 23) | (m << 13);
    memcpy(&v, &bits, 4);
    return sign ? -v : v;
}

/* csrc/ops.c:43-62: round to nearest even; >= 65520 becomes inf; NaN becomes a quiet NaN with the
 * sign kept. Restated with an explicit guard/sticky rounding. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t a = x & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7E00u;
    if (a >= 0x477FF000u) return sign | 0x7C00u;
    int e = (int)(a >> 23) - 127; /* unbiased exponent */
    uint32_t mant = (a & 0x7FFFFFu) | (a >= 0x00800000u ? 0x800000u : 0u);
    if (a == 0) return sign;
    /* value = mant * 2^(e - 23); target unit is 2^-24 for subnormal halves, 2^(e-10) for normal. */
    int shift;
    uint32_t base;
    if (e < -14) { /* subnormal half: quantum 2^-24 */
        shift = -24 - (e - 23);  /* bits to drop from mant */
        base = 0;
    } else {
        shift = 13;
        base = (uint32_t)(e + 15) << 10;
        mant &= 0x7FFFFFu;
    }
    if (e >= -14) {
        uint32_t q = mant >> 13, rem = mant & 0x1FFFu;
        uint32_t r = base | q;
        if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) r++;
        return sign | (uint16_t)r;
    }
    if (shift >= 32) return sign; /* far below half the smallest subnormal */
    uint32_t q = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return sign | (uint16_t)q;
}

void orc_f16_to_f32_n(const uint16_t *x, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(x[i]);
}

#define H2F orc_f16_to_f32

/* ------------------------------------------------------------------ sizes (csrc/ops.c:329-365) */
int orc_block_size(int type) {
    switch (type) {
    case ORC_F32: case ORC_F16: case ORC_BF16: return 1;
    case ORC_Q8_0: case ORC_Q4_0: case ORC_Q5_0: return 32;
    case ORC_Q4_K: case ORC_Q6_K: case ORC_Q8_K: return 256;
    default: return 0;
    }
}

size_t orc_block_bytes(int type) {
    switch (type) {
    case ORC_F32: return 4;
    case ORC_F16: case ORC_BF16: return 2;
    case ORC_Q8_0: return 34;
    case ORC_Q4_0: return 18;
    case ORC_Q5_0: return 22;
    case ORC_Q4_K: return 144;
    case ORC_Q6_K: return 210;
    case ORC_Q8_K: return 292;
    default: return 0;
    }
}

size_t orc_row_size(int type, int n) {
    int b = orc_block_size(type);
    return b ? (size_t)(n / b) * orc_block_bytes(type) : 0;
}

int orc_vec_dot_type(int wtype) {
    if (wtype == ORC_Q8_0 || wtype == ORC_Q4_0 || wtype == ORC_Q5_0) return ORC_Q8_0;
    if (wtype == ORC_Q4_K || wtype == ORC_Q6_K) return ORC_Q8_K;
    return ORC_F32;
}

/* ------------------------------------------------------------------ unpacking helpers */

/* Six-bit scale and min of Q4_K sub-block j (csrc/quant.h:72-80). */
static void q4k_sm(const uint8_t *s, int j, int *sc, int *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* Q6_K values -32..31 in element order (csrc/quant.c:62-75). Element e of a 128-half: column
 * l = e % 32 and quarter k = e / 32; quarters 0/2 use ql[l], 1/3 use ql[l+32]; quarters 2/3 take
 * the high nibble; the two high bits are bits 2k..2k+1 of qh[l]. */
static void q6k_vals(const orc_q6_K *b, int v[256]) {
    for (int half = 0; half < 2; half++) {
        const uint8_t *ql = b->ql + 64 * half, *qh = b->qh + 32 * half;
        for (int e = 0; e < 128; e++) {
            int l = e & 31, k = e >> 5;
            int lo = ql[l + ((k & 1) ? 32 : 0)];
            lo = (k >= 2) ? (lo >> 4) : (lo & 15);
            int hi = (qh[l] >> (2 * k)) & 3;
            v[128 * half + e] = (lo | (hi << 4)) - 32;
        }
    }
}

/* Q5_0 values -16..15 (csrc/quant.c:23-34). */
static void q5_0_vals(const orc_q5_0 *b, int v[32]) {
    uint32_t qh = (uint32_t)b->qh[0] | ((uint32_t)b->qh[1] << 8) | ((uint32_t)b->qh[2] << 16) |
                  ((uint32_t)b->qh[3] << 24);
    for (int e = 0; e < 32; e++) {
        int nib = e < 16 ? (b->qs[e] & 15) : (b->qs[e - 16] >> 4);
        v[e] = (nib | (int)(((qh >> e) & 1u) << 4)) - 16;
    }
}

static void q4_0_vals(const orc_q4_0 *b, int v[32]) {
    for (int e = 0; e < 32; e++) v[e] = (e < 16 ? (b->qs[e] & 15) : (b->qs[e - 16] >> 4)) - 8;
}

/* ------------------------------------------------------------------ dequantisation
 * csrc/quant.c:13-94. Every product is rounded before the subtraction (no contraction). */
static float bf16_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void orc_row_to_f32(const void *row, int type, float *out, size_t n) {
    switch (type) {
    case ORC_F32: memcpy(out, row, n * 4); return;
    case ORC_F16: orc_f16_to_f32_n(row, out, n); return;
    case ORC_BF16:
        for (size_t i = 0; i < n; i++) out[i] = bf16_f32(((const uint16_t *)row)[i]);
        return;
    case ORC_Q8_0: {
        const orc_q8_0 *b = row;
        for (size_t i = 0; i < n / 32; i++) {
            float d = H2F(b[i].d);
            for (int e = 0; e < 32; e++) out[32 * i + e] = (float)b[i].qs[e] * d;
        }
        return;
    }
    case ORC_Q4_0: {
        const orc_q4_0 *b = row;
        int v[32];
        for (size_t i = 0; i < n / 32; i++) {
            float d = H2F(b[i].d);
            q4_0_vals(&b[i], v);
            for (int e = 0; e < 32; e++) out[32 * i + e] = (float)v[e] * d;
        }
        return;
    }
    case ORC_Q5_0: {
        const orc_q5_0 *b = row;
        int v[32];
        for (size_t i = 0; i < n / 32; i++) {
            float d = H2F(b[i].d);
            q5_0_vals(&b[i], v);
            for (int e = 0; e < 32; e++) out[32 * i + e] = (float)v[e] * d;
        }
        return;
    }
    case ORC_Q4_K: {
        const orc_q4_K *b = row;
        for (size_t i = 0; i < n / 256; i++) {
            float d = H2F(b[i].d), dmin = H2F(b[i].dmin);
            for (int j = 0; j < 8; j++) { /* sub-block j: byte group j/2, low nibble if j even */
                int sc, m;
                q4k_sm(b[i].scales, j, &sc, &m);
                float dj = d * (float)sc, mj = dmin * (float)m;
                const uint8_t *q = b[i].qs + 32 * (j / 2);
                for (int l = 0; l < 32; l++) {
                    int nib = (j & 1) ? (q[l] >> 4) : (q[l] & 15);
                    float prod = dj * (float)nib;
                    out[256 * i + 32 * j + l] = prod - mj;
                }
            }
        }
        return;
    }
    case ORC_Q6_K: {
        const orc_q6_K *b = row;
        int v[256];
        for (size_t i = 0; i < n / 256; i++) {
            float d = H2F(b[i].d);
            q6k_vals(&b[i], v);
            for (int e = 0; e < 256; e++) {
                float ds = d * (float)b[i].scales[e / 16];
                out[256 * i + e] = ds * (float)v[e];
            }
        }
        return;
    }
    default: return;
    }
}

/* ------------------------------------------------------------------ activation quantisers */

/* csrc/quant.c:98-108: d = amax/127 stored as f16; q = roundf(x / d) computed with the float
 * reciprocal of the unrounded d; roundf rounds halves away from zero. */
void orc_quant_q8_0(const float *x, void *dst, int n) {
    orc_q8_0 *y = dst;
    for (int i = 0; i < n / 32; i++) {
        const float *xb = x + 32 * i;
        float amax = 0.0f;
        for (int e = 0; e < 32; e++) {
            float a = fabsf(xb[e]);
            amax = a > amax ? a : amax;
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = orc_f32_to_f16(d);
        for (int e = 0; e < 32; e++) y[i].qs[e] = (int8_t)roundf(xb[e] * id);
    }
}

/* csrc/quant.c:111-144: the first element of largest magnitude sets the signed max;
 * iscale = -127/max; q = round-half-even(iscale*x) clamped above at 127; d = 1/iscale;
 * bsums are the sums of 16-element groups; an all-zero block becomes all zero bytes. */
void orc_quant_q8_K(const float *x, void *dst, int n) {
    orc_q8_K *y = dst;
    for (int i = 0; i < n / 256; i++) {
        const float *xb = x + 256 * i;
        float amax = 0.0f, vmax = 0.0f;
        for (int e = 0; e < 256; e++)
            if (fabsf(xb[e]) > amax) {
                amax = fabsf(xb[e]);
                vmax = xb[e];
            }
        if (amax == 0.0f) {
            memset(&y[i], 0, sizeof(y[i]));
            continue;
        }
        float iscale = -127.0f / vmax;
        for (int e = 0; e < 256; e++) {
            long r = lrintf(iscale * xb[e]); /* current mode: round to nearest even */
            y[i].qs[e] = (int8_t)(r < 127 ? r : 127);
        }
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int e = 0; e < 16; e++) s += y[i].qs[16 * g + e];
            y[i].bsums[g] = (int16_t)s;
        }
        y[i].d = 1.0f / iscale;
    }
}

void orc_quantize_rows(int vtype, const float *x, void *xq, int n_in, int t0, int t1) {
    size_t row = orc_row_size(vtype, n_in);
    for (int t = t0; t < t1; t++) {
        void *dst = (uint8_t *)xq + (size_t)t * row;
        if (vtype == ORC_Q8_0) orc_quant_q8_0(x + (size_t)t * n_in, dst, n_in);
        else orc_quant_q8_K(x + (size_t)t * n_in, dst, n_in);
    }
}

/* ------------------------------------------------------------------ scalar dots (csrc/quant.c:148-235) */

static int q0_vals(int wtype, const void *blk, int v[32]) {
    if (wtype == ORC_Q8_0) {
        const orc_q8_0 *b = blk;
        for (int e = 0; e < 32; e++) v[e] = b->qs[e];
        return 0;
    }
    if (wtype == ORC_Q4_0) {
        q4_0_vals(blk, v);
        return 8;
    }
    q5_0_vals(blk, v);
    return 16;
}

/* Integer part and f16 scale of Q0 block i. */
static int32_t q0_isum(int wtype, const void *w, int i, const orc_q8_0 *x, float *dw) {
    const uint8_t *blk = (const uint8_t *)w + (size_t)i * orc_block_bytes(wtype);
    int v[32];
    q0_vals(wtype, blk, v);
    uint16_t d;
    memcpy(&d, blk, 2); /* every Q0 block starts with its f16 scale */
    *dw = H2F(d);
    int32_t s = 0;
    for (int e = 0; e < 32; e++) s += v[e] * x[i].qs[e];
    return s;
}

/* K-quant super-block integer parts (csrc/quant.c:191-235). */
static void q4k_parts(const orc_q4_K *a, const orc_q8_K *b, int32_t *isum, int32_t *msum) {
    int32_t is = 0, ms = 0;
    for (int j = 0; j < 8; j++) {
        int sc, m;
        q4k_sm(a->scales, j, &sc, &m);
        const uint8_t *q = a->qs + 32 * (j / 2);
        int32_t s = 0;
        for (int l = 0; l < 32; l++) s += ((j & 1) ? (q[l] >> 4) : (q[l] & 15)) * b->qs[32 * j + l];
        is += sc * s;
        ms += m * (b->bsums[2 * j] + b->bsums[2 * j + 1]);
    }
    *isum = is;
    *msum = ms;
}

static int32_t q6k_isum(const orc_q6_K *a, const orc_q8_K *b) {
    int v[256];
    q6k_vals(a, v);
    int32_t is = 0;
    for (int g = 0; g < 16; g++) {
        int32_t s = 0;
        for (int e = 0; e < 16; e++) s += v[16 * g + e] * b->qs[16 * g + e];
        is += a->scales[g] * s;
    }
    return is;
}

/* f32 combine of one super-block, in the expression order of csrc/quant.h:84-91. */
static float q4k_comb(float acc, float yd, float d, float dmin, int32_t isum, int32_t msum) {
    float dall = yd * d, dmn = yd * dmin;
    float t1 = dall * (float)isum, t2 = dmn * (float)msum;
    return acc + (t1 - t2);
}

static float q6k_comb(float acc, float yd, float d, int32_t isum) {
    float yd_d = yd * d;
    return acc + yd_d * (float)isum;
}

static float dot_kquant(int wtype, const void *w, const void *xq, int n) {
    const orc_q8_K *b = xq;
    float acc = 0.0f;
    for (int i = 0; i < n / 256; i++) {
        if (wtype == ORC_Q4_K) {
            const orc_q4_K *a = (const orc_q4_K *)w + i;
            int32_t is, ms;
            q4k_parts(a, &b[i], &is, &ms);
            acc = q4k_comb(acc, b[i].d, H2F(a->d), H2F(a->dmin), is, ms);
        } else {
            const orc_q6_K *a = (const orc_q6_K *)w + i;
            acc = q6k_comb(acc, b[i].d, H2F(a->d), q6k_isum(a, &b[i]));
        }
    }
    return acc;
}

float orc_dot_scalar(int wtype, const void *w, const void *xq, int n) {
    if (wtype == ORC_Q4_K || wtype == ORC_Q6_K) return dot_kquant(wtype, w, xq, n);
    const orc_q8_0 *x = xq;
    float acc = 0.0f;
    for (int i = 0; i < n / 32; i++) {
        float dw;
        int32_t s = q0_isum(wtype, w, i, x, &dw);
        float dd = dw * H2F(x[i].d);
        acc += (float)s * dd;
    }
    return acc;
}

/* ------------------------------------------------------------------ AVX2 order of the Q0 dots
 * csrc/quant_avx2.c:90-205. Emulated lane by lane: a block contributes to lane v the exact integer
 * sum of its elements 4v..4v+3 (of the biased unsigned values for Q4_0/Q5_0), converted to float
 * and fused-multiply-added with the float product d_w*d_x. */

static float hsum8(const float v[8]) { /* csrc/quant_avx2.c:22-27 reduction tree */
    float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
    float t0 = s0 + s2, t1 = s1 + s3;
    return t0 + t1;
}

static int q0_bias(int wtype) { return wtype == ORC_Q4_0 ? 8 : wtype == ORC_Q5_0 ? 16 : 0; }

/* lane terms of block i: unsigned biased values for Q4_0/Q5_0, signed values for Q8_0 */
static void q0_lane_terms(int wtype, const void *w, int i, const orc_q8_0 *x, float term[8]) {
    const uint8_t *blk = (const uint8_t *)w + (size_t)i * orc_block_bytes(wtype);
    int v[32];
    int bias = q0_vals(wtype, blk, v);
    for (int lane = 0; lane < 8; lane++) {
        int32_t s = 0;
        for (int e = 4 * lane; e < 4 * lane + 4; e++) s += (v[e] + bias) * x[i].qs[e];
        term[lane] = (float)s;
    }
}

static uint16_t q0_d(int wtype, const void *w, int i) {
    uint16_t d;
    memcpy(&d, (const uint8_t *)w + (size_t)i * orc_block_bytes(wtype), 2);
    return d;
}

/* activation_info (csrc/quant_avx2.c:90-97) */
static void act_info(const orc_q8_0 *x, int nb, float *dx, float *sx) {
    for (int i = 0; i < nb; i++) {
        dx[i] = H2F(x[i].d);
        int s = 0;
        for (int e = 0; e < 32; e++) s += x[i].qs[e];
        sx[i] = dx[i] * (float)s;
    }
}

/* dot_rows_##S (csrc/quant_avx2.c:107-129): two accumulators, even and odd blocks */
static float q0_dot_rows(int wtype, const void *w, const orc_q8_0 *x, const float *dx, const float *sx, int nb) {
    float acc0[8] = {0}, acc1[8] = {0}, term[8];
    float corr = 0.0f;
    int bias = q0_bias(wtype), i = 0;
    for (; i + 2 <= nb; i += 2) {
        float d0 = H2F(q0_d(wtype, w, i)), d1 = H2F(q0_d(wtype, w, i + 1));
        float s0 = d0 * dx[i], s1 = d1 * dx[i + 1];
        q0_lane_terms(wtype, w, i, x, term);
        for (int l = 0; l < 8; l++) acc0[l] = fmaf(s0, term[l], acc0[l]);
        q0_lane_terms(wtype, w, i + 1, x, term);
        for (int l = 0; l < 8; l++) acc1[l] = fmaf(s1, term[l], acc1[l]);
        if (bias) {
            float p0 = d0 * sx[i], p1 = d1 * sx[i + 1];
            corr += p0 + p1;
        }
    }
    for (; i < nb; i++) {
        float d0 = H2F(q0_d(wtype, w, i));
        float s0 = d0 * dx[i];
        q0_lane_terms(wtype, w, i, x, term);
        for (int l = 0; l < 8; l++) acc0[l] = fmaf(s0, term[l], acc0[l]);
        if (bias) corr += d0 * sx[i];
    }
    float sum[8];
    for (int l = 0; l < 8; l++) sum[l] = acc0[l] + acc1[l];
    float biasf = (float)bias;
    return hsum8(sum) - biasf * corr;
}

#define ORC_DX_MAX 8192

/* quant_dot_##S##_avx2 (csrc/quant_avx2.c:131-144), including the chunking of very long rows */
static float q0_dot_avx2(int wtype, const void *w, const void *xq, int n) {
    int nb = n / 32;
    if (nb > ORC_DX_MAX / 4) {
        float s = 0.0f;
        for (int i = 0; i < nb; i += ORC_DX_MAX / 4) {
            int m = nb - i < ORC_DX_MAX / 4 ? nb - i : ORC_DX_MAX / 4;
            s += q0_dot_avx2(wtype, (const uint8_t *)w + (size_t)i * orc_block_bytes(wtype),
                             (const orc_q8_0 *)xq + i, m * 32);
        }
        return s;
    }
    float *dx = malloc(sizeof(float) * (size_t)(nb ? nb : 1)), *sx = malloc(sizeof(float) * (size_t)(nb ? nb : 1));
    act_info(xq, nb, dx, sx);
    float r = q0_dot_rows(wtype, w, xq, dx, sx, nb);
    free(dx);
    free(sx);
    return r;
}

float orc_dot_avx2(int wtype, const void *w, const void *xq, int n) {
    if (wtype == ORC_Q4_K || wtype == ORC_Q6_K) return dot_kquant(wtype, w, xq, n);
    return q0_dot_avx2(wtype, w, xq, n);
}

/* quant_matmul_rows_##S##_avx2 (csrc/quant_avx2.c:146-201): four tokens share one pass over a
 * row's blocks with one accumulator each (no even/odd split); leftover tokens take dot_rows. */
static void q0_matmul_avx2(float *out, const void *xq, const void *w, int wtype, int n_tok, int n_in, int n_out,
                           int row0, int row1) {
    int nb = n_in / 32;
    const orc_q8_0 *x = xq;
    size_t wrow = orc_row_size(wtype, n_in);
    if ((size_t)n_tok * nb > ORC_DX_MAX) {
        int step = ORC_DX_MAX / nb < 4 ? 1 : ORC_DX_MAX / nb / 4 * 4;
        if (nb > ORC_DX_MAX) step = 0;
        if (step == 0) {
            for (int j = row0; j < row1; j++)
                for (int t = 0; t < n_tok; t++)
                    out[(size_t)t * n_out + j] = q0_dot_avx2(wtype, (const uint8_t *)w + (size_t)j * wrow,
                                                             x + (size_t)t * nb, n_in);
            return;
        }
        for (int t = 0; t < n_tok; t += step) {
            int m = n_tok - t < step ? n_tok - t : step;
            q0_matmul_avx2(out + (size_t)t * n_out, x + (size_t)t * nb, w, wtype, m, n_in, n_out, row0, row1);
        }
        return;
    }
    size_t tot = (size_t)n_tok * nb;
    float *dx = malloc(sizeof(float) * (tot ? tot : 1)), *sx = malloc(sizeof(float) * (tot ? tot : 1));
    act_info(x, (int)tot, dx, sx);
    int bias = q0_bias(wtype);
    float biasf = (float)bias, term[8];
    for (int j = row0; j < row1; j++) {
        const uint8_t *wj = (const uint8_t *)w + (size_t)j * wrow;
        int t = 0;
        for (; t + 4 <= n_tok; t += 4) {
            float a[4][8] = {{0}}, c[4] = {0};
            for (int i = 0; i < nb; i++) {
                float dw = H2F(q0_d(wtype, wj, i));
                for (int tt = 0; tt < 4; tt++) {
                    const orc_q8_0 *xt = x + (size_t)(t + tt) * nb;
                    float s = dw * dx[(size_t)(t + tt) * nb + i];
                    q0_lane_terms(wtype, wj, i, xt, term);
                    for (int l = 0; l < 8; l++) a[tt][l] = fmaf(s, term[l], a[tt][l]);
                }
                if (bias)
                    for (int tt = 0; tt < 4; tt++) c[tt] += dw * sx[(size_t)(t + tt) * nb + i];
            }
            for (int tt = 0; tt < 4; tt++) out[(size_t)(t + tt) * n_out + j] = hsum8(a[tt]) - biasf * c[tt];
        }
        for (; t < n_tok; t++)
            out[(size_t)t * n_out + j] = q0_dot_rows(wtype, wj, x + (size_t)t * nb, dx + (size_t)t * nb,
                                                     sx + (size_t)t * nb, nb);
    }
    free(dx);
    free(sx);
}

/* op_matmul_q_rows (csrc/ops.c:403-419) with the reference's kernel choice. */
void orc_matmul_q_rows(float *out, const void *xq, const void *w, int wtype, int n_tok, int n_in, int n_out,
                       int row0, int row1, int simd) {
    if (simd && (wtype == ORC_Q8_0 || wtype == ORC_Q4_0 || wtype == ORC_Q5_0)) {
        q0_matmul_avx2(out, xq, w, wtype, n_tok, n_in, n_out, row0, row1);
        return;
    }
    size_t wrow = orc_row_size(wtype, n_in), xrow = orc_row_size(orc_vec_dot_type(wtype), n_in);
#pragma omp parallel for schedule(static) if ((row1 - row0) * (size_t)n_tok * n_in > (1u << 22))
    for (int j = row0; j < row1; j++) {
        const uint8_t *wj = (const uint8_t *)w + (size_t)j * wrow;
        for (int t = 0; t < n_tok; t++)
            out[(size_t)t * n_out + j] = orc_dot_scalar(wtype, wj, (const uint8_t *)xq + (size_t)t * xrow, n_in);
    }
}

/* Oracle restatement of the reference's float kernels. Test infrastructure only (see oracle.h).
 *
 * Reference files restated here: csrc/ops.c:185-229 (scalar kernels), csrc/ops.c:387-392 and
 * csrc/ops_avx2.c:26-147 (AVX2 matmul/dot/axpy, emulated lane by lane), csrc/ops.c:329-423
 * (bias, norm, softmax, SiLU, RoPE, attention).
 */
#include <math.h>
#include <string.h>

#include "oracle.h"

static float bf16_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float elem(const void *w, int wtype, size_t i) {
    if (wtype == ORC_F32) return ((const float *)w)[i];
    if (wtype == ORC_F16) return orc_f16_to_f32(((const uint16_t *)w)[i]);
    return bf16_f32(((const uint16_t *)w)[i]);
}

static const void *row_ptr(const void *w, int wtype, size_t j, int n_in) {
    size_t es = wtype == ORC_F32 ? 4 : 2;
    return (const uint8_t *)w + j * (size_t)n_in * es;
}

/* 8-lane reduction tree of csrc/ops_avx2.c:27-32 */
static float hsum8(const float v[8]) {
    float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
    float t0 = s0 + s2, t1 = s1 + s3;
    return t0 + t1;
}

/* DEFINE_SCALAR_DOT (csrc/ops.c:189-201): four running sums, combined as (s0+s1)+(s2+s3). */
static float dot_scalar(const float *x, const void *w, int wtype, int n) {
    float s[4] = {0, 0, 0, 0};
    int i = 0;
    for (; i + 4 <= n; i += 4)
        for (int k = 0; k < 4; k++) {
            float p = x[i + k] * elem(w, wtype, (size_t)i + k);
            s[k] += p;
        }
    for (; i < n; i++) {
        float p = x[i] * elem(w, wtype, (size_t)i);
        s[0] += p;
    }
    float a = s[0] + s[1], b = s[2] + s[3];
    return a + b;
}

/* dot_##S (csrc/ops_avx2.c:61-74): four 8-lane FMA chains over 32-element steps, then 8-element
 * steps into the first chain, the lane-wise sum (a0+a1)+(a2+a3), the 8-lane tree, a scalar tail. */
static float dot_avx2(const float *x, const void *w, int wtype, int n) {
    float a[4][8] = {{0}};
    int i = 0;
    for (; i + 32 <= n; i += 32)
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 8; l++) {
                size_t k = (size_t)i + 8 * c + l;
                a[c][l] = fmaf(elem(w, wtype, k), x[k], a[c][l]);
            }
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) a[0][l] = fmaf(elem(w, wtype, (size_t)i + l), x[i + l], a[0][l]);
    float v[8];
    for (int l = 0; l < 8; l++) {
        float p = a[0][l] + a[1][l], q = a[2][l] + a[3][l];
        v[l] = p + q;
    }
    float s = hsum8(v);
    for (; i < n; i++) {
        float p = x[i] * elem(w, wtype, (size_t)i);
        s += p;
    }
    return s;
}

/* block_2x4_##S (csrc/ops_avx2.c:76-111): two rows times four tokens, one 8-lane FMA chain each. */
static void block_2x4(float *out, const float *x, const void *w0, const void *w1, int wtype, int n_in, int n_out) {
    float c[2][4][8] = {{{0}}};
    int i = 0;
    for (; i + 8 <= n_in; i += 8)
        for (int l = 0; l < 8; l++) {
            float b0 = elem(w0, wtype, (size_t)i + l), b1 = elem(w1, wtype, (size_t)i + l);
            for (int t = 0; t < 4; t++) {
                float a = x[(size_t)t * n_in + i + l];
                c[0][t][l] = fmaf(b0, a, c[0][t][l]);
                c[1][t][l] = fmaf(b1, a, c[1][t][l]);
            }
        }
    float s[2][4];
    for (int r = 0; r < 2; r++)
        for (int t = 0; t < 4; t++) s[r][t] = hsum8(c[r][t]);
    for (; i < n_in; i++) {
        float e0 = elem(w0, wtype, (size_t)i), e1 = elem(w1, wtype, (size_t)i);
        for (int t = 0; t < 4; t++) {
            float a = x[(size_t)t * n_in + i];
            float p0 = e0 * a, p1 = e1 * a;
            s[0][t] += p0;
            s[1][t] += p1;
        }
    }
    for (int t = 0; t < 4; t++) {
        out[(size_t)t * n_out] = s[0][t];
        out[(size_t)t * n_out + 1] = s[1][t];
    }
}

/* op_matmul_rows (csrc/ops.c:387-392) with the AVX2 kernel of csrc/ops_avx2.c:113-134 or the
 * scalar one of csrc/ops.c:210-223. */
void orc_matmul_rows(float *out, const float *x, const void *w, int wtype, int n_tok, int n_in, int n_out,
                     int row0, int row1, int simd) {
    if (!simd) {
        for (int j = row0; j < row1; j++)
            for (int t = 0; t < n_tok; t++)
                out[(size_t)t * n_out + j] = dot_scalar(x + (size_t)t * n_in, row_ptr(w, wtype, (size_t)j, n_in),
                                                        wtype, n_in);
        return;
    }
    int j = row0;
    if (n_tok >= 4) {
        for (; j + 2 <= row1; j += 2) {
            const void *w0 = row_ptr(w, wtype, (size_t)j, n_in), *w1 = row_ptr(w, wtype, (size_t)j + 1, n_in);
            int t = 0;
            for (; t + 4 <= n_tok; t += 4)
                block_2x4(out + (size_t)t * n_out + j, x + (size_t)t * n_in, w0, w1, wtype, n_in, n_out);
            for (; t < n_tok; t++) {
                out[(size_t)t * n_out + j] = dot_avx2(x + (size_t)t * n_in, w0, wtype, n_in);
                out[(size_t)t * n_out + j + 1] = dot_avx2(x + (size_t)t * n_in, w1, wtype, n_in);
            }
        }
    }
    for (; j < row1; j++)
        for (int t = 0; t < n_tok; t++)
            out[(size_t)t * n_out + j] = dot_avx2(x + (size_t)t * n_in, row_ptr(w, wtype, (size_t)j, n_in), wtype, n_in);
}

float orc_dot_f32(const float *a, const float *b, int n, int simd) {
    return simd ? dot_avx2(a, b, ORC_F32, n) : dot_scalar(a, b, ORC_F32, n);
}

/* op_axpy: csrc/ops.c:227-229 (scalar) and csrc/ops_avx2.c:142-147 (fused in 8-lane steps) */
void orc_axpy(float *y, float a, const float *x, int n, int simd) {
    int i = 0;
    if (simd)
        for (; i + 8 <= n; i += 8)
            for (int l = 0; l < 8; l++) y[i + l] = fmaf(a, x[i + l], y[i + l]);
    for (; i < n; i++) {
        float p = a * x[i];
        y[i] += p;
    }
}

/* csrc/ops.c:346-351: sum of squares in double, scale rounded to float, out = (x*scale)*w */
void orc_rmsnorm(float *out, const float *x, const float *w, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
    double mean = ss / (double)n + (double)eps;
    float scale = (float)(1.0 / sqrt(mean));
    for (int i = 0; i < n; i++) {
        float t = x[i] * scale;
        out[i] = t * w[i];
    }
}

/* csrc/ops.c:353-364: max-subtracted expf, double sum, multiply by the float reciprocal */
void orc_softmax(float *x, int n) {
    float mx = x[0];
    for (int i = 1; i < n; i++) mx = x[i] > mx ? x[i] : mx;
    double sum = 0.0;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum += (double)x[i];
    }
    float inv = (float)(1.0 / sum);
    for (int i = 0; i < n; i++) x[i] *= inv;
}

/* csrc/ops.c:366-371 */
void orc_silu_mul(float *gate, const float *up, int n) {
    for (int i = 0; i < n; i++) {
        float g = gate[i];
        float s = g / (1.0f + expf(-g));
        gate[i] = s * up[i];
    }
}

/* csrc/ops.c:375-386: angles in double, rounded to float */
void orc_rope_table(float *cos_out, float *sin_out, int n_pos, int head_dim, float theta) {
    int half = head_dim / 2;
    for (int i = 0; i < half; i++) {
        double inv_freq = 1.0 / pow((double)theta, (double)(2 * i) / (double)head_dim);
        for (int p = 0; p < n_pos; p++) {
            double ang = (double)p * inv_freq;
            cos_out[(size_t)p * half + i] = (float)cos(ang);
            sin_out[(size_t)p * half + i] = (float)sin(ang);
        }
    }
}

/* csrc/ops.c:388-401: pairs (2i, 2i+1) when interleaved, else (i, i + hd/2) */
void orc_rope(float *x, int n_heads, int head_dim, const float *cos, const float *sin, int interleaved) {
    int half = head_dim / 2;
    for (int h = 0; h < n_heads; h++) {
        float *v = x + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            int ia = interleaved ? 2 * i : i, ib = interleaved ? 2 * i + 1 : i + half;
            float a = v[ia], b = v[ib];
            float ac = a * cos[i], bs = b * sin[i], as = a * sin[i], bc = b * cos[i];
            v[ia] = ac - bs;
            v[ib] = as + bc;
        }
    }
}

/* csrc/ops.c:405-423: per head, scaled dots, softmax, sum of p*v by axpy; GQA head h reads KV head
 * h / (n_head / n_kv_head). */
void orc_attention(float *out, const float *q, const float *k_cache, const float *v_cache, int n_head,
                   int n_kv_head, int head_dim, int n_kv, int stride, float *scores, int simd) {
    int n_rep = n_head / n_kv_head;
    float scale = 1.0f / sqrtf((float)head_dim);
    for (int h = 0; h < n_head; h++) {
        size_t kv = (size_t)(h / n_rep) * stride * head_dim;
        const float *qh = q + (size_t)h * head_dim, *k = k_cache + kv, *v = v_cache + kv;
        float *o = out + (size_t)h * head_dim;
        for (int j = 0; j < n_kv; j++) scores[j] = orc_dot_f32(qh, k + (size_t)j * head_dim, head_dim, simd) * scale;
        orc_softmax(scores, n_kv);
        memset(o, 0, sizeof(float) * (size_t)head_dim);
        for (int j = 0; j < n_kv; j++) orc_axpy(o, scores[j], v + (size_t)j * head_dim, head_dim, simd);
    }
}

/* Kernel-level entry points of the public ABI (csrc/ops.h:24-74 of the reference): host pointers
 * in and out, computation on the GPU. Each call uploads its operands, runs the gfx950 kernel and
 * copies the result back; the reference's tests and tools call these to check single kernels.
 *
 * These functions have no error return in the reference's ABI. A GPU failure here (no device,
 * out of memory, a HIP error) is reported on stderr and aborts the process: there is no CPU
 * fallback to return instead.
 */
#define _POSIX_C_SOURCE 200809L
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sardyne.h"
#include "sdy_ops.h"
#include "sdy_shim.h"

static sdy_stream g_stream;
static int g_simd = 1;

static void die(const char *what) {
    fprintf(stderr, "libsardyne: %s failed on the GPU: %s\n", what, sdy_last_error());
    abort();
}

#define CK(call, what)         \
    do {                       \
        if ((call) != 0) die(what); \
    } while (0)

static sdy_stream stream(void) {
    if (!g_stream) CK(sdy_stream_new(&g_stream), "stream creation");
    return g_stream;
}

static void *dalloc(size_t n) {
    void *p = NULL;
    CK(sdy_malloc(&p, n), "device allocation");
    return p;
}

static void *dup_to_dev(const void *h, size_t n) {
    void *d = dalloc(n);
    CK(sdy_h2d(d, h, n, stream()), "upload");
    return d;
}

static void to_host(void *h, const void *d, size_t n) {
    CK(sdy_d2h(h, d, n, stream()), "download");
    CK(sdy_sync(stream()), "synchronize");
}

static int is_quant(int t) { return t == OP_Q8_0 || t == OP_Q4_0 || t == OP_Q5_0 || t == OP_Q4_K || t == OP_Q6_K; }

int op_simd(void) { return g_simd; }
int op_set_simd(int enable) {
    g_simd = enable != 0;
    return g_simd;
}

/* csrc/ops.c:329-357 */
static int block_elems(int t) {
    switch (t) {
    case OP_F32: case OP_F16: case OP_BF16: return 1;
    case OP_Q8_0: case OP_Q4_0: case OP_Q5_0: return 32;
    case OP_Q4_K: case OP_Q6_K: case OP_Q8_K: return 256;
    default: return 0;
    }
}

static size_t block_size_bytes(int t) {
    switch (t) {
    case OP_F32: return 4;
    case OP_F16: case OP_BF16: return 2;
    case OP_Q8_0: return 34;
    case OP_Q4_0: return 18;
    case OP_Q5_0: return 22;
    case OP_Q4_K: return 144;
    case OP_Q6_K: return 210;
    case OP_Q8_K: return 292;
    default: return 0;
    }
}

size_t op_row_size(int type, int n) {
    int b = block_elems(type);
    return b ? (size_t)(n / b) * block_size_bytes(type) : 0;
}

static int vec_dot_type(int wtype) {
    if (wtype == OP_Q8_0 || wtype == OP_Q4_0 || wtype == OP_Q5_0) return OP_Q8_0;
    if (wtype == OP_Q4_K || wtype == OP_Q6_K) return OP_Q8_K;
    return OP_F32;
}

void op_f16_to_f32_n(const uint16_t *x, float *out, size_t n) {
    if (!n) return;
    void *dx = dup_to_dev(x, n * 2);
    float *dout = dalloc(n * 4);
    CK(sdy_f16_to_f32(dx, dout, (long)n, stream()), "f16_to_f32");
    to_host(out, dout, n * 4);
    sdy_free(dx);
    sdy_free(dout);
}

uint16_t op_f32_to_f16(float f) {
    float *dx = dup_to_dev(&f, 4);
    uint16_t *dout = dalloc(2), h;
    CK(sdy_f32_to_f16(dx, dout, 1, stream()), "f32_to_f16");
    to_host(&h, dout, 2);
    sdy_free(dx);
    sdy_free(dout);
    return h;
}

void op_row_to_f32(const void *row, int type, float *out, size_t n) {
    if (!n) return;
    size_t raw = op_row_size(type, (int)n);
    if (!raw) die("op_row_to_f32 (unsupported type)");
    sdy_mat m;
    CK(sdy_mat_upload(&m, type, (int)n, 1, row, stream()), "row upload");
    float *dout = dalloc(n * 4);
    CK(sdy_dequant_rows(&m, 0, 1, dout, stream()), "dequant");
    to_host(out, dout, n * 4);
    sdy_mat_free(&m);
    sdy_free(dout);
}

void op_quantize_rows(int vtype, const float *x, void *xq, int n_in, int t0, int t1) {
    if (t1 <= t0) return;
    int n_tok = t1 - t0;
    size_t row = op_row_size(vtype, n_in);
    float *dx = dup_to_dev(x + (size_t)t0 * n_in, (size_t)n_tok * n_in * 4);
    void *dq = dalloc(row * n_tok);
    CK(sdy_quantize(vtype, dx, dq, n_in, n_tok, stream()), "quantize");
    to_host((uint8_t *)xq + (size_t)t0 * row, dq, row * n_tok);
    sdy_free(dx);
    sdy_free(dq);
}

/* rows [row0, row1) of out[n_tok][n_out]; the other rows of out are left untouched */
static void matvec_host(float *out, const void *act, int act_is_f32, const void *w, int wtype, int n_tok, int n_in,
                        int n_out, int row0, int row1) {
    if (row1 <= row0 || n_tok <= 0) return;
    sdy_mat m;
    CK(sdy_mat_upload(&m, wtype, n_in, n_out, w, stream()), "weight upload");
    size_t act_bytes = act_is_f32 ? (size_t)n_tok * n_in * 4 : op_row_size(vec_dot_type(wtype), n_in) * n_tok;
    void *da = dup_to_dev(act, act_bytes);
    float *dout = dup_to_dev(out, (size_t)n_tok * n_out * 4);
    sdy_mv_args a;
    memset(&a, 0, sizeof(a));
    if (act_is_f32) a.x = da;
    else a.xq = da;
    a.n_tok = n_tok;
    a.out = dout;
    a.out_stride = n_out;
    a.row0 = row0;
    a.row1 = row1;
    CK(sdy_matvec(&m, &a, stream()), "matvec");
    to_host(out, dout, (size_t)n_tok * n_out * 4);
    sdy_mat_free(&m);
    sdy_free(da);
    sdy_free(dout);
}

void op_matmul_q_rows(float *out, const void *xq, const void *w, int wtype, int n_tok, int n_in, int n_out, int row0,
                      int row1) {
    if (!is_quant(wtype)) die("op_matmul_q_rows (weight type is not quantized)");
    matvec_host(out, xq, 0, w, wtype, n_tok, n_in, n_out, row0, row1);
}

float op_vec_dot_q(int wtype, const void *w, const void *xq, int n) {
    float r = 0.0f;
    if (!is_quant(wtype)) die("op_vec_dot_q (weight type is not quantized)");
    matvec_host(&r, xq, 0, w, wtype, 1, n, 1, 0, 1);
    return r;
}

void op_matmul_rows(float *out, const float *x, const void *w, int wtype, int n_tok, int n_in, int n_out, int row0,
                    int row1) {
    if (wtype != OP_F32 && wtype != OP_F16 && wtype != OP_BF16) die("op_matmul_rows (weight type)");
    matvec_host(out, x, 1, w, wtype, n_tok, n_in, n_out, row0, row1);
}

void op_matmul(float *out, const float *x, const void *w, int wtype, int n_tok, int n_in, int n_out) {
    int vt = vec_dot_type(wtype);
    if (vt == OP_F32) {
        op_matmul_rows(out, x, w, wtype, n_tok, n_in, n_out, 0, n_out);
        return;
    }
    if (n_tok <= 0 || n_out <= 0) return;
    size_t row = op_row_size(vt, n_in);
    float *dx = dup_to_dev(x, (size_t)n_tok * n_in * 4);
    void *dq = dalloc(row * n_tok);
    CK(sdy_quantize(vt, dx, dq, n_in, n_tok, stream()), "quantize");
    sdy_mat m;
    CK(sdy_mat_upload(&m, wtype, n_in, n_out, w, stream()), "weight upload");
    float *dout = dalloc((size_t)n_tok * n_out * 4);
    sdy_mv_args a;
    memset(&a, 0, sizeof(a));
    a.xq = dq;
    a.n_tok = n_tok;
    a.out = dout;
    a.out_stride = n_out;
    a.row0 = 0;
    a.row1 = n_out;
    CK(sdy_matvec(&m, &a, stream()), "matvec");
    to_host(out, dout, (size_t)n_tok * n_out * 4);
    sdy_mat_free(&m);
    sdy_free(dx);
    sdy_free(dq);
    sdy_free(dout);
}

float op_dot_f32(const float *a, const float *b, int n) {
    float r = 0.0f;
    if (n <= 0) return r;
    float *da = dup_to_dev(a, (size_t)n * 4), *db = dup_to_dev(b, (size_t)n * 4), *dr = dalloc(4);
    CK(sdy_dot(da, db, n, dr, stream()), "dot");
    to_host(&r, dr, 4);
    sdy_free(da);
    sdy_free(db);
    sdy_free(dr);
    return r;
}

void op_axpy(float *y, float a, const float *x, int n) {
    if (n <= 0) return;
    float *dy = dup_to_dev(y, (size_t)n * 4), *dx = dup_to_dev(x, (size_t)n * 4);
    CK(sdy_axpy(dy, a, dx, n, stream()), "axpy");
    to_host(y, dy, (size_t)n * 4);
    sdy_free(dy);
    sdy_free(dx);
}

void op_rmsnorm(float *out, const float *x, const float *w, int n, float eps) {
    if (n <= 0) return;
    float *dx = dup_to_dev(x, (size_t)n * 4), *dw = dup_to_dev(w, (size_t)n * 4), *dout = dalloc((size_t)n * 4);
    CK(sdy_rmsnorm(dx, dw, dout, n, eps, 1, n, n, stream()), "rmsnorm");
    to_host(out, dout, (size_t)n * 4);
    sdy_free(dx);
    sdy_free(dw);
    sdy_free(dout);
}

void op_softmax(float *x, int n) {
    if (n <= 0) return;
    float *dx = dup_to_dev(x, (size_t)n * 4);
    CK(sdy_softmax(dx, n, 1, n, stream()), "softmax");
    to_host(x, dx, (size_t)n * 4);
    sdy_free(dx);
}

void op_silu_mul(float *gate, const float *up, int n) {
    if (n <= 0) return;
    float *dg = dup_to_dev(gate, (size_t)n * 4), *du = dup_to_dev(up, (size_t)n * 4);
    CK(sdy_silu_mul(dg, du, n, stream()), "silu_mul");
    to_host(gate, dg, (size_t)n * 4);
    sdy_free(dg);
    sdy_free(du);
}

/* The table is host work: cos/sin in double through the host libm, as the reference computes it
 * (csrc/ops.c:375-386), so its bits are the reference's. */
void op_rope_table(float *cos_out, float *sin_out, int n_pos, int head_dim, float theta) {
    if (n_pos > 0 && head_dim > 1) sdy_rope_table_host(cos_out, sin_out, n_pos, head_dim, theta);
}

void op_rope(float *x, int n_heads, int head_dim, const float *cos, const float *sin, int interleaved) {
    size_t n = (size_t)n_heads * head_dim, half = (size_t)head_dim / 2;
    if (!n) return;
    float *dx = dup_to_dev(x, n * 4), *dc = dup_to_dev(cos, half * 4), *ds = dup_to_dev(sin, half * 4);
    CK(sdy_rope(dx, n_heads, head_dim, dc, ds, interleaved, stream()), "rope");
    to_host(x, dx, n * 4);
    sdy_free(dx);
    sdy_free(dc);
    sdy_free(ds);
}

void op_attention(float *out, const float *q, const float *k_cache, const float *v_cache, int n_head, int n_kv_head,
                  int head_dim, int n_kv, int stride, float *scores) {
    (void)scores; /* the GPU kernels keep their scores in device scratch */
    if (n_head <= 0 || n_kv <= 0) return;
    size_t qn = (size_t)n_head * head_dim, kvn = (size_t)n_kv_head * stride * head_dim;
    float *dq = dup_to_dev(q, qn * 4), *dk = dup_to_dev(k_cache, kvn * 4), *dv = dup_to_dev(v_cache, kvn * 4);
    float *dout = dalloc(qn * 4);
    float *part = dalloc(sdy_attn_scores_floats(1, n_head, n_kv) * 4);
    CK(sdy_attention(dq, dk, dv, SDY_KV_F32, 1, n_head, n_kv_head, head_dim, n_kv, (long)stride * head_dim, (long)qn,
                     part, dout, (long)qn, stream()),
       "attention");
    to_host(out, dout, qn * 4);
    sdy_free(dq);
    sdy_free(dk);
    sdy_free(dv);
    sdy_free(dout);
    sdy_free(part);
}

/* csrc/engine.h:44-45 */
const char *engine_version(void) { return "0.0.1"; }

void engine_add_f32(const float *a, const float *b, float *out, size_t n) {
    if (!n) return;
    float *da = dup_to_dev(a, n * 4), *db = dup_to_dev(b, n * 4), *dout = dalloc(n * 4);
    CK(sdy_add(da, db, dout, (long)n, stream()), "add");
    to_host(out, dout, n * 4);
    sdy_free(da);
    sdy_free(db);
    sdy_free(dout);
}

/* Kernel-level entry points of the public ABI (csrc/ops.h:24-74 of the reference): host pointers
 * in and out, computation on the GPU. Each call uploads its operands, runs the gfx950 kernel and
 * copies the result back; the reference's tests and tools call these to check single kernels.
 *
 * These functions have no error return in the reference's ABI. A failure here (no device, out of
 * memory, a HIP error, an argument the kernels do not take) ends the call: what it allocated is
 * freed, its float outputs are filled with NaN (a quantised or f16 output is left zeroed / NaN as
 * its type allows), and op_last_error() (this thread's last op_* call) returns the message. The
 * process goes on; there is no CPU fallback.
 */
#define _POSIX_C_SOURCE 200809L
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sardyne.h"
#include "sdy_ops.h"
#include "sdy_shim.h"

static sdy_stream g_stream;
static int g_simd = 1;
static _Thread_local char g_op_err[512];

const char *op_last_error(void) { return g_op_err; }

/* One op_* call: the device buffers and matrices it holds, and whether a step failed (after which
 * no further GPU work is issued). */
typedef struct {
    const char *name;
    void *dev[8];
    int n_dev;
    sdy_mat mat[2];
    int n_mat;
    int failed;
} call;

static void begin(call *c, const char *name) {
    memset(c, 0, sizeof *c);
    c->name = name;
    g_op_err[0] = '\0';
}

static void fail(call *c, const char *fmt, ...) {
    if (c->failed) return;
    c->failed = 1;
    int n = snprintf(g_op_err, sizeof g_op_err, "%s: ", c->name);
    va_list ap;
    va_start(ap, fmt);
    if (n > 0 && (size_t)n < sizeof g_op_err) vsnprintf(g_op_err + n, sizeof g_op_err - (size_t)n, fmt, ap);
    va_end(ap);
}

/* a GPU step: nothing after a failure; a failure records the shim's message */
static int ok(call *c, int rc, const char *what) {
    if (!c->failed && rc != 0) fail(c, "%s failed on the GPU: %s", what, sdy_last_error());
    return !c->failed;
}

static sdy_stream stream(call *c) {
    if (!g_stream && !c->failed) ok(c, sdy_stream_new(&g_stream), "stream creation");
    return g_stream;
}

static void *dalloc(call *c, size_t n) {
    void *p = NULL;
    if (c->failed || !ok(c, sdy_malloc(&p, n), "device allocation")) return NULL;
    c->dev[c->n_dev++] = p;
    return p;
}

static void *dup_to_dev(call *c, const void *h, size_t n) {
    void *d = dalloc(c, n);
    if (d) ok(c, sdy_h2d(d, h, n, stream(c)), "upload");
    return c->failed ? NULL : d;
}

static void to_host(call *c, void *h, const void *d, size_t n) {
    if (c->failed) return;
    if (ok(c, sdy_d2h(h, d, n, stream(c)), "download")) ok(c, sdy_sync(stream(c)), "synchronize");
}

static sdy_mat *upload_mat(call *c, int type, int n_in, long n_rows, const void *w) {
    if (c->failed) return NULL;
    sdy_mat *m = &c->mat[c->n_mat];
    if (!ok(c, sdy_mat_upload(m, type, n_in, n_rows, w, stream(c)), "weight upload")) return NULL;
    c->n_mat++;
    return m;
}

/* frees what the call holds; 0 when it succeeded */
static int end(call *c) {
    for (int i = 0; i < c->n_dev; i++) sdy_free(c->dev[i]);
    for (int i = 0; i < c->n_mat; i++) sdy_mat_free(&c->mat[i]);
    return c->failed;
}

static void nan_fill(float *p, size_t n) {
    for (size_t i = 0; i < n; i++) p[i] = NAN;
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
    call c;
    begin(&c, "op_f16_to_f32_n");
    void *dx = dup_to_dev(&c, x, n * 2);
    float *dout = dalloc(&c, n * 4);
    if (!c.failed) ok(&c, sdy_f16_to_f32(dx, dout, (long)n, stream(&c)), "f16_to_f32");
    to_host(&c, out, dout, n * 4);
    if (end(&c)) nan_fill(out, n);
}

uint16_t op_f32_to_f16(float f) {
    call c;
    begin(&c, "op_f32_to_f16");
    uint16_t h = 0;
    float *dx = dup_to_dev(&c, &f, 4);
    uint16_t *dout = dalloc(&c, 2);
    if (!c.failed) ok(&c, sdy_f32_to_f16(dx, dout, 1, stream(&c)), "f32_to_f16");
    to_host(&c, &h, dout, 2);
    return end(&c) ? (uint16_t)0x7E00u : h; /* (an f16 quiet NaN on failure) */
}

void op_row_to_f32(const void *row, int type, float *out, size_t n) {
    if (!n) return;
    call c;
    begin(&c, "op_row_to_f32");
    if (!op_row_size(type, (int)n)) fail(&c, "type %d with %zu elements is not supported", type, n);
    sdy_mat *m = upload_mat(&c, type, (int)n, 1, row);
    float *dout = dalloc(&c, n * 4);
    if (!c.failed) ok(&c, sdy_dequant_rows(m, 0, 1, dout, stream(&c)), "dequant");
    to_host(&c, out, dout, n * 4);
    if (end(&c)) nan_fill(out, n);
}

void op_quantize_rows(int vtype, const float *x, void *xq, int n_in, int t0, int t1) {
    if (t1 <= t0) return;
    call c;
    begin(&c, "op_quantize_rows");
    int n_tok = t1 - t0;
    size_t row = op_row_size(vtype, n_in);
    if (!row || (vtype != OP_Q8_0 && vtype != OP_Q8_K)) fail(&c, "activation type %d, n_in %d", vtype, n_in);
    float *dx = dup_to_dev(&c, x + (size_t)t0 * n_in, (size_t)n_tok * n_in * 4);
    void *dq = dalloc(&c, row * n_tok);
    if (!c.failed) ok(&c, sdy_quantize(vtype, dx, dq, n_in, n_tok, stream(&c)), "quantize");
    to_host(&c, (uint8_t *)xq + (size_t)t0 * row, dq, row * n_tok);
    if (end(&c) && row) memset((uint8_t *)xq + (size_t)t0 * row, 0, row * n_tok);
}

/* rows [row0, row1) of out[n_tok][n_out]; the other rows of out are left untouched */
/* (the caller began c; a failure marks the call's rows of out with NaN) */
static void matvec_host(call *c, float *out, const void *act, int act_is_f32, const void *w, int wtype, int n_tok,
                        int n_in, int n_out, int row0, int row1) {
    if (row1 <= row0 || n_tok <= 0) return;
    if (row0 < 0 || row1 > n_out) fail(c, "rows [%d, %d) outside %d", row0, row1, n_out);
    sdy_mat *m = upload_mat(c, wtype, n_in, n_out, w);
    size_t act_bytes = act_is_f32 ? (size_t)n_tok * n_in * 4 : op_row_size(vec_dot_type(wtype), n_in) * n_tok;
    void *da = dup_to_dev(c, act, act_bytes);
    float *dout = dup_to_dev(c, out, (size_t)n_tok * n_out * 4);
    sdy_mv_args a;
    memset(&a, 0, sizeof(a));
    if (act_is_f32) a.x = da;
    else a.xq = da;
    a.n_tok = n_tok;
    a.out = dout;
    a.out_stride = n_out;
    a.row0 = row0;
    a.row1 = row1;
    if (!c->failed) ok(c, sdy_matvec(m, &a, stream(c)), "matvec");
    to_host(c, out, dout, (size_t)n_tok * n_out * 4);
    if (end(c) && row0 >= 0 && row1 <= n_out)
        for (int t = 0; t < n_tok; t++) nan_fill(out + (size_t)t * n_out + row0, (size_t)(row1 - row0));
}

void op_matmul_q_rows(float *out, const void *xq, const void *w, int wtype, int n_tok, int n_in, int n_out, int row0,
                      int row1) {
    call c;
    begin(&c, "op_matmul_q_rows");
    if (!is_quant(wtype)) fail(&c, "weight type %d is not quantized", wtype);
    matvec_host(&c, out, xq, 0, w, wtype, n_tok, n_in, n_out, row0, row1);
}

float op_vec_dot_q(int wtype, const void *w, const void *xq, int n) {
    float r = 0.0f;
    call c;
    begin(&c, "op_vec_dot_q");
    if (!is_quant(wtype)) fail(&c, "weight type %d is not quantized", wtype);
    matvec_host(&c, &r, xq, 0, w, wtype, 1, n, 1, 0, 1);
    return r;
}

void op_matmul_rows(float *out, const float *x, const void *w, int wtype, int n_tok, int n_in, int n_out, int row0,
                    int row1) {
    call c;
    begin(&c, "op_matmul_rows");
    if (wtype != OP_F32 && wtype != OP_F16 && wtype != OP_BF16) fail(&c, "weight type %d is not a float type", wtype);
    matvec_host(&c, out, x, 1, w, wtype, n_tok, n_in, n_out, row0, row1);
}

void op_matmul(float *out, const float *x, const void *w, int wtype, int n_tok, int n_in, int n_out) {
    int vt = vec_dot_type(wtype);
    if (vt == OP_F32) {
        op_matmul_rows(out, x, w, wtype, n_tok, n_in, n_out, 0, n_out);
        return;
    }
    if (n_tok <= 0 || n_out <= 0) return;
    call c;
    begin(&c, "op_matmul");
    size_t row = op_row_size(vt, n_in);
    float *dx = dup_to_dev(&c, x, (size_t)n_tok * n_in * 4);
    void *dq = dalloc(&c, row * n_tok);
    if (!c.failed) ok(&c, sdy_quantize(vt, dx, dq, n_in, n_tok, stream(&c)), "quantize");
    sdy_mat *m = upload_mat(&c, wtype, n_in, n_out, w);
    float *dout = dalloc(&c, (size_t)n_tok * n_out * 4);
    sdy_mv_args a;
    memset(&a, 0, sizeof(a));
    a.xq = dq;
    a.n_tok = n_tok;
    a.out = dout;
    a.out_stride = n_out;
    a.row0 = 0;
    a.row1 = n_out;
    if (!c.failed) ok(&c, sdy_matvec(m, &a, stream(&c)), "matvec");
    to_host(&c, out, dout, (size_t)n_tok * n_out * 4);
    if (end(&c)) nan_fill(out, (size_t)n_tok * n_out);
}

float op_dot_f32(const float *a, const float *b, int n) {
    float r = 0.0f;
    if (n <= 0) return r;
    call c;
    begin(&c, "op_dot_f32");
    float *da = dup_to_dev(&c, a, (size_t)n * 4), *db = dup_to_dev(&c, b, (size_t)n * 4), *dr = dalloc(&c, 4);
    if (!c.failed) ok(&c, sdy_dot(da, db, n, dr, stream(&c)), "dot");
    to_host(&c, &r, dr, 4);
    return end(&c) ? NAN : r;
}

void op_axpy(float *y, float a, const float *x, int n) {
    if (n <= 0) return;
    call c;
    begin(&c, "op_axpy");
    float *dy = dup_to_dev(&c, y, (size_t)n * 4), *dx = dup_to_dev(&c, x, (size_t)n * 4);
    if (!c.failed) ok(&c, sdy_axpy(dy, a, dx, n, stream(&c)), "axpy");
    to_host(&c, y, dy, (size_t)n * 4);
    if (end(&c)) nan_fill(y, (size_t)n);
}

void op_rmsnorm(float *out, const float *x, const float *w, int n, float eps) {
    if (n <= 0) return;
    call c;
    begin(&c, "op_rmsnorm");
    float *dx = dup_to_dev(&c, x, (size_t)n * 4), *dw = dup_to_dev(&c, w, (size_t)n * 4);
    float *dout = dalloc(&c, (size_t)n * 4);
    if (!c.failed) ok(&c, sdy_rmsnorm(dx, dw, dout, n, eps, 1, n, n, stream(&c)), "rmsnorm");
    to_host(&c, out, dout, (size_t)n * 4);
    if (end(&c)) nan_fill(out, (size_t)n);
}

void op_softmax(float *x, int n) {
    if (n <= 0) return;
    call c;
    begin(&c, "op_softmax");
    float *dx = dup_to_dev(&c, x, (size_t)n * 4);
    if (!c.failed) ok(&c, sdy_softmax(dx, n, 1, n, stream(&c)), "softmax");
    to_host(&c, x, dx, (size_t)n * 4);
    if (end(&c)) nan_fill(x, (size_t)n);
}

void op_silu_mul(float *gate, const float *up, int n) {
    if (n <= 0) return;
    call c;
    begin(&c, "op_silu_mul");
    float *dg = dup_to_dev(&c, gate, (size_t)n * 4), *du = dup_to_dev(&c, up, (size_t)n * 4);
    if (!c.failed) ok(&c, sdy_silu_mul(dg, du, n, stream(&c)), "silu_mul");
    to_host(&c, gate, dg, (size_t)n * 4);
    if (end(&c)) nan_fill(gate, (size_t)n);
}

/* The table is host work: cos/sin in double through the host libm, as the reference computes it
 * (csrc/ops.c:375-386), so its bits are the reference's. */
void op_rope_table(float *cos_out, float *sin_out, int n_pos, int head_dim, float theta) {
    if (n_pos > 0 && head_dim > 1) sdy_rope_table_host(cos_out, sin_out, n_pos, head_dim, theta);
}

void op_rope(float *x, int n_heads, int head_dim, const float *cos, const float *sin, int interleaved) {
    size_t n = (size_t)n_heads * head_dim, half = (size_t)head_dim / 2;
    if (!n) return;
    call c;
    begin(&c, "op_rope");
    float *dx = dup_to_dev(&c, x, n * 4), *dc = dup_to_dev(&c, cos, half * 4), *ds = dup_to_dev(&c, sin, half * 4);
    if (!c.failed) ok(&c, sdy_rope(dx, n_heads, head_dim, dc, ds, interleaved, stream(&c)), "rope");
    to_host(&c, x, dx, n * 4);
    if (end(&c)) nan_fill(x, n);
}

void op_attention(float *out, const float *q, const float *k_cache, const float *v_cache, int n_head, int n_kv_head,
                  int head_dim, int n_kv, int stride, float *scores) {
    (void)scores; /* the GPU kernels keep their scores in device scratch */
    if (n_head <= 0 || n_kv <= 0) return;
    call c;
    begin(&c, "op_attention");
    size_t qn = (size_t)n_head * head_dim, kvn = (size_t)n_kv_head * stride * head_dim;
    float *dq = dup_to_dev(&c, q, qn * 4), *dk = dup_to_dev(&c, k_cache, kvn * 4);
    float *dv = dup_to_dev(&c, v_cache, kvn * 4), *dout = dalloc(&c, qn * 4);
    float *part = dalloc(&c, sdy_attn_scores_floats(1, n_head, n_kv) * 4);
    if (!c.failed)
        ok(&c, sdy_attention(dq, dk, dv, SDY_KV_F32, 1, n_head, n_kv_head, head_dim, n_kv, (long)stride * head_dim,
                             (long)qn, part, dout, (long)qn, stream(&c)),
           "attention");
    to_host(&c, out, dout, qn * 4);
    if (end(&c)) nan_fill(out, qn);
}

/* csrc/engine.h:44-45 */
const char *engine_version(void) { return "0.0.1"; }

void engine_add_f32(const float *a, const float *b, float *out, size_t n) {
    if (!n) return;
    call c;
    begin(&c, "engine_add_f32");
    float *da = dup_to_dev(&c, a, n * 4), *db = dup_to_dev(&c, b, n * 4), *dout = dalloc(&c, n * 4);
    if (!c.failed) ok(&c, sdy_add(da, db, dout, (long)n, stream(&c)), "add");
    to_host(&c, out, dout, n * 4);
    if (end(&c)) nan_fill(out, n);
}

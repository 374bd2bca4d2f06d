/* Device forward pass: the layer sequence of the reference forward (csrc/model_llama.c:757-832)
 * issued as gfx950 kernels on the context's stream.
 *
 *   embedding rows (dequant gather) -> per layer: RMSNorm -> Q/K/V matvec (+bias) -> q/k norm,
 *   RoPE, KV-cache write -> GQA attention -> O matvec + residual -> RMSNorm -> gate/up matvec ->
 *   SiLU·mul -> down matvec + residual (or the MoE block) -> final RMSNorm -> output matvec.
 *
 * Quantized matrices read activations quantized once per input (Q8_K for K-quants, Q8_0 for the
 * 32-element types), as csrc/model_llama.c:592-611 does.
 */
#define _POSIX_C_SOURCE 200809L
#include <stdlib.h>
#include <string.h>

#include "sdy_engine.h"
#include "sdy_ops.h"
#include "sdy_shim.h"

#define TRY(call)             \
    do {                      \
        int rc_ = (call);     \
        if (rc_) return rc_;  \
    } while (0)

static int vec_dot_type(int wtype) {
    if (wtype == SDY_Q8_0 || wtype == SDY_Q4_0 || wtype == SDY_Q5_0) return SDY_Q8_0;
    if (wtype == SDY_Q4_K || wtype == SDY_Q6_K) return SDY_Q8_K;
    return SDY_F32;
}


static int dalloc(void **p, size_t n) { return sdy_malloc(p, n ? n : 64); }

/* an environment switch: set and not "0" */
static int env_flag(const char *name) {
    const char *v = getenv(name);
    return v && v[0] && strcmp(v, "0") != 0;
}

static int moe_grouped_ok(const engine_ctx *c);

/* Token count from which quantized matrices go through the MFMA GEMM instead of the matvec. */
#define GEMM_MIN_TOKENS 16

int sdy_engine_alloc(engine_ctx *c) {
    const engine_model_info *in = &c->m->info;
    size_t B = (size_t)c->n_batch, S = (size_t)c->max_seq, hd = (size_t)in->head_dim;
    size_t q_dim = (size_t)in->n_head * hd, kv_dim = (size_t)in->n_kv_head * hd;
    size_t kv = (size_t)in->n_layer * in->n_kv_head * S * hd;
    size_t ffn = (size_t)(in->n_expert ? in->ffn_exp_dim : in->ffn_dim);
    size_t max_in = (size_t)in->dim > q_dim ? (size_t)in->dim : q_dim;
    if (ffn > max_in) max_in = ffn;
    size_t logit_rows = c->logits_all ? B : 1;
    /* rows of the FFN activations: n_batch tokens, or for MoE the k routed slots of each of them */
    size_t BR = in->n_expert ? B * (size_t)in->n_expert_used : B;
    const size_t kv_bytes = kv * sdy_kv_elt_bytes(c->kv_type);
    TRY(dalloc(&c->k_cache, kv_bytes));
    TRY(dalloc(&c->v_cache, kv_bytes));
    TRY(dalloc((void **)&c->rope_cos, S * hd / 2 * 4));
    TRY(dalloc((void **)&c->rope_sin, S * hd / 2 * 4));
    TRY(dalloc((void **)&c->x, B * in->dim * 4));
    TRY(dalloc((void **)&c->xb, B * in->dim * 4));
    TRY(dalloc((void **)&c->q, B * q_dim * 4));
    TRY(dalloc((void **)&c->k, B * kv_dim * 4));
    TRY(dalloc((void **)&c->v, B * kv_dim * 4));
    TRY(dalloc((void **)&c->att, B * q_dim * 4));
    TRY(dalloc((void **)&c->hb, BR * ffn * 4));
    TRY(dalloc((void **)&c->hb2, BR * ffn * 4));
    TRY(dalloc((void **)&c->logits_dev, logit_rows * in->n_vocab * 4));
    TRY(dalloc((void **)&c->part, sdy_attn_scores_floats((int)B, in->n_head, (int)S) * 4));
    TRY(dalloc(&c->xq[0], BR * ((max_in + 31) / 32 * 34)));
    TRY(dalloc(&c->xq[1], BR * ((max_in + 255) / 256 * 292)));
    TRY(dalloc((void **)&c->tok_dev, B * 4));
    TRY(sdy_host_alloc((void **)&c->tok_host, B * 4));
    TRY(dalloc((void **)&c->qkv, B * (q_dim + 2 * kv_dim) * 4));
    TRY(dalloc((void **)&c->step_dev, 2 * 4));
    TRY(sdy_host_alloc((void **)&c->step_host, 2 * 4));
    TRY(dalloc(&c->gemm_ws, sdy_gemm_ws_bytes((int)BR, (int)max_in)));
    {
        const size_t split = sdy_attn_decode_split_floats(in->n_head, in->head_dim, c->max_seq);
        const size_t chunked = sdy_attn_chunked_floats(in->n_head, in->head_dim, c->max_seq);
        TRY(dalloc((void **)&c->attn_part, (split > chunked ? split : chunked) * 4));
    }
    TRY(dalloc((void **)&c->attn_count, (size_t)in->n_kv_head * 4));
    TRY(sdy_memset(c->attn_count, 0, (size_t)in->n_kv_head * 4, c->st));
    if (in->n_expert) {
        size_t chosen = B * in->n_expert_used;
        TRY(dalloc((void **)&c->moe_probs, B * in->n_expert * 4));
        TRY(dalloc((void **)&c->moe_w, chosen * 4));
        TRY(dalloc((void **)&c->moe_top, chosen * 4));
        TRY(dalloc((void **)&c->moe_x, BR * in->dim * 4));
        TRY(dalloc((void **)&c->moe_grp_tok, ((size_t)in->n_expert + 1) * 4));
        TRY(dalloc((void **)&c->moe_grp_tile, ((size_t)in->n_expert + 1) * 4));
        TRY(dalloc((void **)&c->moe_src, BR * 4));
        TRY(dalloc((void **)&c->moe_orow, BR * 4));
        TRY(dalloc((void **)&c->moe_y, BR * in->dim * 4));
        TRY(dalloc((void **)&c->moe_sum, B * in->dim * 4));
        TRY(dalloc((void **)&c->moe_gidx, chosen * 4));
        TRY(dalloc((void **)&c->moe_gw, chosen * 4));
        TRY(sdy_host_alloc((void **)&c->moe_top_host, chosen * 4));
        TRY(sdy_host_alloc((void **)&c->moe_w_host, chosen * 4));
        TRY(sdy_host_alloc((void **)&c->moe_gidx_host, chosen * 4));
        TRY(sdy_host_alloc((void **)&c->moe_gw_host, chosen * 4));
    }
    {
        /* RoPE table built on the host with libm (bit-identical to the reference's) and uploaded */
        const size_t nt = S * (hd / 2);
        float *tab = malloc(2 * nt * sizeof(float) + 1);
        if (!tab) return -1;
        sdy_rope_table_host(tab, tab + nt, c->max_seq, in->head_dim, in->rope_theta);
        int rc = sdy_h2d(c->rope_cos, tab, nt * 4, c->st) || sdy_h2d(c->rope_sin, tab + nt, nt * 4, c->st) ||
                 sdy_sync(c->st);
        free(tab);
        TRY(rc ? -1 : 0);
    }
    /* SARDYNE_NO_GROUPED_MOE: many-token MoE blocks grouped on the host instead (same bits) */
    c->moe_grouped_ok = moe_grouped_ok(c) && !env_flag("SARDYNE_NO_GROUPED_MOE");
    TRY(sdy_memset(c->k_cache, 0, kv_bytes, c->st));
    TRY(sdy_memset(c->v_cache, 0, kv_bytes, c->st));
    return sdy_sync(c->st);
}

void sdy_engine_release(engine_ctx *c) {
    if (c->graph) sdy_graph_free(c->graph);
    c->graph = NULL;
    void *dev[] = {c->k_cache, c->v_cache, c->rope_cos, c->rope_sin, c->x, c->xb, c->q, c->k, c->v, c->att, c->hb,
                   c->hb2, c->logits_dev, c->part, c->xq[0], c->xq[1], c->tok_dev, c->moe_probs, c->moe_w,
                   c->moe_top, c->moe_x, c->moe_y, c->moe_sum, c->moe_gidx, c->moe_gw, c->qkv, c->step_dev,
                   c->gemm_ws, c->attn_part, c->attn_count, c->moe_grp_tok, c->moe_grp_tile, c->moe_src,
                   c->moe_orow};
    for (size_t i = 0; i < sizeof dev / sizeof *dev; i++) sdy_free(dev[i]);
    void *host[] = {c->tok_host, c->moe_top_host, c->moe_w_host, c->moe_gidx_host, c->moe_gw_host, c->step_host};
    for (size_t i = 0; i < sizeof host / sizeof *host; i++) sdy_host_free(host[i]);
}

/* Every write of c->xq[] comes with this call: the quantisation cache forgets its sources, and the GEMM
 * workspace's f16 expansion of the activations (recorded with the epoch it was made in) goes stale. */
static void xq_forget(engine_ctx *c) {
    c->xq_src[0] = c->xq_src[1] = NULL;
    c->xq_epoch++;
}

/* gemm_ws now holds the f16 expansion of xq (n_tok rows of n_in), made after the last write of xq[] */
static void gemm_record(engine_ctx *c, const void *xq, int n_tok, int n_in) {
    c->gemm_ready = 1;
    c->gemm_epoch = c->xq_epoch;
    c->gemm_xq = xq;
    c->gemm_n_tok = n_tok;
    c->gemm_n_in = n_in;
}

/* Whether n_tok rows for w take the MFMA GEMM */
static int use_gemm(const dmat *w, int n_tok) { return n_tok >= GEMM_MIN_TOKENS && sdy_gemm_ok(&w->m, n_tok); }

/* out[t][row] = W . x[t] for n_tok rows of x; new_input = 1 when x changed since the last call
 * (the quantized copy of x is then rebuilt), as matmul() in csrc/model_llama.c:592-611. */
static int mm_epi(engine_ctx *c, float *out, const float *x, const dmat *w, int n_tok, const float *bias,
                  const float *resid, int new_input, int epilogue) {
    if (new_input) xq_forget(c);
    sdy_mv_args a;
    memset(&a, 0, sizeof a);
    a.n_tok = n_tok;
    a.out = out;
    a.out_stride = epilogue == SDY_EPI_SWIGLU ? w->n_out / 2 : w->n_out;
    a.epilogue = epilogue;
    a.bias = bias;
    a.resid = resid;
    a.row0 = 0;
    a.row1 = w->n_out;
    int vt = vec_dot_type(w->type);
    if (vt == SDY_F32) {
        a.x = x;
    } else {
        int s = vt == SDY_Q8_0 ? 0 : 1;
        if (c->xq_src[s] != x || c->xq_n_tok[s] != n_tok || c->xq_n_in[s] != w->n_in) {
            /* for the GEMM the quantiser also writes the f16 expansion it reads */
            const int gemm = vt == SDY_Q8_K && use_gemm(w, n_tok);
            if (gemm) TRY(sdy_quantize_gemm(x, c->xq[s], w->n_in, n_tok, c->gemm_ws, c->st));
            else TRY(sdy_quantize(vt, x, c->xq[s], w->n_in, n_tok, c->st));
            c->xq_epoch++;
            if (gemm) gemm_record(c, c->xq[s], n_tok, w->n_in);
            c->xq_src[s] = x;
            c->xq_n_tok[s] = n_tok;
            c->xq_n_in[s] = w->n_in;
        }
        a.xq = c->xq[s];
        /* many tokens of a K-quant matrix: the MFMA GEMM (same bits as the matvec) */
        if (use_gemm(w, n_tok)) {
            /* q, k and v (gate and up) read one quantised input: its f16 expansion is made once */
            a.ws_ready = c->gemm_ready && c->gemm_epoch == c->xq_epoch && c->gemm_xq == a.xq &&
                         c->gemm_n_tok == n_tok && c->gemm_n_in == w->n_in;
            c->gemm_ready = 0;
            TRY(sdy_gemm(&w->m, &a, c->gemm_ws, c->st));
            gemm_record(c, a.xq, n_tok, w->n_in);
            return 0;
        }
    }
    return sdy_matvec(&w->m, &a, c->st);
}

static int mm(engine_ctx *c, float *out, const float *x, const dmat *w, int n_tok, const float *bias,
              const float *resid, int new_input) {
    return mm_epi(c, out, x, w, n_tok, bias, resid, new_input, SDY_EPI_NONE);
}

/* out1 = W1 . x and out2 = W2 . x (+ biases) for n_tok rows of x, which the previous matmul (or norm)
 * quantised already: a layer's q|k and its v. When both take the GEMM on the same quantised rows,
 * one launch multiplies both (sdy_gemm2); otherwise two matmuls. */
static int mm_pair(engine_ctx *c, float *out1, const dmat *w1, const float *b1, float *out2, const dmat *w2,
                   const float *b2, const float *x, int n_tok) {
    const int s = 1;  /* the Q8_K copy */
    if (!(use_gemm(w1, n_tok) && use_gemm(w2, n_tok) && w1->n_in == w2->n_in &&
          vec_dot_type(w1->type) == SDY_Q8_K && vec_dot_type(w2->type) == SDY_Q8_K && c->xq_src[s] == x &&
          c->xq_n_tok[s] == n_tok && c->xq_n_in[s] == w1->n_in)) {
        TRY(mm(c, out1, x, w1, n_tok, b1, NULL, 0));
        return mm(c, out2, x, w2, n_tok, b2, NULL, 0);
    }
    sdy_mv_args a[2];
    const dmat *w[2] = {w1, w2};
    float *out[2] = {out1, out2};
    const float *b[2] = {b1, b2};
    for (int i = 0; i < 2; i++) {
        memset(&a[i], 0, sizeof a[i]);
        a[i].xq = c->xq[s];
        a[i].n_tok = n_tok;
        a[i].out = out[i];
        a[i].out_stride = w[i]->n_out;
        a[i].bias = b[i];
        a[i].row0 = 0;
        a[i].row1 = w[i]->n_out;
        a[i].epilogue = SDY_EPI_NONE;
    }
    a[0].ws_ready = c->gemm_ready && c->gemm_epoch == c->xq_epoch && c->gemm_xq == a[0].xq &&
                    c->gemm_n_tok == n_tok && c->gemm_n_in == w1->n_in;
    c->gemm_ready = 0;
    TRY(sdy_gemm2(&w1->m, &a[0], &w2->m, &a[1], c->gemm_ws, c->st));
    gemm_record(c, a[0].xq, n_tok, w1->n_in);
    return 0;
}

/* xb = RMSNorm(x) * wn for n rows, quantized for the matrix `next` in the same launch; the copy
 * is registered in the activation-quantisation cache, so mm(next, xb, new_input = 0) reuses it. */
static int norm_for(engine_ctx *c, const float *x, const float *wn, const dmat *next, int n) {
    const engine_model_info *in = &c->m->info;
    const int vt = vec_dot_type(next->type);
    xq_forget(c);
    if (vt == SDY_F32) return sdy_norm_quant(x, wn, in->norm_eps, in->dim, n, c->xb, SDY_F32, NULL, c->st);
    const int s = vt == SDY_Q8_0 ? 0 : 1;
    if (vt == SDY_Q8_K && use_gemm(next, n)) { /* with the GEMM's f16 expansion of the rows */
        TRY(sdy_norm_quant_gemm(x, wn, in->norm_eps, in->dim, n, c->xb, c->xq[s], c->gemm_ws, c->st));
        gemm_record(c, c->xq[s], n, in->dim);
    } else {
        TRY(sdy_norm_quant(x, wn, in->norm_eps, in->dim, n, c->xb, vt, c->xq[s], c->st));
    }
    c->xq_src[s] = c->xb;
    c->xq_n_tok[s] = n;
    c->xq_n_in[s] = in->dim;
    return 0;
}

/* One token through two K-quant matrices in one launch (q|k and a v of another type): the Q8_K row
 * of x is the one norm_for just wrote. */
static int mm1_pair(engine_ctx *c, float *out1, const dmat *w1, const float *b1, float *out2, const dmat *w2,
                    const float *b2) {
    sdy_mv_args a1, a2;
    memset(&a1, 0, sizeof a1);
    memset(&a2, 0, sizeof a2);
    a1.xq = a2.xq = c->xq[1];
    a1.n_tok = a2.n_tok = 1;
    a1.out = out1;
    a1.out_stride = w1->n_out;
    a1.bias = b1;
    a1.row1 = w1->n_out;
    a2.out = out2;
    a2.out_stride = w2->n_out;
    a2.bias = b2;
    a2.row1 = w2->n_out;
    return sdy_matvec_pair(&w1->m, &a1, &w2->m, &a2, c->st);
}

/* One-token arguments for a kernel that builds the Q8_K row of x itself (RMS-normalised with nw first
 * when nw is set): the bytes norm_for / sdy_quantize would have written, without their launch. */
static sdy_mv_args fused_args(const engine_ctx *c, float *out, const float *x, const float *nw, const dmat *w,
                              const float *bias, const float *resid, int epilogue) {
    sdy_mv_args a;
    memset(&a, 0, sizeof a);
    a.x = x;
    a.nw = nw;
    a.eps = c->m->info.norm_eps;
    a.n_tok = 1;
    a.out = out;
    a.out_stride = epilogue == SDY_EPI_SWIGLU ? w->n_out / 2 : w->n_out;
    a.bias = bias;
    a.resid = resid;
    a.row1 = w->n_out;
    a.epilogue = epilogue;
    return a;
}

/* out = W . x for one token through the in-kernel quantisation; 1 when it is not available for this
 * matrix (the caller then quantises separately), 0 when done, < 0 on error. */
static int mm1_fused(engine_ctx *c, float *out, const float *x, const float *nw, const dmat *w, const float *bias,
                     const float *resid, int epilogue) {
    sdy_mv_args a = fused_args(c, out, x, nw, w, bias, resid, epilogue);
    if (!c->fuse_act || !sdy_matvec_fused_ok(&w->m, &a, NULL, NULL)) return 1;
    xq_forget(c);
    return sdy_matvec(&w->m, &a, c->st);
}

/* hb[t][i] = silu(gate_i . x) * (up_i . x) for n rows of x (gate/up fused and interleaved, or apart). */
static int ffn_gate_up(engine_ctx *c, const float *x, int n, int new_input, const dmat *gate_up, const dmat *gate,
                       const dmat *up, int ffn) {
    if (gate_up) return mm_epi(c, c->hb, x, gate_up, n, NULL, NULL, new_input, SDY_EPI_SWIGLU);
    TRY(mm(c, c->hb, x, gate, n, NULL, NULL, new_input));
    TRY(mm(c, c->hb2, x, up, n, NULL, NULL, 0));
    return sdy_silu_mul(c->hb, c->hb2, (long)n * ffn, c->st);
}

/* One expert's slice of a stacked [n_expert][n_out][n_in] tensor (rows_per_expert = n_out, or
 * 2 * n_out for the interleaved gate|up tensor). */
static dmat expert(const dmat *w, int e) {
    dmat d = *w;
    d.m = sdy_mat_rows(&w->m, (long)e * w->n_out, w->n_out);
    return d;
}

int sdy_gather_rows(const float *src, const int32_t *idx, int n, int dim, float *dst, sdy_stream s);
int sdy_scatter_axpy(float *dst, const int32_t *idx, const float *w, const float *src, int n, int dim, sdy_stream s);

/* moe_ffn (csrc/model_llama.c:724-751): router, top-k on the device; the (token, slot) pairs are
 * grouped by expert on the host after one small copy, then each chosen expert runs gate/up/down
 * over its tokens and the weighted outputs are accumulated per token in ascending expert order. */
static int moe(engine_ctx *c, const dlayer *L, int n) {
    const engine_model_info *in = &c->m->info;
    const int dim = in->dim, fe = in->ffn_exp_dim, ne = in->n_expert, k = in->n_expert_used, total = n * k;
    TRY(mm(c, c->moe_probs, c->xb, &L->gate_inp, n, NULL, NULL, 0));
    TRY(sdy_moe_route(c->moe_probs, n, ne, k, c->moe_top, c->moe_w, c->st));
    TRY(sdy_d2h(c->moe_top_host, c->moe_top, (size_t)total * 4, c->st));
    TRY(sdy_d2h(c->moe_w_host, c->moe_w, (size_t)total * 4, c->st));
    TRY(sdy_memset(c->moe_sum, 0, (size_t)n * dim * 4, c->st));
    TRY(sdy_sync(c->st));
    int *count = calloc((size_t)ne + 1, sizeof(int));
    if (!count) return -1;
    for (int i = 0; i < total; i++) count[c->moe_top_host[i] + 1]++;
    for (int e = 0; e < ne; e++) count[e + 1] += count[e];
    for (int i = 0; i < total; i++) {
        int slot = count[c->moe_top_host[i]]++;
        c->moe_gidx_host[slot] = i / k;
        c->moe_gw_host[slot] = c->moe_w_host[i];
    }
    memmove(count + 1, count, (size_t)ne * sizeof(int));
    count[0] = 0;
    int rc = sdy_h2d(c->moe_gidx, c->moe_gidx_host, (size_t)total * 4, c->st);
    if (!rc) rc = sdy_h2d(c->moe_gw, c->moe_gw_host, (size_t)total * 4, c->st);
    for (int e = 0; e < ne && !rc; e++) {
        int first = count[e], m = count[e + 1] - first;
        if (!m) continue;
        if ((rc = sdy_gather_rows(c->xb, c->moe_gidx + first, m, dim, c->moe_x, c->st))) break;
        if (L->gu_fused) {
            dmat gu = expert(&L->gate_up, e);
            rc = ffn_gate_up(c, c->moe_x, m, 1, &gu, NULL, NULL, fe);
        } else {
            dmat g = expert(&L->gate, e), u = expert(&L->up, e);
            rc = ffn_gate_up(c, c->moe_x, m, 1, NULL, &g, &u, fe);
        }
        if (rc) break;
        dmat d = expert(&L->down, e);
        if ((rc = mm(c, c->moe_y, c->hb, &d, m, NULL, NULL, 1))) break;
        rc = sdy_scatter_axpy(c->moe_sum, c->moe_gidx + first, c->moe_gw + first, c->moe_y, m, dim, c->st);
    }
    free(count);
    if (!rc) rc = sdy_sync(c->st); /* the pinned index buffers are reused by the next layer */
    return rc;
}

/* The one-token MoE block on the device (csrc/model_llama.c:724-751 for one token): router
 * matvec, softmax + top-k, the k chosen experts' gate|up (SwiGLU) and down as grouped matvecs
 * indexed by the device-side top-k, then the weighted sum in ascending expert order plus the
 * residual. No host round trip, so the step can be recorded as a graph. */
/* The MoE block of n tokens on the device, the residual included (x += the routed experts' sum):
 * router, top-k, the routed pairs sorted by expert, their rows gathered and quantised once, then
 * gate|up + SwiGLU and down as one grouped GEMM each over all routed experts, and the ascending-
 * expert weighted sum (csrc/model_llama.c:724-751; the same bits as moe() below). */
static int moe_grouped(engine_ctx *c, const dlayer *L, int n) {
    const engine_model_info *in = &c->m->info;
    const int dim = in->dim, fe = in->ffn_exp_dim, ne = in->n_expert, k = in->n_expert_used, R = n * k;
    TRY(mm(c, c->moe_probs, c->xb, &L->gate_inp, n, NULL, NULL, 0));
    TRY(sdy_moe_route(c->moe_probs, n, ne, k, c->moe_top, c->moe_w, c->st));
    TRY(sdy_moe_sort(c->moe_top, n, k, ne, sdy_gemm_grouped_tile(), c->moe_grp_tok, c->moe_grp_tile, c->moe_src,
                     c->moe_orow, c->st));
    xq_forget(c); /* xq[1] and the GEMM workspace now hold the n normalised rows */
    c->gemm_ready = 0;
    TRY(sdy_quantize_gemm(c->xb, c->xq[1], dim, n, c->gemm_ws, c->st));
    sdy_mv_args a;
    memset(&a, 0, sizeof a);
    a.xq = c->xq[1];
    a.n_tok = R;
    a.out = c->hb;
    a.out_stride = fe;
    a.epilogue = SDY_EPI_SWIGLU;
    a.ws_ready = 1;
    /* sorted row r reads token moe_src[r]'s row: no gathered copy of the routed rows */
    TRY(sdy_gemm_grouped(&L->gate_up.m, 2L * fe, ne, c->moe_grp_tok, c->moe_grp_tile, NULL, c->moe_src, n, &a,
                         c->gemm_ws, c->st));
    TRY(sdy_quantize_gemm(c->hb, c->xq[1], fe, R, c->gemm_ws, c->st));
    a.out = c->moe_y;
    a.out_stride = dim;
    a.epilogue = SDY_EPI_NONE;
    TRY(sdy_gemm_grouped(&L->down.m, dim, ne, c->moe_grp_tok, c->moe_grp_tile, c->moe_orow, NULL, 0, &a, c->gemm_ws,
                         c->st));
    xq_forget(c);
    return sdy_moe_combine(c->moe_y, c->moe_top, c->moe_w, n, k, dim, c->x, c->x, c->st);
}

/* Whether every MoE layer can take moe_grouped: gate|up stored fused and both expert stacks on the
 * GEMM (K-quant, exactness check passed), an expert width that Q8_K blocks tile. */
static int moe_grouped_ok(const engine_ctx *c) {
    const engine_model_info *in = &c->m->info;
    if (!in->n_expert || in->n_expert_used > 16 || in->n_expert > 512 || in->ffn_exp_dim % 256) return 0;
    for (int l = 0; l < in->n_layer; l++) {
        const dlayer *L = &c->m->layers[l];
        if (!L->gu_fused || !sdy_gemm_ok(&L->gate_up.m, 2) || !sdy_gemm_ok(&L->down.m, 2)) return 0;
    }
    return 1;
}

static int moe_decode(engine_ctx *c, const dlayer *L) {
    const engine_model_info *in = &c->m->info;
    const int dim = in->dim, fe = in->ffn_exp_dim, ne = in->n_expert, k = in->n_expert_used;
    const dmat *first = L->gu_fused ? &L->gate_up : &L->gate;
    if (c->fuse_act && vec_dot_type(first->type) == SDY_Q8_K && dim % 256 == 0 && dim <= 4096) {
        /* the router reads the FFN-normalised row and writes its Q8_K bytes for gate|up */
        sdy_mv_args r;
        memset(&r, 0, sizeof r);
        r.x = c->x;
        r.nw = L->ffn_norm;
        r.eps = in->norm_eps;
        r.n_tok = 1;
        r.out = c->moe_probs;
        r.out_stride = ne;
        r.row1 = ne;
        xq_forget(c);
        TRY(sdy_matvec_float_norm(L->gate_inp.type, (const uint8_t *)L->gate_inp.m.base + L->gate_inp.m.plane_off[0],
                                  dim, &r, c->xq[1], c->st));
    } else {
        TRY(norm_for(c, c->x, L->ffn_norm, first, 1)); /* xb and its Q8_K row */
        TRY(mm(c, c->moe_probs, c->xb, &L->gate_inp, 1, NULL, NULL, 0));
    }
    sdy_mv_args a;
    memset(&a, 0, sizeof a);
    a.n_tok = 1;
    a.xq = c->xq[1];
    a.out = c->hb;
    a.out_stride = fe;
    a.row0 = 0;
    /* gate|up selects its experts from the router's logits itself (writing moe_top / moe_w for down),
       else the route kernel runs first */
    int routed = 1;
    if (L->gu_fused && c->fuse_act && ne <= 128 && k <= 64) {
        a.row1 = 2 * fe;
        a.epilogue = SDY_EPI_SWIGLU;
        routed = sdy_matvec_grouped_route(&L->gate_up.m, &a, c->moe_probs, ne, k, c->moe_top, c->moe_w, 2L * fe, 0,
                                          fe, c->st);
        if (routed < 0) return routed;
    }
    if (routed) {
        TRY(sdy_moe_route(c->moe_probs, 1, ne, k, c->moe_top, c->moe_w, c->st));
        if (L->gu_fused) {
            a.row1 = 2 * fe;
            a.epilogue = SDY_EPI_SWIGLU;
            TRY(sdy_matvec_grouped(&L->gate_up.m, &a, c->moe_top, k, 2L * fe, 0, fe, c->st));
        } else {
            a.row1 = fe;
            TRY(sdy_matvec_grouped(&L->gate.m, &a, c->moe_top, k, fe, 0, fe, c->st));
            a.out = c->hb2;
            TRY(sdy_matvec_grouped(&L->up.m, &a, c->moe_top, k, fe, 0, fe, c->st));
            TRY(sdy_silu_mul(c->hb, c->hb2, (long)k * fe, c->st));
        }
    }
    /* down over the k SwiGLU rows: each slot's workgroups quantise its row themselves, or (when that
       is not available) the rows are quantised first (the Q8_K row of xb is no longer needed) */
    xq_forget(c);
    memset(&a, 0, sizeof a);
    a.n_tok = 1;
    a.x = c->hb;
    a.out = c->moe_y;
    a.out_stride = dim;
    a.row0 = 0;
    a.row1 = dim;
    long x_slot = fe;
    const int fused = c->fuse_act && sdy_matvec_grouped_fused_ok(&L->down.m, &a, k, dim, x_slot);
    if (fused && k <= 8) /* the k down projections and their combine in one launch */
        return sdy_moe_down_combine(&L->down.m, c->hb, c->moe_top, c->moe_w, k, dim, c->x, c->x, c->st);
    if (!fused) {
        TRY(sdy_quantize(SDY_Q8_K, c->hb, c->xq[1], fe, k, c->st));
        a.x = NULL;
        a.xq = c->xq[1];
        x_slot = (long)(fe / 256) * 292;
    }
    TRY(sdy_matvec_grouped(&L->down.m, &a, c->moe_top, k, dim, x_slot, dim, c->st));
    return sdy_moe_combine(c->moe_y, c->moe_top, c->moe_w, 1, k, dim, c->x, c->x, c->st);
}

static int kquant_rows_le_4096(int type, int n_in) {
    return (type == SDY_Q4_K || type == SDY_Q6_K) && n_in % 256 == 0 && n_in <= 4096;
}

/* Whether every MoE layer can take moe_decode: K-quant expert matrices with rows of at most 4096
 * elements (the grouped matvec), an expert width that Q8_K blocks tile, an f32 router. */
int sdy_engine_moe_device_ok(const engine_ctx *c) {
    const engine_model *m = c->m;
    const engine_model_info *in = &m->info;
    if (!in->n_expert || in->n_expert_used > 16) return 0; /* the combine sorts up to 16 slots in registers */
    for (int l = 0; l < in->n_layer; l++) {
        const dlayer *L = &m->layers[l];
        if (L->gate_inp.type != SDY_F32 || !kquant_rows_le_4096(L->down.type, in->ffn_exp_dim)) return 0;
        if (L->gu_fused) {
            if (!kquant_rows_le_4096(L->gate_up.type, in->dim) || (64 / (in->dim / 64)) % 2) return 0;
        } else if (!kquant_rows_le_4096(L->gate.type, in->dim) || !kquant_rows_le_4096(L->up.type, in->dim)) {
            return 0;
        }
    }
    return 1;
}

/* Whether the one-token step can use the fused decode kernels (and be recorded as a graph). */
int sdy_engine_decode_fused_ok(const engine_ctx *c) {
    const engine_model_info *in = &c->m->info;
    return sdy_attn_decode_ok(in->n_head, in->n_kv_head, in->head_dim, c->max_seq);
}

/* The layers and the head for n tokens at positions n_past.. (kernels only: no host copies or
 * synchronisation, so that the one-token step can be recorded as a graph). decode: the fused
 * one-token kernels, with the token and its position read from step_dev. */
static int layers(engine_ctx *c, int n, int out_rows, int decode) {
    const engine_model *m = c->m;
    const engine_model_info *in = &m->info;
    const int dim = in->dim, hd = in->head_dim, q_dim = in->n_head * hd, kv_dim = in->n_kv_head * hd;
    const int pos0 = c->n_past;
    const long head_stride = (long)c->max_seq * hd, layer_stride = (long)in->n_kv_head * head_stride;
    TRY(sdy_dequant_gather(&m->tok_embd.m, decode ? c->step_dev : c->tok_dev, n, c->x, c->st));
    for (int l = 0; l < in->n_layer; l++) {
        const dlayer *L = &m->layers[l];
        const size_t kv_off = (size_t)l * layer_stride * sdy_kv_elt_bytes(c->kv_type);
        void *kc = (char *)c->k_cache + kv_off, *vc = (char *)c->v_cache + kv_off;
        if (decode) {
            /* q | k | v of the token, contiguous in c->qkv */
            float *q = c->qkv, *k = q + q_dim, *v = k + kv_dim;
            const int bias_fused = !in->qkv_bias ||
                                   (L->bk == L->bq + q_dim && (L->qkv_parts < 3 || L->bv == L->bk + kv_dim));
            int qkv_done = 0;
            if (c->fuse_act && L->qkv_parts == 2 && bias_fused &&
                sdy_matvec_pair_ok(&L->wqkv.m, SDY_EPI_NONE, &L->wv.m, SDY_EPI_NONE)) {
                /* attention RMSNorm, quantisation, q|k and v in one launch */
                sdy_mv_args a1 = fused_args(c, q, c->x, L->attn_norm, &L->wqkv, L->bq, NULL, SDY_EPI_NONE);
                sdy_mv_args a2 = fused_args(c, v, c->x, L->attn_norm, &L->wv, L->bv, NULL, SDY_EPI_NONE);
                if (sdy_matvec_fused_ok(&L->wqkv.m, &a1, &L->wv.m, &a2)) {
                    xq_forget(c);
                    TRY(sdy_matvec_pair(&L->wqkv.m, &a1, &L->wv.m, &a2, c->st));
                    qkv_done = 1;
                }
            }
            if (!qkv_done) {
                TRY(norm_for(c, c->x, L->attn_norm, L->qkv_parts >= 2 ? &L->wqkv : &L->wq, 1));
                if (L->qkv_parts == 2 && bias_fused &&
                    sdy_matvec_pair_ok(&L->wqkv.m, SDY_EPI_NONE, &L->wv.m, SDY_EPI_NONE)) {
                    TRY(mm1_pair(c, q, &L->wqkv, L->bq, v, &L->wv, L->bv)); /* q|k and v in one launch */
                } else if (L->qkv_parts >= 2 && bias_fused) {
                    TRY(mm(c, q, c->xb, &L->wqkv, 1, L->bq, NULL, 0));
                    if (L->qkv_parts == 2) TRY(mm(c, v, c->xb, &L->wv, 1, L->bv, NULL, 0));
                } else {
                    TRY(mm(c, q, c->xb, &L->wq, 1, L->bq, NULL, 0));
                    TRY(mm(c, k, c->xb, &L->wk, 1, L->bk, NULL, 0));
                    TRY(mm(c, v, c->xb, &L->wv, 1, L->bv, NULL, 0));
                }
            }
            /* attention into att (and, for a K-quant wo, its Q8_K row: mm then reuses it, unless wo
               quantises att itself: rows of up to 8 super-blocks; a longer row is quantised once by
               the chunked attention's merge instead of by every wo workgroup, measured on the
               30B-A3B's 4096-element row: 398 -> 410 tok/s, while the 3B's 2048 keep the fused form,
               648 against 642) */
            sdy_mv_args awo = fused_args(c, c->x, c->att, NULL, &L->wo, NULL, c->x, SDY_EPI_NONE);
            int wo_fused = c->fuse_act && sdy_matvec_fused_ok(&L->wo.m, &awo, NULL, NULL) &&
                           !(c->attn_mode == SDY_ATTN_CHUNKED && q_dim > 2048);
            int q8k = !wo_fused && vec_dot_type(L->wo.type) == SDY_Q8_K;
            if (c->attn_mode == SDY_ATTN_CHUNKED) {
                TRY(sdy_attn_decode_chunked(q, k, v, L->q_norm, L->k_norm, in->norm_eps, c->rope_cos, c->rope_sin,
                                            c->step_dev, in->n_head, in->n_kv_head, hd, in->rope_interleaved, kc, vc,
                                            c->kv_type, head_stride, c->max_seq, c->attn_part, c->att,
                                            q8k ? c->xq[1] : NULL, c->st));
            } else if (c->attn_mode == SDY_ATTN_SPLIT) {
                /* the split attention's merge writes wo's Q8_K row when wo does not quantise att
                   itself (measured: wo quantising in its prologue is faster than reading the row) */
                q8k = !wo_fused && vec_dot_type(L->wo.type) == SDY_Q8_K && in->n_head / in->n_kv_head * hd % 256 == 0;
                TRY(sdy_attn_decode_split(q, k, v, L->q_norm, L->k_norm, in->norm_eps, c->rope_cos, c->rope_sin,
                                          c->step_dev, in->n_head, in->n_kv_head, hd, in->rope_interleaved, kc, vc,
                                          head_stride, c->max_seq, c->attn_part, c->attn_count, c->att,
                                          q8k ? c->xq[1] : NULL, c->st));
            } else {
                TRY(sdy_attn_decode(q, k, v, L->q_norm, L->k_norm, in->norm_eps, c->rope_cos, c->rope_sin,
                                    c->step_dev, in->n_head, in->n_kv_head, hd, in->rope_interleaved, kc, vc,
                                    c->kv_type, head_stride, c->max_seq, c->part, c->att, q8k ? c->xq[1] : NULL,
                                    c->st));
            }
            xq_forget(c);
            if (q8k) {
                c->xq_src[1] = c->att;
                c->xq_n_tok[1] = 1;
                c->xq_n_in[1] = q_dim;
            }
            if (wo_fused) TRY(sdy_matvec(&L->wo.m, &awo, c->st));
            else TRY(mm(c, c->x, c->att, &L->wo, 1, NULL, c->x, 0));
        } else {
            TRY(norm_for(c, c->x, L->attn_norm, L->qkv_parts >= 2 ? &L->wqkv : &L->wq, n));
            const int bias_fused = !in->qkv_bias ||
                                   (L->bk == L->bq + q_dim && (L->qkv_parts < 3 || L->bv == L->bk + kv_dim));
            float *q = c->q, *k = c->k, *v = c->v;
            long qs = q_dim, ks = kv_dim, vs = kv_dim;
            if (L->qkv_parts >= 2 && bias_fused && use_gemm(&L->wqkv, n)) {
                /* q | k (| v) of every token from one GEMM: rows of c->qkv, wqkv.n_out floats apart; a v of
                   another type in the same launch */
                q = c->qkv;
                k = c->qkv + q_dim;
                qs = ks = L->wqkv.n_out;
                if (L->qkv_parts == 3) {
                    TRY(mm(c, c->qkv, c->xb, &L->wqkv, n, L->bq, NULL, 0));
                    v = c->qkv + q_dim + kv_dim;
                    vs = L->wqkv.n_out;
                } else {
                    TRY(mm_pair(c, c->qkv, &L->wqkv, L->bq, c->v, &L->wv, L->bv, c->xb, n));
                }
            } else {
                TRY(mm(c, c->q, c->xb, &L->wq, n, L->bq, NULL, 0));
                TRY(mm(c, c->k, c->xb, &L->wk, n, L->bk, NULL, 0));
                TRY(mm(c, c->v, c->xb, &L->wv, n, L->bv, NULL, 0));
            }
            TRY(sdy_qk_rope_kv_strided(q, k, v, qs, ks, vs, L->q_norm, L->k_norm, in->norm_eps, c->rope_cos,
                                       c->rope_sin, pos0, n, in->n_head, in->n_kv_head, hd, in->rope_interleaved, kc,
                                       vc, c->kv_type, head_stride, c->st));
            if (c->prefill_flash && (qs & 3) == 0)
                TRY(sdy_attention_flash(q, kc, vc, c->kv_type, n, in->n_head, in->n_kv_head, hd, pos0 + 1, head_stride,
                                        qs, c->att, q_dim, c->st));
            else
                TRY(sdy_attention(q, kc, vc, c->kv_type, n, in->n_head, in->n_kv_head, hd, pos0 + 1, head_stride, qs,
                                  c->part, c->att, q_dim, c->st));
            TRY(mm(c, c->x, c->att, &L->wo, n, NULL, c->x, 1));
        }
        if (in->n_expert && decode && c->moe_device) {
            TRY(moe_decode(c, L));
        } else if (in->n_expert && c->moe_grouped_ok && n * in->n_expert_used >= GEMM_MIN_TOKENS) {
            TRY(norm_for(c, c->x, L->ffn_norm, &L->gate_inp, n));
            TRY(moe_grouped(c, L, n));
        } else if (in->n_expert) {
            TRY(norm_for(c, c->x, L->ffn_norm, &L->gate_inp, n));
            TRY(moe(c, L, n));
            TRY(sdy_add(c->x, c->moe_sum, c->x, (long)n * dim, c->st));
        } else {
            /* one token: the FFN RMSNorm and quantisation inside gate|up, and the hidden row's quantiser
               inside down (its 8-wave workgroups request the row, then their rows' weights, and
               quantise the row while the weights stream: 3B decode 677 against 659-661 tok/s with the
               quantiser's own launch) */
            const int rc = decode && L->gu_fused
                               ? mm1_fused(c, c->hb, c->x, L->ffn_norm, &L->gate_up, NULL, NULL, SDY_EPI_SWIGLU)
                               : 1;
            if (rc < 0) return rc;
            if (rc) {
                TRY(norm_for(c, c->x, L->ffn_norm, L->gu_fused ? &L->gate_up : &L->gate, n));
                TRY(ffn_gate_up(c, c->xb, n, 0, L->gu_fused ? &L->gate_up : NULL, &L->gate, &L->up, in->ffn_dim));
            }
            const int drc = decode ? mm1_fused(c, c->x, c->hb, NULL, &L->down, NULL, c->x, SDY_EPI_NONE) : 1;
            if (drc < 0) return drc;
            if (drc) TRY(mm(c, c->x, c->hb, &L->down, n, NULL, c->x, 1));
        }
    }
    if (out_rows > 0) {
        const float *xs = c->x + (size_t)(n - out_rows) * dim;
        /* one row of logits: the head's workgroups normalise and quantise the row themselves (the
           persistent ring matvec with its norm prologue, the bits of the norm launch + matvec) */
        const int hrc = out_rows == 1 ? mm1_fused(c, c->logits_dev, xs, m->output_norm, &m->output, NULL, NULL,
                                                  SDY_EPI_NONE)
                                      : 1;
        if (hrc < 0) return hrc;
        if (hrc) {
            TRY(norm_for(c, xs, m->output_norm, &m->output, out_rows));
            TRY(mm(c, c->logits_dev, c->xb, &m->output, out_rows, NULL, NULL, 0));
        }
    }
    return 0;
}

int sdy_engine_forward(engine_ctx *c, const int32_t *tokens, int n, int out_rows) {
    const engine_model_info *in = &c->m->info;
    const int decode = n == 1 && c->decode_fused;
    if (decode) {
        c->step_host[0] = tokens[0];
        c->step_host[1] = c->n_past;
        TRY(sdy_h2d(c->step_dev, c->step_host, 2 * 4, c->st));
        /* the first one-token step runs eagerly (it settles every lazily configured kernel); the
           second is recorded as a graph that later steps replay */
        if (c->graph_ok == 0 && c->use_graph && c->n_decode >= 1) {
            TRY(sdy_graph_begin(c->st));
            int rc = layers(c, 1, out_rows, 1);
            if (rc) {
                sdy_graph_abort(c->st);
                c->graph_ok = -1;
                return rc;
            }
            if (sdy_graph_end(c->st, &c->graph)) {
                c->graph = NULL;
                c->graph_ok = -1; /* not recordable here: keep running eagerly */
            } else {
                c->graph_ok = 1;
            }
        }
        if (c->graph_ok == 1 && out_rows == 1) TRY(sdy_graph_launch(c->graph, c->st));
        else TRY(layers(c, 1, out_rows, 1));
        c->n_decode++;
    } else {
        memcpy(c->tok_host, tokens, (size_t)n * 4);
        TRY(sdy_h2d(c->tok_dev, c->tok_host, (size_t)n * 4, c->st));
        TRY(layers(c, n, out_rows, 0));
    }
    if (out_rows > 0) TRY(sdy_d2h(c->logits, c->logits_dev, (size_t)out_rows * in->n_vocab * 4, c->st));
    TRY(sdy_sync(c->st));
    c->n_past += n;
    return 0;
}

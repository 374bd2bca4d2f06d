/* Oracle restatement of the reference's model forward: csrc/model_llama.c:542-886 (matmul with
 * activation quantisation, attention with the causal mask, SwiGLU MLP, qwen3moe router and
 * experts, eval/reset/truncate). Test infrastructure only (see oracle.h).
 *
 * Differences that do not change results: no thread pool (every output element is computed by
 * one sequence of operations, as in the reference), no prefetch, no activation-quantisation cache
 * (quantising the same rows again yields the same bytes).
 */
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

struct orc_model {
    orc_info info;
    orc_tensor tok_embd, output;
    float *output_norm;
    orc_layer *layers;
    float *vec; /* f32 copies of norms and biases */
    float **attn_norm, **ffn_norm, **bq, **bk, **bv, **q_norm, **k_norm;
};

struct orc_ctx {
    const orc_model *m;
    int max_seq, n_batch, logits_all, simd, n_past, n_logits;
    int kv_f16; /* the cache holds each K/V value rounded to f16 (orc_ctx_set_kv_f16) */
    float *k_cache, *v_cache, *rope_cos, *rope_sin;
    float *x, *xb, *q, *k, *v, *att, *hb, *hb2, *scores, *logits;
    float *moe_probs, *moe_w, *moe_x, *moe_y, *moe_sum;
    int32_t *moe_top, *topk_log;
    void *xq;
};

static float *to_f32(orc_tensor t, int n) {
    float *out = malloc(sizeof(float) * (size_t)n);
    if (out && t.data) orc_row_to_f32(t.data, t.type, out, (size_t)n);
    return out;
}

orc_model *orc_model_new(const orc_info *info, orc_tensor tok_embd, orc_tensor output_norm, orc_tensor output,
                         const orc_layer *layers) {
    orc_model *m = calloc(1, sizeof(*m));
    m->info = *info;
    m->tok_embd = tok_embd;
    m->output = info->tied_embeddings ? tok_embd : output;
    int L = info->n_layer, hd = info->head_dim, dim = info->dim;
    int q_dim = info->n_head * hd, kv_dim = info->n_kv_head * hd;
    m->layers = malloc(sizeof(orc_layer) * (size_t)L);
    memcpy(m->layers, layers, sizeof(orc_layer) * (size_t)L);
    m->output_norm = to_f32(output_norm, dim);
    m->attn_norm = calloc((size_t)L, sizeof(float *));
    m->ffn_norm = calloc((size_t)L, sizeof(float *));
    m->bq = calloc((size_t)L, sizeof(float *));
    m->bk = calloc((size_t)L, sizeof(float *));
    m->bv = calloc((size_t)L, sizeof(float *));
    m->q_norm = calloc((size_t)L, sizeof(float *));
    m->k_norm = calloc((size_t)L, sizeof(float *));
    for (int l = 0; l < L; l++) {
        const orc_layer *ly = &layers[l];
        m->attn_norm[l] = to_f32(ly->attn_norm, dim);
        m->ffn_norm[l] = to_f32(ly->ffn_norm, dim);
        if (info->qkv_bias) {
            m->bq[l] = to_f32(ly->bq, q_dim);
            m->bk[l] = to_f32(ly->bk, kv_dim);
            m->bv[l] = to_f32(ly->bv, kv_dim);
        }
        if (info->qk_norm) {
            m->q_norm[l] = to_f32(ly->q_norm, hd);
            m->k_norm[l] = to_f32(ly->k_norm, hd);
        }
    }
    return m;
}

void orc_model_free(orc_model *m) {
    if (!m) return;
    for (int l = 0; l < m->info.n_layer; l++) {
        free(m->attn_norm[l]); free(m->ffn_norm[l]); free(m->bq[l]); free(m->bk[l]); free(m->bv[l]);
        free(m->q_norm[l]); free(m->k_norm[l]);
    }
    free(m->attn_norm); free(m->ffn_norm); free(m->bq); free(m->bk); free(m->bv); free(m->q_norm); free(m->k_norm);
    free(m->output_norm);
    free(m->layers);
    free(m);
}

static float *falloc(size_t n) { return calloc(n ? n : 1, sizeof(float)); }

orc_ctx *orc_ctx_new(const orc_model *m, int max_seq, int n_batch, int logits_all, int simd) {
    const orc_info *in = &m->info;
    if (max_seq < 1 || max_seq > in->max_pos || n_batch < 1) return NULL;
    orc_ctx *c = calloc(1, sizeof(*c));
    c->m = m;
    c->max_seq = max_seq;
    c->n_batch = n_batch;
    c->logits_all = logits_all != 0;
    c->simd = simd;
    size_t B = (size_t)n_batch, S = (size_t)max_seq, hd = (size_t)in->head_dim;
    size_t q_dim = (size_t)in->n_head * hd, kv_dim = (size_t)in->n_kv_head * hd;
    size_t kv = (size_t)in->n_layer * in->n_kv_head * S * hd;
    size_t ffn = (size_t)(in->n_expert ? in->ffn_exp_dim : in->ffn_dim);
    c->k_cache = falloc(kv);
    c->v_cache = falloc(kv);
    c->rope_cos = falloc(S * hd / 2);
    c->rope_sin = falloc(S * hd / 2);
    c->x = falloc(B * in->dim);
    c->xb = falloc(B * in->dim);
    c->q = falloc(B * q_dim);
    c->k = falloc(B * kv_dim);
    c->v = falloc(B * kv_dim);
    c->att = falloc(B * q_dim);
    c->hb = falloc(B * ffn);
    c->hb2 = falloc(B * ffn);
    c->scores = falloc(S);
    c->logits = falloc((c->logits_all ? B : 1) * (size_t)in->n_vocab);
    if (in->n_expert) {
        c->moe_probs = falloc(B * in->n_expert);
        c->moe_w = falloc(B * in->n_expert_used);
        c->moe_x = falloc(B * in->dim);
        c->moe_y = falloc(B * in->dim);
        c->moe_sum = falloc(B * in->dim);
        c->moe_top = calloc(B * in->n_expert_used, sizeof(int32_t));
        c->topk_log = calloc((size_t)in->n_layer * B * in->n_expert_used, sizeof(int32_t));
    }
    size_t max_in = (size_t)in->dim > q_dim ? (size_t)in->dim : q_dim;
    if (ffn > max_in) max_in = ffn;
    c->xq = malloc(B * ((max_in + 31) / 32 * 34 + (max_in + 255) / 256 * 292) + 64);
    orc_rope_table(c->rope_cos, c->rope_sin, max_seq, in->head_dim, in->rope_theta);
    return c;
}

/* Not in the reference: a cache of f16 values, each K/V value rounded with the reference's
 * f32 -> f16 conversion (csrc/ops.c:43-62) when it is written, the model otherwise unchanged. The
 * f16-cache engine is checked against this. */
void orc_ctx_set_kv_f16(orc_ctx *c, int on) { c->kv_f16 = on != 0; }

void orc_ctx_free(orc_ctx *c) {
    if (!c) return;
    free(c->k_cache); free(c->v_cache); free(c->rope_cos); free(c->rope_sin);
    free(c->x); free(c->xb); free(c->q); free(c->k); free(c->v); free(c->att); free(c->hb); free(c->hb2);
    free(c->scores); free(c->logits);
    free(c->moe_probs); free(c->moe_w); free(c->moe_x); free(c->moe_y); free(c->moe_sum); free(c->moe_top);
    free(c->topk_log);
    free(c->xq);
    free(c);
}

/* matmul() (csrc/model_llama.c:592-611): F32/F16/BF16 weights multiply float activations; quantized
 * weights first quantize the activation rows to the weight's dot type. */
static void matmul(orc_ctx *c, float *out, const float *x, orc_tensor w, int n_tok, int n_in, int n_out) {
    int vt = orc_vec_dot_type(w.type);
    if (vt == ORC_F32) {
        orc_matmul_rows(out, x, w.data, w.type, n_tok, n_in, n_out, 0, n_out, c->simd);
        return;
    }
    orc_quantize_rows(vt, x, c->xq, n_in, 0, n_tok);
    orc_matmul_q_rows(out, c->xq, w.data, w.type, n_tok, n_in, n_out, 0, n_out, c->simd);
}

/* moe_select (csrc/model_llama.c:653-666): insertion into a sorted top-k; a later expert must be
 * strictly more probable to pass an earlier one, so ties keep the lower index. */
static void moe_select(const float *probs, int n_expert, int k, int32_t *top, float *w) {
    int n = 0;
    for (int e = 0; e < n_expert; e++) {
        int pos = n;
        while (pos > 0 && probs[e] > probs[top[pos - 1]]) pos--;
        if (pos == k) continue;
        int last = n < k ? n : k - 1;
        for (int j = last; j > pos; j--) top[j] = top[j - 1];
        top[pos] = e;
        if (n < k) n++;
    }
    float sum = 0.0f;
    for (int i = 0; i < k; i++) sum += probs[top[i]];
    for (int i = 0; i < k; i++) w[i] = probs[top[i]] / sum;
}

static orc_tensor expert_slice(orc_tensor w, int e, int n_in, int n_out) {
    orc_tensor t = {(const uint8_t *)w.data + (size_t)e * n_out * orc_row_size(w.type, n_in), w.type};
    return t;
}

/* moe_ffn (csrc/model_llama.c:724-751): experts in ascending order, each over its tokens in
 * ascending order; outputs accumulated with axpy in that order. */
static void moe_ffn(orc_ctx *c, int l, int n) {
    const orc_info *in = &c->m->info;
    const orc_layer *L = &c->m->layers[l];
    int dim = in->dim, fe = in->ffn_exp_dim, ne = in->n_expert, k = in->n_expert_used;
    matmul(c, c->moe_probs, c->xb, L->gate_inp, n, dim, ne);
    for (int t = 0; t < n; t++) {
        float *probs = c->moe_probs + (size_t)t * ne;
        orc_softmax(probs, ne);
        moe_select(probs, ne, k, c->moe_top + (size_t)t * k, c->moe_w + (size_t)t * k);
    }
    memcpy(c->topk_log + (size_t)l * n * k, c->moe_top, sizeof(int32_t) * (size_t)n * k);
    memset(c->moe_sum, 0, sizeof(float) * (size_t)n * dim);
    int32_t *tok = malloc(sizeof(int32_t) * (size_t)(n * k));
    float *wt = malloc(sizeof(float) * (size_t)(n * k));
    for (int e = 0; e < ne; e++) {
        int m = 0;
        for (int i = 0; i < n * k; i++)
            if (c->moe_top[i] == e) {
                tok[m] = i / k;
                wt[m] = c->moe_w[i];
                m++;
            }
        if (!m) continue;
        for (int r = 0; r < m; r++) memcpy(c->moe_x + (size_t)r * dim, c->xb + (size_t)tok[r] * dim, sizeof(float) * dim);
        matmul(c, c->hb, c->moe_x, expert_slice(L->gate, e, dim, fe), m, dim, fe);
        matmul(c, c->hb2, c->moe_x, expert_slice(L->up, e, dim, fe), m, dim, fe);
        orc_silu_mul(c->hb, c->hb2, m * fe);
        matmul(c, c->moe_y, c->hb, expert_slice(L->down, e, fe, dim), m, fe, dim);
        for (int r = 0; r < m; r++)
            orc_axpy(c->moe_sum + (size_t)tok[r] * dim, wt[r], c->moe_y + (size_t)r * dim, dim, c->simd);
    }
    free(tok);
    free(wt);
}

/* forward (csrc/model_llama.c:757-832) */
static void forward(orc_ctx *c, const int32_t *tokens, int n, int out_rows) {
    const orc_model *m = c->m;
    const orc_info *in = &m->info;
    int dim = in->dim, hd = in->head_dim, half = hd / 2;
    int q_dim = in->n_head * hd, kv_dim = in->n_kv_head * hd, pos0 = c->n_past;
    size_t head_stride = (size_t)c->max_seq * hd, layer_stride = (size_t)in->n_kv_head * head_stride;
    size_t emb_row = orc_row_size(m->tok_embd.type, dim);
    for (int t = 0; t < n; t++)
        orc_row_to_f32((const uint8_t *)m->tok_embd.data + (size_t)tokens[t] * emb_row, m->tok_embd.type,
                       c->x + (size_t)t * dim, (size_t)dim);
    for (int l = 0; l < in->n_layer; l++) {
        const orc_layer *L = &m->layers[l];
        float *kc = c->k_cache + l * layer_stride, *vc = c->v_cache + l * layer_stride;
        for (int t = 0; t < n; t++)
            orc_rmsnorm(c->xb + (size_t)t * dim, c->x + (size_t)t * dim, m->attn_norm[l], dim, in->norm_eps);
        matmul(c, c->q, c->xb, L->wq, n, dim, q_dim);
        matmul(c, c->k, c->xb, L->wk, n, dim, kv_dim);
        matmul(c, c->v, c->xb, L->wv, n, dim, kv_dim);
        if (in->qkv_bias)
            for (int t = 0; t < n; t++) {
                for (int i = 0; i < q_dim; i++) c->q[(size_t)t * q_dim + i] += m->bq[l][i];
                for (int i = 0; i < kv_dim; i++) c->k[(size_t)t * kv_dim + i] += m->bk[l][i];
                for (int i = 0; i < kv_dim; i++) c->v[(size_t)t * kv_dim + i] += m->bv[l][i];
            }
        for (int t = 0; t < n; t++) {
            int pos = pos0 + t;
            const float *cs = c->rope_cos + (size_t)pos * half, *sn = c->rope_sin + (size_t)pos * half;
            float *qt = c->q + (size_t)t * q_dim, *kt = c->k + (size_t)t * kv_dim, *vt = c->v + (size_t)t * kv_dim;
            if (in->qk_norm) {
                for (int h = 0; h < in->n_head; h++) orc_rmsnorm(qt + h * hd, qt + h * hd, m->q_norm[l], hd, in->norm_eps);
                for (int h = 0; h < in->n_kv_head; h++) orc_rmsnorm(kt + h * hd, kt + h * hd, m->k_norm[l], hd, in->norm_eps);
            }
            orc_rope(qt, in->n_head, hd, cs, sn, in->rope_interleaved);
            orc_rope(kt, in->n_kv_head, hd, cs, sn, in->rope_interleaved);
            for (int h = 0; h < in->n_kv_head; h++) {
                float *kd = kc + h * head_stride + (size_t)pos * hd, *vd = vc + h * head_stride + (size_t)pos * hd;
                memcpy(kd, kt + (size_t)h * hd, sizeof(float) * hd);
                memcpy(vd, vt + (size_t)h * hd, sizeof(float) * hd);
                if (c->kv_f16)
                    for (int i = 0; i < hd; i++) {
                        kd[i] = orc_f16_to_f32(orc_f32_to_f16(kd[i]));
                        vd[i] = orc_f16_to_f32(orc_f32_to_f16(vd[i]));
                    }
            }
        }
        for (int t = 0; t < n; t++) /* token t sees positions 0..pos0+t */
            orc_attention(c->att + (size_t)t * q_dim, c->q + (size_t)t * q_dim, kc, vc, in->n_head, in->n_kv_head, hd,
                          pos0 + t + 1, c->max_seq, c->scores, c->simd);
        matmul(c, c->xb, c->att, L->wo, n, q_dim, dim);
        for (size_t i = 0; i < (size_t)n * dim; i++) c->x[i] += c->xb[i];
        for (int t = 0; t < n; t++)
            orc_rmsnorm(c->xb + (size_t)t * dim, c->x + (size_t)t * dim, m->ffn_norm[l], dim, in->norm_eps);
        const float *ffn_out = c->xb;
        if (in->n_expert) {
            moe_ffn(c, l, n);
            ffn_out = c->moe_sum;
        } else {
            matmul(c, c->hb, c->xb, L->gate, n, dim, in->ffn_dim);
            matmul(c, c->hb2, c->xb, L->up, n, dim, in->ffn_dim);
            orc_silu_mul(c->hb, c->hb2, n * in->ffn_dim);
            matmul(c, c->xb, c->hb, L->down, n, in->ffn_dim, dim);
        }
        for (size_t i = 0; i < (size_t)n * dim; i++) c->x[i] += ffn_out[i];
    }
    if (out_rows > 0) {
        const float *xs = c->x + (size_t)(n - out_rows) * dim;
        for (int r = 0; r < out_rows; r++)
            orc_rmsnorm(c->xb + (size_t)r * dim, xs + (size_t)r * dim, m->output_norm, dim, in->norm_eps);
        matmul(c, c->logits, c->xb, m->output, out_rows, dim, in->n_vocab);
    }
    c->n_past += n;
}

/* engine_eval (csrc/model_llama.c:834-864): validation leaves the context unchanged; chunks of
 * n_batch tokens; logits of the last chunk only. */
int orc_eval(orc_ctx *c, const int32_t *tokens, int n) {
    if (!c || !tokens || n < 1) return -1;
    if (c->logits_all && n > c->n_batch) return -1;
    if (n > c->max_seq - c->n_past) return -1;
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= c->m->info.n_vocab) return -1;
    for (int done = 0; done < n;) {
        int chunk = n - done < c->n_batch ? n - done : c->n_batch;
        int last = done + chunk == n;
        forward(c, tokens + done, chunk, last ? (c->logits_all ? chunk : 1) : 0);
        done += chunk;
    }
    c->n_logits = c->logits_all ? n : 1;
    return 0;
}

const float *orc_logits(const orc_ctx *c) { return c && c->n_logits ? c->logits : NULL; }
int orc_n_logits(const orc_ctx *c) { return c ? c->n_logits : 0; }
int orc_n_past(const orc_ctx *c) { return c ? c->n_past : 0; }
void orc_reset(orc_ctx *c) {
    if (!c) return;
    c->n_past = 0;
    c->n_logits = 0;
}
int orc_truncate(orc_ctx *c, int n) {
    if (!c || n < 0 || n > c->n_past) return -1;
    c->n_past = n;
    c->n_logits = 0;
    return 0;
}
const int32_t *orc_last_topk(const orc_ctx *c) { return c ? c->topk_log : NULL; }

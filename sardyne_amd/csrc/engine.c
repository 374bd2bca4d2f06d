/* Model runtime on the GPU: GGUF -> device weights, device KV cache, forward pass, eval API.
 *
 * The host side here is the reference's csrc/model_llama.c contract (engine_* of
 * include/sardyne.h) re-implemented around device buffers: the model is uploaded once (every
 * matrix repacked into the device layout of quant_kernels.hip, every expert resident), a context
 * owns the f32 KV cache [n_layer][n_kv_head][max_seq][head_dim] and the activations in device
 * memory, and engine_eval runs the layer sequence of the reference forward
 * (csrc/model_llama.c:757-832) as a stream of gfx950 kernels, copying back only the logits.
 *
 * Validation rules and error messages follow csrc/model_llama.c:225-319 and :468-525, :834-886,
 * because callers match on them (the Python runtime raises them as ValueError).
 */
#define _POSIX_C_SOURCE 200809L
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sardyne.h"
#include "sdy_engine.h"
#include "sdy_ops.h"
#include "sdy_shim.h"

#define MAX_SEQ_LIMIT (1 << 20)
#define MAX_BATCH_LIMIT 4096

static void set_err(char *err, size_t len, const char *fmt, ...) {
    if (!err || !len) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, len, fmt, ap);
    va_end(ap);
}

/* ------------------------------------------------------------------ metadata */

typedef struct {
    const gguf_file *gf;
    const char *arch;
    char *err;
    size_t err_len;
} meta;

static int64_t arch_key(const meta *mt, const char *suffix) {
    char key[128];
    snprintf(key, sizeof key, "%s.%s", mt->arch, suffix);
    return gguf_find_kv(mt->gf, key);
}

/* Required (def < 0) or defaulted positive integer; -1 on error. */
static int64_t meta_int(const meta *mt, const char *suffix, int64_t def) {
    int64_t i = arch_key(mt, suffix);
    uint64_t v;
    if (i < 0) {
        if (def < 0) set_err(mt->err, mt->err_len, "metadato mancante: %s.%s", mt->arch, suffix);
        return def;
    }
    if (gguf_kv_get_u64(mt->gf, i, &v) || v == 0 || v > (1u << 30)) {
        set_err(mt->err, mt->err_len, "metadato non valido: %s.%s", mt->arch, suffix);
        return -1;
    }
    return (int64_t)v;
}

static int meta_float(const meta *mt, const char *suffix, double def, float *out) {
    int64_t i = arch_key(mt, suffix);
    double v = def;
    if (i < 0 && def < 0) {
        set_err(mt->err, mt->err_len, "metadato mancante: %s.%s", mt->arch, suffix);
        return -1;
    }
    if (i >= 0 && gguf_kv_get_f64(mt->gf, i, &v)) {
        set_err(mt->err, mt->err_len, "metadato non valido: %s.%s", mt->arch, suffix);
        return -1;
    }
    if (!(v > 0.0) || v > 1e12) {
        set_err(mt->err, mt->err_len, "valore non valido per %s.%s", mt->arch, suffix);
        return -1;
    }
    *out = (float)v;
    return 0;
}

static const char *const LAYER_TENSORS[] = {
    "attn_norm.weight", "attn_q.weight", "attn_q.bias", "attn_k.weight", "attn_k.bias", "attn_v.weight",
    "attn_v.bias", "attn_q_norm.weight", "attn_k_norm.weight", "attn_output.weight", "ffn_norm.weight",
    "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight", "ffn_gate_inp.weight", "ffn_gate_exps.weight",
    "ffn_up_exps.weight", "ffn_down_exps.weight",
};

/* Unknown tensors mean an architecture variant this runtime does not implement. */
static int known_tensor(const char *name, int n_layer) {
    if (!strcmp(name, "token_embd.weight") || !strcmp(name, "output_norm.weight") || !strcmp(name, "output.weight"))
        return 1;
    if (strncmp(name, "blk.", 4)) return 0;
    const char *p = name + 4;
    if (*p < '0' || *p > '9') return 0;
    long idx = 0;
    for (; *p >= '0' && *p <= '9'; p++)
        if ((idx = idx * 10 + (*p - '0')) >= n_layer) return 0;
    if (*p++ != '.') return 0;
    for (size_t k = 0; k < sizeof LAYER_TENSORS / sizeof *LAYER_TENSORS; k++)
        if (!strcmp(p, LAYER_TENSORS[k])) return 1;
    return 0;
}

static const gguf_tensor *find(const gguf_file *gf, const char *name) {
    int64_t i = gguf_find_tensor(gf, name);
    return i < 0 ? NULL : gguf_get_tensor(gf, (uint64_t)i);
}

static int type_supported(uint32_t t) {
    return t == OP_F32 || t == OP_F16 || t == OP_BF16 || t == OP_Q8_0 || t == OP_Q4_0 || t == OP_Q5_0 ||
           t == OP_Q4_K || t == OP_Q6_K;
}

static int read_config(engine_model *m, char *err, size_t err_len) {
    const gguf_file *gf = m->gf;
    uint64_t len;
    const char *arch = gguf_kv_get_str(gf, gguf_find_kv(gf, "general.architecture"), &len);
    char ab[32];
    if (!arch || len == 0 || len >= sizeof ab) {
        set_err(err, err_len, "general.architecture mancante o non valido");
        return -1;
    }
    memcpy(ab, arch, len);
    ab[len] = '\0';
    engine_model_info *in = &m->info;
    if (!strcmp(ab, "llama")) in->rope_interleaved = 1;
    else if (!strcmp(ab, "qwen2") || !strcmp(ab, "qwen3") || !strcmp(ab, "qwen3moe")) in->rope_interleaved = 0;
    else {
        set_err(err, err_len, "architettura %s non supportata", ab);
        return -1;
    }
    meta mt = {gf, ab, err, err_len};
    const char *scaling = gguf_kv_get_str(gf, arch_key(&mt, "rope.scaling.type"), &len);
    if ((scaling && !(len == 4 && !memcmp(scaling, "none", 4))) || find(gf, "rope_freqs.weight")) {
        set_err(err, err_len, "rope scaling (anche 'llama3' via rope_freqs.weight) non supportato");
        return -1;
    }
    int64_t v;
    if ((v = meta_int(&mt, "embedding_length", -1)) < 0) return -1;
    in->dim = (int32_t)v;
    if ((v = meta_int(&mt, "block_count", -1)) < 0) return -1;
    in->n_layer = (int32_t)v;
    if ((v = meta_int(&mt, "feed_forward_length", -1)) < 0) return -1;
    in->ffn_dim = (int32_t)v;
    if (!strcmp(ab, "qwen3moe")) {
        if ((v = meta_int(&mt, "expert_count", -1)) < 0) return -1;
        in->n_expert = (int32_t)v;
        if ((v = meta_int(&mt, "expert_used_count", -1)) < 0) return -1;
        in->n_expert_used = (int32_t)v;
        if (in->n_expert_used > in->n_expert) {
            set_err(err, err_len, "expert_used_count=%d oltre expert_count=%d", in->n_expert_used, in->n_expert);
            return -1;
        }
        /* the device router keeps a token's expert probabilities in one wave's registers */
        if (in->n_expert > 512 || in->n_expert_used < 1 || in->n_expert_used > 64) {
            set_err(err, err_len, "expert_count=%d / expert_used_count=%d oltre i limiti del dispositivo (512 / 64)",
                    in->n_expert, in->n_expert_used);
            return -1;
        }
        if ((v = meta_int(&mt, "expert_feed_forward_length", in->ffn_dim / in->n_expert_used)) <= 0) {
            if (v == 0) set_err(err, err_len, "dimensione degli esperti nulla");
            return -1;
        }
        in->ffn_exp_dim = (int32_t)v;
    }
    if ((v = meta_int(&mt, "attention.head_count", -1)) < 0) return -1;
    in->n_head = (int32_t)v;
    if ((v = meta_int(&mt, "attention.head_count_kv", in->n_head)) < 0) return -1;
    in->n_kv_head = (int32_t)v;
    if ((v = meta_int(&mt, "attention.key_length", in->dim / in->n_head)) <= 0) {
        if (v == 0) set_err(err, err_len, "head_dim nullo");
        return -1;
    }
    in->head_dim = (int32_t)v;
    if (meta_int(&mt, "attention.value_length", in->head_dim) != in->head_dim) {
        set_err(err, err_len, "key_length diverso da value_length");
        return -1;
    }
    if (meta_int(&mt, "rope.dimension_count", in->head_dim) != in->head_dim) {
        set_err(err, err_len, "RoPE parziale (rope.dimension_count < head_dim) non supportata");
        return -1;
    }
    if ((v = meta_int(&mt, "context_length", 2048)) < 0) return -1;
    in->max_pos = (int32_t)v;
    if (meta_float(&mt, "attention.layer_norm_rms_epsilon", -1.0, &in->norm_eps)) return -1;
    if (meta_float(&mt, "rope.freq_base", 10000.0, &in->rope_theta)) return -1;
    if (in->n_head % in->n_kv_head || in->head_dim % 2) {
        set_err(err, err_len, "teste o head_dim non validi (n_head %% n_kv_head, head_dim pari)");
        return -1;
    }
    const gguf_tensor *emb = find(gf, "token_embd.weight");
    if (!emb || emb->n_dims != 2 || emb->ne[1] == 0 || emb->ne[1] > (1u << 30)) {
        set_err(err, err_len, "token_embd.weight mancante o non valido");
        return -1;
    }
    in->n_vocab = (int32_t)emb->ne[1];
    in->tied_embeddings = find(gf, "output.weight") == NULL;
    in->qkv_bias = find(gf, "blk.0.attn_q.bias") != NULL;
    in->qk_norm = find(gf, "blk.0.attn_q_norm.weight") != NULL;
    for (uint64_t i = 0; i < gguf_n_tensors(gf); i++) {
        const char *name = gguf_get_tensor(gf, i)->name;
        if (!known_tensor(name, in->n_layer)) {
            set_err(err, err_len, "tensore non supportato: %s", name);
            return -1;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ upload */

static int sdy_err(char *err, size_t err_len, const char *what) {
    set_err(err, err_len, "%s: %s", what, sdy_last_error());
    return -1;
}

/* Descriptor of a [n_expert][n_out][n_in] tensor (n_expert = 0: a matrix [n_out][n_in]) of a
 * supported type, or NULL with the reason in err. */
static const gguf_tensor *check_tensor(engine_model *m, const char *name, int n_in, int n_out, int n_expert, char *err,
                                       size_t err_len) {
    const gguf_tensor *t = find(m->gf, name);
    if (!t) {
        set_err(err, err_len, "tensore mancante: %s", name);
        return NULL;
    }
    if (t->n_dims != (n_expert ? 3u : 2u) || t->ne[0] != (uint64_t)n_in || t->ne[1] != (uint64_t)n_out ||
        (n_expert && t->ne[2] != (uint64_t)n_expert)) {
        set_err(err, err_len, "%s: dimensioni [%llu, %llu, %llu], attese [%d, %d, %d]", name,
                (unsigned long long)t->ne[0], (unsigned long long)t->ne[1], (unsigned long long)t->ne[2], n_in, n_out,
                n_expert ? n_expert : 1);
        return NULL;
    }
    if (!type_supported(t->type)) {
        set_err(err, err_len,
                "%s: tipo %s non supportato dal runtime (supportati: F32, F16, BF16, Q8_0, Q4_0, Q5_0, Q4_K, Q6_K)",
                name, gguf_type_name(t->type));
        return NULL;
    }
    return t;
}

static void set_dmat(dmat *d, int type, int n_in, int n_out) {
    d->type = type;
    d->n_in = n_in;
    d->n_out = n_out;
}

static int get_tensor(engine_model *m, const char *name, int n_in, int n_out, int n_expert, dmat *out, char *err,
                      size_t err_len) {
    const gguf_tensor *t = check_tensor(m, name, n_in, n_out, n_expert, err, err_len);
    if (!t) return -1;
    if (sdy_mat_upload(&out->m, (int)t->type, n_in, (long)n_out * (n_expert ? n_expert : 1), t->data, m->st))
        return sdy_err(err, err_len, name);
    set_dmat(out, (int)t->type, n_in, n_out);
    m->device_bytes += out->m.bytes;
    return 0;
}

static int is_quant(uint32_t t) { return t != OP_F32 && t != OP_F16 && t != OP_BF16; }

/* Row view of a fused matrix. */
static dmat view(const dmat *w, long r0, int n_out) {
    dmat d = *w;
    d.m = sdy_mat_rows(&w->m, r0, n_out);
    d.n_out = n_out;
    return d;
}

/* wq, wk, wv. When wq and wk (and wv) have one type they are stored as one matrix whose row ranges
 * are wq, wk (, wv), so that a single matvec computes them together. */
static int get_qkv(engine_model *m, int l, dlayer *L, char *err, size_t err_len) {
    const engine_model_info *in = &m->info;
    const int dim = in->dim, q_dim = in->n_head * in->head_dim, kv_dim = in->n_kv_head * in->head_dim;
    char nq[64], nk[64], nv[64];
    snprintf(nq, sizeof nq, "blk.%d.attn_q.weight", l);
    snprintf(nk, sizeof nk, "blk.%d.attn_k.weight", l);
    snprintf(nv, sizeof nv, "blk.%d.attn_v.weight", l);
    const gguf_tensor *tq = check_tensor(m, nq, dim, q_dim, 0, err, err_len);
    const gguf_tensor *tk = tq ? check_tensor(m, nk, dim, kv_dim, 0, err, err_len) : NULL;
    const gguf_tensor *tv = tk ? check_tensor(m, nv, dim, kv_dim, 0, err, err_len) : NULL;
    if (!tv) return -1;
    if (tq->type != tk->type) {
        L->qkv_parts = 0;
        return get_tensor(m, nq, dim, q_dim, 0, &L->wq, err, err_len) ||
               get_tensor(m, nk, dim, kv_dim, 0, &L->wk, err, err_len) ||
               get_tensor(m, nv, dim, kv_dim, 0, &L->wv, err, err_len) ? -1 : 0;
    }
    const int parts = tv->type == tq->type ? 3 : 2;
    const long rows = (long)q_dim + kv_dim + (parts == 3 ? kv_dim : 0);
    if (sdy_mat_alloc(&L->wqkv.m, (int)tq->type, dim, rows)) return sdy_err(err, err_len, nq);
    set_dmat(&L->wqkv, (int)tq->type, dim, (int)rows);
    L->qkv_parts = parts;
    m->device_bytes += L->wqkv.m.bytes;
    if (sdy_mat_upload_rows(&L->wqkv.m, 0, 1, q_dim, tq->data, m->st)) return sdy_err(err, err_len, nq);
    if (sdy_mat_upload_rows(&L->wqkv.m, q_dim, 1, kv_dim, tk->data, m->st)) return sdy_err(err, err_len, nk);
    L->wq = view(&L->wqkv, 0, q_dim);
    L->wk = view(&L->wqkv, q_dim, kv_dim);
    if (parts == 3) {
        if (sdy_mat_upload_rows(&L->wqkv.m, q_dim + kv_dim, 1, kv_dim, tv->data, m->st))
            return sdy_err(err, err_len, nv);
        L->wv = view(&L->wqkv, q_dim + kv_dim, kv_dim);
        return 0;
    }
    return get_tensor(m, nv, dim, kv_dim, 0, &L->wv, err, err_len);
}

/* gate and up ([n_expert][ffn][dim]). With one quantized type they are stored interleaved, row
 * 2i = gate i and row 2i+1 = up i (per expert), for the SwiGLU matvec epilogue. */
static int get_gate_up(engine_model *m, int l, dlayer *L, int ffn, int n_expert, char *err, size_t err_len) {
    const int dim = m->info.dim;
    char ng[64], nu[64];
    snprintf(ng, sizeof ng, n_expert ? "blk.%d.ffn_gate_exps.weight" : "blk.%d.ffn_gate.weight", l);
    snprintf(nu, sizeof nu, n_expert ? "blk.%d.ffn_up_exps.weight" : "blk.%d.ffn_up.weight", l);
    const gguf_tensor *tg = check_tensor(m, ng, dim, ffn, n_expert, err, err_len);
    const gguf_tensor *tu = tg ? check_tensor(m, nu, dim, ffn, n_expert, err, err_len) : NULL;
    if (!tu) return -1;
    if (tg->type != tu->type || !is_quant(tg->type)) {
        L->gu_fused = 0;
        return get_tensor(m, ng, dim, ffn, n_expert, &L->gate, err, err_len) ||
               get_tensor(m, nu, dim, ffn, n_expert, &L->up, err, err_len) ? -1 : 0;
    }
    const long ne = n_expert ? n_expert : 1, n = ne * ffn;
    if (sdy_mat_alloc(&L->gate_up.m, (int)tg->type, dim, 2 * n)) return sdy_err(err, err_len, ng);
    set_dmat(&L->gate_up, (int)tg->type, dim, 2 * ffn);
    L->gu_fused = 1;
    m->device_bytes += L->gate_up.m.bytes;
    if (sdy_mat_upload_map(&L->gate_up.m, 0, n, 2, ffn, 2L * ffn, tg->data, m->st)) return sdy_err(err, err_len, ng);
    if (sdy_mat_upload_map(&L->gate_up.m, 1, n, 2, ffn, 2L * ffn, tu->data, m->st)) return sdy_err(err, err_len, nu);
    return 0;
}

/* Vector of n elements converted to f32 in device memory. */
static int get_vector(engine_model *m, const char *name, int n, float **dst, char *err, size_t err_len) {
    const gguf_tensor *t = find(m->gf, name);
    if (!t) {
        set_err(err, err_len, "tensore mancante: %s", name);
        return -1;
    }
    if (t->n_dims != 1 || t->ne[0] != (uint64_t)n) {
        set_err(err, err_len, "%s: dimensione %llu, attesa %d", name, (unsigned long long)t->ne[0], n);
        return -1;
    }
    if (!type_supported(t->type)) {
        set_err(err, err_len, "%s: tipo %s non supportato", name, gguf_type_name(t->type));
        return -1;
    }
    float *d = m->vec_cursor;
    m->vec_cursor += (n + 63) & ~63;
    if (t->type == OP_F32) {
        if (sdy_h2d(d, t->data, (size_t)n * 4, m->st)) return sdy_err(err, err_len, name);
    } else {
        sdy_mat tmp;
        if (sdy_mat_upload(&tmp, (int)t->type, n, 1, t->data, m->st) || sdy_dequant_rows(&tmp, 0, 1, d, m->st) ||
            sdy_sync(m->st) || sdy_mat_free(&tmp))
            return sdy_err(err, err_len, name);
    }
    *dst = d;
    return 0;
}

void engine_model_free(engine_model *m) {
    if (!m) return;
    if (m->layers) {
        for (int l = 0; l < m->info.n_layer; l++) {
            dlayer *L = &m->layers[l];
            /* row views of wqkv share its allocation */
            if (L->qkv_parts < 2) sdy_mat_free(&L->wq.m);
            if (L->qkv_parts < 2) sdy_mat_free(&L->wk.m);
            if (L->qkv_parts < 3) sdy_mat_free(&L->wv.m);
            dmat *mats[] = {&L->wqkv, &L->wo, &L->gate, &L->up, &L->gate_up, &L->down, &L->gate_inp};
            for (size_t i = 0; i < sizeof mats / sizeof *mats; i++) sdy_mat_free(&mats[i]->m);
        }
        free(m->layers);
    }
    sdy_mat_free(&m->tok_embd.m);
    if (!m->info.tied_embeddings) sdy_mat_free(&m->output.m);
    sdy_free(m->vectors);
    if (m->st) sdy_stream_free(m->st);
    gguf_close(m->gf);
    free(m);
}

void engine_model_get_info(const engine_model *m, engine_model_info *out) {
    if (m && out) *out = m->info;
}

engine_model *engine_model_load(const char *path, char *err, size_t err_len) {
    if (err && err_len) err[0] = '\0';
    engine_model *m = calloc(1, sizeof *m);
    if (!m) {
        set_err(err, err_len, "memoria esaurita");
        return NULL;
    }
    if (!(m->gf = gguf_open(path, err, err_len)) || read_config(m, err, err_len)) goto fail;
    if (sdy_init() || sdy_stream_new(&m->st)) {
        sdy_err(err, err_len, "GPU");
        goto fail;
    }
    const engine_model_info *in = &m->info;
    int dim = in->dim, q_dim = in->n_head * in->head_dim, kv_dim = in->n_kv_head * in->head_dim;
    size_t per_layer = 2 * (size_t)dim + (in->qkv_bias ? (size_t)q_dim + 2 * (size_t)kv_dim : 0) +
                       (in->qk_norm ? 2 * (size_t)in->head_dim : 0) + 7 * 64;
    size_t n_vec = (size_t)dim + 64 + per_layer * in->n_layer;
    if (sdy_malloc((void **)&m->vectors, n_vec * sizeof(float))) {
        sdy_err(err, err_len, "vettori");
        goto fail;
    }
    m->vec_cursor = m->vectors;
    m->layers = calloc((size_t)in->n_layer, sizeof(dlayer));
    if (!m->layers) {
        set_err(err, err_len, "memoria esaurita");
        goto fail;
    }
    if (get_tensor(m, "token_embd.weight", dim, in->n_vocab, 0, &m->tok_embd, err, err_len) ||
        get_vector(m, "output_norm.weight", dim, &m->output_norm, err, err_len))
        goto fail;
    if (in->tied_embeddings) m->output = m->tok_embd;
    else if (get_tensor(m, "output.weight", dim, in->n_vocab, 0, &m->output, err, err_len)) goto fail;
    for (int l = 0; l < in->n_layer; l++) {
        dlayer *L = &m->layers[l];
        char name[64];
#define NAME(suffix) (snprintf(name, sizeof name, "blk.%d." suffix, l), name)
        if (get_vector(m, NAME("attn_norm.weight"), dim, &L->attn_norm, err, err_len) ||
            get_vector(m, NAME("ffn_norm.weight"), dim, &L->ffn_norm, err, err_len) || get_qkv(m, l, L, err, err_len) ||
            get_tensor(m, NAME("attn_output.weight"), q_dim, dim, 0, &L->wo, err, err_len))
            goto fail;
        if (in->n_expert) {
            int ne = in->n_expert, fe = in->ffn_exp_dim;
            if (get_tensor(m, NAME("ffn_gate_inp.weight"), dim, ne, 0, &L->gate_inp, err, err_len) ||
                get_gate_up(m, l, L, fe, ne, err, err_len) ||
                get_tensor(m, NAME("ffn_down_exps.weight"), fe, dim, ne, &L->down, err, err_len))
                goto fail;
        } else if (get_gate_up(m, l, L, in->ffn_dim, 0, err, err_len) ||
                   get_tensor(m, NAME("ffn_down.weight"), in->ffn_dim, dim, 0, &L->down, err, err_len)) {
            goto fail;
        }
        if (in->qkv_bias && (get_vector(m, NAME("attn_q.bias"), q_dim, &L->bq, err, err_len) ||
                             get_vector(m, NAME("attn_k.bias"), kv_dim, &L->bk, err, err_len) ||
                             get_vector(m, NAME("attn_v.bias"), kv_dim, &L->bv, err, err_len)))
            goto fail;
        if (in->qk_norm && (get_vector(m, NAME("attn_q_norm.weight"), in->head_dim, &L->q_norm, err, err_len) ||
                            get_vector(m, NAME("attn_k_norm.weight"), in->head_dim, &L->k_norm, err, err_len)))
            goto fail;
#undef NAME
    }
    if (sdy_sync(m->st)) {
        sdy_err(err, err_len, "upload");
        goto fail;
    }
    return m;
fail:
    engine_model_free(m);
    return NULL;
}

/* ------------------------------------------------------------------ context */

int32_t engine_ctx_n_threads(const engine_ctx *c) { return c ? c->n_threads : 0; }

void engine_ctx_free(engine_ctx *c) {
    if (!c) return;
    sdy_engine_release(c);
    if (c->st) sdy_stream_free(c->st);
    sdy_host_free(c->logits);
    free(c);
}

engine_ctx *engine_ctx_new(const engine_model *m, int32_t max_seq, int32_t n_batch, int32_t logits_all,
                           int32_t n_threads, char *err, size_t err_len) {
    if (err && err_len) err[0] = '\0';
    if (!m) {
        set_err(err, err_len, "modello NULL");
        return NULL;
    }
    if (max_seq < 1 || max_seq > MAX_SEQ_LIMIT || max_seq > m->info.max_pos) {
        set_err(err, err_len, "max_seq=%d non valido (1..%d)", max_seq,
                m->info.max_pos < MAX_SEQ_LIMIT ? m->info.max_pos : MAX_SEQ_LIMIT);
        return NULL;
    }
    if (n_batch < 1 || n_batch > MAX_BATCH_LIMIT) {
        set_err(err, err_len, "n_batch=%d non valido (1..%d)", n_batch, MAX_BATCH_LIMIT);
        return NULL;
    }
    if (n_threads < 0 || n_threads > 256) {
        set_err(err, err_len, "n_threads=%d non valido (0..256)", n_threads);
        return NULL;
    }
    engine_ctx *c = calloc(1, sizeof *c);
    if (!c) {
        set_err(err, err_len, "memoria esaurita");
        return NULL;
    }
    c->m = m;
    c->max_seq = max_seq;
    c->n_batch = n_batch;
    c->logits_all = logits_all != 0;
    c->n_threads = n_threads ? n_threads : 1;
    size_t n_logit_rows = c->logits_all ? (size_t)n_batch : 1;
    if (sdy_stream_new(&c->st) || sdy_host_alloc((void **)&c->logits, n_logit_rows * m->info.n_vocab * sizeof(float)) ||
        sdy_engine_alloc(c)) {
        set_err(err, err_len, "memoria GPU esaurita o errore del dispositivo: %s", sdy_last_error());
        engine_ctx_free(c);
        return NULL;
    }
    /* SARDYNE_NO_FUSED_DECODE / SARDYNE_NO_GRAPH: run one-token steps with the unfused kernels, or
       without recording them (the results are the same; used to compare the paths) */
    c->decode_fused = !getenv("SARDYNE_NO_FUSED_DECODE") && sdy_engine_decode_fused_ok(c);
    /* SARDYNE_NO_DEVICE_MOE: one-token MoE blocks group their experts on the host, as prefill does */
    c->moe_device = c->decode_fused && !getenv("SARDYNE_NO_DEVICE_MOE") && sdy_engine_moe_device_ok(c);
    c->use_graph = c->decode_fused && (!m->info.n_expert || c->moe_device) && !getenv("SARDYNE_NO_GRAPH");
    c->fuse_act = c->decode_fused && !getenv("SARDYNE_NO_FUSED_ACT");
    return c;
}

/* ------------------------------------------------------------------ eval */

int engine_eval(engine_ctx *c, const int32_t *tokens, int32_t n) {
    if (!c) return -1;
    c->err[0] = '\0';
    if (!tokens || n < 1) {
        snprintf(c->err, sizeof c->err, "nessun token in ingresso");
        return -1;
    }
    if (c->logits_all && n > c->n_batch) {
        snprintf(c->err, sizeof c->err, "con logits_all servono al massimo n_batch=%d token per chiamata", c->n_batch);
        return -1;
    }
    if (n > c->max_seq - c->n_past) {
        snprintf(c->err, sizeof c->err, "contesto pieno: %d + %d > max_seq=%d", c->n_past, n, c->max_seq);
        return -1;
    }
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= c->m->info.n_vocab) {
            snprintf(c->err, sizeof c->err, "token %d fuori dal vocabolario [0, %d)", tokens[i], c->m->info.n_vocab);
            return -1;
        }
    int n_past0 = c->n_past;
    for (int done = 0; done < n;) {
        int chunk = n - done < c->n_batch ? n - done : c->n_batch;
        int last = done + chunk == n;
        if (sdy_engine_forward(c, tokens + done, chunk, last ? (c->logits_all ? chunk : 1) : 0)) {
            snprintf(c->err, sizeof c->err, "errore GPU: %s", sdy_last_error());
            c->n_past = n_past0; /* positions after n_past are rewritten by the next eval */
            c->n_logits = 0;
            return -1;
        }
        done += chunk;
    }
    c->n_logits = c->logits_all ? n : 1;
    return 0;
}

const float *engine_logits(const engine_ctx *c) { return c && c->n_logits ? c->logits : NULL; }
int32_t engine_n_logits(const engine_ctx *c) { return c ? c->n_logits : 0; }
int32_t engine_n_past(const engine_ctx *c) { return c ? c->n_past : 0; }
const char *engine_last_error(const engine_ctx *c) { return c ? c->err : "contesto NULL"; }

void engine_reset(engine_ctx *c) {
    if (!c) return;
    c->n_past = 0;
    c->n_logits = 0;
}

int engine_truncate(engine_ctx *c, int32_t n) {
    if (!c) return -1;
    if (n < 0 || n > c->n_past) {
        snprintf(c->err, sizeof c->err, "posizione %d fuori da [0, %d]", n, c->n_past);
        return -1;
    }
    c->n_past = n;
    c->n_logits = 0;
    return 0;
}

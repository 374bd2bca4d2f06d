/* engine_* of the public ABI: model loading into device memory, contexts, eval.
 *
 * The contract is the reference's csrc/engine.h:43-72: which GGUF files load (architectures,
 * metadata rules, tensor shapes and types), the NULL-on-failure constructors with the reason in
 * the caller's buffer, engine_eval's -1 with the context unchanged, and the error messages callers
 * match on (kept verbatim). The structure is this file's own:
 *
 *   - configuration: a table of metadata keys, each with its field of engine_model_info and its
 *     rule (required, constant default, or a quotient of fields read before it), read in one loop;
 *     cross-field rules follow the table;
 *   - tensors: one schema of per-layer tensors (suffix, rank, shape, when it must exist) serves
 *     both the "unknown tensor" check and the loader, which walks the schema to validate shapes
 *     and types before anything is uploaded;
 *   - upload: every matrix goes from the mmap to the device layout through the shim's uploader;
 *     q|k(|v) of one type become one stacked matrix, gate and up of one quantized type one
 *     interleaved matrix, and a layer's q|k|v biases one contiguous span (what the stacked
 *     matvecs read). Expert stacks are uploaded last, each layer's into device memory while it
 *     leaves room for the contexts and otherwise into pinned host memory, which the same kernels
 *     read in place (so a model larger than the device still loads);
 *   - contexts: argument limits checked from a table; the device state is allocated by forward.c.
 */
#define _POSIX_C_SOURCE 200809L
#include <stdarg.h>
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "sardyne.h"
#include "sdy_engine.h"
#include "sdy_ops.h"
#include "sdy_shim.h"

enum { SEQ_CAP = 1 << 20, BATCH_CAP = 4096, THREADS_CAP = 256, META_INT_CAP = 1 << 30 };

static int say(char *err, size_t len, const char *fmt, ...) {
    if (err && len) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, len, fmt, ap);
        va_end(ap);
    }
    return -1;
}

static const gguf_tensor *tensor(const gguf_file *gf, const char *name) {
    return gguf_get_tensor(gf, (uint64_t)gguf_find_tensor(gf, name));
}

/* ------------------------------------------------------------------ configuration */

#define INFO_FIELD(f) offsetof(engine_model_info, f)
#define FIELD(in, off) (*(int32_t *)((char *)(in) + (off)))

enum rule { REQUIRED, CONSTANT, COPY, QUOTIENT, SAME_AS };

typedef struct {
    const char *suffix;   /* key = "<arch>.<suffix>" */
    int moe_only;
    size_t field;         /* engine_model_info field written (SAME_AS: the field it must equal) */
    enum rule rule;
    int32_t constant;     /* CONSTANT default */
    size_t num, den;      /* COPY default: field num; QUOTIENT default: field num / field den */
    const char *zero;     /* QUOTIENT: message when the default comes out 0 */
    const char *differs;  /* SAME_AS: message when the key holds another value */
} int_key;

/* The keys in the order they are read: COPY, QUOTIENT and SAME_AS rules only name fields above them. */
static const int_key INT_KEYS[] = {
    {"embedding_length", 0, INFO_FIELD(dim), REQUIRED, 0, 0, 0, NULL, NULL},
    {"block_count", 0, INFO_FIELD(n_layer), REQUIRED, 0, 0, 0, NULL, NULL},
    {"feed_forward_length", 0, INFO_FIELD(ffn_dim), REQUIRED, 0, 0, 0, NULL, NULL},
    {"expert_count", 1, INFO_FIELD(n_expert), REQUIRED, 0, 0, 0, NULL, NULL},
    {"expert_used_count", 1, INFO_FIELD(n_expert_used), REQUIRED, 0, 0, 0, NULL, NULL},
    /* as in llama.cpp: without the key, the FFN length is the sum over the chosen experts */
    {"expert_feed_forward_length", 1, INFO_FIELD(ffn_exp_dim), QUOTIENT, 0, INFO_FIELD(ffn_dim),
     INFO_FIELD(n_expert_used), "dimensione degli esperti nulla", NULL},
    {"attention.head_count", 0, INFO_FIELD(n_head), REQUIRED, 0, 0, 0, NULL, NULL},
    {"attention.head_count_kv", 0, INFO_FIELD(n_kv_head), COPY, 0, INFO_FIELD(n_head), 0, NULL, NULL},
    {"attention.key_length", 0, INFO_FIELD(head_dim), QUOTIENT, 0, INFO_FIELD(dim), INFO_FIELD(n_head),
     "head_dim nullo", NULL},
    {"attention.value_length", 0, INFO_FIELD(head_dim), SAME_AS, 0, 0, 0, NULL, "key_length diverso da value_length"},
    {"rope.dimension_count", 0, INFO_FIELD(head_dim), SAME_AS, 0, 0, 0, NULL,
     "RoPE parziale (rope.dimension_count < head_dim) non supportata"},
    {"context_length", 0, INFO_FIELD(max_pos), CONSTANT, 2048, 0, 0, NULL, NULL},
};

typedef struct {
    const gguf_file *gf;
    char arch[32];
    char *err;
    size_t len;
} meta_reader;

/* Index of "<arch>.<suffix>", or -1. */
static int64_t meta_key(const meta_reader *r, const char *suffix) {
    char key[160];
    snprintf(key, sizeof key, "%s.%s", r->arch, suffix);
    return gguf_find_kv(r->gf, key);
}

/* 1 when present and valid (*v set), 0 when absent, -1 when present but not a count in 1..2^30. */
static int meta_count(const meta_reader *r, const char *suffix, int32_t *v) {
    int64_t i = meta_key(r, suffix);
    uint64_t u;
    if (i < 0) return 0;
    if (gguf_kv_get_u64(r->gf, i, &u) || u == 0 || u > META_INT_CAP)
        return say(r->err, r->len, "metadato non valido: %s.%s", r->arch, suffix);
    *v = (int32_t)u;
    return 1;
}

static int read_int_keys(const meta_reader *r, engine_model_info *in, int moe) {
    for (size_t k = 0; k < sizeof INT_KEYS / sizeof *INT_KEYS; k++) {
        const int_key *d = &INT_KEYS[k];
        if (d->moe_only && !moe) continue;
        int32_t v = 0;
        int got = meta_count(r, d->suffix, &v);
        if (got < 0 && d->rule != SAME_AS) return -1;
        if (d->rule == SAME_AS) {
            if (got && v != FIELD(in, d->field)) return say(r->err, r->len, "%s", d->differs);
            if (got < 0) return say(r->err, r->len, "%s", d->differs);
            continue;
        }
        if (!got) {
            if (d->rule == REQUIRED) return say(r->err, r->len, "metadato mancante: %s.%s", r->arch, d->suffix);
            v = d->rule == CONSTANT ? d->constant
                : d->rule == COPY   ? FIELD(in, d->num)
                                    : FIELD(in, d->num) / FIELD(in, d->den);
            if (v == 0) return say(r->err, r->len, "%s", d->zero ? d->zero : d->suffix);
        }
        FIELD(in, d->field) = v;
        if (d->field == INFO_FIELD(n_expert_used)) {
            /* the used count is checked as soon as it is known: the next default divides by it */
            if (in->n_expert_used > in->n_expert)
                return say(r->err, r->len, "expert_used_count=%d oltre expert_count=%d", in->n_expert_used,
                           in->n_expert);
            /* the device router keeps one token's expert probabilities in a wave's registers */
            if (in->n_expert > 512 || in->n_expert_used > 64)
                return say(r->err, r->len,
                           "expert_count=%d / expert_used_count=%d oltre i limiti del dispositivo (512 / 64)",
                           in->n_expert, in->n_expert_used);
        }
    }
    return 0;
}

/* A positive float key (<= 1e12); def < 0: required. */
static int read_float_key(const meta_reader *r, const char *suffix, double def, float *out) {
    int64_t i = meta_key(r, suffix);
    double v = def;
    if (i < 0 && def < 0) return say(r->err, r->len, "metadato mancante: %s.%s", r->arch, suffix);
    if (i >= 0 && gguf_kv_get_f64(r->gf, i, &v)) return say(r->err, r->len, "metadato non valido: %s.%s", r->arch, suffix);
    if (!(v > 0.0 && v <= 1e12)) return say(r->err, r->len, "valore non valido per %s.%s", r->arch, suffix);
    *out = (float)v;
    return 0;
}

/* Architectures and their RoPE pairing (csrc/model_llama.c:235-241). */
static const struct {
    const char *name;
    int interleaved, moe;
} ARCHS[] = {{"llama", 1, 0}, {"qwen2", 0, 0}, {"qwen3", 0, 0}, {"qwen3moe", 0, 1}};

/* ------------------------------------------------------------------ tensor schema */

enum when { ALWAYS, WITH_BIAS, WITH_QK_NORM, DENSE, MOE };
enum dim_src { D_ONE, D_DIM, D_QDIM, D_KVDIM, D_HEAD, D_FFN, D_FFN_EXP, D_EXPERTS };

typedef struct {
    const char *suffix;
    enum when when;
    int rank;             /* 1 vector, 2 matrix, 3 stacked experts */
    enum dim_src ne[3];   /* ne[0] (inner), ne[1], ne[2] */
} layer_tensor;

static const layer_tensor LAYER[] = {
    {"attn_norm.weight", ALWAYS, 1, {D_DIM}},
    {"attn_q.weight", ALWAYS, 2, {D_DIM, D_QDIM}},
    {"attn_q.bias", WITH_BIAS, 1, {D_QDIM}},
    {"attn_k.weight", ALWAYS, 2, {D_DIM, D_KVDIM}},
    {"attn_k.bias", WITH_BIAS, 1, {D_KVDIM}},
    {"attn_v.weight", ALWAYS, 2, {D_DIM, D_KVDIM}},
    {"attn_v.bias", WITH_BIAS, 1, {D_KVDIM}},
    {"attn_q_norm.weight", WITH_QK_NORM, 1, {D_HEAD}},
    {"attn_k_norm.weight", WITH_QK_NORM, 1, {D_HEAD}},
    {"attn_output.weight", ALWAYS, 2, {D_QDIM, D_DIM}},
    {"ffn_norm.weight", ALWAYS, 1, {D_DIM}},
    {"ffn_gate.weight", DENSE, 2, {D_DIM, D_FFN}},
    {"ffn_up.weight", DENSE, 2, {D_DIM, D_FFN}},
    {"ffn_down.weight", DENSE, 2, {D_FFN, D_DIM}},
    {"ffn_gate_inp.weight", MOE, 2, {D_DIM, D_EXPERTS}},
    {"ffn_gate_exps.weight", MOE, 3, {D_DIM, D_FFN_EXP, D_EXPERTS}},
    {"ffn_up_exps.weight", MOE, 3, {D_DIM, D_FFN_EXP, D_EXPERTS}},
    {"ffn_down_exps.weight", MOE, 3, {D_FFN_EXP, D_DIM, D_EXPERTS}},
};
enum { N_LAYER_TENSORS = sizeof LAYER / sizeof *LAYER };

static int64_t dim_of(const engine_model_info *in, enum dim_src d) {
    switch (d) {
    case D_DIM: return in->dim;
    case D_QDIM: return (int64_t)in->n_head * in->head_dim;
    case D_KVDIM: return (int64_t)in->n_kv_head * in->head_dim;
    case D_HEAD: return in->head_dim;
    case D_FFN: return in->ffn_dim;
    case D_FFN_EXP: return in->ffn_exp_dim;
    case D_EXPERTS: return in->n_expert;
    default: return 1;
    }
}

static int needed(const engine_model_info *in, enum when w) {
    switch (w) {
    case WITH_BIAS: return in->qkv_bias;
    case WITH_QK_NORM: return in->qk_norm;
    case DENSE: return !in->n_expert;
    case MOE: return in->n_expert > 0;
    default: return 1;
    }
}

/* Whether the runtime knows a tensor name: the model-level three, or blk.<l>.<schema suffix> with
 * l < n_layer. Anything else is an architecture variant this runtime does not implement. */
static int known_name(const char *name, int n_layer) {
    static const char *const TOP[] = {"token_embd.weight", "output_norm.weight", "output.weight"};
    for (size_t i = 0; i < 3; i++)
        if (!strcmp(name, TOP[i])) return 1;
    if (strncmp(name, "blk.", 4)) return 0;
    const char *p = name + 4;
    long l = 0;
    int digits = 0;
    for (; *p >= '0' && *p <= '9'; p++, digits++)
        if ((l = l * 10 + (*p - '0')) >= n_layer) return 0;
    if (!digits || *p != '.') return 0;
    for (int k = 0; k < N_LAYER_TENSORS; k++)
        if (!strcmp(p + 1, LAYER[k].suffix)) return 1;
    return 0;
}

static int runtime_type(uint32_t t) {
    return t == OP_F32 || t == OP_F16 || t == OP_BF16 || t == OP_Q8_0 || t == OP_Q4_0 || t == OP_Q5_0 ||
           t == OP_Q4_K || t == OP_Q6_K;
}

/* Shape and type of one tensor against what the schema expects; NULL with the reason otherwise. */
static const gguf_tensor *checked(const gguf_file *gf, const char *name, int rank, const int64_t want[3], char *err,
                                  size_t len) {
    const gguf_tensor *t = tensor(gf, name);
    if (!t) {
        say(err, len, "tensore mancante: %s", name);
        return NULL;
    }
    int shape_ok = t->n_dims == (uint32_t)rank;
    for (int d = 0; d < rank && shape_ok; d++) shape_ok = t->ne[d] == (uint64_t)want[d];
    if (!shape_ok) {
        if (rank == 1)
            say(err, len, "%s: dimensione %llu, attesa %lld", name, (unsigned long long)t->ne[0], (long long)want[0]);
        else
            say(err, len, "%s: dimensioni [%llu, %llu, %llu], attese [%lld, %lld, %lld]", name,
                (unsigned long long)t->ne[0], (unsigned long long)t->ne[1], (unsigned long long)t->ne[2],
                (long long)want[0], (long long)want[1], (long long)(rank == 3 ? want[2] : 1));
        return NULL;
    }
    if (!runtime_type(t->type)) {
        if (rank == 1) say(err, len, "%s: tipo %s non supportato", name, gguf_type_name(t->type));
        else
            say(err, len, "%s: tipo %s non supportato dal runtime (supportati: F32, F16, BF16, Q8_0, Q4_0, Q5_0, "
                "Q4_K, Q6_K)", name, gguf_type_name(t->type));
        return NULL;
    }
    return t;
}

static int read_config(engine_model *m, char *err, size_t len) {
    const gguf_file *gf = m->gf;
    engine_model_info *in = &m->info;
    meta_reader r = {.gf = gf, .err = err, .len = len};
    uint64_t n;
    const char *arch = gguf_kv_get_str(gf, gguf_find_kv(gf, "general.architecture"), &n);
    if (!arch || !n || n >= sizeof r.arch) return say(err, len, "general.architecture mancante o non valido");
    memcpy(r.arch, arch, n);
    r.arch[n] = '\0';
    int moe = -1;
    for (size_t a = 0; a < sizeof ARCHS / sizeof *ARCHS; a++)
        if (!strcmp(r.arch, ARCHS[a].name)) {
            in->rope_interleaved = ARCHS[a].interleaved;
            moe = ARCHS[a].moe;
        }
    if (moe < 0) return say(err, len, "architettura %s non supportata", r.arch);
    const char *scaling = gguf_kv_get_str(gf, meta_key(&r, "rope.scaling.type"), &n);
    if ((scaling && !(n == 4 && !memcmp(scaling, "none", 4))) || tensor(gf, "rope_freqs.weight"))
        return say(err, len, "rope scaling (anche 'llama3' via rope_freqs.weight) non supportato");
    if (read_int_keys(&r, in, moe) || read_float_key(&r, "attention.layer_norm_rms_epsilon", -1.0, &in->norm_eps) ||
        read_float_key(&r, "rope.freq_base", 10000.0, &in->rope_theta))
        return -1;
    if (in->n_head % in->n_kv_head || in->head_dim % 2)
        return say(err, len, "teste o head_dim non validi (n_head %% n_kv_head, head_dim pari)");
    const gguf_tensor *emb = tensor(gf, "token_embd.weight");
    if (!emb || emb->n_dims != 2 || emb->ne[1] > META_INT_CAP) return say(err, len, "token_embd.weight mancante o non valido");
    in->n_vocab = (int32_t)emb->ne[1];
    in->tied_embeddings = !tensor(gf, "output.weight");
    in->qkv_bias = tensor(gf, "blk.0.attn_q.bias") != NULL;
    in->qk_norm = tensor(gf, "blk.0.attn_q_norm.weight") != NULL;
    for (uint64_t i = 0; i < gguf_n_tensors(gf); i++) {
        const char *name = gguf_get_tensor(gf, i)->name;
        if (!known_name(name, in->n_layer)) return say(err, len, "tensore non supportato: %s", name);
    }
    return 0;
}

/* Every schema tensor of every layer, plus the model-level ones, checked before any upload. */
static int validate_tensors(const engine_model *m, const gguf_tensor *lt[][N_LAYER_TENSORS], char *err, size_t len) {
    const engine_model_info *in = &m->info;
    char name[96];
    const int64_t emb[3] = {in->dim, in->n_vocab, 1}, vec[3] = {in->dim, 1, 1};
    if (!checked(m->gf, "token_embd.weight", 2, emb, err, len) || !checked(m->gf, "output_norm.weight", 1, vec, err, len))
        return -1;
    if (!in->tied_embeddings && !checked(m->gf, "output.weight", 2, emb, err, len)) return -1;
    for (int l = 0; l < in->n_layer; l++)
        for (int k = 0; k < N_LAYER_TENSORS; k++) {
            lt[l][k] = NULL;
            if (!needed(in, LAYER[k].when)) continue;
            int64_t want[3];
            for (int d = 0; d < 3; d++) want[d] = d < LAYER[k].rank ? dim_of(in, LAYER[k].ne[d]) : 1;
            snprintf(name, sizeof name, "blk.%d.%s", l, LAYER[k].suffix);
            if (!(lt[l][k] = checked(m->gf, name, LAYER[k].rank, want, err, len))) return -1;
        }
    return 0;
}

/* ------------------------------------------------------------------ upload */

enum { T_ATTN_NORM, T_Q, T_QB, T_K, T_KB, T_V, T_VB, T_QN, T_KN, T_O, T_FFN_NORM, T_GATE, T_UP, T_DOWN, T_ROUTER,
       T_GATE_X, T_UP_X, T_DOWN_X };

enum { HOST_AUTO, HOST_NONE, HOST_ALL, HOST_LAST };

typedef struct {
    engine_model *m;
    char *err;
    size_t len;
    sdy_uploader *up; /* pipelined uploads (NULL: one synchronous upload per tensor) */
    int host_mode;    /* where expert stacks go (HOST_*; HOST_LAST: the last host_last layers' in host memory) */
    int host_last;
    size_t reserve;   /* device memory the load leaves free for the contexts (HOST_AUTO) */
} loader;

/* Rows of a tensor from the file mapping into an allocated matrix (the map of sdy_mat_upload_map). */
static int load_rows(loader *ld, sdy_mat *m, long r0, long n, long step, long grp, long gstride, const void *data) {
    return ld->up ? sdy_uploader_rows(ld->up, m, r0, n, step, grp, gstride, data)
                  : sdy_mat_upload_map(m, r0, n, step, grp, gstride, data, ld->m->st);
}

static int device_fail(loader *ld, const char *what) {
    return say(ld->err, ld->len, "%s: %s", what, sdy_last_error());
}

static int is_quant(uint32_t t) { return t != OP_F32 && t != OP_F16 && t != OP_BF16; }

static void describe(dmat *d, int type, int n_in, int n_out) {
    d->type = type;
    d->n_in = n_in;
    d->n_out = n_out;
}

static dmat row_view(const dmat *w, long r0, int n_out) {
    dmat d = *w;
    d.m = sdy_mat_rows(&w->m, r0, n_out);
    d.n_out = n_out;
    return d;
}

/* A matrix allocated in device memory, or (host) in pinned host memory, and counted. */
static int alloc_matrix(loader *ld, sdy_mat *m, int type, int n_in, long rows, int host) {
    if (host ? sdy_mat_alloc_host(m, type, n_in, rows) : sdy_mat_alloc(m, type, n_in, rows)) return -1;
    if (host) ld->m->host_bytes += m->bytes;
    else ld->m->device_bytes += m->bytes;
    return 0;
}

static long file_rows(const gguf_tensor *t) {
    return (long)(t->nbytes / sdy_raw_row_bytes((int)t->type, (int)t->ne[0]));
}

/* One matrix (or expert stack) as it is in the file; host: in pinned host memory. */
static int upload_matrix_in(loader *ld, const gguf_tensor *t, dmat *out, int host) {
    const long rows = file_rows(t);
    if (alloc_matrix(ld, &out->m, (int)t->type, (int)t->ne[0], rows, host)) return device_fail(ld, t->name);
    if (load_rows(ld, &out->m, 0, rows, 1, rows, 0, t->data)) return device_fail(ld, t->name);
    describe(out, (int)t->type, (int)t->ne[0], (int)t->ne[1]);
    return 0;
}

static int upload_matrix(loader *ld, const gguf_tensor *t, dmat *out) { return upload_matrix_in(ld, t, out, 0); }

/* q, k and v. With q and k of one type they are one matrix (and v too when it shares the type),
 * whose row ranges are the three: one launch computes them all. */
static int upload_qkv(loader *ld, const gguf_tensor *const *lt, dlayer *L) {
    const gguf_tensor *tq = lt[T_Q], *tk = lt[T_K], *tv = lt[T_V];
    const int n_in = (int)tq->ne[0], qd = (int)tq->ne[1], kvd = (int)tk->ne[1];
    if (tq->type != tk->type) {
        L->qkv_parts = 0;
        return upload_matrix(ld, tq, &L->wq) || upload_matrix(ld, tk, &L->wk) || upload_matrix(ld, tv, &L->wv) ? -1 : 0;
    }
    const int parts = tv->type == tq->type ? 3 : 2;
    const long rows = (long)qd + kvd + (parts == 3 ? kvd : 0);
    if (alloc_matrix(ld, &L->wqkv.m, (int)tq->type, n_in, rows, 0)) return device_fail(ld, tq->name);
    describe(&L->wqkv, (int)tq->type, n_in, (int)rows);
    L->qkv_parts = parts;
    const gguf_tensor *src[3] = {tq, tk, tv};
    long r0 = 0;
    for (int p = 0; p < parts; p++) {
        const int n = (int)src[p]->ne[1];
        if (load_rows(ld, &L->wqkv.m, r0, n, 1, n, 0, src[p]->data)) return device_fail(ld, src[p]->name);
        dmat *view = p == 0 ? &L->wq : p == 1 ? &L->wk : &L->wv;
        *view = row_view(&L->wqkv, r0, n);
        r0 += n;
    }
    return parts == 3 ? 0 : upload_matrix(ld, tv, &L->wv);
}

/* gate and up ([n_expert][ffn][dim]). With one quantized type they become one matrix with rows
 * interleaved (2i = gate i, 2i+1 = up i, per expert) for the SwiGLU matvec epilogue. host: in
 * pinned host memory. */
static int upload_gate_up(loader *ld, const gguf_tensor *tg, const gguf_tensor *tu, dlayer *L, int host) {
    if (tg->type != tu->type || !is_quant(tg->type)) {
        L->gu_fused = 0;
        return upload_matrix_in(ld, tg, &L->gate, host) || upload_matrix_in(ld, tu, &L->up, host) ? -1 : 0;
    }
    const int n_in = (int)tg->ne[0], ffn = (int)tg->ne[1];
    const long experts = tg->n_dims == 3 ? (long)tg->ne[2] : 1, rows = experts * ffn;
    if (alloc_matrix(ld, &L->gate_up.m, (int)tg->type, n_in, 2 * rows, host)) return device_fail(ld, tg->name);
    describe(&L->gate_up, (int)tg->type, n_in, 2 * ffn);
    L->gu_fused = 1;
    if (load_rows(ld, &L->gate_up.m, 0, rows, 2, ffn, 2L * ffn, tg->data)) return device_fail(ld, tg->name);
    if (load_rows(ld, &L->gate_up.m, 1, rows, 2, ffn, 2L * ffn, tu->data)) return device_fail(ld, tu->name);
    return 0;
}

/* n f32 values from a vector tensor (converted on the device when it is F16/BF16/quantized) into
 * device memory at dst. */
static int upload_vector(loader *ld, const gguf_tensor *t, float *dst) {
    const int n = (int)t->ne[0];
    sdy_stream st = ld->m->st;
    if (t->type == OP_F32) return sdy_h2d(dst, t->data, (size_t)n * 4, st) ? device_fail(ld, t->name) : 0;
    sdy_mat tmp;
    memset(&tmp, 0, sizeof tmp);
    int rc = sdy_mat_upload(&tmp, (int)t->type, n, 1, t->data, st) || sdy_dequant_rows(&tmp, 0, 1, dst, st) ||
             sdy_sync(st);
    sdy_mat_free(&tmp);
    return rc ? device_fail(ld, t->name) : 0;
}

/* Carves n floats from the model's vector block; spans start on 64-float boundaries. */
static float *carve(engine_model *m, size_t n) {
    float *p = m->vec_cursor;
    m->vec_cursor += (n + 63) & ~(size_t)63;
    return p;
}

static int upload_layer(loader *ld, const gguf_tensor *const *lt, dlayer *L) {
    const engine_model_info *in = &ld->m->info;
    const size_t dim = (size_t)in->dim, hd = (size_t)in->head_dim;
    const size_t qd = in->n_head * hd, kvd = in->n_kv_head * hd;
    L->attn_norm = carve(ld->m, dim);
    L->ffn_norm = carve(ld->m, dim);
    if (upload_vector(ld, lt[T_ATTN_NORM], L->attn_norm) || upload_vector(ld, lt[T_FFN_NORM], L->ffn_norm)) return -1;
    if (in->qkv_bias) {
        /* one contiguous span: the stacked q|k(|v) matvec adds it as a single bias vector */
        L->bq = carve(ld->m, qd + 2 * kvd);
        L->bk = L->bq + qd;
        L->bv = L->bk + kvd;
        if (upload_vector(ld, lt[T_QB], L->bq) || upload_vector(ld, lt[T_KB], L->bk) ||
            upload_vector(ld, lt[T_VB], L->bv))
            return -1;
    }
    if (in->qk_norm) {
        L->q_norm = carve(ld->m, hd);
        L->k_norm = carve(ld->m, hd);
        if (upload_vector(ld, lt[T_QN], L->q_norm) || upload_vector(ld, lt[T_KN], L->k_norm)) return -1;
    }
    if (upload_qkv(ld, lt, L) || upload_matrix(ld, lt[T_O], &L->wo)) return -1;
    if (in->n_expert) return upload_matrix(ld, lt[T_ROUTER], &L->gate_inp); /* the experts: upload_experts */
    return upload_gate_up(ld, lt[T_GATE], lt[T_UP], L, 0) || upload_matrix(ld, lt[T_DOWN], &L->down) ? -1 : 0;
}

/* Whether layer l's expert stacks (need bytes) go to pinned host memory: SARDYNE_HOST_EXPERTS=auto
 * (the default) while the device would keep less than the reserve free after them, all, none, or
 * a count n of the last layers. */
static int experts_on_host(loader *ld, int l, size_t need) {
    switch (ld->host_mode) {
    case HOST_NONE: return 0;
    case HOST_ALL: return 1;
    case HOST_LAST: return l >= ld->m->info.n_layer - ld->host_last;
    default: {
        size_t free_b = 0;
        if (sdy_mem_info(&free_b, NULL)) return 0; /* (the allocation then reports the device's state) */
        return free_b < need + ld->reserve;
    }
    }
}

/* A MoE layer's expert stacks (gate|up and down), in device memory or in pinned host memory. */
static int upload_experts(loader *ld, const gguf_tensor *const *lt, dlayer *L, int l) {
    const gguf_tensor *tg = lt[T_GATE_X], *tu = lt[T_UP_X], *td = lt[T_DOWN_X];
    const size_t need = sdy_mat_bytes((int)tg->type, (int)tg->ne[0], file_rows(tg)) +
                        sdy_mat_bytes((int)tu->type, (int)tu->ne[0], file_rows(tu)) +
                        sdy_mat_bytes((int)td->type, (int)td->ne[0], file_rows(td));
    const int host = experts_on_host(ld, l, need);
    if (upload_gate_up(ld, tg, tu, L, host) || upload_matrix_in(ld, td, &L->down, host)) return -1;
    L->down.n_out = ld->m->info.dim; /* an expert's rows; the stack holds n_expert of them */
    ld->m->host_layers += host;
    return 0;
}

void engine_model_free(engine_model *m) {
    if (!m) return;
    for (int l = 0; m->layers && l < m->info.n_layer; l++) {
        dlayer *L = &m->layers[l];
        /* row views of wqkv share its allocation */
        dmat *own[] = {L->qkv_parts < 2 ? &L->wq : NULL, L->qkv_parts < 2 ? &L->wk : NULL,
                       L->qkv_parts < 3 ? &L->wv : NULL, &L->wqkv, &L->wo, &L->gate, &L->up, &L->gate_up, &L->down,
                       &L->gate_inp};
        for (size_t i = 0; i < sizeof own / sizeof *own; i++)
            if (own[i]) sdy_mat_free(&own[i]->m);
    }
    free(m->layers);
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

/* Device memory a load leaves free for the contexts (KV caches, work buffers): SARDYNE_RESERVE_MB,
 * by default an eighth of the device and at least 2 GiB. */
static size_t context_reserve(size_t total) {
    const char *r = getenv("SARDYNE_RESERVE_MB");
    if (r && r[0]) return (size_t)(strtod(r, NULL) * 1048576.0);
    return total / 8 > ((size_t)2 << 30) ? total / 8 : ((size_t)2 << 30);
}

/* The expert placement switch (SARDYNE_HOST_EXPERTS: auto, none, all, or a count of last layers)
 * and the reserve. */
static int placement(loader *ld) {
    size_t total = 0;
    if (sdy_mem_info(NULL, &total)) return device_fail(ld, "GPU");
    ld->reserve = context_reserve(total);
    const char *h = getenv("SARDYNE_HOST_EXPERTS");
    char *end = NULL;
    if (!h || !h[0] || !strcmp(h, "auto")) ld->host_mode = HOST_AUTO;
    else if (!strcmp(h, "none")) ld->host_mode = HOST_NONE;
    else if (!strcmp(h, "all")) ld->host_mode = HOST_ALL;
    else {
        const long n = strtol(h, &end, 10);
        if (*end || n < 0) return say(ld->err, ld->len, "SARDYNE_HOST_EXPERTS=%s not supported (auto, none, all, or a "
                                                        "count of layers)", h);
        ld->host_mode = HOST_LAST;
        ld->host_last = (int)n;
    }
    return 0;
}

/* The prefill GEMM's tiled copies of the layer matrices (Q4_K / Q6_K, sdy_mat_gemm_layout): a second
 * copy of those weights, from which the GEMM's loads read whole cache lines. They only make prompts
 * faster (without one the GEMM reads the planes, with the same results), so they are made where the
 * device has room: the attention and dense FFN matrices of every layer first, then the expert stacks
 * (the bulk of a MoE file) in device memory, each only if it leaves the reserve free for the
 * contexts (SARDYNE_GEMM_RESERVE_MB, else the load's reserve). An allocation that fails all the same
 * skips that copy. SARDYNE_GEMM_COPY_MB caps the copies' total (MiB, fractions allowed; 0: no
 * copies). Expert stacks in host memory have none. */
static int gemm_copies(loader *ld) {
    engine_model *m = ld->m;
    const engine_model_info *in = &m->info;
    size_t free_b = 0;
    if (sdy_mem_info(&free_b, NULL)) return device_fail(ld, "gemm layout");
    size_t reserve = ld->reserve;
    const char *r = getenv("SARDYNE_GEMM_RESERVE_MB");
    if (r && r[0]) reserve = (size_t)(strtod(r, NULL) * 1048576.0);
    size_t cap = (size_t)-1;
    const char *c = getenv("SARDYNE_GEMM_COPY_MB");
    if (c && c[0]) cap = (size_t)(strtod(c, NULL) * 1048576.0);
    for (int experts = 0; experts < 2; experts++) {
        for (int l = 0; l < in->n_layer; l++) {
            dlayer *L = &m->layers[l];
            dmat *own[] = {L->qkv_parts < 2 ? &L->wq : NULL, L->qkv_parts < 2 ? &L->wk : NULL,
                           L->qkv_parts < 3 ? &L->wv : NULL, L->qkv_parts >= 2 ? &L->wqkv : NULL, &L->wo,
                           &L->gate, &L->up, &L->gate_up, &L->down};
            for (size_t i = 0; i < sizeof own / sizeof *own; i++) {
                if (!own[i] || !own[i]->m.base || own[i]->m.hbase) continue;
                if ((in->n_expert && i >= 5) != experts) continue; /* (i >= 5: the FFN matrices) */
                const size_t need = sdy_mat_gemm_layout_bytes(&own[i]->m);
                if (!need) continue;
                if (sdy_mem_info(&free_b, NULL)) return device_fail(ld, "gemm layout");
                const int room = free_b >= need + reserve && m->gemm_bytes + need <= cap;
                const int rc = room ? sdy_mat_gemm_layout(&own[i]->m, m->st) : SDY_ERR_ALLOC;
                if (rc == SDY_ERR_ALLOC) {
                    m->gemm_skipped++;
                    continue;
                }
                if (rc) return device_fail(ld, "gemm layout");
                m->gemm_bytes += own[i]->m.gbytes;
                m->gemm_copies++;
            }
        }
    }
    return sdy_sync(m->st) ? device_fail(ld, "gemm layout") : 0;
}

static int load(engine_model *m, const char *path, char *err, size_t len) {
    if (!(m->gf = gguf_open(path, err, len)) || read_config(m, err, len)) return -1;
    const engine_model_info *in = &m->info;
    const gguf_tensor *(*lt)[N_LAYER_TENSORS] = calloc((size_t)in->n_layer, sizeof *lt);
    m->layers = calloc((size_t)in->n_layer, sizeof *m->layers);
    if (!lt || !m->layers) {
        free(lt);
        return say(err, len, "memoria esaurita");
    }
    loader ld = {m, err, len, NULL, HOST_AUTO, 0, 0};
    int rc = validate_tensors(m, lt, err, len);
    if (!rc && (sdy_init() || sdy_stream_new(&m->st))) rc = device_fail(&ld, "GPU");
    if (!rc) rc = placement(&ld);
    /* weights go through a ring of four 64 MiB pinned/device slot pairs, the host copies split over
       half the online CPUs; SARDYNE_UPLOAD_SYNC=1: one synchronous upload per tensor instead */
    const char *sync_up = getenv("SARDYNE_UPLOAD_SYNC");
    if (!rc && !(sync_up && sync_up[0] && strcmp(sync_up, "0"))) {
        const long online = sysconf(_SC_NPROCESSORS_ONLN);
        const int threads = online > 32 ? 16 : online > 2 ? (int)(online / 2) : 1;
        if (sdy_uploader_new(&ld.up, (size_t)64 << 20, 4, threads, m->st)) rc = device_fail(&ld, "upload");
    }
    /* the f32 vectors of every layer: norms, biases, q/k norms, each span padded to 64 floats */
    const size_t hd = (size_t)in->head_dim, qd = in->n_head * hd, kvd = in->n_kv_head * hd;
    const size_t per_layer = 2 * ((size_t)in->dim + 63) + (in->qkv_bias ? qd + 2 * kvd + 63 : 0) +
                             (in->qk_norm ? 2 * (hd + 63) : 0);
    if (!rc && sdy_malloc((void **)&m->vectors, (((size_t)in->dim + 63) + per_layer * in->n_layer) * sizeof(float)))
        rc = device_fail(&ld, "vettori");
    m->vec_cursor = m->vectors;
    if (!rc) {
        const gguf_tensor *emb = tensor(m->gf, "token_embd.weight");
        m->output_norm = carve(m, (size_t)in->dim);
        rc = upload_matrix(&ld, emb, &m->tok_embd) || upload_vector(&ld, tensor(m->gf, "output_norm.weight"),
                                                                    m->output_norm);
        if (!rc && in->tied_embeddings) m->output = m->tok_embd;
        else if (!rc) rc = upload_matrix(&ld, tensor(m->gf, "output.weight"), &m->output);
    }
    for (int l = 0; !rc && l < in->n_layer; l++) rc = upload_layer(&ld, lt[l], &m->layers[l]);
    for (int l = 0; !rc && in->n_expert && l < in->n_layer; l++) rc = upload_experts(&ld, lt[l], &m->layers[l], l);
    if (!rc && ld.up && sdy_uploader_finish(ld.up)) rc = device_fail(&ld, "upload");
    if (!rc && sdy_sync(m->st)) rc = device_fail(&ld, "upload");
    if (sdy_uploader_free(ld.up) && !rc) rc = device_fail(&ld, "upload");
    if (!rc) rc = gemm_copies(&ld);
    if (!rc) {
        /* views taken before the exactness checks ran: take them again (gemm_ok of the stack) */
        for (int l = 0; l < in->n_layer; l++) {
            dlayer *L = &m->layers[l];
            if (L->qkv_parts >= 2) {
                const int qd_l = L->wq.n_out, kvd_l = L->wk.n_out;
                L->wq = row_view(&L->wqkv, 0, qd_l);
                L->wk = row_view(&L->wqkv, qd_l, kvd_l);
                if (L->qkv_parts == 3) L->wv = row_view(&L->wqkv, (long)qd_l + kvd_l, kvd_l);
            }
        }
        if (in->tied_embeddings) m->output = m->tok_embd;
    }
    free(lt);
    return rc;
}

int sdy_model_host_weights(const engine_model *m, size_t *host_bytes, int *host_layers) {
    if (!m) return -1;
    if (host_bytes) *host_bytes = m->host_bytes;
    if (host_layers) *host_layers = m->host_layers;
    return 0;
}

int sdy_model_memory(const engine_model *m, size_t *weight_bytes, size_t *gemm_copy_bytes, int *n_copies,
                     int *n_skipped) {
    if (!m) return -1;
    if (weight_bytes) *weight_bytes = m->device_bytes;
    if (gemm_copy_bytes) *gemm_copy_bytes = m->gemm_bytes;
    if (n_copies) *n_copies = m->gemm_copies;
    if (n_skipped) *n_skipped = m->gemm_skipped;
    return 0;
}

engine_model *engine_model_load(const char *path, char *err, size_t err_len) {
    if (err && err_len) err[0] = '\0';
    engine_model *m = calloc(1, sizeof *m);
    if (!m) {
        say(err, err_len, "memoria esaurita");
        return NULL;
    }
    if (load(m, path, err, err_len)) {
        engine_model_free(m);
        return NULL;
    }
    return m;
}

/* ------------------------------------------------------------------ contexts */

int32_t engine_ctx_n_threads(const engine_ctx *c) { return c ? c->n_threads : 0; }

void engine_ctx_free(engine_ctx *c) {
    if (!c) return;
    sdy_engine_release(c);
    if (c->st) sdy_stream_free(c->st);
    sdy_host_free(c->logits);
    free(c);
}

/* Reads an on/off switch from the environment: set and not "0" means on. */
static int env_on(const char *name) {
    const char *v = getenv(name);
    return v && v[0] && strcmp(v, "0") != 0;
}

engine_ctx *engine_ctx_new(const engine_model *m, int32_t max_seq, int32_t n_batch, int32_t logits_all,
                           int32_t n_threads, char *err, size_t err_len) {
    if (err && err_len) err[0] = '\0';
    if (!m) {
        say(err, err_len, "modello NULL");
        return NULL;
    }
    const struct {
        const char *name;
        int32_t v, lo, hi;
    } limits[] = {
        {"max_seq", max_seq, 1, m->info.max_pos < SEQ_CAP ? m->info.max_pos : SEQ_CAP},
        {"n_batch", n_batch, 1, BATCH_CAP},
        {"n_threads", n_threads, 0, THREADS_CAP},
    };
    for (size_t i = 0; i < sizeof limits / sizeof *limits; i++)
        if (limits[i].v < limits[i].lo || limits[i].v > limits[i].hi) {
            say(err, err_len, "%s=%d non valido (%d..%d)", limits[i].name, limits[i].v, limits[i].lo, limits[i].hi);
            return NULL;
        }
    engine_ctx *c = calloc(1, sizeof *c);
    if (!c) {
        say(err, err_len, "memoria esaurita");
        return NULL;
    }
    c->m = m;
    c->max_seq = max_seq;
    c->n_batch = n_batch;
    c->logits_all = logits_all != 0;
    if (!n_threads) {
        /* the reference's default, the online CPUs (csrc/threadpool.c:68-71); reported, never used
           to split GPU work */
        long online = sysconf(_SC_NPROCESSORS_ONLN);
        n_threads = online < 1 ? 1 : online > THREADS_CAP ? THREADS_CAP : (int32_t)online;
    }
    c->n_threads = n_threads;
    /* SARDYNE_KV: the KV cache's element type, f32 (the reference's; default) or f16 (each value
       rounded to nearest even when written: half the cache's bytes and its reads) */
    const char *kv = getenv("SARDYNE_KV");
    if (!kv || !kv[0] || !strcmp(kv, "f32")) {
        c->kv_type = SDY_KV_F32;
    } else if (!strcmp(kv, "f16")) {
        c->kv_type = SDY_KV_F16;
    } else {
        say(err, err_len, "SARDYNE_KV=%s not supported (f32, f16)", kv);
        free(c);
        return NULL;
    }
    /* SARDYNE_ATTENTION: the one-token attention. chunked (the default): split over spans of
       positions in two launches, within tolerance of the reference (its f32 rounding only); exact: the
       reference's softmax over every position and its in-order weighted sum, bit for bit, for the
       one-token steps and the prompt alike; split: the chunked form in one launch (f32 cache only).
       Except with exact, the prompt's attention runs in flash form (also within tolerance). */
    const char *attn = getenv("SARDYNE_ATTENTION");
    if (!attn || !attn[0] || !strcmp(attn, "chunked")) {
        c->attn_mode = SDY_ATTN_CHUNKED;
    } else if (!strcmp(attn, "exact")) {
        c->attn_mode = SDY_ATTN_EXACT;
    } else if (!strcmp(attn, "split") && c->kv_type == SDY_KV_F32) {
        c->attn_mode = SDY_ATTN_SPLIT;
    } else {
        say(err, err_len, "SARDYNE_ATTENTION=%s not supported (exact, chunked, split with an f32 cache)", attn);
        free(c);
        return NULL;
    }
    const size_t logit_bytes = (c->logits_all ? (size_t)n_batch : 1) * (size_t)m->info.n_vocab * sizeof(float);
    if (sdy_stream_new(&c->st) || sdy_host_alloc((void **)&c->logits, logit_bytes) || sdy_engine_alloc(c)) {
        say(err, err_len, "memoria GPU esaurita o errore del dispositivo: %s", sdy_last_error());
        engine_ctx_free(c);
        return NULL;
    }
    /* Switches that select between paths with identical results (used to compare them):
       SARDYNE_NO_DEVICE_MOE    one-token MoE blocks grouped on the host, as prefill does;
       SARDYNE_NO_GRAPH         one-token steps issued eagerly instead of replayed;
       SARDYNE_NO_FUSED_ACT     one-token matvecs read activations quantised by a separate launch.
       SARDYNE_NO_FUSED_DECODE  one-token steps on the unfused kernels: they take the exact attention
                                chain, and so does the prompt (the results of SARDYNE_ATTENTION=exact). */
    c->decode_fused = !env_on("SARDYNE_NO_FUSED_DECODE") && sdy_engine_decode_fused_ok(c);
    c->moe_device = c->decode_fused && !env_on("SARDYNE_NO_DEVICE_MOE") && sdy_engine_moe_device_ok(c);
    c->use_graph = c->decode_fused && (!m->info.n_expert || c->moe_device) && !env_on("SARDYNE_NO_GRAPH");
    c->fuse_act = c->decode_fused && !env_on("SARDYNE_NO_FUSED_ACT");
    const engine_model_info *in = &m->info;
    /* the split forms take the fused one-token step and their head layouts; otherwise the exact chain */
    if (!c->decode_fused || (c->attn_mode == SDY_ATTN_CHUNKED && !sdy_attn_chunked_ok(in->n_head, in->n_kv_head,
                                                                                      in->head_dim)) ||
        (c->attn_mode == SDY_ATTN_SPLIT && !sdy_attn_decode_split_ok(in->n_head, in->n_kv_head, in->head_dim)))
        c->attn_mode = SDY_ATTN_EXACT;
    /* the prompt's attention: in flash form on the matrix cores with the split one-token forms; with
       the exact chain the prompt keeps the reference's bits too */
    c->prefill_flash = c->attn_mode != SDY_ATTN_EXACT && sdy_attention_flash_ok(in->n_head, in->n_kv_head, in->head_dim);
    return c;
}

/* ------------------------------------------------------------------ eval */

/* The reason n tokens cannot be evaluated now (written into c->err), or 0. */
static int refuse(engine_ctx *c, const int32_t *tokens, int32_t n) {
    const int vocab = c->m->info.n_vocab;
    if (!tokens || n < 1) return say(c->err, sizeof c->err, "nessun token in ingresso");
    if (c->logits_all && n > c->n_batch)
        return say(c->err, sizeof c->err, "con logits_all servono al massimo n_batch=%d token per chiamata", c->n_batch);
    if (n > c->max_seq - c->n_past)
        return say(c->err, sizeof c->err, "contesto pieno: %d + %d > max_seq=%d", c->n_past, n, c->max_seq);
    for (int32_t i = 0; i < n; i++)
        if ((uint32_t)tokens[i] >= (uint32_t)vocab)
            return say(c->err, sizeof c->err, "token %d fuori dal vocabolario [0, %d)", tokens[i], vocab);
    return 0;
}

int engine_eval(engine_ctx *c, const int32_t *tokens, int32_t n) {
    if (!c) return -1;
    c->err[0] = '\0';
    if (refuse(c, tokens, n)) return -1;
    const int start = c->n_past;
    /* n_batch-token chunks; logits come from the last chunk only (all its rows with logits_all) */
    for (int32_t at = 0; at < n; at += c->n_batch) {
        const int32_t len = n - at < c->n_batch ? n - at : c->n_batch;
        const int out_rows = at + len < n ? 0 : c->logits_all ? len : 1;
        if (sdy_engine_forward(c, tokens + at, len, out_rows)) {
            say(c->err, sizeof c->err, "errore GPU: %s", sdy_last_error());
            c->n_past = start; /* positions past n_past are overwritten by the next eval */
            c->n_logits = 0;
            return -1;
        }
    }
    c->n_logits = c->logits_all ? n : 1;
    return 0;
}

const float *engine_logits(const engine_ctx *c) { return c && c->n_logits ? c->logits : NULL; }
int32_t engine_n_logits(const engine_ctx *c) { return c ? c->n_logits : 0; }
int32_t engine_n_past(const engine_ctx *c) { return c ? c->n_past : 0; }
const char *engine_last_error(const engine_ctx *c) { return c ? c->err : "contesto NULL"; }

void engine_reset(engine_ctx *c) {
    if (c) c->n_past = c->n_logits = 0;
}

int engine_truncate(engine_ctx *c, int32_t n) {
    if (!c) return -1;
    if (n < 0 || n > c->n_past) return say(c->err, sizeof c->err, "posizione %d fuori da [0, %d]", n, c->n_past);
    c->n_past = n;
    c->n_logits = 0;
    return 0;
}

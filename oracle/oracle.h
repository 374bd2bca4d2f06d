/* Oracle: a clean-room CPU restatement of the reference's quantized-matrix path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library (sardyne_amd/) links, loads or calls
 * this code; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and
 * only as the checker.
 *
 * Each function cites the reference file:line whose behaviour it restates (paths relative to the
 * reference repository root). Arithmetic order follows the reference wherever the reference's
 * result depends on it: contraction is off (-ffp-contract=off), f32 combines are written in the
 * reference's expression order, and the AVX2 accumulation orders of the Q8_0/Q4_0/Q5_0 dots and of
 * the f32 matmul / dot / axpy are emulated lane by lane, so the oracle reproduces what the
 * reference computes on an AVX2 host, not only its scalar fallback.
 */
#ifndef SARDYNE_ORACLE_H
#define SARDYNE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF / ggml type ids (csrc/ops.h:21-22). */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q5_0 = 6, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q6_K = 14,
       ORC_Q8_K = 15, ORC_BF16 = 30 };

/* ---- conversions (csrc/ops.c:15-62) */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void orc_f16_to_f32_n(const uint16_t *x, float *out, size_t n);

/* ---- formats (csrc/quant.h:14-56, csrc/ops.c:329-365) */
int orc_block_size(int type);
size_t orc_block_bytes(int type);
size_t orc_row_size(int type, int n);
int orc_vec_dot_type(int wtype);

/* ---- dequantisation (csrc/quant.c:13-94, csrc/ops.c:372-383) */
void orc_row_to_f32(const void *row, int type, float *out, size_t n);

/* ---- activation quantisation (csrc/quant.c:98-144, csrc/ops.c:394-401) */
void orc_quant_q8_0(const float *x, void *dst, int n);
void orc_quant_q8_K(const float *x, void *dst, int n);
void orc_quantize_rows(int vtype, const float *x, void *xq, int n_in, int t0, int t1);

/* ---- quantized dots.
 * orc_dot_scalar: the portable kernels (csrc/quant.c:148-235).
 * orc_dot_avx2:   the kernels an AVX2 host runs (csrc/quant_avx2.c:106-281); identical to the scalar
 *                 ones for Q4_K/Q6_K, different f32 order for Q8_0/Q4_0/Q5_0. */
float orc_dot_scalar(int wtype, const void *w, const void *xq, int n);
float orc_dot_avx2(int wtype, const void *w, const void *xq, int n);
/* out[t][j] for t < n_tok, row0 <= j < row1, with the reference's AVX2 row/token grouping
 * (csrc/ops.c:403-419, csrc/quant_avx2.c:146-201,290-385). simd=0 selects the scalar order. */
void orc_matmul_q_rows(float *out, const void *xq, const void *w, int wtype, int n_tok, int n_in, int n_out,
                       int row0, int row1, int simd);

/* ---- float kernels (csrc/ops.c:387-423 and csrc/ops_avx2.c:60-147; simd selects AVX2 order) */
void orc_matmul_rows(float *out, const float *x, const void *w, int wtype, int n_tok, int n_in, int n_out,
                     int row0, int row1, int simd);
float orc_dot_f32(const float *a, const float *b, int n, int simd);
void orc_axpy(float *y, float a, const float *x, int n, int simd);
void orc_rmsnorm(float *out, const float *x, const float *w, int n, float eps);
void orc_softmax(float *x, int n);
void orc_silu_mul(float *gate, const float *up, int n);
void orc_rope_table(float *cos_out, float *sin_out, int n_pos, int head_dim, float theta);
void orc_rope(float *x, int n_heads, int head_dim, const float *cos, const float *sin, int interleaved);
void orc_attention(float *out, const float *q, const float *k_cache, const float *v_cache, int n_head,
                   int n_kv_head, int head_dim, int n_kv, int stride, float *scores, int simd);

/* ---- model forward (csrc/model_llama.c:542-886).
 * The caller supplies the configuration and host pointers to every tensor's raw bytes in GGUF
 * layout; the oracle keeps its own f32 KV cache. */
typedef struct {
    int32_t n_vocab, dim, n_layer, n_head, n_kv_head, head_dim, ffn_dim, max_pos;
    float norm_eps, rope_theta;
    int32_t rope_interleaved, qkv_bias, tied_embeddings, qk_norm;
    int32_t n_expert, n_expert_used, ffn_exp_dim;
} orc_info; /* same field order as engine_model_info (csrc/engine.h:24-40) */

typedef struct {
    const void *data;
    int32_t type;
} orc_tensor;

typedef struct {
    orc_tensor attn_norm, ffn_norm, bq, bk, bv, q_norm, k_norm;
    orc_tensor wq, wk, wv, wo, gate, up, down, gate_inp;
} orc_layer;

typedef struct orc_model orc_model;
orc_model *orc_model_new(const orc_info *info, orc_tensor tok_embd, orc_tensor output_norm, orc_tensor output,
                         const orc_layer *layers);
void orc_model_free(orc_model *m);

typedef struct orc_ctx orc_ctx;
/* n_threads: OpenMP threads used for row loops (results never depend on it); simd as above. */
orc_ctx *orc_ctx_new(const orc_model *m, int max_seq, int n_batch, int logits_all, int simd);
void orc_ctx_free(orc_ctx *c);
void orc_ctx_set_kv_f16(orc_ctx *c, int on);
int orc_eval(orc_ctx *c, const int32_t *tokens, int n);
const float *orc_logits(const orc_ctx *c);
int orc_n_logits(const orc_ctx *c);
int orc_n_past(const orc_ctx *c);
void orc_reset(orc_ctx *c);
int orc_truncate(orc_ctx *c, int n);
/* MoE instrumentation: expert ids chosen for each token of the last eval, [n_layer][n][k]. */
const int32_t *orc_last_topk(const orc_ctx *c);

#ifdef __cplusplus
}
#endif
#endif

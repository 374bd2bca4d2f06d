/* Launchers of the float-side kernels (ops_kernels.hip). Internal to the library. */
#ifndef SDY_OPS_H
#define SDY_OPS_H
#include <stddef.h>
#include <stdint.h>

#include "sdy_shim.h"

#ifdef __cplusplus
extern "C" {
#endif
int sdy_rmsnorm(const float *x, const float *w, float *out, int n, float eps, int n_rows, long x_stride,
                long out_stride, sdy_stream s);
/* KV-cache element types (kv_type arguments): f32, or f16 with each value rounded to nearest even
 * when written (the reference's f32 -> f16 rules). A layer's cache is [n_kv_head][max_seq][hd]
 * elements; head_stride counts elements. */
enum { SDY_KV_F32 = 0, SDY_KV_F16 = 1 };
size_t sdy_kv_elt_bytes(int kv_type); /* 4, 2, or 0 for an unknown type */
int sdy_qk_rope_kv(float *q, float *k, const float *v, const float *qn, const float *kn, float eps,
                   const float *rope_cos, const float *rope_sin, int pos0, int n_tok, int n_head, int n_kv_head, int hd,
                   int interleaved, void *k_cache, void *v_cache, int kv_type, long head_stride, sdy_stream s);
/* the same with token rows t * q_stride, t * k_stride, t * v_stride floats apart (q|k|v of one GEMM) */
int sdy_qk_rope_kv_strided(float *q, float *k, const float *v, long q_stride, long k_stride, long v_stride,
                           const float *qn, const float *kn, float eps, const float *rope_cos, const float *rope_sin,
                           int pos0, int n_tok, int n_head, int n_kv_head, int hd, int interleaved, void *k_cache,
                           void *v_cache, int kv_type, long head_stride, sdy_stream s);
/* Causal attention of n_tok tokens at positions n_kv0 - 1 + t (q rotated, K/V in the cache) in the
 * reference's arithmetic; scores: sdy_attn_scores_floats(n_tok, n_head, n_kv0 + n_tok - 1) floats of
 * device scratch. head_dim 32, 64, 128 or 256. */
size_t sdy_attn_scores_floats(int n_tok, int n_head, int max_kv);
int sdy_attention(const float *q, const void *k_cache, const void *v_cache, int kv_type, int n_tok, int n_head,
                  int n_kv_head, int hd, int n_kv0, long head_stride, long q_stride, float *scores, float *out,
                  long out_stride, sdy_stream s);
/* The same attention in flash form on the f32 matrix cores (attn_flash.hip): within tolerance of the
 * reference, not its bits; no scratch. head_dim 64 or 128; q rows and both strides 16-byte aligned. */
int sdy_attention_flash_ok(int n_head, int n_kv_head, int hd);
int sdy_attention_flash(const float *q, const void *k_cache, const void *v_cache, int kv_type, int n_tok,
                        int n_head, int n_kv_head, int hd, int n_kv0, long head_stride, long q_stride, float *out,
                        long out_stride, sdy_stream s);
int sdy_silu_mul(float *gate, const float *up, long n, sdy_stream s);
int sdy_add(const float *a, const float *b, float *out, long n, sdy_stream s);
int sdy_axpy(float *y, float a, const float *x, long n, sdy_stream s);
int sdy_dot(const float *a, const float *b, int n, float *out, sdy_stream s);
int sdy_f16_to_f32(const uint16_t *x, float *out, long n, sdy_stream s);
int sdy_f32_to_f16(const float *x, uint16_t *out, long n, sdy_stream s);
int sdy_softmax(float *x, int n, int n_rows, long stride, sdy_stream s);
/* RoPE cos/sin tables [n_pos][hd/2], computed on the host (libm, double) into host memory */
void sdy_rope_table_host(float *cos_out, float *sin_out, int n_pos, int hd, float theta);
int sdy_rope(float *x, int n_heads, int hd, const float *cs, const float *sn, int interleaved, sdy_stream s);
int sdy_moe_route(float *probs, int n_tok, int n_expert, int k, int32_t *top, float *wts, sdy_stream s);
/* The routed (token, slot) pairs of top ([n_tok][k] expert ids) grouped by expert, stably: sorted row
 * r is pair out_row[r] = t * k + s of token src_tok[r]; expert e owns rows grp_tok[e] ..
 * grp_tok[e + 1] - 1 and the bn-row tiles grp_tile[e] .. grp_tile[e + 1] - 1 (arrays of n_expert + 1). */
int sdy_moe_sort(const int32_t *top, int n_tok, int k, int n_expert, int bn, int *grp_tok, int *grp_tile,
                 int32_t *src_tok, int32_t *out_row, sdy_stream s);
int sdy_gather_rows(const float *src, const int32_t *idx, int n, int dim, float *dst, sdy_stream s);
int sdy_moe_combine(const float *y, const int32_t *top, const float *wts, int n_tok, int k, int dim, float *out,
                    const float *resid, sdy_stream s);
/* RMSNorm of n_rows rows of n floats, then the activation quantiser vtype (SDY_Q8_K / SDY_Q8_0)
 * into xq, or vtype SDY_F32: normalise only. xb receives the f32 rows (may be NULL when
 * quantising). Bytes equal sdy_rmsnorm followed by sdy_quantize. */
int sdy_norm_quant(const float *x, const float *w, float eps, int n, int n_rows, float *xb, int vtype, void *xq,
                   sdy_stream s);
/* One-token decode attention at the position held in step_dev[1] (read on the device, so that a
 * recorded step replays for every position): q/k norm + RoPE, the KV-cache write of that position,
 * the scores (scores: sdy_attn_scores_floats(1, n_head, max_seq) floats of scratch), the softmax and
 * the weighted V into out (n_head * hd floats), and with xq_q8k also out's Q8_K row. */
int sdy_attn_decode_ok(int n_head, int n_kv_head, int hd, int max_seq);
int sdy_attn_decode(const float *q, const float *k, const float *v, const float *q_norm, const float *k_norm,
                    float eps, const float *rope_cos, const float *rope_sin, const int32_t *step_dev, int n_head,
                    int n_kv_head, int hd, int interleaved, void *k_cache, void *v_cache, int kv_type,
                    long head_stride, int max_seq, float *scores, float *out, void *xq_q8k, sdy_stream s);
/* One-token decode attention in two launches, split over spans of positions (64, or more for
 * caches beyond 8192 positions) with a deterministic merge in span order (within tolerance of the
 * reference; sdy_attn_decode is the bit-exact form): the same inputs and outputs as
 * sdy_attn_decode, with part (sdy_attn_chunked_floats floats) as scratch. xq_q8k needs
 * n_head * hd % 256 == 0. head_dim 64, 128 or 256, at most 16 query heads per kv head. */
int sdy_attn_chunked_ok(int n_head, int n_kv_head, int hd);
size_t sdy_attn_chunked_floats(int n_head, int hd, int max_seq);
int sdy_attn_decode_chunked(const float *q, const float *k, const float *v, const float *q_norm, const float *k_norm,
                            float eps, const float *rope_cos, const float *rope_sin, const int32_t *step_dev,
                            int n_head, int n_kv_head, int hd, int interleaved, void *k_cache, void *v_cache,
                            int kv_type, long head_stride, int max_seq, float *part, float *out, void *xq_q8k,
                            sdy_stream s);
/* One-token decode attention in one launch, split over 32-position chunks with a deterministic
 * merge (within tolerance of the reference; sdy_attn_decode is the bit-exact form): the same
 * inputs and outputs as sdy_attn_decode (f32 cache only), with part (sdy_attn_decode_split_floats floats) and count
 * (n_kv_head unsigned, zero before the first call; each call leaves them zero) as scratch. xq_q8k
 * needs whole Q8_K blocks per kv group ((n_head / n_kv_head) * hd % 256 == 0). head_dim 64 or 128,
 * at most 16 query heads per kv head. */
int sdy_attn_decode_split_ok(int n_head, int n_kv_head, int hd);
size_t sdy_attn_decode_split_floats(int n_head, int hd, int max_seq);
int sdy_attn_decode_split(const float *q, const float *k, const float *v, const float *q_norm, const float *k_norm,
                          float eps, const float *rope_cos, const float *rope_sin, const int32_t *step_dev, int n_head,
                          int n_kv_head, int hd, int interleaved, float *k_cache, float *v_cache, long head_stride,
                          int max_seq, float *part, unsigned *count, float *out, void *xq_q8k, sdy_stream s);
#ifdef __cplusplus
}
#endif
#endif

/* Public C ABI of libsardyne.so (MI355X build).
 *
 * The declarations below are the drop-in boundary: the same symbols, signatures, struct layouts,
 * ownership and error conventions as the reference's libsardyne.so, so that its ctypes layer
 * (sardyne/capi.py:33-102) binds this library unchanged. Each group cites the reference
 * declaration it replaces. Computation behind engine_* and op_* runs on the GPU (gfx950); there is
 * no CPU compute path in this library.
 */
#ifndef SARDYNE_H
#define SARDYNE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ engine (csrc/engine.h:17-72) */

typedef struct engine_model engine_model;
typedef struct engine_ctx engine_ctx;

/* Field order and types of csrc/engine.h:24-40 (mirrored by sardyne/capi.py:55-60). */
typedef struct {
    int32_t n_vocab;
    int32_t dim;
    int32_t n_layer;
    int32_t n_head;
    int32_t n_kv_head;
    int32_t head_dim;
    int32_t ffn_dim;
    int32_t max_pos;
    float norm_eps;
    float rope_theta;
    int32_t rope_interleaved; /* 1: pairs (2i, 2i+1) ("llama"); 0: pairs (i, i + head_dim/2) (qwen2/qwen3) */
    int32_t qkv_bias;
    int32_t tied_embeddings;
    int32_t qk_norm;
    int32_t n_expert, n_expert_used, ffn_exp_dim;
} engine_model_info;

/* csrc/engine.h:44-45 */
const char *engine_version(void);
void engine_add_f32(const float *a, const float *b, float *out, size_t n);

/* csrc/engine.h:49-51. Loads a llama / qwen2 / qwen3 / qwen3moe GGUF and uploads every weight to
 * device memory; the expert stacks of layers the device has no room for go to pinned host memory,
 * read in place by the kernels (SARDYNE_HOST_EXPERTS, sdy_model_host_weights). NULL on error, with
 * the reason in err. */
engine_model *engine_model_load(const char *path, char *err, size_t err_len);
void engine_model_free(engine_model *m);
void engine_model_get_info(const engine_model *m, engine_model_info *out);

/* csrc/engine.h:57-60. n_threads is validated (0..256) and reported back; results never depend on
 * it. The KV cache and activations live in device memory. */
engine_ctx *engine_ctx_new(const engine_model *m, int32_t max_seq, int32_t n_batch, int32_t logits_all,
                           int32_t n_threads, char *err, size_t err_len);
int32_t engine_ctx_n_threads(const engine_ctx *c);
void engine_ctx_free(engine_ctx *c);

/* csrc/engine.h:65-72. engine_eval returns 0, or -1 with the reason in engine_last_error and the
 * context unchanged. engine_logits points into host memory owned by the context, valid until the
 * next call. */
int engine_eval(engine_ctx *c, const int32_t *tokens, int32_t n);
const float *engine_logits(const engine_ctx *c);
int32_t engine_n_logits(const engine_ctx *c);
int32_t engine_n_past(const engine_ctx *c);
void engine_reset(engine_ctx *c);
int engine_truncate(engine_ctx *c, int32_t n);
const char *engine_last_error(const engine_ctx *c);

/* ------------------------------------------------------------------ GGUF (csrc/gguf.h:22-84) */

enum gguf_value_type {
    GGUF_TYPE_UINT8 = 0, GGUF_TYPE_INT8 = 1, GGUF_TYPE_UINT16 = 2, GGUF_TYPE_INT16 = 3, GGUF_TYPE_UINT32 = 4,
    GGUF_TYPE_INT32 = 5, GGUF_TYPE_FLOAT32 = 6, GGUF_TYPE_BOOL = 7, GGUF_TYPE_STRING = 8, GGUF_TYPE_ARRAY = 9,
    GGUF_TYPE_UINT64 = 10, GGUF_TYPE_INT64 = 11, GGUF_TYPE_FLOAT64 = 12,
};
#define GGUF_MAX_DIMS 4

/* csrc/gguf.h:40-48 (sardyne/capi.py:22-25) */
typedef struct {
    const char *name;
    uint32_t n_dims;
    uint32_t type;
    uint64_t ne[GGUF_MAX_DIMS];
    uint64_t offset;
    uint64_t nbytes;
    const void *data;
} gguf_tensor;

/* csrc/gguf.h:50-57 (sardyne/capi.py:28-30) */
typedef struct {
    const char *key;
    uint32_t type;
    uint32_t arr_type;
    uint64_t n;
    const uint8_t *ptr;
    uint64_t *str_pos;
} gguf_kv;

typedef struct gguf_file gguf_file;

gguf_file *gguf_open(const char *path, char *err, size_t err_len);
void gguf_close(gguf_file *f);
void gguf_prefetch(const void *p, size_t n);
uint32_t gguf_version(const gguf_file *f);
uint32_t gguf_alignment(const gguf_file *f);
uint64_t gguf_data_offset(const gguf_file *f);
uint64_t gguf_n_kv(const gguf_file *f);
uint64_t gguf_n_tensors(const gguf_file *f);
const gguf_kv *gguf_get_kv(const gguf_file *f, uint64_t i);
int64_t gguf_find_kv(const gguf_file *f, const char *key);
const gguf_tensor *gguf_get_tensor(const gguf_file *f, uint64_t i);
int64_t gguf_find_tensor(const gguf_file *f, const char *name);
int gguf_kv_get_u64(const gguf_file *f, int64_t i, uint64_t *out);
int gguf_kv_get_f64(const gguf_file *f, int64_t i, double *out);
const char *gguf_kv_get_str(const gguf_file *f, int64_t i, uint64_t *len);
const char *gguf_kv_get_arr_str(const gguf_file *f, int64_t i, uint64_t j, uint64_t *len);
const char *gguf_type_name(uint32_t ggml_type);

/* ------------------------------------------------------------------ kernels (csrc/ops.h:21-74)
 * Host-pointer entry points used by kernel-level tests. Each call copies its operands to the GPU,
 * runs the gfx950 kernel and copies the result back. */

enum { OP_F32 = 0, OP_F16 = 1, OP_Q4_0 = 2, OP_Q5_0 = 6, OP_Q8_0 = 8, OP_Q4_K = 12, OP_Q6_K = 14,
       OP_Q8_K = 15, OP_BF16 = 30 };

/* csrc/ops.h:25-26. The reference selects scalar or AVX2 CPU kernels. Here op_set_simd records the
 * request and op_simd reports it (1 by default); the GPU kernels are the same either way, and
 * their Q4_K/Q6_K results equal both of the reference's kernel sets, which agree bit for bit. */
int op_simd(void);
int op_set_simd(int enable);
/* No counterpart in the reference (its op_* cannot fail): the message of this thread's last op_*
 * call that failed on the GPU or rejected its arguments, "" after one that succeeded. A failed call
 * frees what it allocated and fills its float outputs with NaN; the process goes on. */
const char *op_last_error(void);
void op_f16_to_f32_n(const uint16_t *x, float *out, size_t n);                     /* csrc/ops.h:36 */
void op_matmul_rows(float *out, const float *x, const void *w, int wtype, int n_tok, int n_in, int n_out,
                    int row0, int row1);                                          /* csrc/ops.h:42-43 */
float op_dot_f32(const float *a, const float *b, int n);                          /* csrc/ops.h:55 */
uint16_t op_f32_to_f16(float f);                                                  /* csrc/ops.h:35 */
void op_row_to_f32(const void *row, int type, float *out, size_t n);              /* csrc/ops.h:37 */
size_t op_row_size(int type, int n);                                              /* csrc/ops.h:30 */
void op_quantize_rows(int vtype, const float *x, void *xq, int n_in, int t0, int t1); /* csrc/ops.h:49 */
void op_matmul_q_rows(float *out, const void *xq, const void *w, int wtype, int n_tok, int n_in, int n_out,
                      int row0, int row1);                                        /* csrc/ops.h:50-51 */
float op_vec_dot_q(int wtype, const void *w, const void *xq, int n);             /* csrc/ops.h:52 */
void op_axpy(float *y, float a, const float *x, int n);                           /* csrc/ops.h:56 */
void op_matmul(float *out, const float *x, const void *w, int wtype, int n_tok, int n_in, int n_out); /* :45 */
void op_rmsnorm(float *out, const float *x, const float *w, int n, float eps);    /* csrc/ops.h:58 */
void op_softmax(float *x, int n);                                                 /* csrc/ops.h:59 */
void op_silu_mul(float *gate, const float *up, int n);                            /* csrc/ops.h:60 */
void op_rope_table(float *cos_out, float *sin_out, int n_pos, int head_dim, float theta); /* csrc/ops.h:63 */
void op_rope(float *x, int n_heads, int head_dim, const float *cos, const float *sin, int interleaved); /* :66 */
void op_attention(float *out, const float *q, const float *k_cache, const float *v_cache, int n_head,
                  int n_kv_head, int head_dim, int n_kv, int stride, float *scores); /* csrc/ops.h:73-74 */

/* ------------------------------------------------------------------ model memory
 * No counterpart in the reference. The device memory a loaded model holds: its weights (the planes
 * of every matrix, the same bytes as the file's tensors) and the prefill GEMM's tiled copies made at
 * load, with the number of matrices that got a copy and that were left without one because the
 * device had no room (the GEMM then reads the planes, with the same results). Returns 0, or -1 for
 * a NULL model. */
int sdy_model_memory(const engine_model *m, size_t *weight_bytes, size_t *gemm_copy_bytes, int *n_copies,
                     int *n_skipped);
/* The expert stacks a loaded model keeps in pinned host memory, read in place by the kernels over
 * the host link (the layers whose experts did not fit the device, or those SARDYNE_HOST_EXPERTS
 * names): their bytes and the number of layers. Stands where the reference reads its weights from
 * the file mapping and prefetches the chosen experts (csrc/model_llama.c:703-721). Returns 0, or
 * -1 for a NULL model. */
int sdy_model_host_weights(const engine_model *m, size_t *host_bytes, int *host_layers);
/* Free and total device memory now (hipMemGetInfo); 0 or a negative code. No counterpart in the
 * reference. */
int sdy_mem_info(size_t *free_bytes, size_t *total_bytes);

/* ------------------------------------------------------------------ measurement
 * No counterpart in the reference: what a persistent decode kernel would pay per phase, against the
 * kernel boundary it would replace (the benchmark's grid_barrier workload).
 *
 * sdy_grid_barrier_probe: a co-resident grid of n_wg workgroups (cooperative launch) runs `rounds`
 * grid barriers of the given form, each publishing 64 floats per workgroup that another workgroup
 * reads back and checks; with stream_mb > 0 the other waves stream that many MiB (four passes) from
 * HBM meanwhile. Every wait is bounded: a timeout ends the grid and is counted. Times come from the
 * GPU's wall clock per round of workgroup 0. */
enum { SDY_BARRIER_FLAT = 0, SDY_BARRIER_TWO_LEVEL = 1, SDY_BARRIER_FENCED = 2 };
typedef struct {
    float us_median, us_mean;   /* per barrier round, over all rounds done */
    float us_mean_streaming;    /* mean over the rounds that ended while the stream still ran */
    float kernel_ms;            /* the whole launch (HIP events) */
    int rounds_done, rounds_streaming;
    unsigned timeouts, mismatches;  /* bounded waits that gave up; data values read back wrong */
} sdy_barrier_stats;
int sdy_grid_barrier_probe(int n_wg, int rounds, int mode, int stream_mb, sdy_barrier_stats *out);
/* n empty kernels back to back on one stream, recorded as a graph and replayed, and issued eagerly:
 * the mean microseconds per kernel of each. */
int sdy_kernel_boundary_us(int n, float *us_graph, float *us_eager);

/* ------------------------------------------------------------------ device-level, no allocation
 * No counterpart in the reference. For callers that cannot allocate device memory: code recorded
 * under graph capture, tight serving loops, harnesses that forbid hipMalloc. The one-token decode
 * attention of the engine (q/k RMSNorm and RoPE, the K/V write at step_dev[1], attention over
 * step_dev[1] + 1 positions split into 32-position chunks, and the Q8_K row of the output when
 * xq_q8k is set), with its partials and counters in a fixed static device buffer instead of
 * caller scratch: at most 1 048 576 floats of partials (n_head * ceil(max_seq / 32) * (head_dim + 4))
 * and 256 kv heads; larger shapes are rejected with an error. It calls no allocator. Every call on a
 * GPU shares that GPU's buffer: calls that overlap on one GPU race. sdy_init sets the buffer up on the
 * device it selects; on another device the first call does (a launch and a wait on the null stream),
 * and returns an error instead when the stream is being captured. A position step_dev[1] outside
 * [0, max_seq) leaves out and the caches untouched. Device pointers; returns 0 or a negative code
 * (the message from the library's last-error call). */
int sdy_attn_decode_split_noalloc(const float *q, const float *k, const float *v, const float *q_norm,
                                  const float *k_norm, float eps, const float *rope_cos, const float *rope_sin,
                                  const int32_t *step_dev, int n_head, int n_kv_head, int head_dim, int interleaved,
                                  float *k_cache, float *v_cache, long head_stride, int max_seq, float *out,
                                  void *xq_q8k, void *stream);

#ifdef __cplusplus
}
#endif
#endif

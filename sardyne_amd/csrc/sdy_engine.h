/* Engine state shared by engine.c (ABI, loading, validation) and forward.c (device forward). */
#ifndef SDY_ENGINE_H
#define SDY_ENGINE_H
#include <stdint.h>

#include "sardyne.h"
#include "sdy_shim.h"

enum { SDY_ATTN_EXACT = 0, SDY_ATTN_CHUNKED = 1, SDY_ATTN_SPLIT = 2 };

typedef struct {
    sdy_mat m;  /* device layout; experts stacked as n_expert * n_out rows */
    int type, n_in, n_out;
} dmat;

typedef struct {
    float *attn_norm, *ffn_norm, *bq, *bk, *bv, *q_norm, *k_norm; /* f32, device */
    dmat wq, wk, wv, wo, gate, up, down, gate_inp;
    /* wq|wk (qkv_parts 2) or wq|wk|wv (3) of one type stored as one matrix; wq, wk (and wv) are
       then row views of it, and bq|bk|bv are contiguous */
    dmat wqkv;
    int qkv_parts;
    /* gate and up of one quantized type stored interleaved (row 2i = gate i, row 2i+1 = up i; per
       expert for MoE): used with the SwiGLU matvec epilogue; gate and up are then unset */
    dmat gate_up;
    int gu_fused;
} dlayer;

struct engine_model {
    gguf_file *gf;
    engine_model_info info;
    dmat tok_embd, output;
    float *output_norm;
    dlayer *layers;
    float *vectors, *vec_cursor; /* one device allocation for every f32 vector */
    sdy_stream st;
    size_t device_bytes;       /* the uploaded weights in device memory (the planes of every matrix) */
    size_t host_bytes;         /* expert stacks kept in pinned host memory (read in place by the kernels) */
    int host_layers;           /* layers whose expert stacks are in host memory */
    size_t gemm_bytes;         /* the prefill GEMM's tiled copies made at load */
    int gemm_copies, gemm_skipped;
};

struct engine_ctx {
    const engine_model *m;
    int max_seq, n_batch, logits_all, n_past, n_logits, n_threads;
    sdy_stream st;
    float *logits; /* host (pinned), [n_logits][n_vocab] */
    /* device state */
    void *k_cache, *v_cache;    /* [n_layer][n_kv_head][max_seq][head_dim] of kv_type elements */
    int kv_type;                /* SDY_KV_F32 (the reference's), or SDY_KV_F16 (SARDYNE_KV=f16) */
    float *rope_cos, *rope_sin;
    float *x, *xb, *q, *k, *v, *att, *hb, *hb2, *logits_dev, *part;
    void *xq[2];                /* quantized activations: [0] Q8_0, [1] Q8_K */
    const float *xq_src[2];
    int xq_n_tok[2], xq_n_in[2];
    unsigned xq_epoch;          /* bumped at every write of xq[] */
    int gemm_ready;             /* gemm_ws holds the f16 expansion of gemm_xq made in epoch gemm_epoch */
    unsigned gemm_epoch;
    const void *gemm_xq;
    int gemm_n_tok, gemm_n_in;
    int32_t *tok_dev, *tok_host;
    /* one-token decode: step_dev = {token, position} read by the kernels, so the recorded graph
       replays for every position */
    int32_t *step_dev, *step_host;
    void *graph;                /* recorded one-token decode step (NULL until recorded) */
    int graph_ok;               /* 0: not tried, 1: recorded, -1: recording failed (run eagerly) */
    int n_decode;               /* one-token evals so far (the first runs eagerly) */
    int decode_fused;           /* one-token steps use the fused decode kernels */
    int use_graph;              /* one-token steps are recorded once and replayed */
    int fuse_act;               /* one-token matvecs quantise (and RMS-normalise) their f32 row in-kernel */
    int moe_device;             /* one-token MoE blocks route, run their experts and combine on the
                                   device (grouped matvec, no host round trip) */
    int attn_mode;              /* one-token attention: SDY_ATTN_EXACT (the reference's bits), or split
                                   over positions within tolerance: SDY_ATTN_CHUNKED (two launches),
                                   SDY_ATTN_SPLIT (one launch) */
    int prefill_flash;          /* many-token attention in flash form (sdy_attention_flash), within tolerance */
    float *attn_part;           /* chunked / split attention: per-span partials */
    unsigned *attn_count;       /* split attention: arrivals per kv head (zero between launches) */
    float *qkv;                 /* q | k | v of one token */
    void *gemm_ws;              /* scratch of the prefill GEMM (f16 activations of n_batch rows) */
    /* MoE */
    float *moe_probs, *moe_w, *moe_x, *moe_y, *moe_sum, *moe_gw;
    int32_t *moe_top, *moe_gidx, *moe_top_host, *moe_gidx_host;
    /* many-token MoE on the device: the routed pairs sorted by expert (sdy_moe_sort) */
    int *moe_grp_tok, *moe_grp_tile;
    int32_t *moe_src, *moe_orow;
    int moe_grouped_ok;         /* every MoE layer's experts take the grouped GEMM */
    float *moe_w_host, *moe_gw_host;
    char err[256];
};

int sdy_engine_alloc(engine_ctx *c);
void sdy_engine_release(engine_ctx *c);
int sdy_engine_forward(engine_ctx *c, const int32_t *tokens, int n, int out_rows);
int sdy_engine_decode_fused_ok(const engine_ctx *c);
int sdy_engine_moe_device_ok(const engine_ctx *c);
#endif

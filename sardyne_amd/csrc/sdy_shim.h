/* Internal C-ABI shim between the C host (engine.c, ops_api.c) and the HIP kernels.
 * Not exported to Python: the public ABI is include/sardyne.h.
 *
 * Every function returns 0 on success or a negative code; sdy_last_error() describes the last
 * failure of the calling thread. Device pointers are opaque `void *`.
 */
#ifndef SDY_SHIM_H
#define SDY_SHIM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { SDY_F32 = 0, SDY_F16 = 1, SDY_Q4_0 = 2, SDY_Q5_0 = 6, SDY_Q8_0 = 8, SDY_Q4_K = 12, SDY_Q6_K = 14,
       SDY_Q8_K = 15, SDY_BF16 = 30 };

typedef struct sdy_stream_s *sdy_stream; /* hipStream_t */

const char *sdy_last_error(void);
int sdy_init(void);                       /* selects the device, checks it is gfx950 */
/* the code sdy_malloc returns when the device has no room */
#define SDY_ERR_ALLOC (-4)
int sdy_malloc(void **p, size_t n);
int sdy_free(void *p);
int sdy_h2d(void *dst, const void *src, size_t n, sdy_stream s);
int sdy_d2h(void *dst, const void *src, size_t n, sdy_stream s);
int sdy_d2d(void *dst, const void *src, size_t n, sdy_stream s);
int sdy_memset(void *p, int v, size_t n, sdy_stream s);
int sdy_sync(sdy_stream s);
int sdy_stream_new(sdy_stream *s);
int sdy_stream_free(sdy_stream s);
int sdy_host_alloc(void **p, size_t n); /* pinned host memory */
/* pinned host memory that kernels read in place: host the allocation (for sdy_host_free), dev its
 * device address; SDY_ERR_ALLOC when the host has no room */
int sdy_host_alloc_mapped(void **host, void **dev, size_t n);
int sdy_host_free(void *p);
int sdy_device_info(int *n_cu, size_t *mem_total);
/* Free and total device memory now (hipMemGetInfo). */
int sdy_mem_info(size_t *free_bytes, size_t *total_bytes);
int sdy_event_new(void **ev);
int sdy_event_record(void *ev, sdy_stream s);
int sdy_event_elapsed(float *ms, void *e0, void *e1); /* waits for e1 */
int sdy_event_free(void *ev);
/* stream capture into a replayable graph (hipGraph): begin, issue kernels on s, end */
int sdy_graph_begin(sdy_stream s);
int sdy_graph_end(sdy_stream s, void **exec);
void sdy_graph_abort(sdy_stream s);
int sdy_graph_launch(void *exec, sdy_stream s);
int sdy_graph_free(void *exec);
/* reads every byte of buf once (HBM bandwidth probe); sink: 4 bytes of device memory. _strided: the
 * same in a grid-strided order over fewer workgroups (the faster one on buffers of a few hundred MB) */
int sdy_membw_read(const void *buf, size_t bytes, void *sink, sdy_stream s);
int sdy_membw_read_strided(const void *buf, size_t bytes, void *sink, sdy_stream s);

/* ---- weight matrices in the device layout (planes, see quant_kernels.hip) */
typedef struct {
    void *base;     /* one allocation holding every plane */
    size_t bytes;
    int type;
    int n_in;       /* elements per row */
    long n_rows;    /* rows (experts stacked: n_expert * n_out) */
    int n_units;    /* 64-element units per row (quantized types) */
    size_t plane_off[5];
    int gemm_ok;    /* Q4_K / Q6_K: 1 when the GEMM's one-fragment scheme is exact for every block,
                       2 when some block needs the wide variant (Q6_K: twice the MFMA work); 0 other types */
    void *gbase;    /* the GEMM's copy of the planes (sdy_mat_gemm_layout) or NULL: rows in tiles of 32,
                       each tile's records unit-major ([tile][unit][32 rows][16 bytes], the per-super-block
                       records [tile][super-block][32 rows]) */
    size_t gbytes;
    long grow0;     /* the first row of a row view in that copy */
    long grows;     /* rows of the matrix the copy was made from */
    void *hbase;    /* a matrix in pinned host memory (sdy_mat_alloc_host): the allocation, whose device
                       address is base; NULL for a matrix in device memory */
} sdy_mat;

/* Bytes of the device layout for a matrix. */
size_t sdy_mat_bytes(int type, int n_in, long n_rows);
/* Upload raw GGUF-layout rows from host memory and repack them on the device. */
int sdy_mat_upload(sdy_mat *m, int type, int n_in, long n_rows, const void *host_raw, sdy_stream s);
/* Allocate a matrix in the device layout (contents undefined until rows are uploaded). */
int sdy_mat_alloc(sdy_mat *m, int type, int n_in, long n_rows);
/* The same layout in pinned host memory that the kernels read in place over the host link (every
 * sdy_mat entry point takes it; no GEMM copy is made of it). */
int sdy_mat_alloc_host(sdy_mat *m, int type, int n_in, long n_rows);
/* Upload n raw rows from host memory into rows r0, r0 + step, ... of an allocated matrix: step 1
 * fills a range (concatenated matrices), step 2 interleaves two matrices row by row. */
int sdy_mat_upload_rows(sdy_mat *m, long r0, long step, long n, const void *host_raw, sdy_stream s);
/* General form: source row i goes to row r0 + (i / grp) * gstride + (i % grp) * step (per-expert
 * interleaving: grp = rows per expert, gstride = destination rows per expert, step 2). */
int sdy_mat_upload_map(sdy_mat *m, long r0, long n, long step, long grp, long gstride, const void *host_raw,
                       sdy_stream s);
/* Same, from raw rows already in device memory. */
int sdy_mat_from_device(sdy_mat *m, int type, int n_in, long n_rows, const void *dev_raw, sdy_stream s);
/* The repack of sdy_mat_upload_map from raw rows in device memory, queued on s (no allocation, no
 * synchronisation, no exactness check). */
int sdy_mat_repack_async(sdy_mat *m, long r0, long n, long step, long grp, long gstride, const void *dev_raw,
                         sdy_stream s);
/* The GEMM's copy of a Q4_K / Q6_K matrix (gbase), made from its planes after the last upload, for
 * the prefill GEMM's loads (a load instruction then reads whole cache lines). Another upload into
 * the matrix frees it (the GEMM reads the planes until it is made again). Other types: no-op. */
int sdy_mat_gemm_layout(sdy_mat *m, sdy_stream s);
/* Bytes sdy_mat_gemm_layout would allocate for m (0: no copy for this type or matrix). */
size_t sdy_mat_gemm_layout_bytes(const sdy_mat *m);

/* Pipelined uploads (upload.hip): a ring of pinned host slots and device slots. A host thread pool
 * copies the next rows from the file mapping into a free pinned slot (advising the kernel to read
 * the rows after them ahead), the DMA engine moves the slot to the device on a copy stream, and the
 * repack runs on the work stream; the three overlap across slots. The GEMM variant checks of the
 * uploaded rows run at sdy_uploader_finish, which waits for everything and sets each matrix's
 * gemm_ok. A matrix must stay at its address until then. */
typedef struct sdy_uploader sdy_uploader;
int sdy_uploader_new(sdy_uploader **u, size_t slot_bytes, int n_slots, int n_threads, sdy_stream work);
/* Rows as sdy_mat_upload_map, from host memory (a GGUF mapping) */
int sdy_uploader_rows(sdy_uploader *u, sdy_mat *m, long r0, long n, long step, long grp, long gstride,
                      const void *host_raw);
int sdy_uploader_finish(sdy_uploader *u); /* waits, runs the checks; the uploader stays usable */
/* bytes uploaded so far, and seconds spent in the host copies and waiting for a free slot */
void sdy_uploader_stats(const sdy_uploader *u, double *bytes, double *host_copy_s, double *slot_wait_s);
int sdy_uploader_free(sdy_uploader *u); /* finishes, then releases the slots and the copy stream */
int sdy_mat_free(sdy_mat *m);
/* Sub-matrix view of rows [r0, r0+n) (e.g. one expert); no copy. */
sdy_mat sdy_mat_rows(const sdy_mat *m, long r0, long n);

/* ---- kernels (all asynchronous on stream s) */
/* rows [r0, r0+n_rows_out) of m dequantised to f32 (bit-exact with the reference). */
int sdy_dequant_rows(const sdy_mat *m, long r0, long n, float *out, sdy_stream s);
/* dequantise the rows listed in idx[0..n) (device int32) into out[n][n_in] */
int sdy_dequant_gather(const sdy_mat *m, const int32_t *idx, int n, float *out, sdy_stream s);
/* activation quantisation in the reference block formats: vtype SDY_Q8_0 or SDY_Q8_K */
int sdy_quantize(int vtype, const float *x, void *xq, int n_in, int n_tok, sdy_stream s);

typedef struct {
    const void *xq;      /* quantized activations, [n_tok][row_size(vtype, n_in)] */
    const float *x;      /* f32 activations for F32/F16/BF16 weights, [n_tok][n_in] */
    int n_tok;
    float *out;          /* out[t * out_stride + row] */
    long out_stride;
    const float *bias;   /* optional, out += bias[row] */
    const float *resid;  /* optional, out = resid[t * out_stride + row] + result */
    long row0, row1;     /* rows computed */
    int epilogue;        /* SDY_EPI_NONE, or SDY_EPI_SWIGLU: rows (2i, 2i+1) of [row0, row1) are the gate and
                            up rows of output i, out[t * out_stride + i] = silu(gate) * up */
    const float *nw;     /* K-quant weights with xq = NULL and x set (one token): the kernel builds the Q8_K
                            row of x itself, RMS-normalised first when nw is set (x / rms(x) * nw, eps), with
                            the bytes sdy_quantize / sdy_norm_quant would write; see sdy_matvec_fused_ok */
    float eps;
    int ws_ready;        /* sdy_gemm: ws already holds this xq's f16 expansion (same n_tok and n_in), written by
                            the previous sdy_gemm on ws with nothing written to xq or ws since: it is not
                            expanded again */
} sdy_mv_args;
enum { SDY_EPI_NONE = 0, SDY_EPI_SWIGLU = 1 };
/* out = W · x for rows [row0, row1) and n_tok tokens. */
int sdy_matvec(const sdy_mat *m, const sdy_mv_args *a, sdy_stream s);
/* 1 when sdy_matvec (and, for two matrices, sdy_matvec_pair) can quantise the f32 row itself for these
 * arguments: one token, Q4_K / Q6_K, 256-element blocks, x (and nw) 16-byte aligned, nw only for
 * rows of at most 4096 elements; a single matrix with more rows than a one-token grid holds at once
 * (an output head) runs on the persistent ring kernel, except with the SwiGLU epilogue; a pair needs
 * a grid the GPU holds at once. m2/a2 may be NULL. */
int sdy_matvec_fused_ok(const sdy_mat *m, const sdy_mv_args *a, const sdy_mat *m2, const sdy_mv_args *a2);
/* Two one-token matvecs in one launch (each with the bits of sdy_matvec): Q4_K / Q6_K matrices of
 * at most 4096-element rows, e.g. a layer's q|k and a v of another type on the same Q8_K row. */
int sdy_matvec_pair_ok(const sdy_mat *m1, int epilogue1, const sdy_mat *m2, int epilogue2);
int sdy_matvec_pair(const sdy_mat *m1, const sdy_mv_args *a1, const sdy_mat *m2, const sdy_mv_args *a2,
                    sdy_stream s);
/* Grouped one-token matvec over routed experts: m stacks experts of slot_rows rows; for each of
 * n_slot slots, rows [row0, row1) of expert slot_expert[slot] (device array) times the slot's
 * Q8_K activation row (a->xq + slot * xq_slot bytes) go to a->out + slot * out_slot. Q4_K / Q6_K,
 * rows of at most 4096 elements; the SwiGLU epilogue as in sdy_matvec. */
int sdy_matvec_grouped(const sdy_mat *m, const sdy_mv_args *a, const int32_t *slot_expert, int n_slot,
                       long slot_rows, long xq_slot, long out_slot, sdy_stream s);
/* sdy_matvec_grouped over the k slots of one token whose experts the kernel selects from the
 * router's n_expert <= 128 logits (device array): the choices and weights of sdy_moe_route, which it
 * also writes to top and wts (k entries each), so no route launch precedes it. The Q8_K row in memory
 * (a->xq), k <= 64. Returns 1, launching nothing, when no one-token grid fits. */
int sdy_matvec_grouped_route(const sdy_mat *m, const sdy_mv_args *a, const float *logits, int n_expert, int k,
                             int32_t *top, float *wts, long slot_rows, long xq_slot, long out_slot, sdy_stream s);
/* 1 when sdy_matvec_grouped can quantise each slot's f32 row itself (a->xq = NULL, a->x set; slot s's
 * row at a->x + s * x_slot floats, passed as xq_slot; RMS-normalised first when a->nw is set) */
int sdy_matvec_grouped_fused_ok(const sdy_mat *m, const sdy_mv_args *a, int n_slot, long slot_rows, long x_slot);
/* The routed experts' down projections of one token and their combine in one launch: slot s's f32
 * row x + s * n_in through expert slot_expert[s] of the stack m (dim rows each), then
 * out = resid + sum over the k <= 8 slots in ascending expert id of wts[s] * y_s (resid may be NULL,
 * or out itself). The bits of sdy_matvec_grouped with in-kernel quantisation, then sdy_moe_combine. */
int sdy_moe_down_combine(const sdy_mat *m, const float *x, const int32_t *slot_expert, const float *wts, int k,
                         long dim, float *out, const float *resid, sdy_stream s);

/* The prefill GEMM (gemm_kernels.hip): the same outputs as sdy_matvec (bit for bit) for
 * n_tok >= 2 tokens of Q8_K activations a->xq on Q4_K / Q6_K matrices with gemm_ok, through
 * MFMA. ws: sdy_gemm_ws_bytes(n_tok, n_in) bytes of device scratch. */
int sdy_gemm_ok(const sdy_mat *m, int n_tok);
size_t sdy_gemm_ws_bytes(int n_tok, int n_in);
int sdy_gemm(const sdy_mat *m, const sdy_mv_args *a, void *ws, sdy_stream s);
/* Two GEMMs over the same activations (a1->xq == a2->xq, the same n_tok and n_in; a layer's q|k and
 * its v): one launch when m1 is Q4_K and m2 Q6_K on small grids, else two sdy_gemm calls. The bits of
 * sdy_gemm(m1, a1) then sdy_gemm(m2, a2 with ws_ready). */
int sdy_gemm2(const sdy_mat *m1, const sdy_mv_args *a1, const sdy_mat *m2, const sdy_mv_args *a2, void *ws,
              sdy_stream s);
/* Q8_K activations for the GEMM in one launch: the bytes of sdy_quantize (of sdy_norm_quant, with xb
 * as there) into xq, and their f16 expansion into ws, so that sdy_gemm on the same rows and ws runs
 * with ws_ready = 1. */
int sdy_quantize_gemm(const float *x, void *xq, int n_in, int n_tok, void *ws, sdy_stream s);
int sdy_norm_quant_gemm(const float *x, const float *w, float eps, int n, int n_rows, float *xb, void *xq, void *ws,
                        sdy_stream s);
/* The GEMM over routed experts in one launch: m stacks n_grp experts of grp_rows rows; rows
 * grp_tok[e] .. grp_tok[e + 1] - 1 (a->n_tok rows in all) multiply expert e, and the results of row
 * t go to output row out_row[t] (or t). Row t's activations are row act_row[t] (or t) of the
 * quantised input (Q8_K in a->xq); with act_row the caller has made the expansion of those n_act
 * rows in ws (sdy_quantize_gemm, a->ws_ready = 1), so the routed rows need no gathered copy. grp_tile: the
 * tiles of sdy_gemm_grouped_tile() rows per expert, as sdy_moe_sort writes them. a->epilogue may be
 * SwiGLU (even grp_rows); no bias or residual. The same bits as sdy_gemm per expert. */
int sdy_gemm_grouped_tile(void);
int sdy_gemm_grouped(const sdy_mat *m, long grp_rows, int n_grp, const int *grp_tok, const int *grp_tile,
                     const int *out_row, const int *act_row, int n_act, const sdy_mv_args *a, void *ws,
                     sdy_stream s);
/* Variant check of rows [r0, r0 + n) of m for the GEMM: *bad_host = 1 when some row has a block
 * that only the wide variant multiplies exactly. */
int sdy_gemm_check_rows(const sdy_mat *m, long r0, long n, int *bad_host, sdy_stream s);
/* The same, queued on s: sets *bad_dev (device int, zero beforehand) to nonzero for such a row */
int sdy_gemm_check_rows_async(const sdy_mat *m, long r0, long n, int *bad_dev, sdy_stream s);

/* raw float-weight matrices (F32/F16/BF16, GGUF row-major layout kept as is) */
int sdy_matvec_float(int wtype, const void *w, int n_in, const sdy_mv_args *a, sdy_stream s);
/* The same for one token of the RMS-normalised row (x / rms(x) * a->nw, with a->eps): the bits of
 * sdy_norm_quant's f32 row followed by sdy_matvec_float; with xq_out, also that row's Q8_K bytes (the
 * ones sdy_norm_quant writes). n_in a multiple of 256, at most 4096; x and nw 16-byte aligned. */
int sdy_matvec_float_norm(int wtype, const void *w, int n_in, const sdy_mv_args *a, void *xq_out, sdy_stream s);

#ifdef __cplusplus
}
#endif
#endif

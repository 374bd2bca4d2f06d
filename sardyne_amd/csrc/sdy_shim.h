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
int sdy_host_free(void *p);
int sdy_device_info(int *n_cu, size_t *mem_total);
int sdy_event_new(void **ev);
int sdy_event_record(void *ev, sdy_stream s);
int sdy_event_elapsed(float *ms, void *e0, void *e1); /* waits for e1 */
int sdy_event_free(void *ev);
/* reads every byte of buf once (HBM bandwidth probe); sink: 4 bytes of device memory */
int sdy_membw_read(const void *buf, size_t bytes, void *sink, sdy_stream s);

/* ---- weight matrices in the device layout (planes, see quant_kernels.hip) */
typedef struct {
    void *base;     /* one allocation holding every plane */
    size_t bytes;
    int type;
    int n_in;       /* elements per row */
    long n_rows;    /* rows (experts stacked: n_expert * n_out) */
    int n_units;    /* 64-element units per row (quantized types) */
    size_t plane_off[5];
} sdy_mat;

/* Bytes of the device layout for a matrix. */
size_t sdy_mat_bytes(int type, int n_in, long n_rows);
/* Upload raw GGUF-layout rows from host memory and repack them on the device. `staging` is a
 * device buffer of at least min(raw bytes, staging_bytes) bytes reused for chunked uploads; pass
 * NULL to let the function allocate one. */
int sdy_mat_upload(sdy_mat *m, int type, int n_in, long n_rows, const void *host_raw, sdy_stream s);
/* Same, from raw rows already in device memory. */
int sdy_mat_from_device(sdy_mat *m, int type, int n_in, long n_rows, const void *dev_raw, sdy_stream s);
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
} sdy_mv_args;
/* out = W · x for rows [row0, row1) and n_tok tokens. */
int sdy_matvec(const sdy_mat *m, const sdy_mv_args *a, sdy_stream s);

/* raw float-weight matrices (F32/F16/BF16, GGUF row-major layout kept as is) */
int sdy_matvec_float(int wtype, const void *w, int n_in, const sdy_mv_args *a, sdy_stream s);

#ifdef __cplusplus
}
#endif
#endif

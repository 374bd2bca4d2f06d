// Internal helpers shared by the HIP translation units of the shim (not part of any ABI).
#pragma once
#include <stddef.h>
#include <string.h>

#ifdef __cplusplus
extern "C" {
#endif
/* Records a formatted error for sdy_last_error() and returns rc. */
int sdy_fail(int rc, const char *fmt, ...);
/* Turns a pending kernel-launch error into an sdy error. */
int sdy_check_launch(const char *what);
/* Raises kernel fn's dynamic-LDS limit to `bytes` if *granted (per call site) is below it. */
int sdy_lds_limit(const void *fn, size_t bytes, size_t *granted);
/* The no-alloc attention entry point's set-up on the current device (attn_decode_split.hip). */
int sdy_attn_split_scratch_setup(void);
/* Bytes of one row in the GGUF layout. */
size_t sdy_raw_row_bytes(int type, int n_in);
#ifdef __cplusplus
}
/* The host function of the last matvec / GEMM / attention kernel launched by this thread (the name
 * sdy_last_kernel reports). Set right before the launch: SDY_NOTE_KERNEL((k<A, B>)). */
extern thread_local const void *sdy_last_kernel_fn;
#define SDY_NOTE_KERNEL(k) (sdy_last_kernel_fn = reinterpret_cast<const void *>(&k))
#endif

/* CPU baseline harness (test infrastructure, used only by bench.py's cpu_baseline): one token of the
 * reference's own matmul() (csrc/model_llama.c:569-611) on the reference's own thread pool
 * (csrc/threadpool.c:68-141), timed over rotated weight copies.
 *
 * Per repetition, as matmul() does for a quantized matrix and a new input:
 *   tp_run(quantize part): rows of tokens split evenly over the threads (one token: the last thread
 *                          quantises it) with op_quantize_rows;
 *   tp_run(row part):      output rows split evenly, r0 = n_out * ith / nth, with op_matmul_q_rows;
 * each tp_run ends with the pool's barrier. Linked against oracle/_ref/libsardyne_ref.so, the
 * reference compiled from its sources; the prototypes below are its csrc/threadpool.h:15-25 and
 * csrc/ops.h:25-51 declarations.
 */
#define _POSIX_C_SOURCE 200809L
#include <stddef.h>
#include <stdint.h>
#include <time.h>

typedef struct threadpool threadpool;
typedef void (*tp_fn)(void *arg, int ith, int nth);
threadpool *tp_new(int n_threads);
void tp_free(threadpool *p);
void tp_run(threadpool *p, tp_fn fn, void *arg);
int tp_default_threads(void);
int op_set_simd(int enable);
void op_quantize_rows(int vtype, const float *x, void *xq, int n_in, int t0, int t1);
void op_matmul_q_rows(float *out, const void *xq, const void *w, int wtype, int n_tok, int n_in, int n_out, int row0,
                      int row1);

typedef struct {
    int wtype, vtype, n_in, n_out;
    const float *x;
    void *xq;
    const void *w;
    float *out;
} job;

static void part(int n, int ith, int nth, int *b, int *e) {
    *b = (int)((long long)n * ith / nth);
    *e = (int)((long long)n * (ith + 1) / nth);
}

static void quantize_part(void *arg, int ith, int nth) {
    const job *j = arg;
    int t0, t1;
    part(1, ith, nth, &t0, &t1);
    if (t0 < t1) op_quantize_rows(j->vtype, j->x, j->xq, j->n_in, t0, t1);
}

static void rows_part(void *arg, int ith, int nth) {
    const job *j = arg;
    int r0, r1;
    part(j->n_out, ith, nth, &r0, &r1);
    if (r0 < r1) op_matmul_q_rows(j->out, j->xq, j->w, j->wtype, 1, j->n_in, j->n_out, r0, r1);
}

static double now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + 1e-9 * ts.tv_nsec;
}

/* Seconds per repetition (quantise + matvec) over `seconds` of wall time, rotating the n_copies
 * weight matrices; n_threads 0 = the pool's default (the online CPUs). *reps and *threads report
 * what ran. xq: a buffer of the activation row's quantized size; out: n_out floats. */
double ref_cpu_matvec(int wtype, int vtype, const void *const *copies, int n_copies, const float *x, void *xq,
                      float *out, int n_in, int n_out, double seconds, int n_threads, long *reps, int *threads) {
    if (n_threads <= 0) n_threads = tp_default_threads();
    threadpool *pool = tp_new(n_threads);
    if (!pool) return -1.0;
    op_set_simd(1);
    job j = {wtype, vtype, n_in, n_out, x, xq, copies[0], out};
    tp_run(pool, quantize_part, &j); /* warm: threads up, first copy touched */
    tp_run(pool, rows_part, &j);
    long n = 0;
    const double t0 = now();
    double t;
    do {
        j.w = copies[n % n_copies];
        tp_run(pool, quantize_part, &j);
        tp_run(pool, rows_part, &j);
        n++;
    } while ((t = now() - t0) < seconds);
    tp_free(pool);
    *reps = n;
    *threads = n_threads;
    return t / n;
}

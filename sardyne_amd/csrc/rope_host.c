/* RoPE tables, built on the host at context creation and uploaded once.
 *
 * cos/sin of p * theta^(-2i/head_dim) are evaluated in double with the host libm and rounded to
 * f32, the arithmetic of the reference's table (csrc/ops.c:375-386): 1 / pow(theta, 2i/head_dim)
 * in double, times p in double. Using the same libm on the same host makes the table bit-identical
 * to the reference's; it is O(max_seq * head_dim) work done once per context, not per token.
 */
#include <math.h>
#include <stddef.h>

#include "sdy_ops.h"

void sdy_rope_table_host(float *cos_out, float *sin_out, int n_pos, int head_dim, float theta) {
    const int half = head_dim / 2;
    for (int i = 0; i < half; i++) {
        const double inv_freq = 1.0 / pow((double)theta, (double)(2 * i) / head_dim);
        for (int p = 0; p < n_pos; p++) {
            const double a = (double)p * inv_freq;
            cos_out[(size_t)p * half + i] = (float)cos(a);
            sin_out[(size_t)p * half + i] = (float)sin(a);
        }
    }
}

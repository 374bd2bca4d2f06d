"""sdy_expf (sardyne_amd/csrc/sdy_expf.h), the device's restatement of the host libm expf that the
reference calls in its softmax and SiLU (csrc/ops.c:353-371), against the host expf itself: a C
program built from the header compares the two on a strided sweep of all 2^32 float bit patterns
(every 61st, plus the 2^16 patterns around each special-case boundary). SDY_EXPF_EXHAUSTIVE=1 sweeps
every pattern (about a minute)."""
import os
import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
SRC = r'''
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "sdy_expf.h"
static uint32_t bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static long check(uint32_t b, long *n) {
    float x; memcpy(&x, &b, 4);
    float a = expf(x), m = sdy_expf(x);
    (*n)++;
    if (a != a && m != m) return 0;
    if (bits(a) != bits(m)) { printf("x=%a host=%a device=%a\n", x, a, m); return 1; }
    return 0;
}
int main(int argc, char **argv) {
    const unsigned long step = strtoul(argv[1], NULL, 10);
    long bad = 0, n = 0;
    for (unsigned long u = 0; u < 0x100000000UL; u += step) bad += check((uint32_t)u, &n);
    const float edges[] = {0x1.62e42ep6f, -0x1.9fe368p6f, 0.0f, 87.0f, -87.0f, 1.0f, -1.0f};
    for (int e = 0; e < 7; e++)
        for (int d = -32768; d < 32768; d++) bad += check(bits(edges[e]) + (uint32_t)d, &n);
    printf("%ld of %ld differ\n", bad, n);
    return bad != 0;
}
'''


def test_sdy_expf_equals_host_expf(tmp_path):
    src = tmp_path / "expf_check.c"
    src.write_text(SRC)
    exe = tmp_path / "expf_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", f"-I{ROOT / 'sardyne_amd' / 'csrc'}", str(src), "-o", str(exe),
                    "-lm"], check=True)
    step = "1" if os.environ.get("SDY_EXPF_EXHAUSTIVE") else "61"
    r = subprocess.run([str(exe), step], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:]
    assert " 0 of " in r.stdout or r.stdout.startswith("0 of"), r.stdout

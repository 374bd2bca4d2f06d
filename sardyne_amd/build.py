"""Build of libsardyne.so: HIP kernels for gfx950 (hipcc) plus the C host (gcc), linked in-tree
into build/libsardyne.so. Run as ``python -m sardyne_amd.build``.

HIP flags: contraction off and f16/f32 denormals kept (the dequantisation and the f32 combines
must round exactly like the reference), correctly rounded f32 division/sqrt, packed-FP32
instructions disabled, and MFMA results in ordinary VGPRs (the GEMM combines them with VALU
instructions, which would otherwise first copy them out of the accumulation registers).
"""
from __future__ import annotations

import os
import pathlib
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

ROOT = pathlib.Path(__file__).resolve().parent.parent
CSRC = ROOT / "sardyne_amd" / "csrc"
INCLUDE = ROOT / "include"
OUT_DIR = ROOT / "build"
LIB = OUT_DIR / "libsardyne.so"
OBJ_DIR = OUT_DIR / "obj"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
             "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form", "-Wall",
             f"-I{INCLUDE}", f"-I{CSRC}"]
C_FLAGS = ["-std=c11", "-O2", "-fPIC", "-ffp-contract=off", "-Wall", "-Wextra", f"-I{INCLUDE}", f"-I{CSRC}",
           "-I/opt/rocm/include"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(map(str, cmd))}\n{err}")
    return err


def build(verbose: bool = False) -> pathlib.Path:
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    hip_srcs = sorted(CSRC.glob("*.hip"))
    c_srcs = sorted(CSRC.glob("*.c"))
    jobs = []
    for s in hip_srcs:
        jobs.append([HIPCC, *HIP_FLAGS, "-c", str(s), "-o", str(OBJ_DIR / (s.stem + ".hip.o"))])
    for s in c_srcs:
        jobs.append(["gcc", *C_FLAGS, "-c", str(s), "-o", str(OBJ_DIR / (s.stem + ".c.o"))])
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        outs = list(ex.map(_run, jobs))
    if verbose:
        for o in outs:
            if o.strip():
                print(o)
    objs = [str(OBJ_DIR / (s.stem + ".hip.o")) for s in hip_srcs] + [str(OBJ_DIR / (s.stem + ".c.o")) for s in c_srcs]
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", str(tmp), "-Wl,-rpath,/opt/rocm/lib",
          "-lm", "-lpthread"])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

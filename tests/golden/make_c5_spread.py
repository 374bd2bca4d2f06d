"""Writes c5_simd_spread.npz: how far the reference's own two engines drift apart on the Qwen3-30B-A3B-
shaped model, the yardstick of the tolerance the GPU engine's split one-token attentions are held to
at that shape (tests/test_gpu_configs.py).

The reference selects its CPU kernels once per process (csrc/ops.c:189-197): the AVX2 set, or the
scalar one when ENGINE_NO_SIMD is set. The two differ only in float summation orders (the attention
dot and axpy, the router matvec, the Q8_0-type dots: csrc/ops_avx2.c, csrc/quant_avx2.c); their K-quant
integer dots agree bit for bit. This script runs the reference compiled from its sources
(oracle/_ref/libsardyne_ref.so) on the test's model and tokens in two child processes, one per kernel
set: the same 1024-token context (n_batch 64, the reference's default), then the same 5 one-token
steps. It records, per evaluation (the context's last logits, then each step's), the largest
|AVX2 - scalar| difference, the logit scale max|AVX2| over all of them, and whether the argmax agrees.

Run (in the build container, where oracle/_ref is built; about 20 GB of the model file in /dev/shm and
a few minutes of CPU): python tests/golden/make_c5_spread.py
"""
from __future__ import annotations

import hashlib
import os
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))

N_CTX, N_STEPS, MAX_SEQ, MODEL_SEED, TOKEN_SEED = 1024, 5, 1152, 0, 1


def tokens() -> np.ndarray:
    """The token ids of tests/test_gpu_configs.py's C5 test (seed 1, uniform over the vocabulary)."""
    return np.random.default_rng(TOKEN_SEED).integers(0, 151936, N_CTX + N_STEPS).astype(np.int32)


def child(model: str, out: str) -> None:
    import oracle as O
    toks = tokens()
    ref = O.RefEngine(model, MAX_SEQ, n_batch=64)
    rows = [ref.eval(toks[:N_CTX])] + [ref.eval([int(t)]) for t in toks[N_CTX:]]
    np.save(out, np.stack(rows))


def main() -> None:
    import oracle as O
    from sardyne_amd.gguf_synth import qwen3_30b_a3b, write_model
    if not O.ref_available():
        sys.exit("oracle/_ref is not built (make -C oracle ref)")
    root = Path("/dev/shm") if os.path.isdir("/dev/shm") else Path(tempfile.gettempdir())
    model = root / f"sardyne_c5_spread_{os.getpid()}.gguf"
    res = {}
    try:
        write_model(model, qwen3_30b_a3b(), seed=MODEL_SEED)
        with tempfile.TemporaryDirectory() as td:
            for name, env in (("avx2", {}), ("scalar", {"ENGINE_NO_SIMD": "1"})):
                out = Path(td) / f"{name}.npy"
                e = {k: v for k, v in os.environ.items() if k != "ENGINE_NO_SIMD"}
                e.update(env)
                subprocess.run([sys.executable, __file__, "--child", str(model), str(out)], env=e, check=True)
                res[name] = np.load(out)
    finally:
        model.unlink(missing_ok=True)
    a, s = res["avx2"], res["scalar"]
    scale = float(np.abs(a).max())
    spread = np.abs(a - s).max(axis=1).astype(np.float32)
    np.savez(HERE / "c5_simd_spread.npz", spread=spread, scale=np.float32(scale),
             argmax_equal=(a.argmax(-1) == s.argmax(-1)), n_ctx=N_CTX, n_steps=N_STEPS, model_seed=MODEL_SEED,
             tok_sha=hashlib.sha256(tokens().tobytes()).hexdigest())
    print("spread / scale per evaluation:", (spread / scale).round(6).tolist(), "argmax equal:",
          (a.argmax(-1) == s.argmax(-1)).tolist())


if __name__ == "__main__":
    if len(sys.argv) == 4 and sys.argv[1] == "--child":
        child(sys.argv[2], sys.argv[3])
    else:
        main()

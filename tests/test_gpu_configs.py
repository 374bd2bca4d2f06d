"""The benchmark configurations at their full sizes on the GPU, against the reference.

  C1  Q4_K 2048 x 2048 matvec (seed 0): bit-exact with the reference's output in golden/c1.npz.
  C2  Q6_K and Q8_0 151936 x 2048 head matvecs (seed 0): the inputs are the ones golden/c2.npz
      was made from (sha256), the first 512 outputs equal the reference's there, and every output
      equals the oracle's (Q6_K bit-exact; Q8_0, whose f32 block sums have an order of their own,
      within rel-L2 1e-6 of both the reference's AVX2 and scalar orders).
  C3/C4  the Qwen2.5-3B-shaped Q4_K_M model: one 512-token prompt with n_batch 512 (the MFMA GEMM
      path), then one-token steps (replayed from the recorded decode graph after the first):
      logits bit-identical to the reference engine compiled from its sources, and within 1e-4 of
      the logit scale (same greedy tokens) with the one-launch split attention.
  C5  the Qwen3-30B-A3B-shaped qwen3moe model (128 experts resident, top-8): a 1024-token context
      (two 512-token chunks), then one-token steps through the device router: the exact chain
      bit-identical, the chunked and split attentions within twice the spread between the
      reference's own AVX2 and scalar engines on the same model and tokens (golden/c5_simd_spread.npz),
      with the same greedy tokens. On a device with room for half its experts, the rest in pinned
      host memory: the bits of the load with every expert on the device.
  C3 and C5 over the decode benchmark's own sequence (its context, then 128 one-token steps): the
      default engine within the same tolerances at every step, with the same greedy tokens.

The models are written to /dev/shm (2.2 GB and 19.8 GB) and deleted afterwards.
"""
import ctypes
import hashlib
import json
import os
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from conftest import engine_env
from sardyne_amd import capi
from sardyne_amd.engine import LoadedModel
from sardyne_amd.gguf_synth import qwen25_3b, qwen3_30b_a3b, random_blocks, write_model

pytestmark = pytest.mark.gpu

TESTS = Path(__file__).resolve().parent
GOLDEN = TESTS / "golden"
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="the reference compiled into oracle/_ref is missing")


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def device_matvec(wt, w, x, n_in):
    L = capi.lib()
    capi.check(L.sdy_init())
    vt = O.VEC_DOT[wt]
    m = capi.DeviceMatrix(wt, n_in, w.shape[0], w)
    dx = capi.DeviceBuffer.from_array(x)
    dq = capi.DeviceBuffer(O.row_size(vt, n_in))
    dy = capi.DeviceBuffer(w.shape[0] * 4)
    capi.check(L.sdy_quantize(vt, dx.ptr, dq.ptr, n_in, 1, None))
    a = capi.SdyMvArgs(xq=dq.ptr, n_tok=1, out=dy.ptr, out_stride=w.shape[0], row0=0, row1=w.shape[0])
    capi.check(L.sdy_matvec(ctypes.byref(m.m), ctypes.byref(a), None))
    capi.check(L.sdy_sync(None))
    return dy.to_array(np.float32, w.shape[0]), O.quantize(x, vt)


def test_c1_q4k_matvec_matches_reference_output():
    g = np.load(GOLDEN / "c1.npz")
    w = random_blocks("Q4_K", 2048 * 2048 // 256, np.random.default_rng(0)).reshape(2048, -1)
    x = np.random.default_rng(1).standard_normal(2048).astype(np.float32)
    assert sha(w) == str(g["w_sha"]) and sha(x) == str(g["x_sha"])
    y, _ = device_matvec(O.Q4_K, w, x, 2048)
    assert np.array_equal(y.view(np.uint32), g["y"].view(np.uint32))


@pytest.mark.parametrize("kind", ["Q6_K", "Q8_0"])
def test_c2_head_matvec_full_shape(kind):
    g = np.load(GOLDEN / "c2.npz")
    t = {"Q6_K": O.Q6_K, "Q8_0": O.Q8_0}[kind]
    e = 256 if kind == "Q6_K" else 32
    w = random_blocks(kind, 151936 * 2048 // e, np.random.default_rng(0)).reshape(151936, -1)
    x = np.random.default_rng(1).standard_normal(2048).astype(np.float32)
    assert sha(w) == str(g[f"{kind}_w_sha"]) and sha(x) == str(g["x_sha"]), "not the inputs of the fixture"
    y, xq = device_matvec(t, w, x, 2048)
    ref512 = g[f"{kind}_y512"]
    exp = O.matmul_q(w, t, xq, 2048, simd=0)[0]  # the oracle over all 151936 rows
    if kind == "Q6_K":
        assert np.array_equal(y[:512].view(np.uint32), ref512.view(np.uint32))
        assert np.array_equal(y.view(np.uint32), exp.view(np.uint32))
    else:
        # Q8_0 sums blocks in f32 in an order of its own (the reference's AVX2 and scalar orders differ
        # too, tests/test_quant.py:156-166): compared by rel-L2, far inside the 1e-3 bar
        exp_avx2 = O.matmul_q(w, t, xq, 2048, simd=1)[0]
        assert np.linalg.norm(y[:512] - ref512) / np.linalg.norm(ref512) < 1e-6
        for e in (exp, exp_avx2):
            assert np.linalg.norm(y - e) / np.linalg.norm(e) < 1e-6
    assert np.array_equal(np.argsort(-y, kind="stable")[:8], np.argsort(-exp, kind="stable")[:8])


def _shm_model(spec, label):
    root = Path("/dev/shm") if os.path.isdir("/dev/shm") else Path(tempfile.gettempdir())
    path = root / f"sardyne_test_{label}_{os.getpid()}.gguf"
    write_model(path, spec, seed=0)
    return path


@pytest.fixture(scope="module")
def qwen25_3b_path():
    p = _shm_model(qwen25_3b(), "qwen25_3b")
    yield p
    p.unlink(missing_ok=True)


def _run_and_compare(path, n_ctx, n_batch, n_steps, max_seq, seed, tol):
    """The engine with the exact attention chain (SARDYNE_ATTENTION=exact) gives the reference's bits
    at every step; with the split one-token attentions (chunked, split), whose prompt runs through
    the flash attention, the logits are within tol of the logit scale, with the same greedy tokens."""
    toks = np.random.default_rng(seed).integers(0, 151936, n_ctx + n_steps).astype(np.int32)
    model = LoadedModel(path)
    runs = {}
    for mode in ("exact", "chunked", "split"):
        env = {"SARDYNE_ATTENTION": mode}
        with engine_env(**env):
            s = model.session(max_seq=max_seq, n_batch=n_batch)
        runs[mode] = [s.feed(toks[:n_ctx])] + [s.step(int(t)) for t in toks[n_ctx:]]
        del s
    del model
    ref = O.RefEngine(path, max_seq, n_batch=64)
    exp = [ref.eval(toks[:n_ctx])] + [ref.eval([int(t)]) for t in toks[n_ctx:]]
    for i, (g, e) in enumerate(zip(runs["exact"], exp)):
        assert np.all(np.isfinite(g)), i
        assert np.array_equal(g.view(np.uint32), e.view(np.uint32)), (i, float(np.abs(g - e).max()))
    exp = np.stack(exp)
    scale = float(np.abs(exp).max())
    for mode in ("chunked", "split"):
        split = np.stack(runs[mode])
        assert float(np.abs(split - exp).max()) <= tol * scale, (mode, float(np.abs(split - exp).max()) / scale)
        assert np.array_equal(split.argmax(-1), exp.argmax(-1)), mode


@needs_ref
def test_c3_c4_qwen25_3b_prefill_512_then_decode(qwen25_3b_path):
    """512-token prompt in one 512-token batch (every projection on the GEMM), then 6 decode steps;
    the split attention within the reference tests' 1e-4 of the logit scale (tests/test_moe.py:297-299)."""
    _run_and_compare(qwen25_3b_path, 512, 512, 6, 640, seed=0, tol=1e-4)


def _default_engine_over_the_decode_benchmark(path, n_ctx, n_steps, tol):
    """The default engine over the decode benchmark's own sequence (bench.py's decode workloads: the
    model written with seed 0, uniform token ids from seed 0, the context in one batch, then n_steps
    one-token steps): each step within tol of the logit scale of the reference engine, with the same
    greedy token."""
    toks = np.random.default_rng(0).integers(0, 151936, n_ctx + n_steps).astype(np.int32)
    model = LoadedModel(path)
    s = model.session(max_seq=n_ctx + n_steps + 1, n_batch=n_ctx)
    s.feed(toks[:n_ctx])
    got = np.stack([s.step(int(t)) for t in toks[n_ctx:]])
    del s, model
    ref = O.RefEngine(path, n_ctx + n_steps + 1, n_batch=64)
    ref.eval(toks[:n_ctx])
    exp = np.stack([ref.eval([int(t)]) for t in toks[n_ctx:]])
    scale = float(np.abs(exp).max())
    err = np.abs(got - exp).max(axis=1) / scale
    assert float(err.max()) <= tol, (int(err.argmax()), float(err.max()), tol)
    assert np.array_equal(got.argmax(-1), exp.argmax(-1))


@needs_ref
def test_c3_default_engine_over_the_decode_benchmark(qwen25_3b_path):
    """The 3B default engine (the flash prompt attention, the chunked one-token attention) over the
    benchmark's 512-token prompt and 128 steps, each within 1e-4 of the logit scale. Over this many
    steps a rounding-level change of the prompt's attention can flip one activation's int8 rounding
    in a later layer and move a step's logits far past that bar, which six steps do not show."""
    _default_engine_over_the_decode_benchmark(qwen25_3b_path, 512, 128, 1e-4)


def fill_device_to(room):
    """Ballast allocations that leave about `room` bytes of device memory free (within 64 MiB): the
    free figure after an allocation can exceed the request's complement (allocation granularity,
    frees still being returned), so it is measured again and topped up."""
    L = capi.lib()
    free = ctypes.c_size_t()
    ballast = []
    for _ in range(4):
        capi.check(L.sdy_mem_info(ctypes.byref(free), None))
        if free.value <= room + (64 << 20):
            break
        ballast.append(capi.DeviceBuffer(free.value - room))
    capi.check(L.sdy_mem_info(ctypes.byref(free), None))
    assert room // 2 < free.value <= room + (64 << 20), (free.value, room)
    return ballast


def _pressure_child(path, room, toks_path, env, out_path):
    """The pressured load of a memory-pressure test, run in a process of its own: a ballast leaves
    `room` bytes free, then the model is loaded with the engine switches `env` (JSON) and fed the
    512-token prompt and one-token steps of toks_path; its logits and memory figures go to out_path.
    A fresh process because the runtime keeps device memory freed by earlier loads for its own
    reuse and reports it as used: a ballast sized in the same process leaves the next load more room
    than it measures."""
    L = capi.lib()
    capi.check(L.sdy_init())
    toks = np.load(toks_path)
    ballast = fill_device_to(int(room))
    with engine_env(**json.loads(env)):
        model = LoadedModel(path)
        s = model.session(max_seq=640, n_batch=512)
    out = np.stack([s.feed(toks[:512])] + [s.step(int(t)) for t in toks[512:]])
    np.savez(out_path, logits=out, **{k: np.int64(v) for k, v in model.memory().items()})
    del s, model, ballast


def run_pressured(path, room, toks, env, tmp):
    """_pressure_child in a child process; returns its logits and memory figures."""
    tp, op = Path(tmp) / "toks.npy", Path(tmp) / "pressured.npz"
    np.save(tp, toks)
    # (conftest puts the repository and the oracle's module directory on the path, as under pytest)
    code = ("import sys; sys.path.insert(0, sys.argv[1]); import conftest; import test_gpu_configs as t; "
            "t._pressure_child(*sys.argv[2:])")
    r = subprocess.run([sys.executable, "-c", code, str(TESTS), str(path), str(room), str(tp), json.dumps(env),
                        str(op)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, (r.returncode, r.stdout[-3000:], r.stderr[-3000:])
    d = np.load(op)
    return d["logits"], {k: int(d[k]) for k in d.files if k != "logits"}


def test_c3_loads_under_memory_pressure(qwen25_3b_path, tmp_path):
    """The Qwen2.5-3B-shaped model on a device with little room: a ballast allocation leaves free only
    the weights, half of the prefill GEMM's tiled copies and 512 MiB, so the weights are more than
    half of the memory left to the model. It loads, the copies are made for what fits (a 256 MiB
    reserve), and the 512-token prompt on the GEMM and two decode steps give the logits bits of the
    load with every copy (the exact attention chain in both; the pressured load in a process of
    its own, _pressure_child)."""
    L = capi.lib()
    capi.check(L.sdy_init())
    toks = np.random.default_rng(3).integers(0, 151936, 514).astype(np.int32)
    env = {"SARDYNE_ATTENTION": "exact", "SARDYNE_GEMM_RESERVE_MB": "256"}
    with engine_env(**env):
        model = LoadedModel(qwen25_3b_path)
        s = model.session(max_seq=640, n_batch=512)
    base = np.stack([s.feed(toks[:512]), s.step(int(toks[512])), s.step(int(toks[513]))])
    mem = model.memory()
    del s, model
    assert mem["gemm_copies"] > 0 and mem["gemm_copies_skipped"] == 0
    room = mem["weight_bytes"] + mem["gemm_copy_bytes"] // 2 + (512 << 20)
    got, mem2 = run_pressured(qwen25_3b_path, room, toks, env, tmp_path)
    assert mem2["weight_bytes"] == mem["weight_bytes"] and mem2["weight_bytes"] > room // 2
    assert mem2["gemm_copies_skipped"] > 0 and 0 < mem2["gemm_copy_bytes"] < mem["gemm_copy_bytes"]
    assert np.all(np.isfinite(base))
    assert np.array_equal(base.view(np.uint32), got.view(np.uint32))


# How far the reference's own AVX2 and scalar engines drift apart on the C5 model and tokens (they
# differ only in float summation orders): written by golden/make_c5_spread.py from the reference
# compiled from its sources. The split one-token attentions change f32 rounding only, and are held to
# SPREAD_MULTIPLE times the largest of that spread.
SPREAD_MULTIPLE = 2.0


def c5_tolerance():
    g = np.load(GOLDEN / "c5_simd_spread.npz")
    toks = np.random.default_rng(1).integers(0, 151936, 1024 + 5).astype(np.int32)
    assert str(g["tok_sha"]) == sha(toks), "the fixture was made for other tokens"
    assert int(g["n_ctx"]) == 1024 and int(g["n_steps"]) == 5 and int(g["model_seed"]) == 0
    assert bool(np.all(g["argmax_equal"]))
    return SPREAD_MULTIPLE * float(g["spread"].max()) / float(g["scale"])


@pytest.fixture(scope="module")
def qwen3_30b_a3b_path():
    p = _shm_model(qwen3_30b_a3b(), "qwen3_30b_a3b")
    yield p
    p.unlink(missing_ok=True)


@needs_ref
def test_c5_qwen3_30b_a3b_context_1024_then_decode(qwen3_30b_a3b_path):
    """48 layers of int8 activation rounding and top-8 routing amplify any change of f32 rounding: the
    exact chain gives the reference's bits, the chunked and split attentions stay within twice the
    reference's own AVX2-vs-scalar spread on this model and token sequence, with the same greedy
    tokens."""
    _run_and_compare(qwen3_30b_a3b_path, 1024, 512, 5, 1152, seed=1, tol=c5_tolerance())


@needs_ref
def test_c5_default_engine_over_the_decode_benchmark(qwen3_30b_a3b_path):
    """The 30B-A3B default engine (the flash prompt attention, the chunked one-token attention, the
    gate|up that routes each token itself) over the benchmark's 1024-token context and 128 steps,
    each within the tolerance derived from the reference's own AVX2-vs-scalar spread."""
    _default_engine_over_the_decode_benchmark(qwen3_30b_a3b_path, 1024, 128, c5_tolerance())


def test_c5_experts_beyond_the_device_memory(qwen3_30b_a3b_path, tmp_path):
    """The Qwen3-30B-A3B-shaped model on a device that holds about half of its expert stacks: a
    ballast allocation leaves free the attention and embedding weights, half the experts and a
    2 GiB reserve. The loader places each layer's experts on the device while the reserve stays
    free and the rest in pinned host memory, which the grouped GEMM and the device-routed decode
    read in place; a 512-token prompt and three decode steps give the logits bits of the load with
    every expert on the device (the exact attention chain in both; the pressured load in a process
    of its own, _pressure_child)."""
    L = capi.lib()
    capi.check(L.sdy_init())
    toks = np.random.default_rng(4).integers(0, 151936, 515).astype(np.int32)
    env = {"SARDYNE_ATTENTION": "exact", "SARDYNE_RESERVE_MB": "2048", "SARDYNE_GEMM_COPY_MB": "0"}
    with engine_env(**env):
        model = LoadedModel(qwen3_30b_a3b_path)
        s = model.session(max_seq=640, n_batch=512)
    base = np.stack([s.feed(toks[:512])] + [s.step(int(t)) for t in toks[512:]])
    mem = model.memory()
    del s, model
    assert mem["host_expert_layers"] == 0 and mem["host_expert_bytes"] == 0
    spec = qwen3_30b_a3b()
    room = mem["weight_bytes"] // 2 + (2048 << 20) + (256 << 20)
    got, mem2 = run_pressured(qwen3_30b_a3b_path, room, toks, env, tmp_path)
    assert 0 < mem2["host_expert_layers"] < spec.n_layer, mem2
    assert mem2["weight_bytes"] + mem2["host_expert_bytes"] == mem["weight_bytes"]
    assert np.all(np.isfinite(base))
    assert np.array_equal(base.view(np.uint32), got.view(np.uint32))

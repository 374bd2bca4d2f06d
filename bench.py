"""Benchmark of the quantized-weight matrix path on one MI355X.

Default workload (one JSON line on stdout): the Q6_K output-head matvec at batch 1, W = 151936 x
2048 in Q6_K super-blocks (255 MB), x ~ N(0, 1). One step = quantize x to Q8_K + the matvec over
one weight copy; 8 distinct copies (2 GB, well above the 256 MB Infinity Cache) are rotated so every
step streams its weights from HBM. value = algorithmic bytes per step / step time.

Other workloads (--workload): q8_0_head (the Q8_0 matvec of the same shape), q4k_matvec (2048 x
2048 Q4_K, measured as one launch over 448 stacked copies), decode_3b (Qwen2.5-3B-shaped Q4_K_M
decode tok/s, 128 tokens after a 512-token context), decode_moe (Qwen3-30B-A3B-shaped MoE decode,
128 tokens after a 1024-token context), decode_moe_host (the same with the expert stacks in pinned
host memory, the placement of a model larger than the device), prefill_3b (one 512-token prompt through the
Qwen2.5-3B-shaped model), grid_barrier (the per-phase synchronisation a persistent decode kernel
would pay, against the kernel boundary).

Every line carries:
  roofline      the dominant kernel's algorithmic bytes / its average duration (HIP events on the
                stream it runs on), against MI355X's 8 TB/s HBM peak;
  cpu_baseline  the reference's own CPU code (compiled from its sources into oracle/_ref) timed
                on this host's cores on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import dataclasses
import ctypes
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))

from sardyne_amd import capi  # noqa: E402
from sardyne_amd.gguf_synth import random_blocks  # noqa: E402

METRIC = "Q4_K/Q6_K matvec GB/s (% of HBM peak); decode tok/s, Qwen2.5-3B shape"
HBM_PEAK_GBPS = 8000.0
PCIE5_X16_GBPS = 64.0  # the host link, one direction (PCIe 5.0 x16)
Q4_K, Q6_K, Q8_0, Q8_K = 12, 14, 8, 15
BLOCK = {Q4_K: (256, 144), Q6_K: (256, 210), Q8_0: (32, 34), Q8_K: (256, 292)}


def row_size(t, n):
    e, b = BLOCK[t]
    return n // e * b


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Events:
    def __init__(self, stream):
        self.L = capi.lib()
        self.s = stream
        self.e0, self.e1 = ctypes.c_void_p(), ctypes.c_void_p()
        capi.check(self.L.sdy_event_new(ctypes.byref(self.e0)))
        capi.check(self.L.sdy_event_new(ctypes.byref(self.e1)))

    def start(self):
        capi.check(self.L.sdy_event_record(self.e0, self.s))

    def stop_ms(self):
        capi.check(self.L.sdy_event_record(self.e1, self.s))
        ms = ctypes.c_float()
        capi.check(self.L.sdy_event_elapsed(ctypes.byref(ms), self.e0, self.e1))
        return ms.value


def per_launch_ms(stream, launch, n):
    """Average duration (ms) of n back-to-back launches on `stream` (the stream the kernel runs on):
    one HIP event before the first and one after the last, so the figure is the kernels' own time
    plus the (small) gaps between consecutive dispatches, without per-launch event overhead."""
    L = capi.lib()
    e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
    capi.check(L.sdy_event_new(ctypes.byref(e0)))
    capi.check(L.sdy_event_new(ctypes.byref(e1)))
    capi.check(L.sdy_event_record(e0, stream))
    for i in range(n):
        launch(i)
    capi.check(L.sdy_event_record(e1, stream))
    ms = ctypes.c_float()
    capi.check(L.sdy_event_elapsed(ctypes.byref(ms), e0, e1))
    for e in (e0, e1):
        capi.check(L.sdy_event_free(e))
    return ms.value / n


def profiled_traffic(name):
    """HBM bytes per launch of a kernel (or per decode token of a step), from the PMC summary committed
    under profiles/ (FETCH_SIZE and WRITE_SIZE scaled by copy-kernel calibration); None when absent."""
    p = ROOT / "profiles" / name
    try:
        for line in p.read_text().splitlines():
            if line.startswith(("traffic_bytes_per_launch:", "traffic_bytes_per_token:")):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def membw_probe(stream, gib=4):
    """The GPU's HBM read rate for a pure read stream (sdy_membw_read) over a gib-GiB buffer, GB/s."""
    L = capi.lib()
    n = gib << 30
    buf = capi.DeviceBuffer(n)
    sink = capi.DeviceBuffer(64)
    capi.check(L.sdy_memset(buf.ptr, 1, n, stream))
    ev = Events(stream)
    for _ in range(2):
        capi.check(L.sdy_membw_read(buf.ptr, n, sink.ptr, stream))
    ev.start()
    for _ in range(5):
        capi.check(L.sdy_membw_read(buf.ptr, n, sink.ptr, stream))
    ms = ev.stop_ms()
    buf.close()
    return 5 * n / (ms * 1e-3) / 1e9


# ---------------------------------------------------------------- CPU baseline (reference code)

def cpu_matvec_baseline(wt, w_copies, x, n_in, seconds, n_threads):
    """The reference's own matmul() for one token: op_quantize_rows, then op_matmul_q_rows with the
    rows split evenly over its thread pool (tp_run, a barrier after each op;
    csrc/model_llama.c:569-611, csrc/threadpool.c:68-141), rotating the weight copies.
    n_threads 0 = the reference's default (the online CPUs). Returns (seconds per rep, reps, threads)."""
    import oracle as O
    return O.ref_cpu_matvec(wt, w_copies, x, n_in, seconds, n_threads)


def host_membw(max_threads=None):
    """Host read bandwidth from the reference's own tool (tools/membw.c with its thread pool, built
    into oracle/_ref/membw): a 512 MB buffer summed with AVX2 by 1..N threads, best of 5 each.
    Returns {"1": GB/s at one thread, "best": GB/s, "best_threads": n, "threads_swept": N} or None."""
    import subprocess
    exe = ROOT / "oracle" / "_ref" / "membw"
    if not exe.exists():
        return None
    n = max_threads or min(os.cpu_count() or 1, 64)
    try:
        out = subprocess.run([str(exe), "512", str(n)], capture_output=True, text=True, timeout=120).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    rows = {}
    for line in out.splitlines():
        f = line.split()
        if len(f) == 2 and f[0].isdigit():
            rows[int(f[0])] = float(f[1])
    if not rows:
        return None
    bt = max(rows, key=rows.get)
    return {"1": rows.get(1), "best": rows[bt], "best_threads": bt, "threads_swept": n,
            "tool": "the reference's tools/membw.c (AVX2 read, 512 MB)"}


def host_cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------- matvec workloads

def bench_matvec(args, wt, n_out, n_in, n_copies, stacked):
    L = capi.lib()
    stream = ctypes.c_void_p()
    capi.check(L.sdy_stream_new(ctypes.byref(stream)))
    st = stream.value
    name = {Q6_K: "Q6_K", Q4_K: "Q4_K", Q8_0: "Q8_0"}[wt]
    e, _ = BLOCK[wt]
    vt = Q8_K if wt in (Q4_K, Q6_K) else Q8_0
    rng = np.random.default_rng(0)
    log(f"[bench] generating {name} {n_out}x{n_in} (seed 0)")
    w0 = random_blocks(name, n_out * n_in // e, rng).reshape(n_out, -1)
    x = np.random.default_rng(1).standard_normal(n_in).astype(np.float32)
    w_bytes = w0.nbytes
    algo_bytes = w_bytes + n_in * 4 + n_out * 4

    # device copies: distinct bytes per copy (a different seed per copy), rotated per step
    mats = []
    if stacked:
        # one matrix of n_copies * n_out rows: each copy is an independent n_out x n_in matvec
        rows = []
        for c in range(n_copies):
            rows.append(w0 if c == 0 else random_blocks(name, n_out * n_in // e, np.random.default_rng(100 + c)).reshape(n_out, -1))
        big = np.concatenate(rows)
        mats.append(capi.DeviceMatrix(wt, n_in, n_out * n_copies, big, st))
        del big, rows
    else:
        for c in range(n_copies):
            wc = w0 if c == 0 else random_blocks(name, n_out * n_in // e, np.random.default_rng(100 + c)).reshape(n_out, -1)
            mats.append(capi.DeviceMatrix(wt, n_in, n_out, wc, st))
    log(f"[bench] uploaded {len(mats)} device matrices ({sum(m.m.bytes for m in mats) / 1e9:.2f} GB)")
    dx = capi.DeviceBuffer.from_array(x, st)
    dq = capi.DeviceBuffer(row_size(vt, n_in))
    out_rows = n_out * (n_copies if stacked else 1)
    dout = capi.DeviceBuffer(out_rows * 4)

    def fused_args(m):
        a = capi.SdyMvArgs(n_tok=1, out=dout.ptr, out_stride=out_rows, row0=0, row1=m.n_rows)
        a.x, a.eps = dx.ptr, 0.0
        return a

    # K-quant weights: one launch whose workgroups quantise the f32 row themselves (the reference's
    # matmul() quantises the activation, then runs the dots); Q8_0: the quantiser's launch, then the
    # matvec on its bytes
    fused = wt in (Q4_K, Q6_K) and L.sdy_matvec_fused_ok(ctypes.byref(mats[0].m), ctypes.byref(fused_args(mats[0])),
                                                          None, None) == 1

    def step(i):
        m = mats[0] if stacked else mats[i % len(mats)]
        if fused:
            capi.check(L.sdy_matvec(ctypes.byref(m.m), ctypes.byref(fused_args(m)), st))
            return
        capi.check(L.sdy_quantize(vt, dx.ptr, dq.ptr, n_in, 1, st))
        a = capi.SdyMvArgs(xq=dq.ptr, n_tok=1, out=dout.ptr, out_stride=out_rows, row0=0, row1=m.n_rows)
        capi.check(L.sdy_matvec(ctypes.byref(m.m), ctypes.byref(a), st))

    def matvec_only(i):
        m = mats[0] if stacked else mats[i % len(mats)]
        if fused:
            capi.check(L.sdy_matvec(ctypes.byref(m.m), ctypes.byref(fused_args(m)), st))
            return
        a = capi.SdyMvArgs(xq=dq.ptr, n_tok=1, out=dout.ptr, out_stride=out_rows, row0=0, row1=m.n_rows)
        capi.check(L.sdy_matvec(ctypes.byref(m.m), ctypes.byref(a), st))

    # parity spot check: the first copy's first 512 rows against the oracle
    step(0)
    capi.check(L.sdy_sync(st))
    y = dout.to_array(np.float32, out_rows, st)
    parity = {}
    try:
        import oracle as O
        if O.available():
            k = min(512, n_out)
            xq = O.quantize(x, vt)
            exp = O.matmul_q(w0[:k], wt, xq, n_in, simd=1)[0]
            if wt in (Q4_K, Q6_K):
                parity = {"rows_checked": k, "bit_exact": bool(np.array_equal(exp.view(np.uint32), y[:k].view(np.uint32)))}
            else:
                rel = float(np.linalg.norm(y[:k] - exp) / np.linalg.norm(exp))
                parity = {"rows_checked": k, "rel_l2_vs_reference_avx2": rel}
    except Exception as ex:  # parity is informative here; the tests are the gate
        parity = {"error": str(ex)}

    ev = Events(st)
    for i in range(args.warmup):
        step(i)
    capi.check(L.sdy_sync(st))
    ev.start()
    for i in range(args.steps):
        step(i)
    ms_total = ev.stop_ms()
    ms_step = ms_total / args.steps
    units = n_copies if stacked else 1
    value = algo_bytes * units / (ms_step * 1e-3) / 1e9

    # dominant kernel alone: each launch bracketed by its own event pair on the kernel's stream,
    # so the average is the launch duration without the gaps between dispatches
    for i in range(3):
        matvec_only(i)
    kernel = L.sdy_last_kernel().decode() or "k_matvec"
    ms_k = per_launch_ms(st, matvec_only, args.steps)
    algo_launch = w_bytes * units + n_in * 4 + n_out * 4 * units
    achieved = algo_launch / (ms_k * 1e-3) / 1e9
    traffic = profiled_traffic(f"k_matvec_{name.lower()}_{'stacked' if stacked else 'head'}.md")
    achievable = membw_probe(st)
    # the read probes over the matrices themselves, one launch per copy in rotation, back to back: a
    # pure read stream of this launch size, with the per-launch ramp and tail the matvec also pays
    # (the faster of the two read orders)
    sink = capi.DeviceBuffer(64)
    achievable_launch = 0.0
    for probe in (L.sdy_membw_read, L.sdy_membw_read_strided):
        def read_copy(i, probe=probe):
            m = mats[i % len(mats)]
            capi.check(probe(ctypes.c_void_p(m.m.base), m.m.bytes, sink.ptr, st))

        for i in range(len(mats)):
            read_copy(i)
        ms_r = per_launch_ms(st, read_copy, max(args.steps, 8 * len(mats)))
        achievable_launch = max(achievable_launch, mats[0].m.bytes / (ms_r * 1e-3) / 1e9)
    back_to_back = None
    if stacked:
        # the same copies as separate n_out x n_in matrices (row views of the stack, each its own region
        # of HBM), one launch per copy, back to back in rotation: per-launch time includes the
        # dispatch gaps that a 2.4 MB matvec cannot hide
        capi.check(L.sdy_quantize(vt, dx.ptr, dq.ptr, n_in, 1, st))  # (the views read the quantised row)
        views = [L.sdy_mat_rows(ctypes.byref(mats[0].m), c * n_out, n_out) for c in range(n_copies)]
        vargs = capi.SdyMvArgs(xq=dq.ptr, n_tok=1, out=dout.ptr, out_stride=n_out, row0=0, row1=n_out)

        def one_copy(i):
            capi.check(L.sdy_matvec(ctypes.byref(views[i % n_copies]), ctypes.byref(vargs), st))

        for i in range(n_copies):
            one_copy(i)
        n_launch = n_copies * max(1, args.steps // 10)
        ms_b = per_launch_ms(st, one_copy, n_launch)
        per = w_bytes + n_in * 4 + n_out * 4
        # the same launches recorded once as a graph and replayed (no host work between them: what a
        # caller that replays its step, as the engine does, pays per launch)
        ms_g = None
        ex = ctypes.c_void_p()
        if L.sdy_graph_begin(st) == 0:
            for i in range(n_copies):
                one_copy(i)
            if L.sdy_graph_end(st, ctypes.byref(ex)) == 0:
                capi.check(L.sdy_graph_launch(ex, st))
                reps = max(1, args.steps // 10)
                ms_g = per_launch_ms(st, lambda _: capi.check(L.sdy_graph_launch(ex, st)), reps) / n_copies
                capi.check(L.sdy_graph_free(ex))
        back_to_back = {"launches": n_launch, "distinct_copies": n_copies, "per_launch_us": round(ms_b * 1e3, 3),
                        "GBps": round(per / (ms_b * 1e-3) / 1e9, 1),
                        "frac_of_hbm_peak": round(per / (ms_b * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                        "kernel": L.sdy_last_kernel().decode()}
        if ms_g:
            back_to_back["graph_replay"] = {"per_launch_us": round(ms_g * 1e3, 3),
                                            "GBps": round(per / (ms_g * 1e-3) / 1e9, 1),
                                            "frac_of_hbm_peak": round(per / (ms_g * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}

    # CPU baseline: the reference's code on this host (all online CPUs, and 1 thread)
    cpu = None
    if args.cpu_seconds > 0:
        try:
            import oracle as O
            if O.ref_available():
                # at least 2 GB of distinct copies, beyond the host's last-level cache
                n_cpu_copies = min(max(2, int(np.ceil(2e9 / w_bytes))), 1024)
                copies = [w0] + [random_blocks(name, n_out * n_in // e, np.random.default_rng(200 + c)).reshape(n_out, -1)
                                 for c in range(n_cpu_copies - 1)]
                dt, reps, n_cpu = cpu_matvec_baseline(wt, copies, x, n_in, args.cpu_seconds, 0)
                dt1, _, _ = cpu_matvec_baseline(wt, copies, x, n_in, max(2.0, args.cpu_seconds / 4), 1)
                cpu = {"value": round(algo_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": n_cpu, "kind": "reference",
                       "sample": f"{reps} reps of the reference's matmul() (quantize + row split on its thread pool) "
                                 f"over {len(copies)} rotated copies ({dt * 1e3:.3f} ms/rep), {host_cpu_model()}",
                       "single_thread_GBps": round(algo_bytes / dt1 / 1e9, 3)}
        except Exception as ex:
            cpu = {"error": str(ex)}

    cfg = {"workload": f"{name} matvec, batch 1, W {n_out}x{n_in}" + (f" x {n_copies} stacked copies" if stacked else
                                                                       f", {n_copies} rotated copies"),
           "weight_type": name, "n_out": n_out, "n_in": n_in, "copies": n_copies,
           "algorithmic_bytes_per_matvec": algo_bytes,
           "step": "one launch quantising the f32 row in its workgroups" if fused else "quantiser launch + matvec"}
    line = {"metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "int8 (Q8_K activations x 6-bit weights, int32 dots, f32 combine)"
            if wt == Q6_K else "int8", "data": "synthetic (seeded random quantized blocks, x ~ N(0,1))",
            "config": cfg, "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBPS, 2),
            "achievable_hbm_GBps": round(achievable, 1),
            "achievable_hbm_GBps_at_launch_size": round(achievable_launch, 1),
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                         "kernel": kernel, "kernel_avg_us": round(ms_k * 1e3, 3),
                         "algorithmic_bytes_per_launch": algo_launch},
            "cpu_baseline": cpu, "parity": parity}
    if back_to_back:
        line["back_to_back"] = back_to_back
    if cpu and "value" in cpu:
        line["gpu_over_cpu"] = round(value / cpu["value"], 1)
    return line


# ---------------------------------------------------------------- decode workloads

def decode_weight_bytes(spec):
    """Weight bytes one decode token reads: per layer the attention matrices, norms and biases, the
    dense FFN or the router plus the k chosen experts' gate/up/down; then the final norm, the output
    head (the tied embedding when there is none) and one embedding row."""
    from sardyne_amd.gguf_synth import row_bytes
    dim, hd = spec.dim, spec.head_dim
    q_dim, kv_dim = spec.n_head * hd, spec.n_kv_head * hd
    td = spec.t_default
    layer = (q_dim * row_bytes(td, dim) + kv_dim * row_bytes(td, dim) + kv_dim * row_bytes(spec.t_attn_v, dim)
             + dim * row_bytes(td, q_dim) + 2 * dim * 4)
    if spec.qkv_bias:
        layer += (q_dim + 2 * kv_dim) * 4
    if spec.qk_norm:
        layer += 2 * hd * 4
    if spec.n_expert:
        fe = spec.ffn_exp_dim
        layer += spec.n_expert * dim * 4 + spec.n_expert_used * (
            2 * fe * row_bytes(td, dim) + dim * row_bytes(spec.t_ffn_down, fe))
    else:
        layer += 2 * spec.ffn_dim * row_bytes(td, dim) + dim * row_bytes(spec.t_ffn_down, spec.ffn_dim)
    head = spec.n_vocab * row_bytes(spec.t_embd if spec.tied else spec.t_output, dim)
    return spec.n_layer * layer + head + dim * 4 + row_bytes(spec.t_embd, dim)


def routed_expert_bytes(spec):
    """Weight bytes of the k routed experts one decode token reads (gate, up and down, every layer)."""
    from sardyne_amd.gguf_synth import row_bytes
    fe = spec.ffn_exp_dim
    return spec.n_layer * spec.n_expert_used * (2 * fe * row_bytes(spec.t_default, spec.dim)
                                                + spec.dim * row_bytes(spec.t_ffn_down, fe))


def host_link_read_GBps(stream, gib=4):
    """The GPU's read rate of pinned host memory: the HBM probe kernel over a buffer the engine would
    hold host-resident experts in (sdy_host_alloc_mapped), best of 3."""
    L = capi.lib()
    h, d = ctypes.c_void_p(), ctypes.c_void_p()
    n = gib << 30
    capi.check(L.sdy_host_alloc_mapped(ctypes.byref(h), ctypes.byref(d), n))
    sink = capi.DeviceBuffer(64)
    try:
        capi.check(L.sdy_memset(d, 0, n, stream))
        ev = Events(stream)
        best = 0.0
        for _ in range(3):
            ev.start()
            capi.check(L.sdy_membw_read(d, n, sink.ptr, stream))
            best = max(best, n / (ev.stop_ms() * 1e-3) / 1e9)
        return best
    finally:
        capi.check(L.sdy_sync(stream))
        capi.check(L.sdy_host_free(h))


def engine_modes():
    """The engine's one-token attention and KV-cache type, as engine_ctx_new reads them."""
    return (os.environ.get("SARDYNE_ATTENTION") or "chunked"), (os.environ.get("SARDYNE_KV") or "f32")


def kv_bytes_per_position(spec):
    elt = 2 if engine_modes()[1] == "f16" else 4
    return 2 * spec.n_layer * spec.n_kv_head * spec.head_dim * elt


def keep_models():
    """SARDYNE_BENCH_KEEP=1: model files are kept after the run and reused by the next one (several
    profiler passes over one workload write the file once)."""
    return os.environ.get("SARDYNE_BENCH_KEEP", "0") not in ("", "0")


def write_bench_model(spec, label):
    from sardyne_amd.gguf_synth import write_model
    tmpdir = Path(os.environ.get("SARDYNE_BENCH_DIR", "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()))
    path = tmpdir / f"sardyne_bench_{label}_{spec.n_layer}l_{spec.scales}.gguf"
    if keep_models() and path.exists():
        log(f"[bench] reusing {path}")
        return path
    t0 = time.perf_counter()
    write_model(path, spec, seed=0)
    log(f"[bench] wrote {path} ({path.stat().st_size / 1e9:.2f} GB) in {time.perf_counter() - t0:.1f}s")
    return path


def drop_bench_model(path):
    if not keep_models():
        path.unlink(missing_ok=True)

def bench_decode(args, spec, ctx_len, n_decode, label, path=None):
    """Decode tok/s after a ctx_len-token context at batch 1 (the method of the reference's
    bench/bench_decode.py:39-48: n_decode / wall time of the decode loop, each step's logits
    returned as a fresh array and dropped). Token ids are uniform over the vocabulary (seeded) and
    fed teacher-forced, so the GPU and the CPU reference see the same sequence; an untimed rerun of
    the same steps keeps the logits, which are compared step by step. The same steps with the f16 KV cache
    (SARDYNE_KV=f16) are compared with the f32 reference too. path: a model file written already
    (kept), else one is written and deleted."""
    from sardyne_amd.engine import LoadedModel
    own_file = path is None
    if own_file:
        path = write_bench_model(spec, label)
    rng = np.random.default_rng(0)
    toks = rng.integers(0, spec.n_vocab, ctx_len + n_decode).astype(np.int32)
    t0 = time.perf_counter()
    model = LoadedModel(path)
    t_load = time.perf_counter() - t0
    mem = model.memory()
    log(f"[bench] GPU model load {t_load:.2f}s")
    n_batch = args.n_batch or ctx_len
    ctx = model.session(max_seq=ctx_len + n_decode + 1, n_batch=n_batch)
    ctx.feed(toks[:ctx_len])  # the prompt kernels' first launches (code loading), untimed
    ctx.clear()
    t0 = time.perf_counter()
    ctx.feed(toks[:ctx_len])
    t_prefill = time.perf_counter() - t0
    # the timed loop drops each step's logits, as the reference's loop does (bench/bench_decode.py:
    # 44-45: every call still returns a fresh copy); kept, the 128 arrays of 608 KB (3B) would add
    # the first-touch faults of fresh memory to every step
    t0 = time.perf_counter()
    for i in range(n_decode):
        last = ctx.feed([int(toks[ctx_len + i])])
    t_dec = time.perf_counter() - t0
    gpu_tok_s = n_decode / t_dec
    log(f"[bench] GPU prefill {ctx_len} tok in {t_prefill:.3f}s, decode {gpu_tok_s:.1f} tok/s")
    # the same prompt and steps again, untimed, keeping every step's logits for the comparison with
    # the reference; the timed run's last step must carry the same bits
    ctx.clear()
    ctx.feed(toks[:ctx_len])
    gpu_logits = [ctx.feed([int(toks[ctx_len + i])]) for i in range(n_decode)]
    rerun_same_bits = bool(np.array_equal(gpu_logits[-1].view(np.uint32), last.view(np.uint32)))
    if not rerun_same_bits:
        log("[bench] decode: the untimed rerun's last logits differ from the timed run's")
    del ctx
    # the same prompt and steps with the f16 cache (untimed: its drift from the f32 reference)
    f16_logits = []
    # (only when the reference runs beside it: the drift is measured against its logits; the split
    # form has no f16 cache)
    if args.cpu_seconds > 0 and engine_modes() in (("chunked", "f32"), ("exact", "f32")):
        saved = os.environ.get("SARDYNE_KV")
        os.environ["SARDYNE_KV"] = "f16"
        try:
            ctx = model.session(max_seq=ctx_len + n_decode + 1, n_batch=n_batch)
        finally:
            if saved is None:
                os.environ.pop("SARDYNE_KV", None)
            else:
                os.environ["SARDYNE_KV"] = saved
        ctx.feed(toks[:ctx_len])
        f16_logits = [ctx.feed([int(toks[ctx_len + i])]) for i in range(n_decode)]
        del ctx
    del model
    cpu = None
    parity = {}
    if args.cpu_seconds > 0:
        try:
            import oracle as O
            if O.ref_available():
                eng = O.RefEngine(path, ctx_len + n_decode + 1, n_batch=64, n_threads=0)
                t0 = time.perf_counter()
                eng.eval(toks[:ctx_len])
                t_pre_cpu = time.perf_counter() - t0
                n_cpu_steps, cpu_logits = 0, []
                t0 = time.perf_counter()
                while n_cpu_steps < n_decode and (time.perf_counter() - t0 < args.cpu_seconds or n_cpu_steps < 4):
                    cpu_logits.append(eng.eval([int(toks[ctx_len + n_cpu_steps])]))
                    n_cpu_steps += 1
                t_cpu = time.perf_counter() - t0
                n_thr = eng.n_threads
                del eng
                # one thread (bounded: a 16-token context, then a few steps)
                eng1 = O.RefEngine(path, 64, n_batch=16, n_threads=1)
                eng1.eval(toks[:16])
                n1 = 0
                t0 = time.perf_counter()
                while n1 < 32 and (time.perf_counter() - t0 < max(2.0, args.cpu_seconds / 4) or n1 < 2):
                    eng1.eval([int(toks[16 + n1])])
                    n1 += 1
                t1 = time.perf_counter() - t0
                del eng1
                cpu = {"value": round(n_cpu_steps / t_cpu, 3), "unit": "tok/s", "cores": n_thr,
                       "kind": "reference",
                       "sample": f"reference engine, {n_cpu_steps} decode steps after a {ctx_len}-token prefill "
                                 f"(prefill {ctx_len / t_pre_cpu:.1f} tok/s, n_batch 64), {host_cpu_model()}",
                       "single_thread": {"value": round(n1 / t1, 3), "unit": "tok/s",
                                         "sample": f"{n1} decode steps after a 16-token context (one thread)"}}
                hb = host_membw()
                if hb:
                    cpu["host_read_GBps"] = hb
                g = np.stack(gpu_logits[:n_cpu_steps])
                c = np.stack(cpu_logits)
                scale = float(np.abs(c).max())
                maxabs = float(np.abs(g - c).max())
                parity = {"steps_compared": n_cpu_steps, "timed_run_last_step_same_bits": rerun_same_bits,
                          "logits_max_abs": maxabs,
                          "logits_max_abs_over_max_ref": maxabs / scale,
                          "greedy_argmax_agreement": float(np.mean(g.argmax(-1) == c.argmax(-1)))}
                if f16_logits:
                    h = np.stack(f16_logits[:n_cpu_steps])
                    d = float(np.abs(h - c).max())
                    parity["kv_f16_vs_f32_reference"] = {
                        "logits_max_abs": d, "logits_max_abs_over_max_ref": d / scale,
                        "rel_l2": float(np.linalg.norm(h - c) / np.linalg.norm(c)),
                        "greedy_argmax_agreement": float(np.mean(h.argmax(-1) == c.argmax(-1)))}
        except Exception as ex:
            cpu = {"error": str(ex)}
    size = path.stat().st_size
    load = {"s": round(t_load, 3), "file_bytes": size, "gb_per_s": round(size / t_load / 1e9, 2),
            "device_weight_bytes": mem["weight_bytes"], "gemm_copy_bytes": mem["gemm_copy_bytes"],
            "gemm_copies": mem["gemm_copies"], "gemm_copies_skipped": mem["gemm_copies_skipped"],
            "host_expert_bytes": mem["host_expert_bytes"], "host_expert_layers": mem["host_expert_layers"],
            "upload": "synchronous per tensor" if os.environ.get("SARDYNE_UPLOAD_SYNC", "0") not in ("", "0")
            else "pipelined (4 x 64 MiB pinned slots)",
            "file": "tmpfs" if str(path).startswith("/dev/shm") else "disk"}
    if own_file:
        drop_bench_model(path)
    return gpu_tok_s, t_prefill, cpu, parity, load


# the decode profiles under profiles/ (their per-token PMC traffic), by workload label
DECODE_PROFILE = {"qwen25_3b": "decode_qwen25_3b.md", "qwen3_30b_a3b": "decode_qwen3_30b_a3b_moe.md"}


def decode_line(args, spec, label, ctx_len, desc, n_dec=None, path=None):
    n_dec = n_dec or max(args.steps, 8)
    tok_s, t_pre, cpu, parity, load = bench_decode(args, spec, ctx_len, n_dec, label, path)
    w_bytes = decode_weight_bytes(spec)
    kv_mean = kv_bytes_per_position(spec) * (ctx_len + n_dec / 2)
    gbps = (w_bytes + kv_mean) * tok_s / 1e9
    cfg = {"workload": f"{desc} decode, batch 1, {n_dec} tokens after a {ctx_len}-token context",
           "n_layer": spec.n_layer, "dim": spec.dim, "heads": f"{spec.n_head}/{spec.n_kv_head}",
           "vocab": spec.n_vocab, "weight_bytes_per_token": w_bytes, "mean_kv_bytes_per_token": int(kv_mean),
           "attention": engine_modes()[0], "kv_cache": engine_modes()[1]}
    if spec.n_expert:
        cfg.update({"experts": f"{spec.n_expert} (top-{spec.n_expert_used})", "expert_ffn": spec.ffn_exp_dim})
    else:
        cfg["ffn"] = spec.ffn_dim
    line = {"metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": n_dec,
            "warmup": 0, "ms_per_step": round(1e3 / tok_s, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "int8 activations x Q4_K/Q6_K weights, f32 elsewhere",
            "data": "synthetic (random-init Q4_K_M weights, uniform token ids)", "config": cfg,
            f"prefill_{ctx_len}_s": round(t_pre, 4),
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": profiled_traffic(DECODE_PROFILE.get(label, f"decode_{label}.md")),
                         "traffic_unit": "HBM bytes per decode token (PMC, profiles/)",
                         "kernel": "whole decode step (weights + mean KV bytes per token)"},
            "cpu_baseline": cpu, "parity": parity, "model_load": load}
    if cpu and "value" in cpu:
        line["gpu_over_cpu"] = round(tok_s / cpu["value"], 1)
    return line


def prefill_flops(spec, n):
    """GEMM flops of an n-token prefill (2 n x matrix parameters, head for the last token only)
    plus the causal attention's QK and PV flops."""
    dim, hd = spec.dim, spec.head_dim
    q_dim, kv_dim = spec.n_head * hd, spec.n_kv_head * hd
    params = dim * q_dim * 2 + dim * kv_dim * 2 + 3 * dim * spec.ffn_dim
    attn = spec.n_layer * spec.n_head * 2 * 2 * hd * (n * (n + 1) // 2)
    return 2 * n * params * spec.n_layer + 2 * spec.n_vocab * dim + attn


def gemm_gate_up_ms(spec, n_tok, reps):
    """The prefill's dominant kernel at its real shape: the interleaved gate|up Q4_K matrix
    (2 ffn x dim) times n_tok Q8_K rows with the SwiGLU epilogue, each launch timed by its own
    HIP event pair on the stream it runs on."""
    L = capi.lib()
    stream = ctypes.c_void_p()
    capi.check(L.sdy_stream_new(ctypes.byref(stream)))
    st = stream.value
    rows, n_in = 2 * spec.ffn_dim, spec.dim
    w = random_blocks("Q4_K", rows * n_in // 256, np.random.default_rng(3), spec.scales).reshape(rows, -1)
    m = capi.DeviceMatrix(Q4_K, n_in, rows, w, st)
    if not L.sdy_gemm_ok(ctypes.byref(m.m), n_tok):
        return None
    x = np.random.default_rng(4).standard_normal((n_tok, n_in)).astype(np.float32)
    dx = capi.DeviceBuffer.from_array(x, st)
    dq = capi.DeviceBuffer(n_tok * row_size(Q8_K, n_in))
    capi.check(L.sdy_quantize(Q8_K, dx.ptr, dq.ptr, n_in, n_tok, st))
    ws = capi.DeviceBuffer(L.sdy_gemm_ws_bytes(n_tok, n_in))
    dout = capi.DeviceBuffer(n_tok * spec.ffn_dim * 4)
    a = capi.SdyMvArgs(xq=dq.ptr, n_tok=n_tok, out=dout.ptr, out_stride=spec.ffn_dim, row0=0, row1=rows,
                       epilogue=capi.EPI_SWIGLU)

    def launch(_):
        capi.check(L.sdy_gemm(ctypes.byref(m.m), ctypes.byref(a), ws.ptr, st))

    launch(0)  # makes the activations' f16 expansion in ws; the timed launches reuse it (GEMM alone)
    a.ws_ready = 1
    for i in range(2):
        launch(i)
    kernel = L.sdy_last_kernel().decode()
    return per_launch_ms(st, launch, reps), 2.0 * rows * n_in * n_tok, kernel


def prefill_line(args, spec, label, n_prompt, desc, path=None):
    """Prefill tok/s of one n_prompt-token eval (n_batch = n_prompt), the median over --steps
    fresh evals, with the whole prefill's MFMA utilisation and the dominant GEMM's roofline. path: a
    model file written already (kept), else one is written and deleted."""
    from sardyne_amd.engine import LoadedModel
    MFMA_PEAK = 2500.0  # TFLOP/s, dense f16/bf16
    own_file = path is None
    if own_file:
        path = write_bench_model(spec, label)
    toks = np.random.default_rng(0).integers(0, spec.n_vocab, n_prompt).astype(np.int32)
    model = LoadedModel(path)
    ctx = model.session(max_seq=n_prompt + 1, n_batch=n_prompt)
    for _ in range(max(1, args.warmup)):
        ctx.clear()
        gpu_logits = ctx.feed(toks)
    times = []
    for _ in range(args.steps):
        ctx.clear()
        t0 = time.perf_counter()
        ctx.feed(toks)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    tok_s = n_prompt / t
    log(f"[bench] GPU prefill {n_prompt} tok: {t * 1e3:.2f} ms median of {len(times)} ({tok_s:.0f} tok/s)")
    del ctx, model
    flops = prefill_flops(spec, n_prompt)
    k = gemm_gate_up_ms(spec, n_prompt, args.steps)
    roof = None
    if k:
        ms_k, fl, kname = k
        ach = fl / (ms_k * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 2), "peak": MFMA_PEAK, "unit": "TFLOP/s",
                "frac": round(ach / MFMA_PEAK, 4), "traffic": None, "kernel": f"{kname} (gate|up, SwiGLU)",
                "kernel_avg_us": round(ms_k * 1e3, 2), "algorithmic_flops_per_launch": fl}
    cpu, parity = None, {}
    if args.cpu_seconds > 0:
        try:
            import oracle as O
            if O.ref_available():
                eng = O.RefEngine(path, n_prompt + 1, n_batch=n_prompt, n_threads=0)
                t0 = time.perf_counter()
                c = eng.eval(toks)
                t_cpu = time.perf_counter() - t0
                cpu = {"value": round(n_prompt / t_cpu, 3), "unit": "tok/s", "cores": eng.n_threads,
                       "kind": "reference", "sample": f"reference engine, one {n_prompt}-token prefill "
                                                      f"(n_batch {n_prompt}), {host_cpu_model()}"}
                maxabs = float(np.abs(gpu_logits - c).max())
                parity = {"logits_max_abs": maxabs, "logits_max_abs_over_max_ref": maxabs / float(np.abs(c).max()),
                          "greedy_argmax_agreement": float(gpu_logits.argmax() == c.argmax())}
        except Exception as ex:
            cpu = {"error": str(ex)}
    if own_file:
        drop_bench_model(path)
    line = {"metric": METRIC, "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(t * 1e3, 3), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "int8 activations x Q4_K/Q6_K weights on f16 MFMA (exact integer sums)",
            "data": "synthetic (random-init Q4_K_M weights, uniform token ids)",
            "config": {"workload": f"{desc} prefill, one {n_prompt}-token prompt", "n_layer": spec.n_layer,
                       "dim": spec.dim, "ffn": spec.ffn_dim, "vocab": spec.n_vocab, "flops": flops,
                       "kquant_scales": spec.scales},
            "mfma_utilisation": round(flops / t / 1e12 / MFMA_PEAK, 4),
            "roofline": roof, "cpu_baseline": cpu, "parity": parity}
    if cpu and "value" in cpu:
        line["gpu_over_cpu"] = round(tok_s / cpu["value"], 1)
    return line


def barrier_line(args):
    """What a persistent decode kernel would pay per phase: grid barriers over co-resident grids of
    256 and 512 workgroups (one and two per CU), flat, two-level (per XCD, then the grid) and two-level
    with the XCD leaders' release/acquire fences, each publishing data that is read back and checked;
    idle and while the other waves stream 4 GiB from HBM (four passes). Beside them, the kernel
    boundary they would replace: empty kernels back to back from a replayed graph and eagerly."""
    L = capi.lib()
    rounds = 2000
    forms = ((0, "flat"), (1, "two_level"), (2, "two_level_fenced"))
    results = []
    for n_wg in (256, 512):
        for mode, name in forms:
            for stream_mb in (0, 4096):
                st = capi.SdyBarrierStats()
                capi.check(L.sdy_grid_barrier_probe(n_wg, rounds, mode, stream_mb, ctypes.byref(st)))
                r = {"workgroups": n_wg, "form": name, "hbm_stream": bool(stream_mb),
                     "us_median": round(st.us_median, 3), "us_mean": round(st.us_mean, 3),
                     "rounds": st.rounds_done, "timeouts": st.timeouts, "mismatches": st.mismatches}
                if stream_mb:
                    r.update({"us_mean_while_streaming": round(st.us_mean_streaming, 3),
                              "rounds_while_streaming": st.rounds_streaming})
                results.append(r)
                log(f"[bench] barrier {n_wg} {name} stream={bool(stream_mb)}: {r}")
    ug, ue = ctypes.c_float(), ctypes.c_float()
    capi.check(L.sdy_kernel_boundary_us(2000, ctypes.byref(ug), ctypes.byref(ue)))
    best = next(r for r in results if r["workgroups"] == 256 and r["form"] == "two_level_fenced" and not r["hbm_stream"])
    return {"metric": METRIC, "value": best["us_median"], "unit": "us per grid barrier (256 workgroups, idle)",
            "n_gpus": 1, "steps": rounds, "warmup": 0, "ms_per_step": round(best["us_median"] / 1e3, 6),
            "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "n/a (synchronisation)",
            "data": "synthetic (64 floats per workgroup per round, checked)",
            "config": {"workload": "grid barrier of a persistent kernel vs the kernel boundary"},
            "kernel_boundary_us": {"graph_replay": round(ug.value, 3), "eager": round(ue.value, 3)},
            "barriers": results, "roofline": None, "cpu_baseline": None}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default: 50; decode workloads: 128 generated tokens)")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="q6k_head",
                    choices=["q6k_head", "q8_0_head", "q4k_matvec", "decode_3b", "decode_moe", "decode_moe_host",
                             "prefill_3b", "grid_barrier"])
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--n-batch", type=int, default=0,
                    help="GPU prefill chunk (decode workloads; 0: the whole context in one batch)")
    ap.add_argument("--layers", type=int, default=0, help="override the layer count (smoke runs only)")
    ap.add_argument("--scales", default="workload", choices=["workload", "file"],
                    help="K-quant scale distribution of the prefill model: the workload's, or the "
                         "normalised scales of quantized model files (the GEMM's wide variant)")
    ap.add_argument("--no-decode", action="store_true",
                    help="default workload: leave out the decode_3b / decode_moe sub-objects")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported in this build "
              "(the multi-GPU sharding of this path is a design note, not an implementation)", file=sys.stderr)
        sys.exit(2)
    if args.steps is None:
        args.steps = 128 if args.workload.startswith("decode") else 50
    capi.check(capi.lib().sdy_init())
    if args.workload == "q6k_head":
        line = bench_matvec(args, Q6_K, 151936, 2048, 8, stacked=False)
        if not args.no_decode:
            # the metric's second half: decode tok/s of the Qwen2.5-3B shape (and the MoE shape), each
            # 128 tokens after its context, with the reference engine on the host beside it; and the
            # 3B model's 512-token prefill on the GEMM (configuration 4)
            from sardyne_amd.gguf_synth import qwen25_3b, qwen3_30b_a3b
            sub = ("value", "unit", "ms_per_step", "roofline", "cpu_baseline", "parity", "model_load",
                   "mfma_utilisation", "gpu_over_cpu")
            p3b = write_bench_model(qwen25_3b(), "qwen25_3b")
            try:
                d = decode_line(args, qwen25_3b(), "qwen25_3b", 512, "Qwen2.5-3B-shaped Q4_K_M", n_dec=128,
                                path=p3b)
                line["decode_3b"] = {k: d[k] for k in sub if k in d}
                line["decode_3b"]["workload"] = d["config"]["workload"]
                pargs = argparse.Namespace(**{**vars(args), "steps": 20, "warmup": 2})
                d = prefill_line(pargs, qwen25_3b(), "qwen25_3b", 512, "Qwen2.5-3B-shaped Q4_K_M", path=p3b)
                line["prefill_3b"] = {k: d[k] for k in sub if k in d}
                line["prefill_3b"]["workload"] = d["config"]["workload"]
            finally:
                drop_bench_model(p3b)
            d = decode_line(args, qwen3_30b_a3b(), "qwen3_30b_a3b", 1024,
                            "Qwen3-30B-A3B-shaped qwen3moe Q4_K_M (128 experts resident, top-8)", n_dec=128)
            line["decode_moe"] = {k: d[k] for k in sub if k in d}
            line["decode_moe"]["workload"] = d["config"]["workload"]
    elif args.workload == "grid_barrier":
        line = barrier_line(args)
    elif args.workload == "q8_0_head":
        line = bench_matvec(args, Q8_0, 151936, 2048, 8, stacked=False)
    elif args.workload == "q4k_matvec":
        line = bench_matvec(args, Q4_K, 2048, 2048, 448, stacked=True)
    elif args.workload == "decode_3b":
        from sardyne_amd.gguf_synth import qwen25_3b
        line = decode_line(args, qwen25_3b(args.layers or 36), "qwen25_3b", 512, "Qwen2.5-3B-shaped Q4_K_M")
    elif args.workload == "decode_moe":
        from sardyne_amd.gguf_synth import qwen3_30b_a3b
        line = decode_line(args, qwen3_30b_a3b(args.layers or 48), "qwen3_30b_a3b", 1024,
                           "Qwen3-30B-A3B-shaped qwen3moe Q4_K_M (128 experts resident, top-8)")
    elif args.workload == "decode_moe_host":
        # the same decode with every expert stack in pinned host memory (a model larger than the
        # device): the routed experts' weights cross the host link each token
        from sardyne_amd.gguf_synth import qwen3_30b_a3b
        os.environ["SARDYNE_HOST_EXPERTS"] = os.environ.get("SARDYNE_HOST_EXPERTS") or "all"
        spec = qwen3_30b_a3b(args.layers or 48)
        line = decode_line(args, spec, "qwen3_30b_a3b_host", 1024,
                           "Qwen3-30B-A3B-shaped qwen3moe Q4_K_M (experts in pinned host memory, top-8)")
        eb = routed_expert_bytes(spec)
        gbps = eb * line["value"] / 1e9
        line["roofline"] = {"bound": "host_link", "achieved": round(gbps, 1), "peak": PCIE5_X16_GBPS,
                            "unit": "GB/s", "frac": round(gbps / PCIE5_X16_GBPS, 4), "traffic": None,
                            "kernel": "routed experts' weights read in place from pinned host memory",
                            "routed_expert_bytes_per_token": eb,
                            "achievable_GBps": round(host_link_read_GBps(None), 1),
                            "host_expert_layers": line["model_load"]["host_expert_layers"]}
    else:
        from sardyne_amd.gguf_synth import qwen25_3b
        spec = dataclasses.replace(qwen25_3b(args.layers or 36), scales=args.scales)
        line = prefill_line(args, spec, "qwen25_3b", 512, "Qwen2.5-3B-shaped Q4_K_M")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

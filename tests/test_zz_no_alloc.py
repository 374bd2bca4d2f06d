"""The no-allocation entry point (sdy_attn_decode_split_noalloc, include/sardyne.h) against the
entry point it varies (sdy_attn_decode_split, scratch from the caller): the same output, cache
rows and Q8_K bytes bit for bit, on two calls in a row, the second with a smaller shape, so the
shared static scratch is reused; and a shape beyond its fixed size is rejected with an error."""
import ctypes

import numpy as np
import pytest

from sardyne_amd import capi

pytestmark = pytest.mark.gpu


def _inputs(rng, n_head, n_kv_head, hd, max_seq):
    L = capi.lib()
    half = hd // 2
    cs, sn = np.empty(max_seq * half, np.float32), np.empty(max_seq * half, np.float32)
    L.op_rope_table(cs.ctypes.data, sn.ctypes.data, max_seq, hd, 1e6)
    return dict(q=rng.standard_normal(n_head * hd).astype(np.float32) * 2,
                k=rng.standard_normal(n_kv_head * hd).astype(np.float32) * 2,
                v=rng.standard_normal(n_kv_head * hd).astype(np.float32),
                kc=rng.standard_normal((n_kv_head, max_seq, hd)).astype(np.float32),
                vc=rng.standard_normal((n_kv_head, max_seq, hd)).astype(np.float32),
                cs=cs, sn=sn, qn=(1 + 0.2 * rng.standard_normal(hd)).astype(np.float32),
                kn=(1 + 0.2 * rng.standard_normal(hd)).astype(np.float32))


def _run(entry, inp, n_head, n_kv_head, hd, max_seq, pos, qk_norm):
    L = capi.lib()
    dev = {n: capi.DeviceBuffer.from_array(a) for n, a in inp.items()}
    step = capi.DeviceBuffer.from_array(np.array([0, pos], np.int32))
    out = capi.DeviceBuffer(n_head * hd * 4)
    n_blk = n_head * hd // 256
    xq = capi.DeviceBuffer(n_blk * 292)
    args = (dev["q"].ptr, dev["k"].ptr, dev["v"].ptr, dev["qn"].ptr if qk_norm else None,
            dev["kn"].ptr if qk_norm else None, 1e-6, dev["cs"].ptr, dev["sn"].ptr, step.ptr, n_head, n_kv_head, hd, 0,
            dev["kc"].ptr, dev["vc"].ptr, max_seq * hd, max_seq)
    if entry == "noalloc":
        capi.check(L.sdy_attn_decode_split_noalloc(*args, out.ptr, xq.ptr, None))
    else:
        part = capi.DeviceBuffer(L.sdy_attn_decode_split_floats(n_head, hd, max_seq) * 4)
        count = capi.DeviceBuffer.from_array(np.zeros(n_kv_head, np.uint32))
        capi.check(L.sdy_attn_decode_split(*args, part.ptr, count.ptr, out.ptr, xq.ptr, None))
    capi.check(L.sdy_sync(None))
    return (out.to_array(np.float32, n_head * hd), dev["kc"].to_array(np.float32, inp["kc"].shape),
            dev["vc"].to_array(np.float32, inp["vc"].shape), xq.to_array(np.uint8, n_blk * 292))


def test_noalloc_matches_scratch_entry_point_twice():
    capi.check(capi.lib().sdy_init())
    rng = np.random.default_rng(5)
    # a Qwen3-30B-A3B-shaped call, then a smaller Qwen2.5-3B-shaped one on the same static scratch
    for n_head, n_kv_head, hd, max_seq, pos, qk_norm in ((32, 4, 128, 1152, 1100, True),
                                                         (16, 2, 128, 640, 300, False)):
        inp = _inputs(rng, n_head, n_kv_head, hd, max_seq)
        got = _run("noalloc", inp, n_head, n_kv_head, hd, max_seq, pos, qk_norm)
        exp = _run("scratch", inp, n_head, n_kv_head, hd, max_seq, pos, qk_norm)
        for g, e in zip(got, exp):
            assert np.array_equal(np.ascontiguousarray(g).view(np.uint8), np.ascontiguousarray(e).view(np.uint8))
        assert np.all(np.isfinite(got[0]))


def test_noalloc_rejects_shapes_beyond_its_scratch():
    L = capi.lib()
    capi.check(L.sdy_init())
    # 64 heads x 131072 positions x (128 + 4) floats: far above the fixed 1 048 576 floats
    rc = L.sdy_attn_decode_split_noalloc(None, None, None, None, None, 1e-6, None, None, None, 64, 8, 128, 0, None,
                                         None, 131072 * 128, 131072, None, None, None)
    assert rc != 0
    assert b"scratch" in L.sdy_last_error()


def test_noalloc_position_outside_the_cache_changes_nothing():
    """A device-side position at or past max_seq (or below 0): every workgroup returns before it
    writes or counts, so the output buffer and the caches keep their bytes, and the next call, with
    a valid position, gives the scratch entry point's result (the shared counters stayed at zero)."""
    capi.check(capi.lib().sdy_init())
    rng = np.random.default_rng(9)
    n_head, n_kv_head, hd, max_seq = 16, 2, 128, 640
    inp = _inputs(rng, n_head, n_kv_head, hd, max_seq)
    for pos in (max_seq, max_seq + 100, -1):
        out, kc, vc, _ = _run("noalloc", inp, n_head, n_kv_head, hd, max_seq, pos, False)
        assert np.array_equal(kc, inp["kc"]) and np.array_equal(vc, inp["vc"])
        # (the output buffer is fresh device memory: it was not written, so it is not the result of
        # any position; the check that matters is the next call)
    got = _run("noalloc", inp, n_head, n_kv_head, hd, max_seq, 200, False)
    exp = _run("scratch", inp, n_head, n_kv_head, hd, max_seq, 200, False)
    for g, e in zip(got, exp):
        assert np.array_equal(np.ascontiguousarray(g).view(np.uint8), np.ascontiguousarray(e).view(np.uint8))

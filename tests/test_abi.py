"""The drop-in boundary on the CPU: build/libsardyne.so loads, exports every function that
include/sardyne.h declares, binds the reference's ctypes table (sardyne/capi.py:33-102) unchanged,
and its GGUF reader (pure host code) accepts and rejects files like the reference's parser
(tests/test_gguf.py of the reference: truncation, fuzz, duplicates, alignment). No kernel is run
here; without a GPU the engine refuses to load a model with an explicit error."""
import ctypes
import re
import struct
import subprocess

import numpy as np
import pytest

from sardyne_amd import capi
from sardyne_amd.gguf_synth import GGUFBuilder, ModelSpec, read_tensors, write_model

ROOT = __import__("pathlib").Path(__file__).resolve().parent.parent
needs_lib = pytest.mark.skipif(not capi.available(), reason="build/libsardyne.so not built")


def header_functions():
    text = (ROOT / "include" / "sardyne.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b([a-z_][a-z0-9_]*)\s*\([^;{]*\)\s*;", text)
    return sorted(set(n for n in names if n not in ("sizeof",)))


def test_header_declares_the_reference_abi():
    names = header_functions()
    for n in capi._SIGNATURES:
        assert n in names, n
    assert "gguf_prefetch" in names


@needs_lib
def test_every_declared_symbol_is_exported():
    out = subprocess.run(["nm", "-D", "--defined-only", str(capi.lib_path())], capture_output=True, text=True).stdout
    exported = set(line.split()[-1] for line in out.splitlines() if " T " in line)
    missing = [n for n in header_functions() if n not in exported]
    assert not missing, missing


@needs_lib
def test_ctypes_table_binds_and_version():
    lib = capi.lib()
    for name in list(capi._SIGNATURES) + list(capi._DEVICE_SIGNATURES):
        assert getattr(lib, name)
    assert capi.version() == "0.0.1"
    assert lib.op_row_size(12, 2048) == 8 * 144 and lib.op_row_size(14, 11008) == 43 * 210
    assert lib.op_row_size(8, 2048) == 64 * 34 and lib.op_row_size(15, 512) == 2 * 292
    assert lib.op_set_simd(0) == 0 and lib.op_simd() == 0
    assert lib.op_set_simd(1) == 1 and lib.op_simd() == 1


def test_missing_library_gives_clear_error(monkeypatch, tmp_path):
    monkeypatch.setenv("SARDYNE_LIB", str(tmp_path / "missing.so"))
    monkeypatch.setattr(capi, "_lib", None)
    assert not capi.available()
    with pytest.raises(OSError, match="make"):
        capi.version()


def gpu_present():
    import os
    return os.path.exists("/dev/kfd")


@needs_lib
@pytest.mark.skipif(gpu_present(), reason="checks the no-GPU error path")
def test_engine_fails_loudly_without_gpu(tmp_path):
    from sardyne_amd.engine import LoadedModel
    p = tmp_path / "m.gguf"
    write_model(p, ModelSpec(n_vocab=100, dim=256, n_layer=1, n_head=4, n_kv_head=2, head_dim=64, ffn_dim=256,
                             context=32), seed=1)
    with pytest.raises(ValueError, match="HIP device|gfx950"):
        LoadedModel(p)


@needs_lib
def test_op_rejects_bad_arguments_without_aborting():
    """A host-pointer op_* that cannot run (here a weight type the kernels do not take, checked before
    any GPU work) returns instead of ending the process: its outputs are NaN and op_last_error names
    the call; the next call clears the message."""
    L = capi.lib()
    out = np.zeros(4, np.float32)
    w = np.zeros(64, np.uint8)
    x = np.zeros(256, np.float32)
    L.op_matmul_rows(out.ctypes.data, x.ctypes.data, w.ctypes.data, 12, 1, 256, 4, 0, 4)  # Q4_K: not a float type
    assert np.all(np.isnan(out))
    assert b"op_matmul_rows" in L.op_last_error() and b"float type" in L.op_last_error()
    out = np.zeros(256, np.float32)
    L.op_row_to_f32(w.ctypes.data, 99, out.ctypes.data, 256)  # no such type
    assert np.all(np.isnan(out)) and b"op_row_to_f32" in L.op_last_error()


@needs_lib
@pytest.mark.skipif(gpu_present(), reason="checks the no-GPU error path")
def test_op_without_gpu_reports_instead_of_aborting():
    """Without a GPU the host-pointer op_* report the failure (NaN outputs, op_last_error) and the
    process goes on, where they used to abort."""
    L = capi.lib()
    x = np.ones(64, np.float32)
    out = np.zeros(64, np.float32)
    L.op_rmsnorm(out.ctypes.data, x.ctypes.data, x.ctypes.data, 64, ctypes.c_float(1e-6))
    assert np.all(np.isnan(out))
    assert b"op_rmsnorm" in L.op_last_error() and b"GPU" in L.op_last_error()
    r = L.op_dot_f32(x.ctypes.data, x.ctypes.data, 64)
    assert np.isnan(r)


# ---------------------------------------------------------------- GGUF reader (host code)

class CGGUF:
    def __init__(self, path):
        self.lib = capi.lib()
        err = ctypes.create_string_buffer(256)
        self.h = self.lib.gguf_open(str(path).encode(), err, len(err))
        self.err = err.value.decode()

    def close(self):
        if self.h:
            self.lib.gguf_close(self.h)
            self.h = None


@needs_lib
def test_gguf_reader_matches_python_reader(tmp_path):
    p = tmp_path / "m.gguf"
    write_model(p, ModelSpec(arch="qwen3moe", n_vocab=100, dim=256, n_layer=2, n_head=4, n_kv_head=2, head_dim=64,
                             ffn_dim=512, context=32, n_expert=4, n_expert_used=2, ffn_exp_dim=256, qkv_bias=False,
                             qk_norm=True), seed=2)
    meta, tensors, data_off, align = read_tensors(p)
    g = CGGUF(p)
    assert g.h, g.err
    L = g.lib
    assert L.gguf_version(g.h) == 3 and L.gguf_alignment(g.h) == align and L.gguf_data_offset(g.h) == data_off
    assert L.gguf_n_tensors(g.h) == len(tensors) and L.gguf_n_kv(g.h) == len(meta)
    raw = np.fromfile(p, np.uint8)
    for i in range(L.gguf_n_tensors(g.h)):
        t = L.gguf_get_tensor(g.h, i).contents
        ne, tid, off = tensors[t.name.decode()]
        assert tuple(t.ne[:t.n_dims]) == ne and t.type == tid and t.offset == off
        assert ctypes.string_at(t.data, min(64, t.nbytes)) == raw[data_off + off:data_off + off + min(64, t.nbytes)].tobytes()
    i = L.gguf_find_kv(g.h, b"qwen3moe.expert_count")
    v = ctypes.c_uint64()
    assert L.gguf_kv_get_u64(g.h, i, ctypes.byref(v)) == 0 and v.value == 4
    f = ctypes.c_double()
    assert L.gguf_kv_get_f64(g.h, L.gguf_find_kv(g.h, b"qwen3moe.rope.freq_base"), ctypes.byref(f)) == 0
    n = ctypes.c_uint64()
    s = L.gguf_kv_get_str(g.h, L.gguf_find_kv(g.h, b"general.architecture"), ctypes.byref(n))
    assert ctypes.string_at(s, n.value) == b"qwen3moe"
    assert L.gguf_kv_get_u64(g.h, L.gguf_find_kv(g.h, b"general.architecture"), ctypes.byref(v)) == -1
    assert L.gguf_find_tensor(g.h, b"nope") == -1 and not L.gguf_get_tensor(g.h, 10 ** 6)
    assert L.gguf_type_name(14) == b"Q6_K" and L.gguf_type_name(4) is None
    g.close()
    # NULL-tolerant accessors
    assert L.gguf_version(None) == 0 and L.gguf_n_tensors(None) == 0 and L.gguf_find_kv(None, b"x") == -1


def small_file(tmp_path, **kw):
    b = GGUFBuilder(tmp_path / "s.gguf")
    b.add_str("general.architecture", "llama")
    b.add_u32("llama.block_count", 1)
    b.add_tensor("a.weight", (64, 2), "F32", lambda: np.ones(128, np.float32).tobytes())
    b.add_tensor("b.weight", (256, 1), "Q4_K", lambda: bytes(144))
    for k, v in kw.items():
        b.add_u32(k, v)
    return b.write()


@needs_lib
def test_gguf_truncation_is_rejected(tmp_path):
    path = small_file(tmp_path)
    data = path.read_bytes()
    _, tensors, data_off, _ = read_tensors(path)
    end = max(data_off + off + (144 if tid == 12 else 512) for ne, tid, off in tensors.values())
    for cut in range(0, end, 7):  # every cut before the end of the last tensor's data
        p = tmp_path / "cut.gguf"
        p.write_bytes(data[:cut])
        g = CGGUF(p)
        assert not g.h, cut
        assert g.err


@needs_lib
def test_gguf_header_fuzz_never_crashes(tmp_path):
    data = bytearray(small_file(tmp_path).read_bytes())
    rng = np.random.default_rng(42)
    p = tmp_path / "fuzz.gguf"
    for _ in range(1500):
        d = bytearray(data)
        for _ in range(int(rng.integers(1, 4))):
            d[int(rng.integers(0, 200))] = int(rng.integers(0, 256))
        p.write_bytes(bytes(d))
        g = CGGUF(p)
        g.close()


@needs_lib
def test_gguf_rejections(tmp_path):
    data = small_file(tmp_path).read_bytes()
    p = tmp_path / "x.gguf"
    p.write_bytes(b"GGUX" + data[4:])
    assert "magic" in CGGUF(p).err
    p.write_bytes(data[:4] + struct.pack("<I", 7) + data[8:])
    assert "versione" in CGGUF(p).err
    p.write_bytes(data[:4] + struct.pack(">I", 3) + data[8:])
    assert "big-endian" in CGGUF(p).err
    q = small_file(tmp_path, **{"general.alignment": 48})
    assert "alignment" in CGGUF(q).err
    g = CGGUF(tmp_path / "does-not-exist.gguf")
    assert "impossibile aprire" in g.err
    b = GGUFBuilder(tmp_path / "dup.gguf")
    b.add_u32("k", 1)
    b.add_u32("k", 2)
    assert "duplicato" in CGGUF(b.write()).err


# ---------------------------------------------------------------- GGUF reader vs the reference's reader

def _gguf_binding(path):
    """ctypes view of the gguf_* functions of a library (this build's or the reference's)."""
    h = ctypes.CDLL(str(path))
    for name, (res, args) in capi._SIGNATURES.items():
        if name.startswith("gguf_"):
            fn = getattr(h, name)
            fn.restype, fn.argtypes = res, args
    return h


def _summary(L, path):
    """Everything a caller reads from an open file, or None when the reader rejects it."""
    err = ctypes.create_string_buffer(256)
    h = L.gguf_open(str(path).encode(), err, len(err))
    if not h:
        assert err.value, "rejected without a message"
        return None
    try:
        kvs = []
        for i in range(L.gguf_n_kv(h)):
            kv = L.gguf_get_kv(h, i).contents
            key = kv.key
            assert L.gguf_find_kv(h, key) == i
            u, f, n = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_uint64()
            val = (L.gguf_kv_get_u64(h, i, ctypes.byref(u)), u.value if L.gguf_kv_get_u64(h, i, ctypes.byref(u)) == 0
                   else None, L.gguf_kv_get_f64(h, i, ctypes.byref(f)), f.value if kv.type in (6, 12) else None)
            s = L.gguf_kv_get_str(h, i, ctypes.byref(n))
            sv = ctypes.string_at(s, n.value) if s else None
            arr = []
            if kv.type == 9 and kv.arr_type == 8:
                for j in range(min(kv.n, 8)):
                    p = L.gguf_kv_get_arr_str(h, i, j, ctypes.byref(n))
                    arr.append(ctypes.string_at(p, n.value))
                assert not L.gguf_kv_get_arr_str(h, i, kv.n, ctypes.byref(n))
            kvs.append((key, kv.type, kv.arr_type if kv.type == 9 else None, kv.n, val, sv, tuple(arr)))
        ts = []
        for i in range(L.gguf_n_tensors(h)):
            t = L.gguf_get_tensor(h, i).contents
            assert L.gguf_find_tensor(h, t.name) == i
            ts.append((t.name, t.n_dims, t.type, tuple(t.ne), t.offset, t.nbytes,
                       t.data - L.gguf_get_tensor(h, 0).contents.data if ts else 0))
        return (L.gguf_version(h), L.gguf_alignment(h), L.gguf_data_offset(h), tuple(kvs), tuple(ts))
    finally:
        L.gguf_close(h)


def _rich_file(path):
    """A file that exercises every value kind: scalars of each width and sign, f32/f64, bool, a
    string, scalar arrays and a string array (with a multi-byte UTF-8 element), and tensors of
    several types and ranks."""
    b = GGUFBuilder(path)
    b.add_str("general.architecture", "qwen2")
    b.add_raw("u8", 0, struct.pack("<B", 200))
    b.add_raw("i8", 1, struct.pack("<b", -3))
    b.add_raw("u16", 2, struct.pack("<H", 40000))
    b.add_raw("i16", 3, struct.pack("<h", 1234))
    b.add_raw("i32", 5, struct.pack("<i", -7))
    b.add_raw("i64", 11, struct.pack("<q", 1 << 40))
    b.add_raw("u64", 10, struct.pack("<Q", 1 << 62))
    b.add_raw("f64", 12, struct.pack("<d", 2.5))
    b.add_raw("ok", 7, b"\x01")
    b.add_f32("f32", 0.125)
    b.add_raw("arr.i32", 9, struct.pack("<IQ", 5, 3) + struct.pack("<3i", 1, -2, 3))
    b.add_str_array("tokenizer.tokens", ["a", "bé", "", "€x"])
    b.add_u32("general.alignment", 64)
    b.add_tensor("t.f32", (64, 2), "F32", lambda: np.ones(128, np.float32).tobytes())
    b.add_tensor("t.q4k", (256, 1), "Q4_K", lambda: bytes(144))
    b.add_tensor("t.q8", (32, 2, 3), "Q8_0", lambda: bytes(6 * 34))
    return b.write()


needs_ref_gguf = pytest.mark.skipif(
    not capi.available() or not (ROOT / "oracle" / "_ref" / "libsardyne_ref.so").exists(),
    reason="needs build/libsardyne.so and the reference compiled into oracle/_ref")


@needs_ref_gguf
def test_gguf_reader_agrees_with_reference_reader(tmp_path):
    """The reference's own parser (csrc/gguf.c, compiled from its sources) and this build's read
    the same fields from a valid file, and accept or reject the same corrupted files: truncations
    at every byte of the header and 1500 random header mutations (seed 42), the method of the
    reference's tests/test_gguf.py:144-173 with its C parser as the other side."""
    ours = _gguf_binding(capi.lib_path())
    ref = _gguf_binding(ROOT / "oracle" / "_ref" / "libsardyne_ref.so")
    path = _rich_file(tmp_path / "rich.gguf")
    good = _summary(ref, path)
    assert good is not None and _summary(ours, path) == good
    data = path.read_bytes()
    header_end = good[2]
    bad = tmp_path / "bad.gguf"
    for n in range(0, header_end + 1):
        bad.write_bytes(data[:n])
        assert _summary(ours, bad) == _summary(ref, bad), n
    rng = np.random.default_rng(42)
    accepted = 0
    for _ in range(1500):
        d = bytearray(data)
        for pos in rng.integers(4, header_end, size=rng.integers(1, 4)):
            d[pos] = int(rng.integers(0, 256))
        bad.write_bytes(bytes(d))
        r = _summary(ref, bad)
        assert _summary(ours, bad) == r
        accepted += r is not None
    assert 0 < accepted < 1500


@needs_ref_gguf
@pytest.mark.parametrize("n_pos,hd,theta", [(640, 128, 1e6), (1152, 128, 1e6), (300, 64, 1e4), (50, 16, 10000.0)],
                         ids=["qwen25-3b-ctx640", "qwen3-30b-a3b-ctx1152", "llama-hd64", "small"])
def test_rope_table_bits_equal_reference(n_pos, hd, theta):
    """op_rope_table (host libm in double, the table the engine uploads at context creation) has the
    bits of the reference's op_rope_table (csrc/ops.c:375-386, compiled from its sources) at the
    tables of the Qwen2.5-3B (640 positions) and Qwen3-30B-A3B (1152 positions) workloads."""
    import oracle as O
    got = [np.empty((n_pos, hd // 2), np.float32) for _ in range(2)]
    exp = [np.empty((n_pos, hd // 2), np.float32) for _ in range(2)]
    capi.lib().op_rope_table(got[0].ctypes.data, got[1].ctypes.data, n_pos, hd, theta)
    O.ref_lib().op_rope_table(exp[0].ctypes.data, exp[1].ctypes.data, n_pos, hd, theta)
    for g, e in zip(got, exp):
        assert np.array_equal(g.view(np.uint32), e.view(np.uint32))
    # the mathematics: position 0 is the identity rotation, and pair i turns by theta^(-2i/hd) per position
    assert np.all(got[0][0] == 1.0) and np.all(got[1][0] == 0.0)
    ang = np.arange(n_pos)[:, None] * theta ** (-np.arange(hd // 2) * 2.0 / hd)[None, :]
    np.testing.assert_allclose(got[0], np.cos(ang), atol=2e-7)
    np.testing.assert_allclose(got[1], np.sin(ang), atol=2e-7)

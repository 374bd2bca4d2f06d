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
    from sardyne_amd.runtime import Model
    p = tmp_path / "m.gguf"
    write_model(p, ModelSpec(n_vocab=100, dim=256, n_layer=1, n_head=4, n_kv_head=2, head_dim=64, ffn_dim=256,
                             context=32), seed=1)
    with pytest.raises(ValueError, match="HIP device|gfx950"):
        Model(p)


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

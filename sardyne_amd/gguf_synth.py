"""Synthetic GGUF models and quantized blocks for tests and benchmarks.

The GGUF v3 container (magic, counts, typed metadata, tensor table, 32-byte aligned data) is the
format the reference reads (csrc/gguf.c:250-320); tensor ``ne`` lists the innermost dimension
first, so a [n_out][n_in] matrix has ne = (n_in, n_out). Weights are random bytes shaped by the
distributions of the benchmark workloads:

- Q4_K: f16 ``d``/``dmin`` = |N(0, 0.02)|, uniform ``scales[12]`` bytes (uniform 6-bit scales and
  mins), uniform ``qs`` bytes (uniform 4-bit quants);
- Q6_K: uniform ``ql``/``qh`` bytes (uniform 6-bit quants), int8 scales uniform in [-32, 31],
  f16 ``d`` = |N(0, 0.01)|;
- Q8_0: f16 scale = |N(0, 0.01)|, int8 quants uniform in [-127, 127];
- Q4_0 / Q5_0: f16 scale = |N(0, 0.01)|, uniform quant bytes.

``scales="file"`` gives the K-quant scales the shape they have in quantized model files, where each
super-block's scales are normalised to the largest one: Q6_K int8 scales with the sub-block of
largest amplitude at -128 and the others in [-128, 127] by their signed amplitude; Q4_K 6-bit scales
and minima with the largest at 63. Sub-block amplitudes are the maxima of 16 |N(0, 1)| draws.

Everything is produced block-row by block-row from a seeded ``numpy.random.Generator``, so a
model of several GB is written without holding it in memory.
"""
from __future__ import annotations

import math
import os
import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

# ggml type id -> (name, elements per block, bytes per block); ids are GGUF's.
GGML_TYPES = {0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 6: ("Q5_0", 32, 22),
              8: ("Q8_0", 32, 34), 12: ("Q4_K", 256, 144), 14: ("Q6_K", 256, 210), 15: ("Q8_K", 256, 292),
              30: ("BF16", 1, 2)}
TYPE_ID = {name: tid for tid, (name, _, _) in GGML_TYPES.items()}
ALIGN = 32


def row_bytes(type_name: str, n: int) -> int:
    _, blk, size = GGML_TYPES[TYPE_ID[type_name]]
    assert n % blk == 0, (type_name, n)
    return n // blk * size


def _f16_abs_normal(rng, std, n):
    return np.abs(rng.standard_normal(n) * std).astype(np.float16).view(np.uint8).reshape(n, 2)


def _amplitudes(rng, n_blocks, n_sub):
    """[n_blocks, n_sub] sub-block amplitudes: the largest |N(0, 1)| of 16 draws."""
    return np.abs(rng.standard_normal((n_blocks, n_sub, 16))).max(axis=2)


def _q4k_pack(sc, mn):
    """The 12 scale bytes of Q4_K from 8 six-bit scales and minima per block: bytes 0-3 hold
    scales 0-3 (low 6 bits) and the top 2 bits of scales 4-7; bytes 4-7 minima 0-3 and the top bits
    of minima 4-7; bytes 8-11 the low 4 bits of scales 4-7 and (high nibble) of minima 4-7."""
    sc, mn = sc.astype(np.uint8), mn.astype(np.uint8)
    out = np.empty((sc.shape[0], 12), np.uint8)
    out[:, 0:4] = sc[:, 0:4] | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = mn[:, 0:4] | ((mn[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    return out


def random_blocks(type_name: str, n_blocks: int, rng: np.random.Generator, scales: str = "workload") -> np.ndarray:
    """[n_blocks, block_bytes] uint8 with the workload distributions above (K-quant scales as in
    model files with scales="file")."""
    _, _, size = GGML_TYPES[TYPE_ID[type_name]]
    b = np.frombuffer(rng.bytes(n_blocks * size), np.uint8).reshape(n_blocks, size).copy()
    if scales not in ("workload", "file"):
        raise ValueError(scales)
    if type_name == "Q4_K":
        b[:, 0:2] = _f16_abs_normal(rng, 0.02, n_blocks)
        b[:, 2:4] = _f16_abs_normal(rng, 0.02, n_blocks)
        if scales == "file":
            a, m = _amplitudes(rng, n_blocks, 8), _amplitudes(rng, n_blocks, 8)
            sc = np.rint(63 * a / a.max(axis=1, keepdims=True))
            mn = np.rint(63 * m / m.max(axis=1, keepdims=True))
            b[:, 4:16] = _q4k_pack(sc, mn)
    elif type_name == "Q6_K":
        if scales == "file":
            a = _amplitudes(rng, n_blocks, 16) * rng.choice([-1.0, 1.0], (n_blocks, 16))
            top = a[np.arange(n_blocks), np.abs(a).argmax(axis=1)][:, None]
            b[:, 192:208] = np.minimum(127, np.rint(-128 * a / top)).astype(np.int8).view(np.uint8)
        else:
            b[:, 192:208] = rng.integers(-32, 32, (n_blocks, 16), dtype=np.int8).view(np.uint8)
        b[:, 208:210] = _f16_abs_normal(rng, 0.01, n_blocks)
    elif type_name == "Q8_0":
        b[:, 0:2] = _f16_abs_normal(rng, 0.01, n_blocks)
        b[:, 2:34] = rng.integers(-127, 128, (n_blocks, 32), dtype=np.int8).view(np.uint8)
    elif type_name in ("Q4_0", "Q5_0"):
        b[:, 0:2] = _f16_abs_normal(rng, 0.01, n_blocks)
    else:
        raise ValueError(type_name)
    return b


def random_matrix(type_name: str, n_out: int, n_in: int, seed: int) -> np.ndarray:
    """Raw [n_out, row_bytes] matrix."""
    _, blk, _ = GGML_TYPES[TYPE_ID[type_name]]
    rng = np.random.default_rng(seed)
    return random_blocks(type_name, n_out * n_in // blk, rng).reshape(n_out, -1)


# ---------------------------------------------------------------- GGUF writer

_VT_U32, _VT_F32, _VT_STR, _VT_U64 = 4, 6, 8, 10


@dataclass
class _Tensor:
    name: str
    ne: tuple
    type_id: int
    nbytes: int
    produce: object  # callable -> bytes-like, or a writer(fileobj)


@dataclass
class GGUFBuilder:
    path: Path
    kv: list = field(default_factory=list)
    tensors: list = field(default_factory=list)

    def add_u32(self, key, v):
        self.kv.append((key, _VT_U32, struct.pack("<I", int(v))))

    def add_f32(self, key, v):
        self.kv.append((key, _VT_F32, struct.pack("<f", float(v))))

    def add_str(self, key, s):
        b = s.encode()
        self.kv.append((key, _VT_STR, struct.pack("<Q", len(b)) + b))

    def add_raw(self, key, vt, payload: bytes):
        """A metadata value of GGUF value type `vt` whose encoded bytes are `payload`."""
        self.kv.append((key, vt, payload))

    def add_str_array(self, key, items):
        enc = [s.encode() for s in items]
        self.kv.append((key, 9, struct.pack("<IQ", _VT_STR, len(enc)) + b"".join(struct.pack("<Q", len(e)) + e
                                                                                for e in enc)))

    def add_tensor(self, name, ne, type_name, produce):
        tid = TYPE_ID[type_name]
        _, blk, size = GGML_TYPES[tid]
        n = int(np.prod(ne))
        assert ne[0] % blk == 0
        self.tensors.append(_Tensor(name, tuple(int(d) for d in ne), tid, n // blk * size, produce))

    def add_array(self, name, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        tname = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16"}[arr.dtype]
        self.add_tensor(name, tuple(reversed(arr.shape)), tname, lambda a=arr: a.tobytes())

    def write(self):
        align = ALIGN
        for key, vt, payload in self.kv:
            if key == "general.alignment" and vt == _VT_U32:
                align = struct.unpack("<I", payload)[0]
        head = [b"GGUF", struct.pack("<IQQ", 3, len(self.tensors), len(self.kv))]
        for key, vt, payload in self.kv:
            k = key.encode()
            head += [struct.pack("<Q", len(k)), k, struct.pack("<I", vt), payload]
        off = 0
        for t in self.tensors:
            nm = t.name.encode()
            head += [struct.pack("<Q", len(nm)), nm, struct.pack("<I", len(t.ne)),
                     struct.pack(f"<{len(t.ne)}Q", *t.ne), struct.pack("<IQ", t.type_id, off)]
            off += -(-t.nbytes // align) * align
        header = b"".join(head)
        tmp = Path(str(self.path) + ".tmp")
        with open(tmp, "wb") as f:
            f.write(header)
            f.write(b"\0" * (-len(header) % align))
            for t in self.tensors:
                start = f.tell()
                res = t.produce()
                if res is not None:
                    f.write(res if isinstance(res, (bytes, bytearray, memoryview)) else bytes(res))
                else:  # produce() wrote nothing: it is a generator of chunks
                    pass
                written = f.tell() - start
                if written != t.nbytes:
                    raise ValueError(f"{t.name}: wrote {written} bytes, expected {t.nbytes}")
                f.write(b"\0" * (-t.nbytes % align))
        os.replace(tmp, self.path)
        return self.path


# ---------------------------------------------------------------- model shapes

@dataclass
class ModelSpec:
    arch: str = "qwen2"
    n_vocab: int = 151936
    dim: int = 2048
    n_layer: int = 36
    n_head: int = 16
    n_kv_head: int = 2
    head_dim: int = 128
    ffn_dim: int = 11008
    context: int = 4096
    rope_theta: float = 1e6
    eps: float = 1e-6
    n_expert: int = 0
    n_expert_used: int = 0
    ffn_exp_dim: int = 0
    qkv_bias: bool = True
    qk_norm: bool = False
    tied: bool = False
    # weight types
    t_default: str = "Q4_K"
    t_attn_v: str = "Q6_K"
    t_ffn_down: str = "Q6_K"
    t_output: str = "Q6_K"
    t_embd: str = "Q4_K"
    router_std: float = 0.02
    norm_value: float = 1.0
    bias_std: float = 0.02
    type_fn: object = None  # optional name -> weight type override for quantized matrices
    same_experts: bool = False  # every expert of a layer gets the blocks of expert 0 (the dense matrix of its seed)
    scales: str = "workload"  # K-quant scale distribution: "workload" or "file" (random_blocks)


def qwen25_3b(n_layer=36) -> ModelSpec:
    """Qwen2.5-3B shape, Q4_K_M mix (Q6_K for attn_v, ffn_down, output)."""
    return ModelSpec(n_layer=n_layer)


def qwen3_30b_a3b(n_layer=48) -> ModelSpec:
    """Qwen3-30B-A3B shape: qwen3moe, 32/4 heads, q/k norm, 128 experts top-8, expert FFN 768."""
    return ModelSpec(arch="qwen3moe", dim=2048, n_layer=n_layer, n_head=32, n_kv_head=4, head_dim=128,
                     ffn_dim=6144, n_expert=128, n_expert_used=8, ffn_exp_dim=768, qkv_bias=False, qk_norm=True,
                     rope_theta=1e6)


def _matrix_producer(type_name, n_out, n_in, seed, n_expert=0, same=False, scales="workload"):
    """Random blocks of an n_out x n_in matrix (n_expert stacked ones). same: one matrix drawn from
    the seed, repeated for every expert, so each expert equals the dense matrix of that seed."""
    def produce():
        rng = np.random.default_rng(seed)
        _, blk, _ = GGML_TYPES[TYPE_ID[type_name]]
        if same:
            one = random_blocks(type_name, n_out * (n_in // blk), rng, scales)
            return np.tile(one.reshape(1, -1), (max(1, n_expert), 1)).tobytes()
        rows = n_out * max(1, n_expert)
        nb = rows * (n_in // blk)
        return random_blocks(type_name, nb, rng, scales).tobytes()
    return produce


def write_model(path, spec: ModelSpec, seed: int = 0) -> Path:
    """Random-init GGUF of the given shape. Matrices are random quantized blocks; norms are
    ``norm_value``; q/k/v biases N(0, bias_std); the MoE router is F32 N(0, router_std)."""
    b = GGUFBuilder(Path(path))
    a = spec.arch
    b.add_str("general.architecture", a)
    b.add_u32(f"{a}.context_length", spec.context)
    b.add_u32(f"{a}.embedding_length", spec.dim)
    b.add_u32(f"{a}.block_count", spec.n_layer)
    b.add_u32(f"{a}.feed_forward_length", spec.ffn_dim)
    b.add_u32(f"{a}.attention.head_count", spec.n_head)
    b.add_u32(f"{a}.attention.head_count_kv", spec.n_kv_head)
    b.add_u32(f"{a}.attention.key_length", spec.head_dim)
    b.add_u32(f"{a}.attention.value_length", spec.head_dim)
    b.add_f32(f"{a}.rope.freq_base", spec.rope_theta)
    b.add_f32(f"{a}.attention.layer_norm_rms_epsilon", spec.eps)
    if spec.n_expert:
        b.add_u32(f"{a}.expert_count", spec.n_expert)
        b.add_u32(f"{a}.expert_used_count", spec.n_expert_used)
        b.add_u32(f"{a}.expert_feed_forward_length", spec.ffn_exp_dim)
    rng = np.random.default_rng(seed + 7919)
    dim, hd = spec.dim, spec.head_dim
    q_dim, kv_dim = spec.n_head * hd, spec.n_kv_head * hd
    s = [seed * 1000003]

    def nxt():
        s[0] += 1
        return s[0]

    norm = lambda n: np.full(n, spec.norm_value, np.float32)
    orig_add = b.add_tensor

    def add_matrix(name, ne, tname, produce):
        t = spec.type_fn(name) if spec.type_fn else None
        if t and t != tname and tname not in ("F32", "F16", "BF16"):
            n_out = int(np.prod(ne[1:]))
            produce = _matrix_producer(t, n_out, ne[0], nxt(), scales=spec.scales)
            tname = t
        orig_add(name, ne, tname, produce)

    b.add_tensor = add_matrix
    b.add_tensor("token_embd.weight", (dim, spec.n_vocab), spec.t_embd,
                 _matrix_producer(spec.t_embd, spec.n_vocab, dim, nxt(), scales=spec.scales))
    b.add_array("output_norm.weight", norm(dim))
    if not spec.tied:
        b.add_tensor("output.weight", (dim, spec.n_vocab), spec.t_output,
                     _matrix_producer(spec.t_output, spec.n_vocab, dim, nxt(), scales=spec.scales))
    for l in range(spec.n_layer):
        p = f"blk.{l}."
        b.add_array(p + "attn_norm.weight", norm(dim))
        b.add_array(p + "ffn_norm.weight", norm(dim))
        b.add_tensor(p + "attn_q.weight", (dim, q_dim), spec.t_default, _matrix_producer(spec.t_default, q_dim, dim, nxt(), scales=spec.scales))
        b.add_tensor(p + "attn_k.weight", (dim, kv_dim), spec.t_default, _matrix_producer(spec.t_default, kv_dim, dim, nxt(), scales=spec.scales))
        b.add_tensor(p + "attn_v.weight", (dim, kv_dim), spec.t_attn_v, _matrix_producer(spec.t_attn_v, kv_dim, dim, nxt(), scales=spec.scales))
        b.add_tensor(p + "attn_output.weight", (q_dim, dim), spec.t_default,
                     _matrix_producer(spec.t_default, dim, q_dim, nxt(), scales=spec.scales))
        if spec.qkv_bias:
            b.add_array(p + "attn_q.bias", (rng.standard_normal(q_dim) * spec.bias_std).astype(np.float32))
            b.add_array(p + "attn_k.bias", (rng.standard_normal(kv_dim) * spec.bias_std).astype(np.float32))
            b.add_array(p + "attn_v.bias", (rng.standard_normal(kv_dim) * spec.bias_std).astype(np.float32))
        if spec.qk_norm:
            b.add_array(p + "attn_q_norm.weight", norm(hd))
            b.add_array(p + "attn_k_norm.weight", norm(hd))
        if spec.n_expert:
            ne, fe = spec.n_expert, spec.ffn_exp_dim
            b.add_array(p + "ffn_gate_inp.weight", (rng.standard_normal((ne, dim)) * spec.router_std).astype(np.float32))
            b.add_tensor(p + "ffn_gate_exps.weight", (dim, fe, ne), spec.t_default,
                         _matrix_producer(spec.t_default, fe, dim, nxt(), ne, spec.same_experts, spec.scales))
            b.add_tensor(p + "ffn_up_exps.weight", (dim, fe, ne), spec.t_default,
                         _matrix_producer(spec.t_default, fe, dim, nxt(), ne, spec.same_experts, spec.scales))
            b.add_tensor(p + "ffn_down_exps.weight", (fe, dim, ne), spec.t_ffn_down,
                         _matrix_producer(spec.t_ffn_down, dim, fe, nxt(), ne, spec.same_experts, spec.scales))
        else:
            b.add_tensor(p + "ffn_gate.weight", (dim, spec.ffn_dim), spec.t_default,
                         _matrix_producer(spec.t_default, spec.ffn_dim, dim, nxt(), scales=spec.scales))
            b.add_tensor(p + "ffn_up.weight", (dim, spec.ffn_dim), spec.t_default,
                         _matrix_producer(spec.t_default, spec.ffn_dim, dim, nxt(), scales=spec.scales))
            b.add_tensor(p + "ffn_down.weight", (spec.ffn_dim, dim), spec.t_ffn_down,
                         _matrix_producer(spec.t_ffn_down, dim, spec.ffn_dim, nxt(), scales=spec.scales))
    return b.write()


# ---------------------------------------------------------------- GGUF reader (tensor table only)

_SCALAR = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}


def read_tensors(path):
    """Parse a GGUF v2/v3 file: returns (metadata dict of scalars/strings, {name: (ne, type_id, offset)},
    data_offset, alignment)."""
    data = np.memmap(path, np.uint8, mode="r")
    pos = 0

    def rd(fmt):
        nonlocal pos
        n = struct.calcsize(fmt)
        v = struct.unpack_from(fmt, data, pos)
        pos += n
        return v if len(v) > 1 else v[0]

    def rstr():
        nonlocal pos
        n = rd("<Q")
        s = bytes(data[pos:pos + n]).decode()
        pos += n
        return s

    assert bytes(data[:4]) == b"GGUF"
    pos = 4
    version, n_t, n_kv = rd("<IQQ")
    meta, align = {}, ALIGN
    fmts = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
    for _ in range(n_kv):
        key = rstr()
        vt = rd("<I")
        if vt == 8:
            meta[key] = rstr()
        elif vt == 9:
            et, n = rd("<IQ")
            if et == 8:
                meta[key] = [rstr() for _ in range(n)]
            else:
                pos += n * _SCALAR[et]
        else:
            meta[key] = rd(fmts[vt])
        if key == "general.alignment":
            align = int(meta[key])
    tensors = {}
    for _ in range(n_t):
        name = rstr()
        nd = rd("<I")
        ne = tuple(rd("<Q") for _ in range(nd))
        tid, off = rd("<IQ")
        tensors[name] = (ne, tid, off)
    data_off = -(-pos // align) * align
    return meta, tensors, data_off, align

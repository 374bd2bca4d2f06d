"""The oracle (oracle/, CPU restatement of the reference) pinned three ways:
1. against the golden fixtures written from the reference compiled from its own sources
   (tests/golden/make_golden.py);
2. against that compiled reference live, when oracle/_ref has been built here;
3. against closed forms and invariants restated independently in NumPy (dequantisation formulas,
   quantiser invariants, exact integer dots on small inputs, exhaustive f16 conversion), chosen so
   that a dropped term, a wrong sign, index or rounding mode fails one of them.
CPU only."""
import hashlib
import math

import numpy as np
import pytest

import oracle as O
from sardyne_amd.gguf_synth import random_blocks

GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"
TYPES = {"Q8_0": O.Q8_0, "Q4_0": O.Q4_0, "Q5_0": O.Q5_0, "Q4_K": O.Q4_K, "Q6_K": O.Q6_K}
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs the reference sources)")


@pytest.fixture(scope="module")
def kern():
    return np.load(GOLDEN / "kernels.npz")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ---------------------------------------------------------------- 1. golden fixtures

@pytest.mark.parametrize("kind", list(TYPES))
@pytest.mark.parametrize("gen", ["ref", "workload"])
def test_golden_dequant_and_matmul(kern, kind, gen):
    t = TYPES[kind]
    w = kern[f"{kind}_{gen}_w"]
    deq = np.stack([O.dequant(r, t, 512) for r in w])
    assert np.array_equal(bits(deq), bits(kern[f"{kind}_{gen}_deq"]))
    xq = O.quantize(kern[f"{kind}_{gen}_x"], O.VEC_DOT[t])
    for simd in (0, 1):
        got = O.matmul_q(w, t, xq, 512, simd=simd)
        assert np.array_equal(bits(got), bits(kern[f"{kind}_{gen}_mm{simd}"])), (kind, gen, simd)


def test_golden_activation_quantization(kern):
    x = kern["act_x"]
    assert np.array_equal(O.quantize(x, O.Q8_0), kern["act_q8_0"])
    assert np.array_equal(O.quantize(x, O.Q8_K), kern["act_q8_k"])


def test_golden_c1():
    g = np.load(GOLDEN / "c1.npz")
    w = random_blocks("Q4_K", 2048 * 2048 // 256, np.random.default_rng(0)).reshape(2048, -1)
    x = np.random.default_rng(1).standard_normal(2048).astype(np.float32)
    assert hashlib.sha256(w.tobytes()).hexdigest() == str(g["w_sha"])
    assert hashlib.sha256(x.tobytes()).hexdigest() == str(g["x_sha"])
    y = O.matmul_q(w, O.Q4_K, O.quantize(x, O.Q8_K), 2048)[0]
    assert np.array_equal(bits(y), bits(g["y"]))


def test_golden_small_models(tmp_path):
    import sys
    sys.path.insert(0, str(GOLDEN))
    from make_golden import PROMPT, SMALL_MODELS
    from sardyne_amd.gguf_synth import write_model
    g = np.load(GOLDEN / "model.npz")
    for name, spec in SMALL_MODELS.items():
        p = tmp_path / f"{name}.gguf"
        write_model(p, spec, seed=11)
        assert hashlib.sha256(p.read_bytes()).hexdigest() == str(g[f"{name}_sha"]), name
        logits = O.OracleContext(p, 32, len(PROMPT), logits_all=True).eval(PROMPT)
        assert np.array_equal(bits(logits), bits(g[f"{name}_logits"])), name
        ctx = O.OracleContext(p, 32, 64)
        lg, gen = ctx.eval(PROMPT[:4]), []
        for _ in range(8):
            gen.append(int(np.argmax(lg)))
            lg = ctx.eval([gen[-1]])
        assert gen == g[f"{name}_greedy"].tolist(), name


# ---------------------------------------------------------------- 2. the compiled reference, live

@needs_ref
@pytest.mark.parametrize("kind", list(TYPES))
@pytest.mark.parametrize("n_tok", [1, 3, 4, 7, 9])
def test_live_reference_kernels(kind, n_tok):
    t = TYPES[kind]
    n = 1024
    rng = np.random.default_rng(n_tok)
    w = random_blocks(kind, 9 * n // O.QK[t], rng).reshape(9, -1)
    x = rng.standard_normal((n_tok, n)).astype(np.float32)
    x[0, :256] *= 1e3
    xq = O.quantize(x, O.VEC_DOT[t])
    assert np.array_equal(xq, O.quantize(x, O.VEC_DOT[t], use_ref=True))
    for simd in (0, 1):
        a, b = O.matmul_q(w, t, xq, n, simd), O.matmul_q(w, t, xq, n, simd, use_ref=True)
        assert np.array_equal(bits(a), bits(b))
    assert np.array_equal(bits(O.dequant(w[0], t, n)), bits(O.dequant(w[0], t, n, use_ref=True)))


@needs_ref
def test_live_reference_float_ops():
    L, R = O.lib(), O.ref_lib()
    p = O.ptr
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(300) * 5).astype(np.float32)
    w = rng.standard_normal(300).astype(np.float32)
    a, b = np.empty_like(x), np.empty_like(x)
    L.orc_rmsnorm(p(a), p(x), p(w), 300, 1e-6)
    R.op_rmsnorm(p(b), p(x), p(w), 300, 1e-6)
    assert np.array_equal(bits(a), bits(b))
    s1 = (rng.standard_normal(77) * 30).astype(np.float32)
    s2 = s1.copy()
    L.orc_softmax(p(s1), 77)
    R.op_softmax(p(s2), 77)
    assert np.array_equal(bits(s1), bits(s2))
    for hd, theta in ((16, 1e4), (128, 1e6)):
        c1, n1 = np.empty((50, hd // 2), np.float32), np.empty((50, hd // 2), np.float32)
        c2, n2 = np.empty_like(c1), np.empty_like(n1)
        L.orc_rope_table(p(c1), p(n1), 50, hd, theta)
        R.op_rope_table(p(c2), p(n2), 50, hd, theta)
        assert np.array_equal(bits(c1), bits(c2)) and np.array_equal(bits(n1), bits(n2))
    q = rng.standard_normal((6, 8)).astype(np.float32)
    kc = rng.standard_normal((2, 20, 8)).astype(np.float32)
    vc = rng.standard_normal((2, 20, 8)).astype(np.float32)
    o1, o2, sc = np.empty_like(q), np.empty_like(q), np.empty(20, np.float32)
    L.orc_attention(p(o1), p(q), p(kc), p(vc), 6, 2, 8, 13, 20, p(sc), 1)
    R.op_attention(p(o2), p(q), p(kc), p(vc), 6, 2, 8, 13, 20, p(sc))
    assert np.array_equal(bits(o1), bits(o2))


@needs_ref
@pytest.mark.parametrize("variant", ["dense_q0", "moe_q8"])
def test_live_reference_forward(tmp_path, variant):
    from sardyne_amd.gguf_synth import ModelSpec, write_model
    spec = {"dense_q0": ModelSpec(n_vocab=200, dim=256, n_layer=2, n_head=4, n_kv_head=2, head_dim=64, ffn_dim=512,
                                  context=64, t_default="Q8_0", t_attn_v="Q4_0", t_ffn_down="Q5_0", t_output="Q8_0",
                                  t_embd="Q4_0"),
            "moe_q8": ModelSpec(arch="qwen3moe", n_vocab=200, dim=128, n_layer=2, n_head=4, n_kv_head=2, head_dim=32,
                                ffn_dim=256, context=64, n_expert=8, n_expert_used=3, ffn_exp_dim=64, qkv_bias=False,
                                qk_norm=True, t_default="Q8_0", t_attn_v="Q8_0", t_ffn_down="Q8_0", t_output="Q8_0",
                                t_embd="Q8_0", router_std=0.3)}[variant]
    p = tmp_path / "m.gguf"
    write_model(p, spec, seed=3)
    toks = [3, 14, 15, 9, 26, 5, 35, 8, 2, 7]
    for n_batch, la in ((10, True), (3, True), (4, False)):
        a = O.OracleContext(p, 32, n_batch, la).eval(toks)
        b = O.RefEngine(p, 32, n_batch, la).eval(toks)
        assert np.array_equal(bits(a), bits(b)), (n_batch, la)


# ---------------------------------------------------------------- 3. closed forms and invariants

def f16(b):
    return np.ascontiguousarray(b).view(np.float16).astype(np.float32).reshape(-1)


def test_f16_to_f32_exhaustive():
    h = np.arange(1 << 16, dtype=np.uint16)
    out = np.empty(1 << 16, np.float32)
    O.lib().orc_f16_to_f32_n(O.ptr(h), O.ptr(out), h.size)
    exp = h.view(np.float16).astype(np.float32)
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(out), nan)
    assert np.array_equal(bits(out)[~nan], bits(exp)[~nan])


def test_f32_to_f16_matches_numpy_rounding():
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000)).astype(np.float32)
    v = np.concatenate([v, np.array([65504, 65519, 65520, 7e4, 6e-8, 3e-8, 2.98e-8, 0, -0.0, 5.96e-8, np.inf, -np.inf],
                                    np.float32)])
    got = np.array([O.lib().orc_f32_to_f16(float(x)) for x in v], np.uint16)
    with np.errstate(over="ignore"):
        assert np.array_equal(got, v.astype(np.float16).view(np.uint16))


def np_q4k_scales(s):
    s = s.astype(np.int32)
    sc, m = np.empty((s.shape[0], 8), np.int32), np.empty((s.shape[0], 8), np.int32)
    sc[:, :4], m[:, :4] = s[:, 0:4] & 63, s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, m


def np_q6k_values(b):
    out = np.empty((b.shape[0], 256), np.int32)
    for half in range(2):
        ql = b[:, 64 * half:64 * half + 64].astype(np.int32)
        qh = b[:, 128 + 32 * half:160 + 32 * half].astype(np.int32)
        for k in range(4):
            lo = ql[:, 32 * (k & 1):32 * (k & 1) + 32]
            lo = (lo >> 4) if k >= 2 else (lo & 15)
            out[:, 128 * half + 32 * k:128 * half + 32 * k + 32] = lo | (((qh >> (2 * k)) & 3) << 4)
    return out - 32


def test_dequant_closed_forms():
    rng = np.random.default_rng(11)
    b = random_blocks("Q4_K", 64, rng)
    d, dmin = f16(b[:, 0:2]), f16(b[:, 2:4])
    sc, m = np_q4k_scales(b[:, 4:16])
    qs = b[:, 16:].reshape(-1, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32).astype(np.float32)
    d1 = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
    m1 = (dmin[:, None] * m.astype(np.float32)).astype(np.float32)
    exp = ((d1[:, :, None] * q).astype(np.float32) - m1[:, :, None]).reshape(-1)
    assert np.array_equal(bits(O.dequant(b, O.Q4_K, 64 * 256)), bits(exp))
    b = random_blocks("Q6_K", 64, rng)
    d = f16(b[:, 208:210])
    s = b[:, 192:208].view(np.int8).astype(np.float32)
    exp = (((d[:, None] * s)[:, :, None]) * np_q6k_values(b).reshape(-1, 16, 16).astype(np.float32)).reshape(-1)
    assert np.array_equal(bits(O.dequant(b, O.Q6_K, 64 * 256)), bits(exp.astype(np.float32)))
    b = random_blocks("Q8_0", 64, rng)
    exp = (b[:, 2:].view(np.int8).astype(np.float32) * f16(b[:, 0:2])[:, None]).reshape(-1)
    assert np.array_equal(bits(O.dequant(b, O.Q8_0, 64 * 32)), bits(exp))


def test_q8k_quantizer_invariants():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((6, 256)).astype(np.float32) * np.array([[1], [1e-3], [50], [1], [1], [1]], np.float32)
    x[3] = 0
    x[4, 5], x[4, 9] = -7.0, 7.0       # equal magnitudes: the first sets the sign
    x[5, :] = 0.5
    x[5, 3] = 2.0                      # +127 exactly, others 0.5*127/2 = 31.75 -> 32
    q = O.quantize(x, O.Q8_K).reshape(6, 292)
    d = q[:, 0:4].copy().view("<f4")[:, 0]
    qs = q[:, 4:260].view(np.int8).astype(np.int32)
    bs = q[:, 260:292].copy().view("<i2").astype(np.int32)
    assert np.array_equal(bs, qs.reshape(6, 16, 16).sum(axis=2))
    assert np.all(q[3] == 0)
    for r in (0, 1, 2, 4, 5):
        vmax = x[r][np.argmax(np.abs(x[r]))]
        iscale = np.float32(-127) / np.float32(vmax)
        exp = np.minimum(127, np.rint((x[r] * iscale).astype(np.float32))).astype(np.int32)
        assert np.array_equal(qs[r], exp), r
        assert d[r] == np.float32(1) / iscale
    assert qs[4, 5] == -127 and qs[4, 9] == 127 and d[4] > 0  # sign of the first maximum (-7)


def test_q8_0_quantizer_closed_form():
    rng = np.random.default_rng(13)
    x = (rng.standard_normal((4, 64)) * 3).astype(np.float32)
    x[1, :32] = 0
    x[2, 0] = 0.5 * 127 / 127  # exact halves round away from zero
    q = O.quantize(x, O.Q8_0).reshape(-1, 34)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, 1), 0).astype(np.float32)
    v = (xb * inv[:, None]).astype(np.float64)
    exp = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int8)
    assert np.array_equal(q[:, 2:].view(np.int8), exp)
    assert np.array_equal(q[:, 0:2].copy().view(np.float16).reshape(-1), d.astype(np.float16))


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
def test_kquant_dot_exact_integer_parts(kind):
    """Brute-force int64 super-block sums and the documented f32 combine order reproduce the
    oracle's dot bit for bit; perturbing a scale index or a sign breaks it."""
    rng = np.random.default_rng(14)
    n = 1024
    w = random_blocks(kind, n // 256, rng)
    x = rng.standard_normal(n).astype(np.float32)
    xq = O.quantize(x, O.Q8_K).reshape(-1, 292)
    yd = xq[:, 0:4].copy().view("<f4")[:, 0]
    y = xq[:, 4:260].view(np.int8).astype(np.int64)
    acc = np.float32(0)
    for i in range(n // 256):
        if kind == "Q4_K":
            sc, m = np_q4k_scales(w[i:i + 1, 4:16])
            qs = w[i, 16:].reshape(4, 32).astype(np.int64)
            q = np.stack([qs & 15, qs >> 4], axis=1).reshape(8, 32)
            isum = int((sc[0].astype(np.int64) * (q * y[i].reshape(8, 32)).sum(axis=1)).sum())
            bsum = y[i].reshape(16, 16).sum(axis=1).reshape(8, 2).sum(axis=1)
            msum = int((m[0].astype(np.int64) * bsum).sum())
            d, dmin = f16(w[i, 0:2])[0], f16(w[i, 2:4])[0]
            dall, dmn = np.float32(yd[i] * d), np.float32(yd[i] * dmin)
            acc = np.float32(acc + np.float32(np.float32(dall * np.float32(isum)) - np.float32(dmn * np.float32(msum))))
        else:
            v = np_q6k_values(w[i:i + 1])[0].astype(np.int64).reshape(16, 16)
            s = w[i, 192:208].view(np.int8).astype(np.int64)
            isum = int((s * (v * y[i].reshape(16, 16)).sum(axis=1)).sum())
            d = f16(w[i, 208:210])[0]
            acc = np.float32(acc + np.float32(np.float32(yd[i] * d) * np.float32(isum)))
    t = O.Q4_K if kind == "Q4_K" else O.Q6_K
    got = O.lib().orc_dot_scalar(t, O.ptr(np.ascontiguousarray(w.reshape(-1))), O.ptr(np.ascontiguousarray(xq.reshape(-1))), n)
    assert np.float32(got) == acc


def test_rmsnorm_and_softmax_closed_form():
    rng = np.random.default_rng(15)
    x = (rng.standard_normal(2048) * 7).astype(np.float32)
    w = rng.standard_normal(2048).astype(np.float32)
    out = np.empty_like(x)
    O.lib().orc_rmsnorm(O.ptr(out), O.ptr(x), O.ptr(w), 2048, 1e-6)
    ss = math.fsum(float(v) * float(v) for v in x)
    scale = np.float32(1.0 / math.sqrt(ss / 2048 + float(np.float32(1e-6))))
    np.testing.assert_array_equal(out, (x * scale).astype(np.float32) * w)
    s = (rng.standard_normal(100) * 20).astype(np.float32)
    e = np.exp((s - s.max()).astype(np.float64))  # the subtraction rounds in f32, as in the reference
    O.lib().orc_softmax(O.ptr(s), 100)
    np.testing.assert_allclose(s, e / e.sum(), rtol=2e-6, atol=1e-40)  # f32 subnormals lose relative precision


def test_rope_table_closed_form():
    c, s = np.empty((64, 64), np.float32), np.empty((64, 64), np.float32)
    O.lib().orc_rope_table(O.ptr(c), O.ptr(s), 64, 128, 1e6)
    inv = 1.0 / np.power(np.float64(np.float32(1e6)), np.arange(0, 128, 2) / 128.0)
    ang = np.arange(64)[:, None] * inv[None, :]
    np.testing.assert_allclose(c, np.cos(ang), atol=1e-7)
    np.testing.assert_allclose(s, np.sin(ang), atol=1e-7)


def test_oracle_moe_invariants(tmp_path):
    """The oracle's MoE against what the mathematics fixes, with the same cases as the GPU tests
    (tests/test_moe.py:147-157, 370-406 of the reference): NaN-poisoned unused experts change no bit;
    identical experts equal the dense MLP within rounding; an all-zero router routes to the lowest k
    experts (poisoning the others changes no bit), with the reference engine's bits."""
    import dataclasses
    from moe_cases import MOE, PROMPT, STEPS, poison_experts, used_experts
    from sardyne_amd.gguf_synth import write_model

    def run(p):
        r = O.OracleContext(p, 48, n_batch=16)
        return np.stack([r.eval(PROMPT)] + [r.eval([t]) for t in STEPS])

    clean_p = write_model(tmp_path / "c.gguf", MOE, seed=3)
    unused = [sorted(set(range(MOE.n_expert)) - u) for u in used_experts(clean_p)]
    dirty_p = write_model(tmp_path / "d.gguf", MOE, seed=3)
    poison_experts(dirty_p, unused)
    a, b = run(clean_p), run(dirty_p)
    assert np.all(np.isfinite(a)) and np.array_equal(a.view(np.uint32), b.view(np.uint32))
    moe = dataclasses.replace(MOE, n_expert=8, n_expert_used=3, same_experts=True)
    dense = dataclasses.replace(MOE, arch="qwen3", ffn_dim=MOE.ffn_exp_dim, n_expert=0, n_expert_used=0, ffn_exp_dim=0)
    g, e = run(write_model(tmp_path / "m.gguf", moe, seed=4)), run(write_model(tmp_path / "n.gguf", dense, seed=4))
    np.testing.assert_allclose(g, e, atol=1e-4 * max(1.0, float(np.abs(e).max())), rtol=0)
    spec = dataclasses.replace(MOE, n_expert=16, n_expert_used=4, router_std=0.0)
    z = write_model(tmp_path / "z.gguf", spec, seed=5)
    h = write_model(tmp_path / "h.gguf", spec, seed=5)
    poison_experts(h, [range(4, 16)] * spec.n_layer)
    a, b = run(z), run(h)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    if O.ref_available():
        R = O.RefEngine(z, 48, n_batch=16)
        r = np.stack([R.eval(PROMPT)] + [R.eval([t]) for t in STEPS])
        assert np.array_equal(a.view(np.uint32), r.view(np.uint32))


def test_c5_spread_fixture_is_for_the_c5_test():
    """golden/c5_simd_spread.npz (made by golden/make_c5_spread.py from the reference compiled from its
    sources) is the AVX2-vs-scalar spread of the reference engine on the C5 test's model and tokens:
    its token digest matches the test's tokens, both engines agree on every argmax, and the spread is
    a rounding-level drift (between 1e-4 and 1e-2 of the logit scale) that the test's bound follows."""
    g = np.load(GOLDEN / "c5_simd_spread.npz")
    toks = np.random.default_rng(1).integers(0, 151936, 1024 + 5).astype(np.int32)
    assert str(g["tok_sha"]) == hashlib.sha256(toks.tobytes()).hexdigest()
    assert g["spread"].shape == (6,) and bool(np.all(g["argmax_equal"]))
    rel = float(g["spread"].max()) / float(g["scale"])
    assert 1e-4 < rel < 1e-2

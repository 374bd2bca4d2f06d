"""GPU kernels against the oracle (oracle/, a CPU restatement of the reference pinned to the
compiled reference): dequantisation and activation quantisation bit/byte-exact, K-quant matvec
bit-exact, 32-element-block matvec within rel 1e-5, float kernels within the tolerances of the
reference's own tests (tests/test_runtime.py:100-152, tests/test_quant.py:120-205).

Every test calls the C ABI of build/libsardyne.so (op_* host entry points or the sdy_* device
entry points)."""
import ctypes

import numpy as np
import pytest

import oracle as O
from sardyne_amd import capi
from sardyne_amd.gguf_synth import random_blocks

pytestmark = pytest.mark.gpu

TYPES = {"Q8_0": O.Q8_0, "Q4_0": O.Q4_0, "Q5_0": O.Q5_0, "Q4_K": O.Q4_K, "Q6_K": O.Q6_K}


def lib():
    return capi.lib()


def ptr(a):
    return a.ctypes.data


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def ref_blocks(kind, n_blocks, seed):
    """The reference's test generator distribution (tests/test_quant.py:24-36): uniform bytes, f16
    scales U(1e-4, 1e-2), Q6_K int8 scales in [-60, 60)."""
    rng = np.random.default_rng(seed)
    size = O.BLOCK_BYTES[TYPES[kind]]
    b = rng.integers(0, 256, (n_blocks, size), dtype=np.uint8)
    scale = lambda: rng.uniform(1e-4, 1e-2, n_blocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
    if kind in ("Q8_0", "Q4_0", "Q5_0"):
        b[:, 0:2] = scale()
    elif kind == "Q4_K":
        b[:, 0:2], b[:, 2:4] = scale(), scale()
    elif kind == "Q6_K":
        b[:, 208:210] = scale()
        b[:, 192:208] = rng.integers(-60, 60, (n_blocks, 16)).astype(np.int8).view(np.uint8)
    return b


def test_f16_to_f32_all_values():
    h = np.arange(1 << 16, dtype=np.uint16)
    out = np.empty(1 << 16, np.float32)
    lib().op_f16_to_f32_n(ptr(h), ptr(out), h.size)
    exp = np.empty_like(out)
    O.lib().orc_f16_to_f32_n(ptr(h), ptr(exp), h.size)
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(out), nan)
    assert np.array_equal(bits(out)[~nan], bits(exp)[~nan])


def test_f32_to_f16_edge_values():
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(200) * 10.0 ** rng.integers(-9, 6, 200)).astype(np.float32)
    v = np.concatenate([v, np.array([65504, 65519, 65520, 7e4, 6e-8, 3e-8, 2.98e-8, 0, -0.0, 5.96e-8, np.inf,
                                     -np.inf, 1e-45, -3.1e-5], np.float32)])
    got = np.array([lib().op_f32_to_f16(float(x)) for x in v], np.uint16)
    exp = np.array([O.lib().orc_f32_to_f16(float(x)) for x in v], np.uint16)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("kind", list(TYPES))
@pytest.mark.parametrize("gen", ["reference", "workload"])
def test_dequant_bit_exact(kind, gen):
    t = TYPES[kind]
    n = 2048
    nb = n // O.QK[t]
    raw = ref_blocks(kind, nb, 4) if gen == "reference" else random_blocks(kind, nb, np.random.default_rng(4))
    raw = np.ascontiguousarray(raw).reshape(-1)
    out = np.empty(n, np.float32)
    lib().op_row_to_f32(ptr(raw), t, ptr(out), n)
    assert np.array_equal(bits(out), bits(O.dequant(raw, t, n)))


@pytest.mark.parametrize("vt", [O.Q8_0, O.Q8_K], ids=["Q8_0", "Q8_K"])
def test_activation_quantization_byte_exact(vt):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((5, 512)) * np.array([[1e-3], [1.0], [300.0], [1.0], [1e-30]])).astype(np.float32)
    x[1, :256] = 0  # all-zero block
    x[2, 7] = 1e4  # one dominant value
    x[3, 10], x[3, 20] = -4.0, 4.0  # equal magnitudes: the first one sets the sign
    x[3, 300] = 2.5
    x = np.concatenate([x, _quant_edge_rows(512, np.random.default_rng(6))])
    n_rows, n = x.shape
    out = np.zeros(O.row_size(vt, n) * n_rows, np.uint8)
    lib().op_quantize_rows(vt, ptr(x), ptr(out), n, 0, n_rows)
    assert out.tobytes() == O.quantize(x, vt).tobytes()
    if O.ref_available():
        assert out.tobytes() == O.quantize(x, vt, use_ref=True).tobytes()


def _quant_edge_rows(n, rng):
    """Rows whose 256-element blocks hold the quantisers' edge cases: NaN elements beside finite
    ones (NaN never sets the scale), a block of NaN but one finite element, an all-NaN block (all
    zero bytes), equal magnitudes of opposite sign in one lane and across lanes (the first one in
    index order sets the sign), infinities (the scale from an infinite maximum), a block holding
    only a value of the smallest subnormal magnitude."""
    x = rng.standard_normal((4, n)).astype(np.float32)
    x[0, [3, 100, 255]] = np.nan
    x[0, 256:512] = np.nan
    x[0, 256 + 77] = -3.0
    x[1, 0:256] = np.nan
    x[1, 256 + 8], x[1, 256 + 10] = -5.0, 5.0  # one lane (elements 8..11)
    x[1, 256 + 40], x[1, 256 + 200] = 5.0, -5.0  # later lanes, the same magnitude
    x[2, 50] = np.inf
    x[2, 256 + 4], x[2, 256 + 9] = -np.inf, np.inf
    x[3, 0:256] = 0.0
    x[3, 17] = -1e-45
    return x


def _matvec_case(kind, n_in, n_out, n_tok, seed, gen="workload"):
    t = TYPES[kind]
    nb = n_out * n_in // O.QK[t]
    if gen == "workload":
        w = random_blocks(kind, nb, np.random.default_rng(seed)).reshape(n_out, -1)
    else:
        w = ref_blocks(kind, nb, seed).reshape(n_out, -1)
    x = np.random.default_rng(seed + 1).standard_normal((n_tok, n_in)).astype(np.float32)
    xq = O.quantize(x, O.VEC_DOT[t])
    return t, w, xq


@pytest.mark.parametrize("kind", list(TYPES))
@pytest.mark.parametrize("n_in,n_out,n_tok", [(256, 13, 1), (512, 13, 3), (2048, 37, 1), (768, 20, 5),
                                              (11008, 9, 2), (4096, 16, 9), (2048, 64, 8), (768, 41, 1),
                                              (1280, 23, 1), (2560, 7, 1), (11008, 33, 1), (8192, 20, 1),
                                              (16384, 5, 1)])
def test_matvec_vs_oracle(kind, n_in, n_out, n_tok):
    if kind in ("Q8_0", "Q4_0", "Q5_0") and n_in % 32:
        pytest.skip("row not a whole number of blocks")
    t, w, xq = _matvec_case(kind, n_in, n_out, n_tok, seed=n_in + n_out)
    out = np.full((n_tok, n_out), np.nan, np.float32)
    lib().op_matmul_q_rows(ptr(out), ptr(xq), ptr(w), t, n_tok, n_in, n_out, 0, n_out)
    if t in (O.Q4_K, O.Q6_K):
        # integer super-block sums and the reference's f32 combine order: identical bits
        exp = O.matmul_q(w, t, xq, n_in, simd=1)
        assert np.array_equal(bits(out), bits(exp))
    else:
        exp = O.matmul_q(w, t, xq, n_in, simd=0)
        np.testing.assert_allclose(out, exp, rtol=1e-5, atol=1e-5 * float(np.abs(exp).max()))
        exp2 = O.matmul_q(w, t, xq, n_in, simd=1)
        np.testing.assert_allclose(out, exp2, rtol=1e-5, atol=1e-5 * float(np.abs(exp).max()))


@pytest.mark.parametrize("kind", list(TYPES))
def test_matvec_row_ranges(kind):
    n_in, n_out, n_tok = 512, 13, 3
    t, w, xq = _matvec_case(kind, n_in, n_out, n_tok, seed=10, gen="reference")
    full = np.empty((n_tok, n_out), np.float32)
    lib().op_matmul_q_rows(ptr(full), ptr(xq), ptr(w), t, n_tok, n_in, n_out, 0, n_out)
    parts = np.full_like(full, np.nan)
    for r0, r1 in [(0, 5), (5, 6), (6, n_out)]:
        lib().op_matmul_q_rows(ptr(parts), ptr(xq), ptr(w), t, n_tok, n_in, n_out, r0, r1)
    assert np.array_equal(bits(parts), bits(full))


@pytest.mark.parametrize("kind", list(TYPES))
def test_vec_dot(kind):
    t = TYPES[kind]
    n = 1024
    w = ref_blocks(kind, n // O.QK[t], 6).reshape(-1)
    x = np.random.default_rng(7).standard_normal(n).astype(np.float32)
    xq = O.quantize(x, O.VEC_DOT[t]).reshape(-1)
    got = lib().op_vec_dot_q(t, ptr(w), ptr(xq), n)
    exp = float(O.matmul_q(w, t, xq, n, simd=0)[0, 0])
    assert got == pytest.approx(exp, rel=1e-5, abs=1e-5)
    wd = O.dequant(w, t, n).astype(np.float64)
    assert abs(got - float(wd @ x)) <= 0.01 * float(np.linalg.norm(wd) * np.linalg.norm(x))


def test_matvec_device_api_deterministic():
    """Same inputs, two launches, identical bits; also checks the device-resident entry points."""
    t = O.Q6_K
    n_in, n_out = 2048, 1000
    w = random_blocks("Q6_K", n_out * n_in // 256, np.random.default_rng(1)).reshape(n_out, -1)
    x = np.random.default_rng(2).standard_normal(n_in).astype(np.float32)
    L = lib()
    m = capi.DeviceMatrix(t, n_in, n_out, w)
    dx = capi.DeviceBuffer.from_array(x)
    dq = capi.DeviceBuffer(O.row_size(O.Q8_K, n_in))
    dout = capi.DeviceBuffer(n_out * 4)
    capi.check(L.sdy_quantize(O.Q8_K, dx.ptr, dq.ptr, n_in, 1, None))
    a = capi.SdyMvArgs(xq=dq.ptr, n_tok=1, out=dout.ptr, out_stride=n_out, row0=0, row1=n_out)
    capi.check(L.sdy_matvec(ctypes.byref(m.m), ctypes.byref(a), None))
    y1 = dout.to_array(np.float32, n_out)
    capi.check(L.sdy_matvec(ctypes.byref(m.m), ctypes.byref(a), None))
    y2 = dout.to_array(np.float32, n_out)
    assert np.array_equal(bits(y1), bits(y2))
    exp = O.matmul_q(w, t, O.quantize(x, O.Q8_K), n_in)[0]
    assert np.array_equal(bits(y1), bits(exp))


@pytest.mark.parametrize("wtype", [O.F32, O.F16, O.BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("n_tok", [1, 3, 4, 9])
@pytest.mark.parametrize("n_in", [67, 96, 2048, 2340])
def test_float_matmul(wtype, n_tok, n_in):
    rng = np.random.default_rng(0)
    n_out = 45
    x = rng.standard_normal((n_tok, n_in)).astype(np.float32)
    w32 = rng.standard_normal((n_out, n_in)).astype(np.float32)
    if wtype == O.F16:
        w = w32.astype(np.float16)
        w_ref = w.astype(np.float32)
    elif wtype == O.BF16:
        b = w32.view(np.uint32)
        w = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
        w_ref = (w.astype(np.uint32) << 16).view(np.float32)
    else:
        w, w_ref = w32, w32
    w = np.ascontiguousarray(w)
    out = np.empty((n_tok, n_out), np.float32)
    lib().op_matmul(ptr(out), ptr(x), ptr(w), wtype, n_tok, n_in, n_out)
    exact = x.astype(np.float64) @ w_ref.T.astype(np.float64)
    if n_in <= 96:  # the reference's own sizes and tolerance (tests/test_runtime.py:100-152)
        np.testing.assert_allclose(out, x @ w_ref.T, rtol=1e-5, atol=1e-5)
    else:  # long rows: the f32 error bound of n_in / 64 chained FMAs per lane and a 6-level tree
        bound = (n_in / 64 + 8) * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(w_ref).T)
        assert np.all(np.abs(out - exact) <= bound)
    parts = np.full_like(out, np.nan)
    for r0, r1 in [(0, 10), (10, 30), (30, n_out)]:
        lib().op_matmul_rows(ptr(parts), ptr(x), ptr(w), wtype, n_tok, n_in, n_out, r0, r1)
    assert np.array_equal(bits(parts), bits(out))


def test_rmsnorm_softmax_silu():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(300) * 5).astype(np.float32)
    w = rng.standard_normal(300).astype(np.float32)
    out = np.empty_like(x)
    lib().op_rmsnorm(ptr(out), ptr(x), ptr(w), x.size, 1e-5)
    exp = np.empty_like(x)
    O.lib().orc_rmsnorm(ptr(exp), ptr(x), ptr(w), x.size, 1e-5)
    assert np.array_equal(bits(out), bits(exp))  # double sum, one float rounding: same bits
    s = np.array([1000.0, 1001.0, -50.0, 3.0], np.float32)
    e = s.copy()
    O.lib().orc_softmax(ptr(e), e.size)
    lib().op_softmax(ptr(s), s.size)
    np.testing.assert_allclose(s, e, rtol=1e-6)
    g = np.array([-100.0, -1.0, 0.0, 2.0, 50.0], np.float32)
    up = np.array([3.0, 2.0, 1.0, -1.0, 0.5], np.float32)
    e = g.copy()
    O.lib().orc_silu_mul(ptr(e), ptr(up), g.size)
    lib().op_silu_mul(ptr(g), ptr(up), g.size)
    np.testing.assert_allclose(g, e, rtol=1e-6, atol=1e-30)


@pytest.mark.parametrize("interleaved", [0, 1], ids=["neox", "interleaved"])
def test_rope(interleaved):
    n_pos, hd, n_heads, theta = 40, 16, 3, 10000.0
    cos, sin = np.empty((n_pos, hd // 2), np.float32), np.empty((n_pos, hd // 2), np.float32)
    lib().op_rope_table(ptr(cos), ptr(sin), n_pos, hd, theta)
    ec, es = np.empty_like(cos), np.empty_like(sin)
    O.lib().orc_rope_table(ptr(ec), ptr(es), n_pos, hd, theta)
    assert np.array_equal(bits(cos), bits(ec)) and np.array_equal(bits(sin), bits(es))
    x = np.random.default_rng(2).standard_normal((n_heads, hd)).astype(np.float32)
    e = x.copy()
    rc, rs = np.ascontiguousarray(ec[33]), np.ascontiguousarray(es[33])
    O.lib().orc_rope(ptr(e), n_heads, hd, ptr(rc), ptr(rs), interleaved)
    lib().op_rope(ptr(x), n_heads, hd, ptr(rc), ptr(rs), interleaved)
    assert np.array_equal(bits(x), bits(e))


@pytest.mark.parametrize("n_kv", [1, 13, 64, 65, 200])
def test_attention_gqa(n_kv):
    rng = np.random.default_rng(3)
    n_head, n_kv_head, hd, stride = 6, 2, 8, 256
    q = rng.standard_normal((n_head, hd)).astype(np.float32)
    kc = rng.standard_normal((n_kv_head, stride, hd)).astype(np.float32)
    vc = rng.standard_normal((n_kv_head, stride, hd)).astype(np.float32)
    out = np.empty_like(q)
    scores = np.empty(stride, np.float32)
    lib().op_attention(ptr(out), ptr(q), ptr(kc), ptr(vc), n_head, n_kv_head, hd, n_kv, stride, ptr(scores))
    exp = np.empty_like(q)
    O.lib().orc_attention(ptr(exp), ptr(q), ptr(kc), ptr(vc), n_head, n_kv_head, hd, n_kv, stride, ptr(scores), 1)
    # the reference's arithmetic (AVX2 dot, libm expf, in-order axpy): the same bits
    assert np.array_equal(bits(out), bits(exp))


def test_dot_axpy_add():
    rng = np.random.default_rng(4)
    for n in (1, 7, 8, 64, 100):
        a, b = rng.standard_normal((2, n)).astype(np.float32)
        assert lib().op_dot_f32(ptr(a), ptr(b), n) == pytest.approx(float(a.astype(np.float64) @ b), rel=1e-5, abs=1e-5)
        y = rng.standard_normal(n).astype(np.float32)
        expected = y + np.float32(0.5) * a
        lib().op_axpy(ptr(y), 0.5, ptr(a), n)
        np.testing.assert_allclose(y, expected, rtol=1e-6, atol=1e-6)
    a = rng.standard_normal(1023).astype(np.float32)
    b = rng.standard_normal(1023).astype(np.float32)
    np.testing.assert_array_equal(capi.add(a, b), a + b)


@pytest.mark.parametrize("vt,n,n_rows", [(O.Q8_K, 2048, 1), (O.Q8_K, 4096, 3), (O.Q8_0, 2048, 2), (O.Q8_0, 96, 1),
                                         (O.F32, 200, 2)], ids=["q8k", "q8k-3rows", "q8_0", "q8_0-odd", "f32"])
def test_norm_quant_equals_rmsnorm_then_quantize(vt, n, n_rows):
    """The fused RMSNorm + activation quantiser writes the bytes of the two separate kernels, and
    those equal the oracle's rmsnorm followed by the reference quantiser."""
    L = lib()
    rng = np.random.default_rng(n + n_rows)
    x = (rng.standard_normal((n_rows, n)) * 3).astype(np.float32)
    x[0, 5] = 40.0  # a dominant element
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    dx, dw = capi.DeviceBuffer.from_array(x), capi.DeviceBuffer.from_array(w)
    db1, db2 = capi.DeviceBuffer(x.nbytes), capi.DeviceBuffer(x.nbytes)
    qbytes = O.row_size(vt, n) * n_rows if vt != O.F32 else 64
    dq1, dq2 = capi.DeviceBuffer(qbytes), capi.DeviceBuffer(qbytes)
    capi.check(L.sdy_rmsnorm(dx.ptr, dw.ptr, db1.ptr, n, 1e-6, n_rows, n, n, None))
    if vt != O.F32:
        capi.check(L.sdy_quantize(vt, db1.ptr, dq1.ptr, n, n_rows, None))
    capi.check(L.sdy_norm_quant(dx.ptr, dw.ptr, 1e-6, n, n_rows, db2.ptr, vt, dq2.ptr if vt != O.F32 else None, None))
    xb1, xb2 = db1.to_array(np.float32, (n_rows, n)), db2.to_array(np.float32, (n_rows, n))
    assert np.array_equal(bits(xb1), bits(xb2))
    exp = np.empty_like(x)
    for r in range(n_rows):
        O.lib().orc_rmsnorm(ptr(exp[r]), ptr(x[r]), ptr(w), n, 1e-6)
    assert np.array_equal(bits(xb2), bits(exp))
    if vt != O.F32:
        q1, q2 = dq1.to_array(np.uint8, qbytes), dq2.to_array(np.uint8, qbytes)
        assert np.array_equal(q1, q2)
        assert np.array_equal(q2, O.quantize(exp, vt).reshape(-1))


@pytest.mark.parametrize("k1,k2", [("Q4_K", "Q6_K"), ("Q6_K", "Q4_K"), ("Q4_K", "Q4_K"), ("Q6_K", "Q6_K")])
@pytest.mark.parametrize("n_in,n1,n2,swiglu", [(2048, 2560, 256, False), (768, 70, 33, False), (2048, 40, 96, True),
                                               (4096, 40, 96, False), (256, 17, 1000, False)])
def test_matvec_pair(k1, k2, n_in, n1, n2, swiglu):
    """Two one-token matvecs on one Q8_K row in one launch (a layer's q|k and v): each output has
    the bits of its own sdy_matvec call (bias on the first, residual or SwiGLU on the second)."""
    L = lib()
    rng = np.random.default_rng(n_in + n1 + n2)
    w1 = random_blocks(k1, n1 * n_in // 256, rng).reshape(n1, -1)
    w2 = random_blocks(k2, n2 * n_in // 256, rng).reshape(n2, -1)
    m1, m2 = capi.DeviceMatrix(TYPES[k1], n_in, n1, w1), capi.DeviceMatrix(TYPES[k2], n_in, n2, w2)
    x = rng.standard_normal((1, n_in)).astype(np.float32)
    dq = capi.DeviceBuffer.from_array(O.quantize(x, O.Q8_K))
    bias = capi.DeviceBuffer.from_array(rng.standard_normal(n1).astype(np.float32))
    o2 = n2 // 2 if swiglu else n2
    resid = capi.DeviceBuffer.from_array(rng.standard_normal(o2).astype(np.float32))
    epi2 = capi.EPI_SWIGLU if swiglu else capi.EPI_NONE
    assert L.sdy_matvec_pair_ok(ctypes.byref(m1.m), capi.EPI_NONE, ctypes.byref(m2.m), epi2) == 1
    outs = [capi.DeviceBuffer.from_array(np.full(n, np.nan, np.float32)) for n in (n1, o2, n1, o2)]
    args = []
    for i in (0, 2):
        a1 = capi.SdyMvArgs(xq=dq.ptr, n_tok=1, out=outs[i].ptr, out_stride=n1, bias=bias.ptr, row0=0, row1=n1)
        a2 = capi.SdyMvArgs(xq=dq.ptr, n_tok=1, out=outs[i + 1].ptr, out_stride=o2, resid=None if swiglu else resid.ptr,
                            row0=0, row1=n2, epilogue=epi2)
        args.append((a1, a2))
    capi.check(L.sdy_matvec_pair(ctypes.byref(m1.m), ctypes.byref(args[0][0]), ctypes.byref(m2.m),
                                 ctypes.byref(args[0][1]), None))
    capi.check(L.sdy_matvec(ctypes.byref(m1.m), ctypes.byref(args[1][0]), None))
    capi.check(L.sdy_matvec(ctypes.byref(m2.m), ctypes.byref(args[1][1]), None))
    got = [outs[i].to_array(np.float32, n) for i, n in enumerate((n1, o2, n1, o2))]
    assert np.array_equal(bits(got[0]), bits(got[2]))
    assert np.array_equal(bits(got[1]), bits(got[3]))
    assert not np.isnan(got[0]).any() and not np.isnan(got[1]).any()


def test_matvec_pair_rejects_unsupported():
    """The paired launch is for Q4_K / Q6_K rows of at most 64 units and one token."""
    L = lib()
    rng = np.random.default_rng(5)
    a = capi.DeviceMatrix(O.Q4_K, 11008, 4, random_blocks("Q4_K", 4 * 43, rng).reshape(4, -1))
    b = capi.DeviceMatrix(O.Q8_0, 256, 4, random_blocks("Q8_0", 4 * 8, rng).reshape(4, -1))
    c = capi.DeviceMatrix(O.Q6_K, 256, 4, random_blocks("Q6_K", 4, rng).reshape(4, -1))
    assert L.sdy_matvec_pair_ok(ctypes.byref(a.m), capi.EPI_NONE, ctypes.byref(c.m), capi.EPI_NONE) == 0
    assert L.sdy_matvec_pair_ok(ctypes.byref(c.m), capi.EPI_NONE, ctypes.byref(b.m), capi.EPI_NONE) == 0
    out = capi.DeviceBuffer(64)
    x = capi.DeviceBuffer(292)
    a1 = capi.SdyMvArgs(xq=x.ptr, n_tok=2, out=out.ptr, out_stride=4, row0=0, row1=4)
    assert L.sdy_matvec_pair(ctypes.byref(c.m), ctypes.byref(a1), ctypes.byref(c.m), ctypes.byref(a1), None) != 0


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("n_in,n_out", [(2048, 22016), (1024, 40000), (1024, 72000), (1024, 110000), (768, 30000),
                                        (512, 151936)])
def test_matvec_one_token_large(kind, n_in, n_out):
    """One-token matvecs with enough rows that a wave takes several row iterations (up to the
    persistent kernel at the largest): every row has the oracle's bits, also with a bias and a
    residual over a row range whose ends are not iteration boundaries; rows outside stay untouched."""
    L = lib()
    t, w, xq = _matvec_case(kind, n_in, n_out, 1, seed=n_out)
    exp = O.matmul_q(w, t, xq, n_in, simd=1)[0]
    rng = np.random.default_rng(n_out + 1)
    bias = rng.standard_normal(n_out).astype(np.float32)
    resid = rng.standard_normal(n_out).astype(np.float32)
    m = capi.DeviceMatrix(t, n_in, n_out, w)
    dq, db, dr = capi.DeviceBuffer.from_array(xq), capi.DeviceBuffer.from_array(bias), capi.DeviceBuffer.from_array(resid)
    for r0, r1, with_br in [(0, n_out, False), (3, n_out - 5, True)]:
        dout = capi.DeviceBuffer.from_array(np.full(n_out, np.nan, np.float32))
        a = capi.SdyMvArgs(xq=dq.ptr, n_tok=1, out=dout.ptr, out_stride=n_out, row0=r0, row1=r1,
                           bias=db.ptr if with_br else None, resid=dr.ptr if with_br else None)
        capi.check(L.sdy_matvec(ctypes.byref(m.m), ctypes.byref(a), None))
        got = dout.to_array(np.float32, n_out)
        e = exp.copy()
        if with_br:
            e = resid + (e + bias)  # the kernel's order: acc + bias, then resid + that
        assert np.array_equal(bits(got[r0:r1]), bits(e[r0:r1]))
        assert np.isnan(got[:r0]).all() and np.isnan(got[r1:]).all()
    m.close()


Q8K_TYPE = 15


def _fused_case(kind, n_in, n_out, seed):
    t = TYPES[kind]
    rng = np.random.default_rng(seed)
    w = random_blocks(kind, n_out * n_in // O.QK[t], rng).reshape(n_out, -1)
    x = (3.0 * rng.standard_normal(n_in)).astype(np.float32)
    nw = (1.0 + 0.5 * rng.standard_normal(n_in)).astype(np.float32)
    return t, w, x, nw


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("n_in,n_out,mode", [
    (2048, 2560, "norm_bias"), (2048, 22016, "norm_swiglu"), (2048, 2048, "quant_resid"), (11008, 2048, "quant_resid"),
    (768, 2048, "norm"), (4096, 2048, "quant_resid"), (4096, 512, "norm"), (1024, 40000, "quant_bias"),
    (256, 300, "norm_swiglu"), (11008, 37, "quant"), (2048, 5, "norm")])
def test_matvec_fused_activation(kind, n_in, n_out, mode):
    """A one-token matvec whose workgroups build the Q8_K row of the f32 input themselves (RMS-
    normalised first for 'norm') has the bits of sdy_norm_quant / sdy_quantize followed by
    sdy_matvec, with a bias, a residual or the SwiGLU epilogue."""
    L = lib()
    t, w, x, nw = _fused_case(kind, n_in, n_out, n_in + n_out)
    norm, swiglu = mode.startswith("norm"), mode.endswith("swiglu")
    eps = 1e-6
    m = capi.DeviceMatrix(t, n_in, n_out, w)
    dx, dnw = capi.DeviceBuffer.from_array(x), capi.DeviceBuffer.from_array(nw)
    rng = np.random.default_rng(n_out)
    extra = capi.DeviceBuffer.from_array(rng.standard_normal(n_out).astype(np.float32))
    dq = capi.DeviceBuffer(n_in // 256 * 292)
    if norm:
        capi.check(L.sdy_norm_quant(dx.ptr, dnw.ptr, eps, n_in, 1, None, Q8K_TYPE, dq.ptr, None))
    else:
        capi.check(L.sdy_quantize(Q8K_TYPE, dx.ptr, dq.ptr, n_in, 1, None))
    n_res = n_out // 2 if swiglu else n_out
    outs = []
    for fused in (False, True):
        dout = capi.DeviceBuffer.from_array(np.full(n_res, np.nan, np.float32))
        a = capi.SdyMvArgs(n_tok=1, out=dout.ptr, out_stride=n_res, row0=0, row1=n_out,
                           epilogue=capi.EPI_SWIGLU if swiglu else capi.EPI_NONE,
                           bias=extra.ptr if mode.endswith("bias") else None,
                           resid=extra.ptr if mode.endswith("resid") else None)
        if fused:
            a.x, a.nw, a.eps = dx.ptr, dnw.ptr if norm else None, eps
            assert L.sdy_matvec_fused_ok(ctypes.byref(m.m), ctypes.byref(a), None, None) == 1
        else:
            a.xq = dq.ptr
        capi.check(L.sdy_matvec(ctypes.byref(m.m), ctypes.byref(a), None))
        outs.append(dout.to_array(np.float32, n_res))
    assert not np.isnan(outs[0]).any()
    assert np.array_equal(bits(outs[1]), bits(outs[0]))
    m.close()


@pytest.mark.parametrize("kind,n_in", [("Q6_K", 11008), ("Q4_K", 2048), ("Q4_K", 768)])
def test_matvec_fused_quantiser_edge_cases(kind, n_in):
    """The workgroup quantisers of the fused one-token matvecs (several blocks per wave in one set
    of cross-lane reductions and divisions) write the bytes of the one-block quantiser on rows of
    NaN elements, all-NaN blocks, equal magnitudes of opposite sign, infinities and subnormals: the
    matvec outputs through both carry the same bits (NaN where an infinite scale makes them NaN)."""
    L = lib()
    t = TYPES[kind]
    n_out = 2048
    rng = np.random.default_rng(n_in)
    w = random_blocks(kind, n_out * n_in // O.QK[t], rng).reshape(n_out, -1)
    rows = _quant_edge_rows(n_in, rng)
    m = capi.DeviceMatrix(t, n_in, n_out, w)
    for xr in rows:
        x = np.ascontiguousarray(xr)
        dx = capi.DeviceBuffer.from_array(x)
        dq = capi.DeviceBuffer(n_in // 256 * 292)
        capi.check(L.sdy_quantize(Q8K_TYPE, dx.ptr, dq.ptr, n_in, 1, None))
        assert dq.to_array(np.uint8, n_in // 256 * 292).tobytes() == O.quantize(x[None], O.Q8_K).tobytes()
        outs = []
        for fused in (False, True):
            dout = capi.DeviceBuffer.from_array(np.full(n_out, 7.0, np.float32))
            a = capi.SdyMvArgs(n_tok=1, out=dout.ptr, out_stride=n_out, row0=0, row1=n_out, epilogue=capi.EPI_NONE)
            if fused:
                a.x, a.nw, a.eps = dx.ptr, None, 1e-6
                assert L.sdy_matvec_fused_ok(ctypes.byref(m.m), ctypes.byref(a), None, None) == 1
            else:
                a.xq = dq.ptr
            capi.check(L.sdy_matvec(ctypes.byref(m.m), ctypes.byref(a), None))
            outs.append(dout.to_array(np.float32, n_out))
        nan = np.isnan(outs[0])
        assert np.array_equal(np.isnan(outs[1]), nan)
        assert np.array_equal(bits(outs[1])[~nan], bits(outs[0])[~nan])
    m.close()


@pytest.mark.parametrize("norm", [True, False])
def test_matvec_pair_fused_activation(norm):
    """The paired one-token matvec (q|k Q4_K and v Q6_K) building its own Q8_K row: the bits of the
    pair on the row sdy_norm_quant / sdy_quantize wrote."""
    L = lib()
    n_in, n1, n2, eps = 2048, 2560, 256, 1e-6
    _, w1, x, nw = _fused_case("Q4_K", n_in, n1, 5)
    _, w2, _, _ = _fused_case("Q6_K", n_in, n2, 6)
    m1, m2 = capi.DeviceMatrix(O.Q4_K, n_in, n1, w1), capi.DeviceMatrix(O.Q6_K, n_in, n2, w2)
    dx, dnw = capi.DeviceBuffer.from_array(x), capi.DeviceBuffer.from_array(nw)
    b1 = capi.DeviceBuffer.from_array(np.random.default_rng(1).standard_normal(n1).astype(np.float32))
    b2 = capi.DeviceBuffer.from_array(np.random.default_rng(2).standard_normal(n2).astype(np.float32))
    dq = capi.DeviceBuffer(n_in // 256 * 292)
    if norm:
        capi.check(L.sdy_norm_quant(dx.ptr, dnw.ptr, eps, n_in, 1, None, Q8K_TYPE, dq.ptr, None))
    else:
        capi.check(L.sdy_quantize(Q8K_TYPE, dx.ptr, dq.ptr, n_in, 1, None))
    res = []
    for fused in (False, True):
        o1, o2 = capi.DeviceBuffer(n1 * 4), capi.DeviceBuffer(n2 * 4)
        a1 = capi.SdyMvArgs(n_tok=1, out=o1.ptr, out_stride=n1, row0=0, row1=n1, bias=b1.ptr)
        a2 = capi.SdyMvArgs(n_tok=1, out=o2.ptr, out_stride=n2, row0=0, row1=n2, bias=b2.ptr)
        for a in (a1, a2):
            if fused:
                a.x, a.nw, a.eps = dx.ptr, dnw.ptr if norm else None, eps
            else:
                a.xq = dq.ptr
        if fused:
            assert L.sdy_matvec_fused_ok(ctypes.byref(m1.m), ctypes.byref(a1), ctypes.byref(m2.m), ctypes.byref(a2)) == 1
        capi.check(L.sdy_matvec_pair(ctypes.byref(m1.m), ctypes.byref(a1), ctypes.byref(m2.m), ctypes.byref(a2), None))
        res.append((o1.to_array(np.float32, n1), o2.to_array(np.float32, n2)))
    for r0, r1 in zip(res[0], res[1]):
        assert np.array_equal(bits(r0), bits(r1))


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("norm", [False, True], ids=["quant", "norm"])
def test_matvec_ring_fused_activation(kind, norm):
    """Rows too many for a one-token grid the GPU holds at once (an output head) on the persistent
    ring kernel whose workgroups build the Q8_K row of the f32 input themselves: the bits of
    sdy_quantize / sdy_norm_quant followed by sdy_matvec, with a residual."""
    L = lib()
    n_in, n_out = 2048, 100003
    t, w, x, nw = _fused_case(kind, n_in, n_out, 17)
    eps = 1e-6
    m = capi.DeviceMatrix(t, n_in, n_out, w)
    dx, dnw = capi.DeviceBuffer.from_array(x), capi.DeviceBuffer.from_array(nw)
    extra = capi.DeviceBuffer.from_array(np.random.default_rng(3).standard_normal(n_out).astype(np.float32))
    dq = capi.DeviceBuffer(n_in // 256 * 292)
    if norm:
        capi.check(L.sdy_norm_quant(dx.ptr, dnw.ptr, eps, n_in, 1, None, Q8K_TYPE, dq.ptr, None))
    else:
        capi.check(L.sdy_quantize(Q8K_TYPE, dx.ptr, dq.ptr, n_in, 1, None))
    outs = []
    for fused in (False, True):
        dout = capi.DeviceBuffer.from_array(np.full(n_out, np.nan, np.float32))
        a = capi.SdyMvArgs(n_tok=1, out=dout.ptr, out_stride=n_out, row0=0, row1=n_out, epilogue=capi.EPI_NONE,
                           resid=extra.ptr)
        if fused:
            a.x, a.nw, a.eps = dx.ptr, dnw.ptr if norm else None, eps
            assert L.sdy_matvec_fused_ok(ctypes.byref(m.m), ctypes.byref(a), None, None) == 1
        else:
            a.xq = dq.ptr
        capi.check(L.sdy_matvec(ctypes.byref(m.m), ctypes.byref(a), None))
        if fused:
            assert "k_matvec_ring" in L.sdy_last_kernel().decode()
        outs.append(dout.to_array(np.float32, n_out))
    assert not np.isnan(outs[0]).any()
    assert np.array_equal(bits(outs[1]), bits(outs[0]))
    m.close()


def test_matvec_fused_activation_rejects():
    """Arguments the in-kernel quantisation does not cover are refused (no launch): other weight
    types, several tokens, a misaligned row, RMSNorm of rows above 4096 elements, SwiGLU on long rows."""
    L = lib()
    x = capi.DeviceBuffer.from_array(np.ones(8192 + 64, np.float32))
    out = capi.DeviceBuffer(4 * 4096)
    cases = [("Q8_0", 2048, 1, 0, False, capi.EPI_NONE), ("Q4_K", 2048, 2, 0, False, capi.EPI_NONE),
             ("Q4_K", 2048, 1, 4, False, capi.EPI_NONE), ("Q4_K", 8192, 1, 0, True, capi.EPI_NONE),
             ("Q6_K", 11008, 1, 0, False, capi.EPI_SWIGLU)]
    for kind, n_in, n_tok, off, norm, epi in cases:
        t = TYPES[kind]
        w = random_blocks(kind, 8 * n_in // O.QK[t], np.random.default_rng(0)).reshape(8, -1)
        m = capi.DeviceMatrix(t, n_in, 8, w)
        a = capi.SdyMvArgs(x=x.ptr + off, nw=x.ptr if norm else None, eps=1e-6, n_tok=n_tok, out=out.ptr, out_stride=8,
                           row0=0, row1=8, epilogue=epi)
        assert L.sdy_matvec_fused_ok(ctypes.byref(m.m), ctypes.byref(a), None, None) == 0, (kind, n_in, n_tok, off)
        assert L.sdy_matvec(ctypes.byref(m.m), ctypes.byref(a), None) != 0, (kind, n_in, n_tok, off)
        m.close()


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("n_in,ffn", [(2048, 11008), (1024, 20000), (1024, 36000), (256, 70000)])
def test_swiglu_epilogue_large(kind, n_in, ffn):
    """The one-token SwiGLU epilogue when a wave gathers the outputs of several row iterations (and
    several (gate, up) pairs per iteration for short rows): the bits of the separate gate and up
    matvecs followed by the SiLU op."""
    t = TYPES[kind]
    L = lib()
    rng = np.random.default_rng(ffn)
    nb = ffn * n_in // O.QK[t]
    g = random_blocks(kind, nb, rng).reshape(ffn, -1)
    u = random_blocks(kind, nb, rng).reshape(ffn, -1)
    x = rng.standard_normal((1, n_in)).astype(np.float32)
    xq = O.quantize(x, O.VEC_DOT[t])
    m = capi.SdyMat()
    capi.check(L.sdy_mat_alloc(ctypes.byref(m), t, n_in, 2 * ffn))
    capi.check(L.sdy_mat_upload_map(ctypes.byref(m), 0, ffn, 2, ffn, 0, ptr(g), None))
    capi.check(L.sdy_mat_upload_map(ctypes.byref(m), 1, ffn, 2, ffn, 0, ptr(u), None))
    dq = capi.DeviceBuffer.from_array(xq)
    dout = capi.DeviceBuffer(ffn * 4)
    a = capi.SdyMvArgs(xq=dq.ptr, n_tok=1, out=dout.ptr, out_stride=ffn, row0=0, row1=2 * ffn,
                       epilogue=capi.EPI_SWIGLU)
    capi.check(L.sdy_matvec(ctypes.byref(m), ctypes.byref(a), None))
    got = dout.to_array(np.float32, ffn)
    eg, eu = O.matmul_q(g, t, xq, n_in, simd=1)[0], O.matmul_q(u, t, xq, n_in, simd=1)[0]
    exp = eg.copy()
    L.op_silu_mul(ptr(exp), ptr(eu), exp.size)
    assert np.array_equal(bits(got), bits(exp))
    L.sdy_mat_free(ctypes.byref(m))


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K", "Q8_0", "Q5_0"])
@pytest.mark.parametrize("n_in,ffn,n_tok", [(2048, 96, 1), (1024, 40, 3), (11008, 8, 2), (768, 20, 1)])
def test_swiglu_epilogue(kind, n_in, ffn, n_tok):
    """gate and up uploaded interleaved (row 2i = gate i, 2i+1 = up i) and multiplied with the
    SwiGLU epilogue give silu(gate.x) * (up.x) with the bits of the separate matvecs followed by
    the SiLU kernel; the matvecs themselves are checked against the oracle."""
    if kind in ("Q8_0", "Q5_0") and n_in % 32:
        pytest.skip("row not a whole number of blocks")
    t = TYPES[kind]
    L = lib()
    rng = np.random.default_rng(n_in + ffn)
    nb = ffn * n_in // O.QK[t]
    g = random_blocks(kind, nb, rng).reshape(ffn, -1)
    u = random_blocks(kind, nb, rng).reshape(ffn, -1)
    x = rng.standard_normal((n_tok, n_in)).astype(np.float32)
    xq = O.quantize(x, O.VEC_DOT[t])
    m = capi.SdyMat()
    capi.check(L.sdy_mat_alloc(ctypes.byref(m), t, n_in, 2 * ffn))
    capi.check(L.sdy_mat_upload_map(ctypes.byref(m), 0, ffn, 2, ffn, 0, ptr(g), None))
    capi.check(L.sdy_mat_upload_map(ctypes.byref(m), 1, ffn, 2, ffn, 0, ptr(u), None))
    dq = capi.DeviceBuffer.from_array(xq)
    dout = capi.DeviceBuffer(n_tok * ffn * 4)
    a = capi.SdyMvArgs(xq=dq.ptr, n_tok=n_tok, out=dout.ptr, out_stride=ffn, row0=0, row1=2 * ffn,
                       epilogue=capi.EPI_SWIGLU)
    capi.check(L.sdy_matvec(ctypes.byref(m), ctypes.byref(a), None))
    got = dout.to_array(np.float32, (n_tok, ffn))
    # separate path: both halves through the plain matvec, then the SiLU kernel
    gm, um = capi.DeviceMatrix(t, n_in, ffn, g), capi.DeviceMatrix(t, n_in, ffn, u)
    dg, du = capi.DeviceBuffer(n_tok * ffn * 4), capi.DeviceBuffer(n_tok * ffn * 4)
    for mat, buf in ((gm, dg), (um, du)):
        a2 = capi.SdyMvArgs(xq=dq.ptr, n_tok=n_tok, out=buf.ptr, out_stride=ffn, row0=0, row1=ffn)
        capi.check(L.sdy_matvec(ctypes.byref(mat.m), ctypes.byref(a2), None))
    yg, yu = dg.to_array(np.float32, (n_tok, ffn)), du.to_array(np.float32, (n_tok, ffn))
    hg = yg.copy()
    L.op_silu_mul(ptr(hg), ptr(yu), hg.size)
    assert np.array_equal(bits(got), bits(hg))
    simd = 1 if t in (O.Q4_K, O.Q6_K) else 0
    eg, eu = O.matmul_q(g, t, xq, n_in, simd=simd), O.matmul_q(u, t, xq, n_in, simd=simd)
    if t in (O.Q4_K, O.Q6_K):
        assert np.array_equal(bits(yg), bits(eg)) and np.array_equal(bits(yu), bits(eu))
    exp = eg.copy()
    O.lib().orc_silu_mul(ptr(exp), ptr(eu), exp.size)
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5 * float(np.abs(exp).max()))
    L.sdy_mat_free(ctypes.byref(m))


@pytest.mark.parametrize("kind,n_in,e_rows,swiglu,rows", [
    ("Q4_K", 2048, 96, True, None), ("Q6_K", 768, 200, False, None), ("Q4_K", 768, 64, False, (3, 61)),
    ("Q6_K", 256, 40, True, None), ("Q4_K", 1280, 30, False, None), ("Q6_K", 4096, 16, False, None)])
def test_grouped_matvec(kind, n_in, e_rows, swiglu, rows):
    """The routed-expert grouped matvec: slot s computes rows of expert top[s] of a stacked
    matrix with its own activation row (down) or one shared row (gate|up with SwiGLU), with the
    bits of the plain matvec on that expert's rows, which are the oracle's."""
    t = TYPES[kind]
    L = lib()
    n_exp = 12
    top = np.array([7, 2, 11, 2, 0], np.int32)  # expert 2 twice, as two tokens' slots could
    k = len(top)
    rng = np.random.default_rng(n_in + e_rows)
    w = random_blocks(kind, n_exp * e_rows * n_in // 256, rng).reshape(n_exp * e_rows, -1)
    x = rng.standard_normal((1 if swiglu else k, n_in)).astype(np.float32)
    xq = O.quantize(x, O.Q8_K)
    xrow = O.row_size(O.Q8_K, n_in)
    r0, r1 = rows or (0, e_rows)
    n_out = (r1 - r0) // 2 if swiglu else e_rows
    epi = capi.EPI_SWIGLU if swiglu else capi.EPI_NONE
    m = capi.DeviceMatrix(t, n_in, n_exp * e_rows, w)
    dq, dtop = capi.DeviceBuffer.from_array(xq), capi.DeviceBuffer.from_array(top)
    dout = capi.DeviceBuffer.from_array(np.full((k, n_out), np.nan, np.float32))
    a = capi.SdyMvArgs(xq=dq.ptr, n_tok=1, out=dout.ptr, out_stride=n_out, row0=r0, row1=r1, epilogue=epi)
    capi.check(L.sdy_matvec_grouped(ctypes.byref(m.m), ctypes.byref(a), dtop.ptr, k, e_rows, 0 if swiglu else xrow,
                                    n_out, None))
    got = dout.to_array(np.float32, (k, n_out))
    # the plain matvec writes out[row] for row in [row0, row1) (out[(row - row0) / 2] with SwiGLU)
    n1 = n_out if swiglu else n_exp * e_rows
    d1 = capi.DeviceBuffer.from_array(np.full(n1, np.nan, np.float32))
    for s, e in enumerate(top):
        xs = 0 if swiglu else s
        a1 = capi.SdyMvArgs(xq=dq.ptr + xs * xrow, n_tok=1, out=d1.ptr, out_stride=n1, row0=e * e_rows + r0,
                            row1=e * e_rows + r1, epilogue=epi)
        capi.check(L.sdy_matvec(ctypes.byref(m.m), ctypes.byref(a1), None))
        one = d1.to_array(np.float32, n1)
        if swiglu:
            assert np.array_equal(bits(got[s]), bits(one)), s
        else:
            assert np.array_equal(bits(got[s, r0:r1]), bits(one[e * e_rows + r0:e * e_rows + r1])), s
            assert np.isnan(got[s, :r0]).all() and np.isnan(got[s, r1:]).all()
            exp = O.matmul_q(w[e * e_rows + r0:e * e_rows + r1], t, xq[xs:xs + 1], n_in, simd=1)[0]
            assert np.array_equal(bits(got[s, r0:r1]), bits(exp)), s
    if swiglu:  # the gate and up rows of each slot through the oracle, then SiLU (libm expf: 1e-5)
        for s, e in enumerate(top):
            y = O.matmul_q(w[e * e_rows + r0:e * e_rows + r1], t, xq, n_in, simd=1)[0]
            g, u = y[0::2].copy(), y[1::2].copy()
            O.lib().orc_silu_mul(ptr(g), ptr(u), g.size)
            np.testing.assert_allclose(got[s], g, rtol=1e-5, atol=1e-5 * float(np.abs(g).max()))


@pytest.mark.parametrize("kind,n_in,e_rows,swiglu,n_exp,k,case", [
    ("Q4_K", 2048, 96, True, 128, 8, "normal"), ("Q4_K", 2048, 96, True, 128, 8, "ties"),
    ("Q4_K", 2048, 64, True, 128, 16, "equal"), ("Q6_K", 768, 40, False, 60, 4, "normal"),
    ("Q6_K", 256, 24, True, 8, 8, "ties"), ("Q4_K", 4096, 32, False, 100, 64, "normal")])
def test_grouped_matvec_routes_itself(kind, n_in, e_rows, swiglu, n_exp, k, case):
    """The grouped matvec that selects its experts from the router's logits: its choices and weights
    are sdy_moe_route's bit for bit (exact ties, all-equal logits: the lowest experts), and its
    outputs are sdy_matvec_grouped's on those choices."""
    t = TYPES[kind]
    L = lib()
    rng = np.random.default_rng(n_in + n_exp + k)
    w = random_blocks(kind, n_exp * e_rows * n_in // 256, rng).reshape(n_exp * e_rows, -1)
    x = rng.standard_normal((1, n_in)).astype(np.float32)
    xq = O.quantize(x, O.Q8_K)
    logits = (rng.standard_normal(n_exp) * 2).astype(np.float32)
    if case == "ties":
        logits[1:n_exp:3] = logits.max()
    elif case == "equal":
        logits[:] = -0.25
    n_out = e_rows // 2 if swiglu else e_rows
    epi = capi.EPI_SWIGLU if swiglu else capi.EPI_NONE
    m = capi.DeviceMatrix(t, n_in, n_exp * e_rows, w)
    dq, dl = capi.DeviceBuffer.from_array(xq), capi.DeviceBuffer.from_array(logits)
    outs = []
    for routed in (False, True):
        dtop = capi.DeviceBuffer.from_array(np.full(k, -7, np.int32))
        dw = capi.DeviceBuffer.from_array(np.full(k, np.nan, np.float32))
        dout = capi.DeviceBuffer.from_array(np.full((k, n_out), np.nan, np.float32))
        a = capi.SdyMvArgs(xq=dq.ptr, n_tok=1, out=dout.ptr, out_stride=n_out, row0=0, row1=e_rows, epilogue=epi)
        if routed:
            capi.check(L.sdy_matvec_grouped_route(ctypes.byref(m.m), ctypes.byref(a), dl.ptr, n_exp, k, dtop.ptr, dw.ptr,
                                                  e_rows, 0, n_out, None))
        else:
            capi.check(L.sdy_moe_route(dl.ptr, 1, n_exp, k, dtop.ptr, dw.ptr, None))
            capi.check(L.sdy_matvec_grouped(ctypes.byref(m.m), ctypes.byref(a), dtop.ptr, k, e_rows, 0, n_out, None))
        outs.append((dtop.to_array(np.int32, k), dw.to_array(np.float32, k), dout.to_array(np.float32, (k, n_out))))
    (t0, w0, y0), (t1, w1, y1) = outs
    assert t1.tolist() == t0.tolist()
    assert np.array_equal(bits(w1), bits(w0)) and np.array_equal(bits(y1), bits(y0))
    p = logits.copy()
    O.lib().orc_softmax(ptr(p), n_exp)
    assert t1.tolist() == np.argsort(-p, kind="stable")[:k].tolist()
    if case == "equal":
        assert t1.tolist() == list(range(k))
    assert not np.isnan(y1).any()
    # the checks of the entry point: more than 128 experts, more than 64 choices, no Q8_K row
    a = capi.SdyMvArgs(xq=dq.ptr, n_tok=1, out=dout.ptr, out_stride=n_out, row0=0, row1=e_rows, epilogue=epi)
    assert L.sdy_matvec_grouped_route(ctypes.byref(m.m), ctypes.byref(a), dl.ptr, 129, k, dtop.ptr, dw.ptr, e_rows, 0,
                                      n_out, None) < 0
    assert L.sdy_matvec_grouped_route(ctypes.byref(m.m), ctypes.byref(a), dl.ptr, n_exp, 65, dtop.ptr, dw.ptr, e_rows,
                                      0, n_out, None) < 0
    a.xq = None
    a.x = dq.ptr
    assert L.sdy_matvec_grouped_route(ctypes.byref(m.m), ctypes.byref(a), dl.ptr, n_exp, k, dtop.ptr, dw.ptr, e_rows, 0,
                                      n_out, None) < 0


@pytest.mark.parametrize("kind,n_in,e_rows,mode", [
    ("Q6_K", 768, 2048, "quant"), ("Q4_K", 2048, 1536, "norm_swiglu"), ("Q4_K", 1024, 300, "quant"),
    ("Q6_K", 2048, 96, "norm")])
def test_grouped_matvec_fused_activation(kind, n_in, e_rows, mode):
    """The grouped matvec whose workgroups quantise their slot's f32 row (one row per slot, or one
    shared row RMS-normalised first): the bits of the grouped matvec on the rows sdy_quantize /
    sdy_norm_quant wrote."""
    t = TYPES[kind]
    L = lib()
    n_exp, eps = 10, 1e-6
    top = np.array([7, 2, 9, 2, 0, 4, 5, 1], np.int32)
    k = len(top)
    norm, swiglu = mode.startswith("norm"), mode.endswith("swiglu")
    rng = np.random.default_rng(n_in + e_rows)
    w = random_blocks(kind, n_exp * e_rows * n_in // 256, rng).reshape(n_exp * e_rows, -1)
    n_x = 1 if norm else k
    x = (2.0 * rng.standard_normal((n_x, n_in))).astype(np.float32)
    nw = (1.0 + 0.3 * rng.standard_normal(n_in)).astype(np.float32)
    m = capi.DeviceMatrix(t, n_in, n_exp * e_rows, w)
    dx, dnw, dtop = capi.DeviceBuffer.from_array(x), capi.DeviceBuffer.from_array(nw), capi.DeviceBuffer.from_array(top)
    xrow = O.row_size(O.Q8_K, n_in)
    dq = capi.DeviceBuffer(n_x * xrow)
    if norm:
        capi.check(L.sdy_norm_quant(dx.ptr, dnw.ptr, eps, n_in, 1, None, Q8K_TYPE, dq.ptr, None))
    else:
        capi.check(L.sdy_quantize(Q8K_TYPE, dx.ptr, dq.ptr, n_in, k, None))
    n_out = e_rows // 2 if swiglu else e_rows
    epi = capi.EPI_SWIGLU if swiglu else capi.EPI_NONE
    res = []
    for fused in (False, True):
        dout = capi.DeviceBuffer.from_array(np.full((k, n_out), np.nan, np.float32))
        a = capi.SdyMvArgs(n_tok=1, out=dout.ptr, out_stride=n_out, row0=0, row1=e_rows, epilogue=epi)
        if fused:
            a.x, a.nw, a.eps = dx.ptr, dnw.ptr if norm else None, eps
            x_slot = 0 if norm else n_in
            assert L.sdy_matvec_grouped_fused_ok(ctypes.byref(m.m), ctypes.byref(a), k, e_rows, x_slot) == 1
        else:
            a.xq = dq.ptr
            x_slot = 0 if norm else xrow
        capi.check(L.sdy_matvec_grouped(ctypes.byref(m.m), ctypes.byref(a), dtop.ptr, k, e_rows, x_slot, n_out, None))
        res.append(dout.to_array(np.float32, (k, n_out)))
    assert not np.isnan(res[0]).any()
    assert np.array_equal(bits(res[1]), bits(res[0]))


@pytest.mark.parametrize("kind,n_in,dim,k,resid", [
    ("Q6_K", 768, 2048, 8, "inplace"), ("Q4_K", 768, 2050, 8, "sep"), ("Q6_K", 2048, 300, 5, "none"),
    ("Q4_K", 512, 77, 1, "inplace"), ("Q6_K", 4096, 130, 3, "sep"), ("Q4_K", 1280, 1000, 7, "inplace")])
def test_moe_down_combine_bit_exact(kind, n_in, dim, k, resid):
    """The routed experts' down projections and their combine in one launch: the bits of the grouped
    matvec (each slot's f32 row quantised in the kernel) followed by sdy_moe_combine, with the
    residual separate, absent or the output itself."""
    t = TYPES[kind]
    L = lib()
    n_exp = 11
    rng = np.random.default_rng(n_in + dim + k)
    top = rng.permutation(n_exp)[:k].astype(np.int32)
    wts = rng.random(k).astype(np.float32)
    w = random_blocks(kind, n_exp * dim * n_in // 256, rng).reshape(n_exp * dim, -1)
    x = (2.0 * rng.standard_normal((k, n_in))).astype(np.float32)
    r = rng.standard_normal(dim).astype(np.float32)
    m = capi.DeviceMatrix(t, n_in, n_exp * dim, w)
    dx, dtop, dw = capi.DeviceBuffer.from_array(x), capi.DeviceBuffer.from_array(top), capi.DeviceBuffer.from_array(wts)
    # separate: grouped matvec into y [k][dim], then the combine
    dy = capi.DeviceBuffer.from_array(np.full((k, dim), np.nan, np.float32))
    a = capi.SdyMvArgs(n_tok=1, x=dx.ptr, out=dy.ptr, out_stride=dim, row0=0, row1=dim)
    assert L.sdy_matvec_grouped_fused_ok(ctypes.byref(m.m), ctypes.byref(a), k, dim, n_in) == 1
    capi.check(L.sdy_matvec_grouped(ctypes.byref(m.m), ctypes.byref(a), dtop.ptr, k, dim, n_in, dim, None))
    dr = capi.DeviceBuffer.from_array(r)
    de = capi.DeviceBuffer.from_array(np.full(dim, np.nan, np.float32))
    capi.check(L.sdy_moe_combine(dy.ptr, dtop.ptr, dw.ptr, 1, k, dim, de.ptr, None if resid == "none" else dr.ptr,
                                 None))
    exp = de.to_array(np.float32, dim)
    assert not np.isnan(exp).any()
    if resid == "inplace":
        dout = capi.DeviceBuffer.from_array(r)
        rp = dout.ptr
    else:
        dout = capi.DeviceBuffer.from_array(np.full(dim, np.nan, np.float32))
        rp = dr.ptr if resid == "sep" else None
    capi.check(L.sdy_moe_down_combine(ctypes.byref(m.m), dx.ptr, dtop.ptr, dw.ptr, k, dim, dout.ptr, rp, None))
    assert np.array_equal(bits(dout.to_array(np.float32, dim)), bits(exp))


FLOAT_TYPES = {"F32": (0, np.float32), "F16": (1, np.float16), "BF16": (30, None)}


@pytest.mark.parametrize("wname,n_in,n_rows", [("F32", 2048, 128), ("F16", 1024, 64), ("BF16", 4096, 17),
                                               ("F32", 256, 3), ("F32", 4096, 13), ("F32", 1024, 70),
                                               ("F32", 2048, 5)])
def test_matvec_float_norm(wname, n_in, n_rows):
    """The float matvec of the RMS-normalised row (the MoE router reading the FFN norm's output):
    the bits of sdy_norm_quant's f32 row followed by sdy_matvec_float, and the Q8_K bytes
    sdy_norm_quant writes (row counts that leave the last workgroup partial among them)."""
    L = lib()
    wt, dt = FLOAT_TYPES[wname]
    rng = np.random.default_rng(n_in + n_rows)
    w32 = rng.standard_normal((n_rows, n_in)).astype(np.float32)
    w = w32.astype(dt) if dt else (w32.view(np.uint32) >> 16).astype(np.uint16)
    x = (2.0 * rng.standard_normal(n_in)).astype(np.float32)
    nw = (1.0 + 0.3 * rng.standard_normal(n_in)).astype(np.float32)
    eps = 1e-6
    dw, dx, dnw = capi.DeviceBuffer.from_array(w), capi.DeviceBuffer.from_array(x), capi.DeviceBuffer.from_array(nw)
    xrow = n_in // 256 * 292
    # separate path: norm_quant (f32 row and Q8_K), then the float matvec of the f32 row
    dxb, dq = capi.DeviceBuffer(n_in * 4), capi.DeviceBuffer(xrow)
    capi.check(L.sdy_norm_quant(dx.ptr, dnw.ptr, eps, n_in, 1, dxb.ptr, Q8K_TYPE, dq.ptr, None))
    d1 = capi.DeviceBuffer(n_rows * 4)
    a = capi.SdyMvArgs(x=dxb.ptr, n_tok=1, out=d1.ptr, out_stride=n_rows, row0=0, row1=n_rows)
    capi.check(L.sdy_matvec_float(wt, dw.ptr, n_in, ctypes.byref(a), None))
    d2, dq2 = capi.DeviceBuffer(n_rows * 4), capi.DeviceBuffer(xrow)
    a2 = capi.SdyMvArgs(x=dx.ptr, nw=dnw.ptr, eps=eps, n_tok=1, out=d2.ptr, out_stride=n_rows, row0=0, row1=n_rows)
    capi.check(L.sdy_matvec_float_norm(wt, dw.ptr, n_in, ctypes.byref(a2), dq2.ptr, None))
    assert np.array_equal(bits(d2.to_array(np.float32, n_rows)), bits(d1.to_array(np.float32, n_rows)))
    assert np.array_equal(dq2.to_array(np.uint8, xrow), dq.to_array(np.uint8, xrow))


def test_grouped_matvec_rejects_bad_shapes():
    L = lib()
    w = random_blocks("Q4_K", 4 * 10 * 2048 // 256, np.random.default_rng(0)).reshape(40, -1)
    m = capi.DeviceMatrix(O.Q4_K, 2048, 40, w)
    top = capi.DeviceBuffer.from_array(np.zeros(2, np.int32))
    a = capi.SdyMvArgs(xq=None, n_tok=1, out=None, out_stride=10, row0=0, row1=10)
    assert L.sdy_matvec_grouped(ctypes.byref(m.m), ctypes.byref(a), top.ptr, 2, 7, 0, 10, None) != 0  # 40 % 7
    a.row1 = 11
    assert L.sdy_matvec_grouped(ctypes.byref(m.m), ctypes.byref(a), top.ptr, 2, 10, 0, 10, None) != 0
    a.row1, a.n_tok = 10, 2
    assert L.sdy_matvec_grouped(ctypes.byref(m.m), ctypes.byref(a), top.ptr, 2, 10, 0, 10, None) != 0


@pytest.mark.parametrize("wtype", [O.F32, O.F16, O.BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("n_in,n_out,n_tok,r0,r1", [(2048, 128, 1, 0, 128), (2340, 45, 9, 0, 45),
                                                  (67, 45, 4, 3, 42), (768, 33, 17, 0, 33), (96, 10, 3, 1, 10),
                                                  (2048, 128, 1024, 0, 128), (2048, 128, 512, 0, 128),
                                                  (2340, 45, 37, 0, 45), (300, 35, 19, 1, 34), (16, 16, 16, 0, 16)])
def test_float_matmul_reference_order_bit_exact(wtype, n_in, n_out, n_tok, r0, r1):
    """F32/F16/BF16 weights (the MoE router) in the reference's AVX2 order: block_2x4 for paired
    rows x groups of four tokens, dot for the rest, with the hsum tree and the scalar tail; the
    bits of the oracle's restatement of csrc/ops_avx2.c. Blocks of at least 16 rows and tokens run
    on the LDS-tiled kernel (partial tiles and a partial last 256-element chunk included)."""
    rng = np.random.default_rng(n_in + n_tok + r0)
    x = rng.standard_normal((n_tok, n_in)).astype(np.float32)
    w32 = (rng.standard_normal((n_out, n_in)) * 0.02).astype(np.float32)
    if wtype == O.F16:
        w = w32.astype(np.float16)
    elif wtype == O.BF16:
        w = (w32.view(np.uint32) >> 16).astype(np.uint16)
    else:
        w = w32
    w = np.ascontiguousarray(w)
    L = lib()
    dw, dx = capi.DeviceBuffer.from_array(w), capi.DeviceBuffer.from_array(x)
    dout = capi.DeviceBuffer.from_array(np.full((n_tok, n_out), np.nan, np.float32))
    a = capi.SdyMvArgs(x=dx.ptr, n_tok=n_tok, out=dout.ptr, out_stride=n_out, row0=r0, row1=r1)
    capi.check(L.sdy_matvec_float(wtype, dw.ptr, n_in, ctypes.byref(a), None))
    got = dout.to_array(np.float32, (n_tok, n_out))
    exp = np.full((n_tok, n_out), np.nan, np.float32)
    O.lib().orc_matmul_rows(ptr(exp), ptr(x), ptr(w), wtype, n_tok, n_in, n_out, r0, r1, 1)
    assert np.array_equal(bits(got[:, r0:r1]), bits(exp[:, r0:r1]))


@pytest.mark.parametrize("n_expert,k", [(128, 8), (60, 4), (256, 16), (512, 64), (8, 3)])
def test_moe_route_and_combine(n_expert, k):
    """Router softmax + top-k (ties to the lowest expert) and the weighted sum of the chosen experts'
    outputs in ascending expert order, against the oracle's softmax, a stable sort and the oracle's
    AVX2 axpy (fused in 8-lane steps, rounded product and sum in the tail: dim 2050)."""
    L = lib()
    n_tok, dim = 5, 2050
    rng = np.random.default_rng(n_expert + k)
    logits = (rng.standard_normal((n_tok, n_expert)) * 2).astype(np.float32)
    logits[1, 1:min(n_expert, 40):3] = logits[1, 0]  # exact ties
    logits[2, :] = 0.5                               # all equal: experts 0 .. k-1
    dl = capi.DeviceBuffer.from_array(logits)
    dtop, dw = capi.DeviceBuffer(n_tok * k * 4), capi.DeviceBuffer(n_tok * k * 4)
    capi.check(L.sdy_moe_route(dl.ptr, n_tok, n_expert, k, dtop.ptr, dw.ptr, None))
    top, w = dtop.to_array(np.int32, (n_tok, k)), dw.to_array(np.float32, (n_tok, k))
    for t in range(n_tok):
        p = logits[t].copy()
        O.lib().orc_softmax(ptr(p), n_expert)
        et = np.argsort(-p, kind="stable")[:k]
        assert top[t].tolist() == et.tolist(), t
        # the device's expf is the host libm's, so its probabilities are the oracle's softmax bit for
        # bit, and the weights divide them by their sequential float sum in rank order
        pc = p
        sc = np.float32(0)
        for e in et:
            sc = np.float32(sc + pc[e])
        assert np.array_equal(bits(w[t]), bits(pc[et] / sc)), t
        s = np.float32(0)
        for e in et:
            s = np.float32(s + p[e])
        np.testing.assert_allclose(w[t], p[et] / s, rtol=1e-6)
    if k > 16:
        return
    y = rng.standard_normal((n_tok, k, dim)).astype(np.float32)
    resid = rng.standard_normal((n_tok, dim)).astype(np.float32)
    dy, dr = capi.DeviceBuffer.from_array(y), capi.DeviceBuffer.from_array(resid)
    dout = capi.DeviceBuffer(n_tok * dim * 4)
    capi.check(L.sdy_moe_combine(dy.ptr, dtop.ptr, dw.ptr, n_tok, k, dim, dout.ptr, dr.ptr, None))
    got = dout.to_array(np.float32, (n_tok, dim))
    for t in range(n_tok):
        acc = np.zeros(dim, np.float32)
        for i in np.argsort(top[t]):
            yi = np.ascontiguousarray(y[t, i])
            O.lib().orc_axpy(ptr(acc), float(w[t, i]), ptr(yi), dim, 1)
        assert np.array_equal(bits(got[t]), bits(resid[t] + acc)), t


@pytest.mark.parametrize("n_head,n_kv_head,hd", [(16, 2, 128), (4, 2, 64), (32, 4, 128), (4, 4, 64), (6, 2, 64),
                                             (4, 2, 32), (2, 1, 256), (6, 3, 80)])
@pytest.mark.parametrize("n_tok,n_kv0", [(16, 1), (40, 70), (77, 3)])
@pytest.mark.parametrize("kv", ["f32", "f16"])
def test_prefill_attention_tokens_bit_identical(n_head, n_kv_head, hd, n_tok, n_kv0, kv):
    """Causal attention of n_tok tokens in one call gives the bits of one call per token and those of
    the oracle's op_attention_head (the reference's AVX2 dot, libm expf, in-order axpy), and follows a
    float64 softmax. With an f16 cache, the oracle runs on the f32 values of the same f16 cache."""
    L = lib()
    rng = np.random.default_rng(n_head * 1000 + n_tok + hd)
    max_seq = 160
    q = rng.standard_normal((n_tok, n_head * hd)).astype(np.float32)
    kc = rng.standard_normal((n_kv_head, max_seq, hd)).astype(np.float32)
    vc = rng.standard_normal((n_kv_head, max_seq, hd)).astype(np.float32)
    kv_type = capi.KV_F16 if kv == "f16" else capi.KV_F32
    if kv == "f16":
        kc16, vc16 = kc.astype(np.float16), vc.astype(np.float16)
        dk, dv = capi.DeviceBuffer.from_array(kc16), capi.DeviceBuffer.from_array(vc16)
        kc, vc = kc16.astype(np.float32), vc16.astype(np.float32)
    else:
        dk, dv = capi.DeviceBuffer.from_array(kc), capi.DeviceBuffer.from_array(vc)
    dq = capi.DeviceBuffer.from_array(q)
    dpart = capi.DeviceBuffer(L.sdy_attn_scores_floats(n_tok, n_head, max_seq) * 4)
    dout = capi.DeviceBuffer(n_tok * n_head * hd * 4)
    q_dim = n_head * hd
    capi.check(L.sdy_attention(dq.ptr, dk.ptr, dv.ptr, kv_type, n_tok, n_head, n_kv_head, hd, n_kv0, max_seq * hd,
                               q_dim, dpart.ptr, dout.ptr, q_dim, None))
    got = dout.to_array(np.float32, (n_tok, q_dim))
    one = np.empty_like(got)
    d1 = capi.DeviceBuffer(q_dim * 4)
    for t in range(n_tok):
        capi.check(L.sdy_attention(dq.ptr + 4 * t * q_dim, dk.ptr, dv.ptr, kv_type, 1, n_head, n_kv_head, hd,
                                   n_kv0 + t, max_seq * hd, q_dim, dpart.ptr, d1.ptr, q_dim, None))
        one[t] = d1.to_array(np.float32, q_dim)
    assert np.array_equal(bits(got), bits(one))
    exp_o = np.empty((n_tok, q_dim), np.float32)
    scores = np.empty(max_seq, np.float32)
    for t in range(n_tok):
        qt = np.ascontiguousarray(q[t])
        O.lib().orc_attention(ptr(exp_o[t]), ptr(qt), ptr(kc), ptr(vc), n_head, n_kv_head, hd, n_kv0 + t, max_seq,
                              ptr(scores), 1)
    assert np.array_equal(bits(got), bits(exp_o))
    n_rep = n_head // n_kv_head
    for t in range(0, n_tok, 7):
        for h in range(n_head):
            kk, vv = kc[h // n_rep, :n_kv0 + t].astype(np.float64), vc[h // n_rep, :n_kv0 + t].astype(np.float64)
            sc = kk @ q[t, h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            exp = (p / p.sum()) @ vv
            np.testing.assert_allclose(got[t, h * hd:(h + 1) * hd], exp, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("n_head,n_kv_head,hd", [(16, 2, 128), (32, 4, 128), (4, 2, 64), (4, 4, 64), (6, 2, 64)])
@pytest.mark.parametrize("n_tok,n_kv0", [(16, 1), (40, 70), (77, 3), (512, 1), (100, 900)])
@pytest.mark.parametrize("kv", ["f32", "f16"])
def test_prefill_attention_flash(n_head, n_kv_head, hd, n_tok, n_kv0, kv):
    """The flash-form prompt attention (f32 matrix cores, eight waves per 32 queries over key tiles
    of 32, merged in wave order) is within 1e-5 of the output scale of the reference's arithmetic
    (sdy_attention, bit-exact with the oracle), for partial query blocks and key tiles, q rows at a
    stride wider than the heads (the engine's q|k|v rows) and both cache types; it is deterministic."""
    L = lib()
    assert L.sdy_attention_flash_ok(n_head, n_kv_head, hd)
    rng = np.random.default_rng(n_head * 7 + n_tok + n_kv0 + hd)
    max_seq = n_kv0 + n_tok + 5
    q_dim = n_head * hd
    q_stride = q_dim + 2 * n_kv_head * hd
    q = rng.standard_normal((n_tok, q_stride)).astype(np.float32)
    ct = np.float16 if kv == "f16" else np.float32
    kc = rng.standard_normal((n_kv_head, max_seq, hd)).astype(ct)
    vc = rng.standard_normal((n_kv_head, max_seq, hd)).astype(ct)
    kv_type = capi.KV_F16 if kv == "f16" else capi.KV_F32
    dq, dk, dv = (capi.DeviceBuffer.from_array(a) for a in (q, kc, vc))
    dpart = capi.DeviceBuffer(L.sdy_attn_scores_floats(n_tok, n_head, max_seq) * 4)
    dexp, dgot = capi.DeviceBuffer(n_tok * q_dim * 4), capi.DeviceBuffer(n_tok * q_dim * 4)
    capi.check(L.sdy_attention(dq.ptr, dk.ptr, dv.ptr, kv_type, n_tok, n_head, n_kv_head, hd, n_kv0, max_seq * hd,
                               q_stride, dpart.ptr, dexp.ptr, q_dim, None))
    exp = dexp.to_array(np.float32, (n_tok, q_dim))
    outs = []
    for _ in range(2):
        capi.check(L.sdy_attention_flash(dq.ptr, dk.ptr, dv.ptr, kv_type, n_tok, n_head, n_kv_head, hd, n_kv0,
                                         max_seq * hd, q_stride, dgot.ptr, q_dim, None))
        outs.append(dgot.to_array(np.float32, (n_tok, q_dim)))
    assert np.array_equal(bits(outs[0]), bits(outs[1]))
    np.testing.assert_allclose(outs[0], exp, rtol=0, atol=1e-5 * float(np.abs(exp).max()))


def test_prefill_attention_flash_rejects_layouts():
    """head_dim other than 64 / 128, GQA groups that do not divide, unaligned q rows: an error, no launch."""
    L = lib()
    assert not L.sdy_attention_flash_ok(4, 2, 32) and not L.sdy_attention_flash_ok(6, 4, 64)
    assert L.sdy_attention_flash(None, None, None, capi.KV_F32, 4, 4, 2, 32, 1, 64, 128, None, 128, None) != 0
    assert L.sdy_attention_flash(None, None, None, capi.KV_F32, 4, 4, 2, 64, 1, 64, 258, None, 256, None) != 0


@pytest.mark.parametrize("n_head,n_kv_head,hd,qk_norm", [(16, 2, 128, False), (32, 4, 128, True), (6, 2, 64, False)])
@pytest.mark.parametrize("pos", [0, 15, 16, 1000, 2047, 2048, 2110])
@pytest.mark.parametrize("kv", ["f32", "f16"])
def test_decode_attention_long_context(n_head, n_kv_head, hd, qk_norm, pos, kv):
    """One-token decode attention through sdy_attn_decode (q/k RMSNorm, RoPE, the KV write, scores,
    softmax, weighted V and the output's Q8_K row) at positions up to the last slot of a 2111-position
    cache: past the 2048 positions whose softmax stays in registers, and over a cache whose size is not
    a multiple of 16 or 64. The output, the written cache rows and the Q8_K bytes have the bits of the
    oracle's decode step (orc_model.c: norm, rope, cache write, orc_attention over pos + 1 positions).
    With an f16 cache: the new row is written as the f16 rounding of the oracle's (the reference's
    f32 -> f16 rules, here numpy's, equal for these finite values) and the output has the oracle's
    bits over the f32 values of the f16 cache."""
    L = lib()
    max_seq, eps, half = 2111, 1e-6, hd // 2
    assert L.sdy_attn_decode_ok(n_head, n_kv_head, hd, max_seq)
    rng = np.random.default_rng(pos * 7 + n_head)
    cs, sn = np.empty(max_seq * half, np.float32), np.empty(max_seq * half, np.float32)
    O.lib().orc_rope_table(ptr(cs), ptr(sn), max_seq, hd, 1e6)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    k = rng.standard_normal(n_kv_head * hd).astype(np.float32)
    v = rng.standard_normal(n_kv_head * hd).astype(np.float32)
    kc = rng.standard_normal((n_kv_head, max_seq, hd)).astype(np.float32)
    vc = rng.standard_normal((n_kv_head, max_seq, hd)).astype(np.float32)
    qn = (1 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    ct = np.float16 if kv == "f16" else np.float32
    kc, vc = kc.astype(ct), vc.astype(ct)
    dev = {n: capi.DeviceBuffer.from_array(a) for n, a in
           dict(q=q, k=k, v=v, kc=kc, vc=vc, cs=cs, sn=sn, qn=qn, kn=kn, step=np.array([0, pos], np.int32)).items()}
    dscores = capi.DeviceBuffer(L.sdy_attn_scores_floats(1, n_head, max_seq) * 4)
    dout = capi.DeviceBuffer(n_head * hd * 4)
    with_q8k = n_head * hd % 256 == 0
    dxq = capi.DeviceBuffer(n_head * hd // 256 * 292) if with_q8k else None
    capi.check(L.sdy_attn_decode(dev["q"].ptr, dev["k"].ptr, dev["v"].ptr, dev["qn"].ptr if qk_norm else None,
                                 dev["kn"].ptr if qk_norm else None, eps, dev["cs"].ptr, dev["sn"].ptr,
                                 dev["step"].ptr, n_head, n_kv_head, hd, 0, dev["kc"].ptr, dev["vc"].ptr,
                                 capi.KV_F16 if kv == "f16" else capi.KV_F32, max_seq * hd, max_seq, dscores.ptr,
                                 dout.ptr, dxq.ptr if with_q8k else None, None))
    got = dout.to_array(np.float32, n_head * hd)
    qe, ke = q.copy(), k.copy()
    if qk_norm:
        for h in range(n_head):
            O.lib().orc_rmsnorm(ptr(qe) + 4 * h * hd, ptr(qe) + 4 * h * hd, ptr(qn), hd, eps)
        for h in range(n_kv_head):
            O.lib().orc_rmsnorm(ptr(ke) + 4 * h * hd, ptr(ke) + 4 * h * hd, ptr(kn), hd, eps)
    O.lib().orc_rope(ptr(qe), n_head, hd, ptr(cs) + 4 * pos * half, ptr(sn) + 4 * pos * half, 0)
    O.lib().orc_rope(ptr(ke), n_kv_head, hd, ptr(cs) + 4 * pos * half, ptr(sn) + 4 * pos * half, 0)
    kc[:, pos] = ke.reshape(n_kv_head, hd)
    vc[:, pos] = v.reshape(n_kv_head, hd)
    kc32, vc32 = np.ascontiguousarray(kc, np.float32), np.ascontiguousarray(vc, np.float32)
    exp = np.empty(n_head * hd, np.float32)
    scores = np.empty(max_seq, np.float32)
    O.lib().orc_attention(ptr(exp), ptr(qe), ptr(kc32), ptr(vc32), n_head, n_kv_head, hd, pos + 1, max_seq,
                          ptr(scores), 1)
    assert np.array_equal(bits(got), bits(exp)), float(np.abs(got - exp).max())
    assert dev["kc"].to_array(ct, kc.shape).tobytes() == kc.tobytes()
    assert dev["vc"].to_array(ct, vc.shape).tobytes() == vc.tobytes()
    if with_q8k:
        assert dxq.to_array(np.uint8, n_head * hd // 256 * 292).tobytes() == O.quantize(exp, O.Q8_K).tobytes()


def _gemm_case(kind, n_in, n_out, n_tok, seed, gen="workload"):
    t = TYPES[kind]
    rng = np.random.default_rng(seed)
    nb = n_out * n_in // O.QK[t]
    w = (random_blocks(kind, nb, rng) if gen == "workload" else ref_blocks(kind, nb, seed)).reshape(n_out, -1)
    x = np.random.default_rng(seed + 1).standard_normal((n_tok, n_in)).astype(np.float32)
    return t, w, O.quantize(x, O.Q8_K)


def _gemm_run(t, w, xq, n_in, n_out, n_tok, row0=0, row1=None, bias=None, resid=None, epilogue=0):
    L = lib()
    row1 = n_out if row1 is None else row1
    m = capi.DeviceMatrix(t, n_in, n_out, w)
    assert L.sdy_gemm_ok(ctypes.byref(m.m), n_tok), "matrix failed the GEMM exactness check"
    out_cols = (row1 - row0) // 2 if epilogue else n_out
    dq = capi.DeviceBuffer.from_array(xq)
    dout = capi.DeviceBuffer.from_array(np.full((n_tok, out_cols), np.nan, np.float32))
    ws = capi.DeviceBuffer(L.sdy_gemm_ws_bytes(n_tok, n_in))
    db = capi.DeviceBuffer.from_array(bias) if bias is not None else None
    dr = capi.DeviceBuffer.from_array(resid) if resid is not None else None
    a = capi.SdyMvArgs(xq=dq.ptr, n_tok=n_tok, out=dout.ptr, out_stride=out_cols, row0=row0, row1=row1,
                       bias=db.ptr if db else None, resid=dr.ptr if dr else None, epilogue=epilogue)
    capi.check(L.sdy_gemm(ctypes.byref(m.m), ctypes.byref(a), ws.ptr, None))
    return dout.to_array(np.float32, (n_tok, out_cols))


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("n_in,n_out,n_tok", [(256, 40, 16), (2048, 128, 33), (2048, 300, 64), (768, 96, 100),
                                              (11008, 64, 20), (4096, 200, 200), (2048, 37, 129)])
def test_gemm_bit_exact(kind, n_in, n_out, n_tok):
    """The MFMA prefill GEMM gives the reference's bits (integer super-block dots, f32 combine in
    super-block order) for every token and row, including partial row and token tiles."""
    t, w, xq = _gemm_case(kind, n_in, n_out, n_tok, seed=n_in + n_out + n_tok)
    got = _gemm_run(t, w, xq, n_in, n_out, n_tok)
    exp = O.matmul_q(w, t, xq, n_in, simd=1)
    assert np.array_equal(bits(got), bits(exp))


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
def test_gemm_bit_exact_with_subnormal_scale_products(kind):
    """Tokens whose activations are scaled by 2^-80 .. 2^-119: their Q8_K scales yd reach 2^-127, and
    the combine's products yd*d and yd*dmin (formed on the matrix cores for one wave per row tile)
    and the sums after them run through f32 subnormals. The bits stay the oracle's."""
    n_in, n_out, n_tok = 512, 96, 40
    t = TYPES[kind]
    rng = np.random.default_rng(77)
    w = random_blocks(kind, n_out * n_in // O.QK[t], rng).reshape(n_out, -1)
    x = np.random.default_rng(78).standard_normal((n_tok, n_in)).astype(np.float32)
    x *= np.float32(2.0) ** -(80 + np.arange(n_tok, dtype=np.float32))[:, None]
    xq = O.quantize(x, O.Q8_K)
    got = _gemm_run(t, w, xq, n_in, n_out, n_tok)
    exp = O.matmul_q(w, t, xq, n_in, simd=1)
    # the smallest tokens' yd times the rows' d scales (an f16 at byte 0 of a Q4_K block, 208 of a
    # Q6_K one) are f32 subnormals: the case reaches the range it is about
    yd = np.ascontiguousarray(xq.reshape(n_tok, -1)[:, :4]).view(np.float32)[:, 0]
    off = 0 if kind == "Q4_K" else 208
    d = np.ascontiguousarray(w.reshape(-1, w.shape[1] // (n_in // 256))[:, off:off + 2]).view(np.float16)[:, 0]
    prods = np.abs(yd[-1]).astype(np.float64) * np.abs(d.astype(np.float64))
    assert np.any((prods > 0) & (prods < np.finfo(np.float32).tiny))
    assert np.all(np.isfinite(exp))
    assert np.array_equal(bits(got), bits(exp))


@pytest.mark.parametrize("n_in,n_tok", [(2048, 512), (11008, 33), (256, 16)])
def test_gemm_ws_ready_reuses_expansion(n_in, n_tok):
    """ws_ready = 1 skips the f16 expansion of the activations: a Q6_K GEMM that reuses the workspace
    a Q4_K GEMM on the same Q8_K input just filled gives the bits of its own full call and of the
    oracle; after a different input has been expanded into the workspace, a full call is needed again."""
    L = lib()
    t4, w4, xq = _gemm_case("Q4_K", n_in, 96, n_tok, seed=n_in + n_tok)
    t6, w6, _ = _gemm_case("Q6_K", n_in, 70, n_tok, seed=n_in + n_tok + 5)
    m4, m6 = capi.DeviceMatrix(t4, n_in, 96, w4), capi.DeviceMatrix(t6, n_in, 70, w6)
    assert L.sdy_gemm_ok(ctypes.byref(m4.m), n_tok) and L.sdy_gemm_ok(ctypes.byref(m6.m), n_tok)
    dq = capi.DeviceBuffer.from_array(xq)
    ws = capi.DeviceBuffer(L.sdy_gemm_ws_bytes(n_tok, n_in))
    d4, d6 = capi.DeviceBuffer(n_tok * 96 * 4), capi.DeviceBuffer(n_tok * 70 * 4)

    def run(m, dout, n_out, ready, xq_ptr=dq.ptr):
        a = capi.SdyMvArgs(xq=xq_ptr, n_tok=n_tok, out=dout.ptr, out_stride=n_out, row0=0, row1=n_out,
                           ws_ready=ready)
        capi.check(L.sdy_gemm(ctypes.byref(m.m), ctypes.byref(a), ws.ptr, None))
        return dout.to_array(np.float32, (n_tok, n_out))

    got4 = run(m4, d4, 96, 0)
    got6_reused = run(m6, d6, 70, 1)
    exp6 = O.matmul_q(w6, t6, xq, n_in, simd=1)
    assert np.array_equal(bits(got4), bits(O.matmul_q(w4, t4, xq, n_in, simd=1)))
    assert np.array_equal(bits(got6_reused), bits(exp6))
    assert np.array_equal(bits(run(m6, d6, 70, 0)), bits(exp6))
    # another input expanded into the workspace: the reused result follows that input
    xq2 = O.quantize(np.random.default_rng(n_in).standard_normal((n_tok, n_in)).astype(np.float32), O.Q8_K)
    dq2 = capi.DeviceBuffer.from_array(xq2)
    run(m4, d4, 96, 0, dq2.ptr)
    assert np.array_equal(bits(run(m6, d6, 70, 1)), bits(O.matmul_q(w6, t6, xq2, n_in, simd=1)))
    assert np.array_equal(bits(run(m6, d6, 70, 0)), bits(exp6))


@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("n_in,n_tok", [(2048, 512), (11008, 40), (4096, 17)])
def test_quantize_gemm_expansion(norm, n_in, n_tok):
    """sdy_quantize_gemm / sdy_norm_quant_gemm write the Q8_K bytes (and the normalised rows) of
    sdy_quantize / sdy_norm_quant, plus the GEMM's expansion of them: a GEMM with ws_ready = 1 after
    them gives the bits of a full GEMM on those bytes and of the oracle. Rows include all-zero ones."""
    L = lib()
    rng = np.random.default_rng(n_in + n_tok + norm)
    x = rng.standard_normal((n_tok, n_in)).astype(np.float32)
    x[1] = 0.0
    wn = (1 + 0.3 * rng.standard_normal(n_in)).astype(np.float32)
    t, w, _ = _gemm_case("Q4_K", n_in, 64, n_tok, seed=n_in + 3)
    m = capi.DeviceMatrix(t, n_in, 64, w)
    assert L.sdy_gemm_ok(ctypes.byref(m.m), n_tok)
    dx, dw = capi.DeviceBuffer.from_array(x), capi.DeviceBuffer.from_array(wn)
    qb = n_tok * n_in // 256 * 292
    dq1, dq2 = capi.DeviceBuffer(qb), capi.DeviceBuffer(qb)
    db1, db2 = capi.DeviceBuffer(x.nbytes), capi.DeviceBuffer(x.nbytes)
    ws = capi.DeviceBuffer(L.sdy_gemm_ws_bytes(n_tok, n_in))
    if norm:
        capi.check(L.sdy_norm_quant(dx.ptr, dw.ptr, 1e-6, n_in, n_tok, db1.ptr, O.Q8_K, dq1.ptr, None))
        capi.check(L.sdy_norm_quant_gemm(dx.ptr, dw.ptr, 1e-6, n_in, n_tok, db2.ptr, dq2.ptr, ws.ptr, None))
        assert np.array_equal(bits(db2.to_array(np.float32, x.shape)), bits(db1.to_array(np.float32, x.shape)))
    else:
        capi.check(L.sdy_quantize(O.Q8_K, dx.ptr, dq1.ptr, n_in, n_tok, None))
        capi.check(L.sdy_quantize_gemm(dx.ptr, dq2.ptr, n_in, n_tok, ws.ptr, None))
    q1 = dq1.to_array(np.uint8, qb)
    assert dq2.to_array(np.uint8, qb).tobytes() == q1.tobytes()
    dout = capi.DeviceBuffer(n_tok * 64 * 4)

    def gemm(ready):
        a = capi.SdyMvArgs(xq=dq2.ptr, n_tok=n_tok, out=dout.ptr, out_stride=64, row0=0, row1=64, ws_ready=ready)
        capi.check(L.sdy_gemm(ctypes.byref(m.m), ctypes.byref(a), ws.ptr, None))
        return dout.to_array(np.float32, (n_tok, 64))

    reused = gemm(1)
    exp = O.matmul_q(w, t, q1.reshape(n_tok, -1), n_in, simd=1)
    assert np.array_equal(bits(reused), bits(exp))
    assert np.array_equal(bits(gemm(0)), bits(exp))


@pytest.mark.parametrize("wide1,wide2", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("n_in,rows1,rows2,n_tok", [(2048, 2304, 256, 512), (1024, 200, 77, 45)])
def test_gemm2_pair_launch_bit_exact(n_in, rows1, rows2, n_tok, wide1, wide2):
    """sdy_gemm2 (a layer's Q4_K q|k and Q6_K v on the same activations, one launch) gives each matrix
    the oracle's bits, bias included, in the one-fragment and wide forms of either matrix, and with
    row counts that do not fill the 64-row tiles."""
    L = lib()
    rng = np.random.default_rng(rows1 + rows2 + n_tok)
    def mat(kind, rows, wide, seed):
        if wide:
            return _full_range_blocks(kind, rows, n_in, seed)
        return _gemm_case(kind, n_in, rows, n_tok, seed=seed)[1]
    w1, w2 = mat("Q4_K", rows1, wide1, 3), mat("Q6_K", rows2, wide2, 4)
    x = rng.standard_normal((n_tok, n_in)).astype(np.float32)
    xq = O.quantize(x, O.Q8_K)
    b1 = rng.standard_normal(rows1).astype(np.float32)
    b2 = rng.standard_normal(rows2).astype(np.float32)
    m1, m2 = capi.DeviceMatrix(O.Q4_K, n_in, rows1, w1), capi.DeviceMatrix(O.Q6_K, n_in, rows2, w2)
    assert m1.m.gemm_ok == (2 if wide1 else 1) and m2.m.gemm_ok == (2 if wide2 else 1)
    dq = capi.DeviceBuffer.from_array(xq)
    ws = capi.DeviceBuffer(L.sdy_gemm_ws_bytes(n_tok, n_in))
    d1 = capi.DeviceBuffer.from_array(np.full((n_tok, rows1), np.nan, np.float32))
    d2 = capi.DeviceBuffer.from_array(np.full((n_tok, rows2), np.nan, np.float32))
    db1, db2 = capi.DeviceBuffer.from_array(b1), capi.DeviceBuffer.from_array(b2)
    a1 = capi.SdyMvArgs(xq=dq.ptr, n_tok=n_tok, out=d1.ptr, out_stride=rows1, row0=0, row1=rows1, bias=db1.ptr)
    a2 = capi.SdyMvArgs(xq=dq.ptr, n_tok=n_tok, out=d2.ptr, out_stride=rows2, row0=0, row1=rows2, bias=db2.ptr)
    capi.check(L.sdy_gemm2(ctypes.byref(m1.m), ctypes.byref(a1), ctypes.byref(m2.m), ctypes.byref(a2), ws.ptr, None))
    got1, got2 = d1.to_array(np.float32, (n_tok, rows1)), d2.to_array(np.float32, (n_tok, rows2))
    assert np.array_equal(bits(got1), bits(O.matmul_q(w1, O.Q4_K, xq, n_in, simd=1) + b1))
    assert np.array_equal(bits(got2), bits(O.matmul_q(w2, O.Q6_K, xq, n_in, simd=1) + b2))


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
def test_gemm_layout_copy_and_planes_same_bits(kind):
    """The GEMM reads the tiled copy that sdy_mat_gemm_layout makes (the default of DeviceMatrix and
    of the engine) or, without one, the planes: the same bits, the oracle's, with a row count that
    is not a multiple of the 32-row tile and a row range; an upload into the matrix drops the copy
    (it would be stale) and the GEMM goes on with the planes."""
    L = lib()
    n_in, n_out, n_tok = 1024, 77, 45
    t, w, xq = _gemm_case(kind, n_in, n_out, n_tok, seed=21)
    exp = O.matmul_q(w, t, xq, n_in, simd=1)
    dq = capi.DeviceBuffer.from_array(xq)
    ws = capi.DeviceBuffer(L.sdy_gemm_ws_bytes(n_tok, n_in))

    def run(m, row0=0, row1=n_out):
        dout = capi.DeviceBuffer.from_array(np.full((n_tok, n_out), np.nan, np.float32))
        a = capi.SdyMvArgs(xq=dq.ptr, n_tok=n_tok, out=dout.ptr, out_stride=n_out, row0=row0, row1=row1)
        capi.check(L.sdy_gemm(ctypes.byref(m.m), ctypes.byref(a), ws.ptr, None))
        return dout.to_array(np.float32, (n_tok, n_out))

    tiled = capi.DeviceMatrix(t, n_in, n_out, w)
    assert tiled.m.gbase and tiled.m.grows == n_out
    planes = capi.DeviceMatrix(t, n_in, n_out, w, gemm_layout=False)
    assert not planes.m.gbase
    assert np.array_equal(bits(run(tiled)), bits(exp))
    assert np.array_equal(bits(run(planes)), bits(exp))
    assert np.array_equal(bits(run(tiled, 33, 70)[:, 33:70]), bits(exp[:, 33:70]))
    raw = np.ascontiguousarray(w[5:6]).view(np.uint8)
    capi.check(L.sdy_mat_upload_rows(ctypes.byref(tiled.m), 5, 1, 1, raw.ctypes.data, None))
    assert not tiled.m.gbase
    assert np.array_equal(bits(run(tiled)), bits(exp))


@pytest.mark.parametrize("kind", list(TYPES))
def test_matrix_in_host_memory_same_bits(kind):
    """A matrix in pinned host memory (sdy_mat_alloc_host, read in place by the kernels over the host
    link, as the engine keeps expert stacks the device has no room for): its dequantised rows, its
    one-token and 40-token matvecs and, for the K-quants, the GEMM (the wide variant: a host matrix is
    not checked, and keeps no tiled copy) have the bits of the same matrix in device memory."""
    L = lib()
    n_in, n_out, n_tok = 2048, 70, 40
    t, w, xq = _matvec_case(kind, n_in, n_out, n_tok, seed=31)
    dev = capi.DeviceMatrix(t, n_in, n_out, w, gemm_layout=False)
    host = capi.SdyMat()
    capi.check(L.sdy_mat_alloc_host(ctypes.byref(host), t, n_in, n_out))
    try:
        assert host.hbase and host.base
        raw = np.ascontiguousarray(w).view(np.uint8)
        capi.check(L.sdy_mat_upload_rows(ctypes.byref(host), 0, 1, n_out, raw.ctypes.data, None))
        capi.check(L.sdy_mat_gemm_layout(ctypes.byref(host), None))
        assert not host.gbase
        kq = t in (O.Q4_K, O.Q6_K)
        assert host.gemm_ok == (2 if kq else 0)

        def dequant(m):
            d = capi.DeviceBuffer(n_out * n_in * 4)
            capi.check(L.sdy_dequant_rows(ctypes.byref(m), 0, n_out, d.ptr, None))
            return d.to_array(np.float32, (n_out, n_in))

        def matvec(m, n, gemm=False):
            q = capi.DeviceBuffer.from_array(xq[:n] if not gemm else O.quantize(
                np.random.default_rng(32).standard_normal((n, n_in)).astype(np.float32), O.Q8_K))
            out = capi.DeviceBuffer.from_array(np.full((n, n_out), np.nan, np.float32))
            a = capi.SdyMvArgs(xq=q.ptr, n_tok=n, out=out.ptr, out_stride=n_out, row0=0, row1=n_out)
            if gemm:
                ws = capi.DeviceBuffer(L.sdy_gemm_ws_bytes(n, n_in))
                capi.check(L.sdy_gemm(ctypes.byref(m), ctypes.byref(a), ws.ptr, None))
            else:
                capi.check(L.sdy_matvec(ctypes.byref(m), ctypes.byref(a), None))
            capi.check(L.sdy_sync(None))
            return out.to_array(np.float32, (n, n_out))

        assert np.array_equal(bits(dequant(host)), bits(dequant(dev.m)))
        for n in (1, n_tok):
            got = matvec(host, n)
            assert np.all(np.isfinite(got))
            assert np.array_equal(bits(got), bits(matvec(dev.m, n))), n
        if kq:
            got = matvec(host, n_tok, gemm=True)
            assert np.array_equal(bits(got), bits(matvec(dev.m, n_tok, gemm=True)))
            assert np.array_equal(bits(got), bits(O.matmul_q(w, t, O.quantize(
                np.random.default_rng(32).standard_normal((n_tok, n_in)).astype(np.float32), O.Q8_K), n_in, simd=1)))
    finally:
        L.sdy_mat_free(ctypes.byref(host))


@pytest.mark.parametrize("variant", ["11", "12", "13", "14", "15", "16", "17", "18", "19", "20"])
@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
def test_gemm_tile_variants_bit_exact(kind, variant, monkeypatch):
    """Every workgroup tile shape of the GEMM (forced through SARDYNE_GEMM_VARIANT; 17, 18 and 20 split
    each super-block's units between two waves, 19 and 20 keep two super-blocks in flight) gives the
    reference's bits, with partial row and token tiles (1 to 43 super-blocks: every remainder of the
    rounds of three), in its one-fragment and wide forms, and with the SwiGLU and residual epilogues."""
    monkeypatch.setenv("SARDYNE_GEMM_VARIANT", variant)
    for n_in, n_out, n_tok in [(256, 64, 40), (512, 96, 33), (2048, 300, 200), (768, 40, 17), (11008, 70, 130)]:
        t, w, xq = _gemm_case(kind, n_in, n_out, n_tok, seed=n_in + n_out + n_tok + 1)
        got = _gemm_run(t, w, xq, n_in, n_out, n_tok)
        exp = O.matmul_q(w, t, xq, n_in, simd=1)
        assert np.array_equal(bits(got), bits(exp)), (n_in, n_out, n_tok)
    sw = _gemm_run(t, w, xq, n_in, n_out, n_tok, epilogue=capi.EPI_SWIGLU)
    g, u = exp[:, 0::2].copy(), exp[:, 1::2].copy()
    lib().op_silu_mul(ptr(g), ptr(u), g.size)
    assert np.array_equal(bits(sw), bits(g))
    resid = np.random.default_rng(5).standard_normal((n_tok, n_out)).astype(np.float32)
    assert np.array_equal(bits(_gemm_run(t, w, xq, n_in, n_out, n_tok, resid=resid)), bits(resid + exp))
    n_in, n_out, n_tok = 1024, 200, 150
    w = _full_range_blocks(kind, n_out, n_in, 11)
    xq = O.quantize(np.random.default_rng(12).standard_normal((n_tok, n_in)).astype(np.float32), O.Q8_K)
    got = _gemm_run(t, w, xq, n_in, n_out, n_tok)
    assert np.array_equal(bits(got), bits(O.matmul_q(w, t, xq, n_in, simd=1)))


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
def test_gemm_bias_resid_rows_swiglu(kind):
    n_in, n_out, n_tok = 512, 96, 40
    t, w, xq = _gemm_case(kind, n_in, n_out, n_tok, seed=7)
    exp = O.matmul_q(w, t, xq, n_in, simd=1)
    rng = np.random.default_rng(8)
    bias = rng.standard_normal(n_out).astype(np.float32)
    resid = rng.standard_normal((n_tok, n_out)).astype(np.float32)
    got = _gemm_run(t, w, xq, n_in, n_out, n_tok, bias=bias, resid=resid)
    assert np.array_equal(bits(got), bits(resid + (exp + bias)))
    part = _gemm_run(t, w, xq, n_in, n_out, n_tok, row0=32, row1=70)
    assert np.array_equal(bits(part[:, 32:70]), bits(exp[:, 32:70]))
    # SwiGLU over rows (2i, 2i+1)
    sw = _gemm_run(t, w, xq, n_in, n_out, n_tok, epilogue=capi.EPI_SWIGLU)
    g, u = exp[:, 0::2].copy(), exp[:, 1::2].copy()
    lib().op_silu_mul(ptr(g), ptr(u), g.size)
    assert np.array_equal(bits(sw), bits(g))


def _full_range_blocks(kind, n_out, n_in, seed):
    """Blocks with scales over the whole range the format stores: Q6_K int8 scales in [-128, 127]
    (row 0 all -128 with quants 0, i.e. values -32; row 1 all 127 with quants 63), Q4_K 6-bit scales
    and minima in [0, 63] (rows 0 and 1 all 63 with quants 15)."""
    rng = np.random.default_rng(seed)
    w = random_blocks(kind, n_out * n_in // 256, rng).reshape(n_out, n_in // 256, -1)
    if kind == "Q6_K":
        w[:, :, 192:208] = rng.integers(-128, 128, w.shape[:2] + (16,)).astype(np.int8).view(np.uint8)
        w[0, :, 0:192], w[0, :, 192:208] = 0, np.uint8(0x80)
        w[1, :, 0:192], w[1, :, 192:208] = 0xFF, 127
    else:
        w[:, :, 4:16] = rng.integers(0, 256, w.shape[:2] + (12,), dtype=np.uint8)
        w[0:2, :, 4:144] = 0xFF
    return w.reshape(n_out, -1)


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("n_in,n_out,n_tok", [(2048, 96, 40), (1024, 37, 129), (256, 64, 2)])
def test_gemm_wide_variant_bit_exact(kind, n_in, n_out, n_tok):
    """Matrices whose blocks the one-fragment scheme would round (Q6_K |sc * (q - 32)| above 2048,
    partial sums of 2^24 and more) are flagged for the wide variant (gemm_ok 2), which keeps
    the oracle's bits for every row and token: scales over the whole stored range, a token of one
    sign (Q8_K values all -127) that drives the extreme rows' sums to their bounds. The same shapes
    with the workload's scales take the one-fragment variant (gemm_ok 1)."""
    L = lib()
    t = TYPES[kind]
    w = _full_range_blocks(kind, n_out, n_in, n_in + n_out)
    x = np.random.default_rng(n_tok).standard_normal((n_tok, n_in)).astype(np.float32)
    x[0] = 1.0
    xq = O.quantize(x, O.Q8_K)
    m = capi.DeviceMatrix(t, n_in, n_out, w)
    assert m.m.gemm_ok == 2
    got = _gemm_run(t, w, xq, n_in, n_out, n_tok)
    exp = O.matmul_q(w, t, xq, n_in, simd=1)
    assert np.array_equal(bits(got), bits(exp))
    if n_out % 2 == 0:
        sw = _gemm_run(t, w, xq, n_in, n_out, n_tok, epilogue=capi.EPI_SWIGLU)
        g, u = exp[:, 0::2].copy(), exp[:, 1::2].copy()
        lib().op_silu_mul(ptr(g), ptr(u), g.size)
        assert np.array_equal(bits(sw), bits(g))
    _, w1, _ = _gemm_case(kind, n_in, n_out, n_tok, seed=n_in + n_out)
    assert capi.DeviceMatrix(t, n_in, n_out, w1).m.gemm_ok == 1


def test_gemm_variant_check_flags_rows():
    """One Q6_K block with scales -128 anywhere in the matrix selects the wide variant;
    ordinary rows keep the one-fragment one."""
    L = lib()
    w = random_blocks("Q6_K", 8 * 4, np.random.default_rng(3)).reshape(8, -1)
    ok = capi.DeviceMatrix(O.Q6_K, 1024, 8, w)
    assert L.sdy_gemm_ok(ctypes.byref(ok.m), 32) and ok.m.gemm_ok == 1
    w2 = w.copy().reshape(-1, 210)
    w2[5, 192:208] = np.uint8(0x80)  # scales -128: |-128 * (q - 32)| reaches 4096
    split = capi.DeviceMatrix(O.Q6_K, 1024, 8, w2.reshape(8, -1))
    assert L.sdy_gemm_ok(ctypes.byref(split.m), 32) and split.m.gemm_ok == 2


@pytest.mark.parametrize("interleaved", [0, 1], ids=["neox", "llama"])
@pytest.mark.parametrize("qk_norm", [False, True], ids=["plain", "qknorm"])
@pytest.mark.parametrize("v_in_stack", [True, False], ids=["v-stacked", "v-apart"])
def test_qk_rope_kv_strided_equals_packed(interleaved, qk_norm, v_in_stack):
    """The strided RoPE + KV write (token rows of q|k|v interleaved at the GEMM's stride
    q_dim + 2 kv_dim, or v in a buffer of its own with another stride) gives the bits of the packed
    form on contiguous copies: rotated q and k rows, and both caches."""
    import ctypes
    from sardyne_amd import capi
    L = capi.lib()
    capi.check(L.sdy_init())
    n_tok, n_head, n_kv, hd, pos0, max_seq = 5, 4, 2, 64, 3, 16
    qd, kvd = n_head * hd, n_kv * hd
    rng = np.random.default_rng(9)
    stack = rng.standard_normal((n_tok, qd + 2 * kvd)).astype(np.float32)
    v_apart = rng.standard_normal((n_tok, kvd + 32)).astype(np.float32)  # stride kvd + 32
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    cs, sn = np.empty((max_seq, hd // 2), np.float32), np.empty((max_seq, hd // 2), np.float32)
    L.op_rope_table(cs.ctypes.data, sn.ctypes.data, max_seq, hd, 1e6)
    head_stride = max_seq * hd
    D = capi.DeviceBuffer.from_array
    dcs, dsn, dqn, dkn = D(cs), D(sn), D(qn), D(kn)
    qn_p, kn_p = (dqn.ptr, dkn.ptr) if qk_norm else (None, None)
    # strided: q, k (and v) in the stacked rows
    dstack = D(stack)
    dv_apart = D(v_apart)
    kc1 = capi.DeviceBuffer.from_array(np.zeros(n_kv * head_stride, np.float32))
    vc1 = capi.DeviceBuffer.from_array(np.zeros(n_kv * head_stride, np.float32))
    row = qd + 2 * kvd
    v_ptr, v_stride = ((dstack.ptr + 4 * (qd + kvd), row) if v_in_stack else (dv_apart.ptr, kvd + 32))
    capi.check(L.sdy_qk_rope_kv_strided(dstack.ptr, dstack.ptr + 4 * qd, v_ptr, row, row, v_stride, qn_p, kn_p, 1e-6,
                                        dcs.ptr, dsn.ptr, pos0, n_tok, n_head, n_kv, hd, interleaved, kc1.ptr,
                                        vc1.ptr, capi.KV_F32, head_stride, None))
    # packed: contiguous copies
    q = np.ascontiguousarray(stack[:, :qd])
    k = np.ascontiguousarray(stack[:, qd:qd + kvd])
    v = np.ascontiguousarray(stack[:, qd + kvd:] if v_in_stack else v_apart[:, :kvd])
    dq, dk, dv = D(q), D(k), D(v)
    kc2 = capi.DeviceBuffer.from_array(np.zeros(n_kv * head_stride, np.float32))
    vc2 = capi.DeviceBuffer.from_array(np.zeros(n_kv * head_stride, np.float32))
    capi.check(L.sdy_qk_rope_kv(dq.ptr, dk.ptr, dv.ptr, qn_p, kn_p, 1e-6, dcs.ptr, dsn.ptr, pos0, n_tok, n_head, n_kv,
                                hd, interleaved, kc2.ptr, vc2.ptr, capi.KV_F32, head_stride, None))
    capi.check(L.sdy_sync(None))
    got = dstack.to_array(np.float32, stack.size).reshape(stack.shape)
    assert np.array_equal(bits(got[:, :qd]), bits(dq.to_array(np.float32, q.size).reshape(q.shape)))
    assert np.array_equal(bits(got[:, qd:qd + kvd]), bits(dk.to_array(np.float32, k.size).reshape(k.shape)))
    for a, b in ((kc1, kc2), (vc1, vc2)):
        assert np.array_equal(bits(a.to_array(np.float32, n_kv * head_stride)),
                              bits(b.to_array(np.float32, n_kv * head_stride)))
    # the rotation did happen, and the cache rows outside [pos0, pos0 + n_tok) stayed zero
    assert not np.array_equal(got[:, :qd], stack[:, :qd])
    kc = kc1.to_array(np.float32, n_kv * head_stride).reshape(n_kv, max_seq, hd)
    assert np.all(kc[:, :pos0] == 0) and np.all(kc[:, pos0 + n_tok:] == 0) and np.any(kc[:, pos0] != 0)


def _decode_expected(q, k, v, kc, vc, qn, kn, cs, sn, p, n_head, n_kv_head, hd, qk_norm, interleaved, eps):
    """The oracle's decode step (orc_model.c: q/k norm, RoPE, the cache write of position p, then
    orc_attention over p + 1 positions) on copies of the caches kc / vc (f32 or f16: the new row is
    rounded to the cache's type first). Returns (out, kc, vc) with the caches as written."""
    half = hd // 2
    qe, ke = q.copy(), k.copy()
    if qk_norm:
        for h in range(n_head):
            O.lib().orc_rmsnorm(ptr(qe) + 4 * h * hd, ptr(qe) + 4 * h * hd, ptr(qn), hd, eps)
        for h in range(n_kv_head):
            O.lib().orc_rmsnorm(ptr(ke) + 4 * h * hd, ptr(ke) + 4 * h * hd, ptr(kn), hd, eps)
    O.lib().orc_rope(ptr(qe), n_head, hd, ptr(cs) + 4 * p * half, ptr(sn) + 4 * p * half, interleaved)
    O.lib().orc_rope(ptr(ke), n_kv_head, hd, ptr(cs) + 4 * p * half, ptr(sn) + 4 * p * half, interleaved)
    kc, vc = kc.copy(), vc.copy()
    kc[:, p] = ke.reshape(n_kv_head, hd)
    vc[:, p] = v.reshape(n_kv_head, hd)
    kc32, vc32 = np.ascontiguousarray(kc, np.float32), np.ascontiguousarray(vc, np.float32)
    out = np.empty(n_head * hd, np.float32)
    scores = np.empty(kc.shape[1], np.float32)
    O.lib().orc_attention(ptr(out), ptr(qe), ptr(kc32), ptr(vc32), n_head, n_kv_head, hd, p + 1, kc.shape[1],
                          ptr(scores), 1)
    return out, kc, vc


CHUNKED_LAYOUTS = [(16, 2, 128, False, 0), (32, 4, 128, True, 0), (6, 2, 64, False, 1), (4, 4, 64, True, 0),
                   (32, 2, 128, False, 0), (8, 2, 256, True, 0)]
CHUNKED_IDS = ["qwen25-3b", "qwen3-30b-a3b", "llama-gqa3", "mha", "gqa16", "hd256"]


@pytest.mark.parametrize("n_head,n_kv_head,hd,qk_norm,interleaved", CHUNKED_LAYOUTS, ids=CHUNKED_IDS)
@pytest.mark.parametrize("max_seq,pos", [(2111, p) for p in (0, 63, 64, 65, 640, 1151, 2110)] +
                         [(9000, p) for p in (127, 128, 5000, 8999)])
@pytest.mark.parametrize("kv", ["f32", "f16"])
def test_decode_attention_chunked(n_head, n_kv_head, hd, qk_norm, interleaved, max_seq, pos, kv):
    """The two-launch chunked attention (64-position spans, or 128 for a 9000-position cache, partials
    merged in span order) against the oracle's decode step on the same cache: output within 1e-5 of
    the output scale, the new position's K/V rows bit-exact (f32), or the f16 rounding of the
    oracle's (f16 cache, whose f32 values the oracle then attends over), the Q8_K bytes those of the
    output it wrote. Two calls in a row (the second at pos - 1 over a fresh copy of the cache): the
    partials of one call do not leak into the next."""
    L = lib()
    eps = 1e-6
    assert L.sdy_attn_chunked_ok(n_head, n_kv_head, hd)
    rng = np.random.default_rng(pos * 13 + n_head + hd)
    cs, sn = np.empty(max_seq * hd // 2, np.float32), np.empty(max_seq * hd // 2, np.float32)
    L.op_rope_table(ptr(cs), ptr(sn), max_seq, hd, 1e6)
    ct = np.float16 if kv == "f16" else np.float32
    kc0 = rng.standard_normal((n_kv_head, max_seq, hd)).astype(ct)
    vc0 = rng.standard_normal((n_kv_head, max_seq, hd)).astype(ct)
    qn = (1 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    part = capi.DeviceBuffer(L.sdy_attn_chunked_floats(n_head, hd, max_seq) * 4)
    with_q8k = n_head * hd % 256 == 0
    for p in (pos, max(pos - 1, 0)):
        q = rng.standard_normal(n_head * hd).astype(np.float32) * 3
        k = rng.standard_normal(n_kv_head * hd).astype(np.float32) * 3
        v = rng.standard_normal(n_kv_head * hd).astype(np.float32)
        dev = {n: capi.DeviceBuffer.from_array(a) for n, a in
               dict(q=q, k=k, v=v, kc=kc0, vc=vc0, cs=cs, sn=sn, qn=qn, kn=kn,
                    step=np.array([0, p], np.int32)).items()}
        dout = capi.DeviceBuffer(n_head * hd * 4)
        dxq = capi.DeviceBuffer(n_head * hd // 256 * 292) if with_q8k else None
        capi.check(L.sdy_attn_decode_chunked(dev["q"].ptr, dev["k"].ptr, dev["v"].ptr,
                                             dev["qn"].ptr if qk_norm else None, dev["kn"].ptr if qk_norm else None,
                                             eps, dev["cs"].ptr, dev["sn"].ptr, dev["step"].ptr, n_head, n_kv_head, hd,
                                             interleaved, dev["kc"].ptr, dev["vc"].ptr,
                                             capi.KV_F16 if kv == "f16" else capi.KV_F32, max_seq * hd, max_seq,
                                             part.ptr, dout.ptr, dxq.ptr if with_q8k else None, None))
        got = dout.to_array(np.float32, n_head * hd)
        exp, kc, vc = _decode_expected(q, k, v, kc0, vc0, qn, kn, cs, sn, p, n_head, n_kv_head, hd, qk_norm,
                                       interleaved, eps)
        np.testing.assert_allclose(got, exp, rtol=0, atol=1e-5 * float(np.abs(exp).max()))
        assert dev["kc"].to_array(ct, kc.shape).tobytes() == kc.tobytes()
        assert dev["vc"].to_array(ct, vc.shape).tobytes() == vc.tobytes()
        if with_q8k:
            assert dxq.to_array(np.uint8, n_head * hd // 256 * 292).tobytes() == O.quantize(got, O.Q8_K).tobytes()


@pytest.mark.parametrize("n_head,n_kv_head,hd,qk_norm,interleaved",
                         [(16, 2, 128, False, 0), (32, 4, 128, True, 0), (6, 2, 64, False, 1), (4, 4, 64, True, 0),
                          (32, 2, 128, False, 0)],
                         ids=["qwen25-3b", "qwen3-30b-a3b", "llama-gqa3", "mha", "gqa16"])
@pytest.mark.parametrize("pos", [0, 63, 64, 65, 640, 1151, 2110])
def test_decode_attention_split(n_head, n_kv_head, hd, qk_norm, interleaved, pos):
    """The one-launch split attention (32-position chunks, partials merged in chunk order by the last
    workgroup of each kv group) against the oracle's exact decode step: output within 1e-5 of the
    output scale, the new position's K/V rows bit-exact (the same norm and rotation), the Q8_K bytes
    those of the output it wrote. Two calls in a row (the second at pos - 1 over a fresh copy of the
    cache) check that each call leaves the arrival counters at zero for the next."""
    L = lib()
    max_seq, eps, half = 2111, 1e-6, hd // 2
    assert L.sdy_attn_decode_split_ok(n_head, n_kv_head, hd)
    rng = np.random.default_rng(pos * 11 + n_head)
    cs, sn = np.empty(max_seq * half, np.float32), np.empty(max_seq * half, np.float32)
    L.op_rope_table(ptr(cs), ptr(sn), max_seq, hd, 1e6)
    kc0 = rng.standard_normal((n_kv_head, max_seq, hd)).astype(np.float32)
    vc0 = rng.standard_normal((n_kv_head, max_seq, hd)).astype(np.float32)
    qn = (1 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    part = capi.DeviceBuffer(L.sdy_attn_decode_split_floats(n_head, hd, max_seq) * 4)
    count = capi.DeviceBuffer.from_array(np.zeros(n_kv_head, np.uint32))
    with_q8k = (n_head // n_kv_head) * hd % 256 == 0
    for p in (pos, max(pos - 1, 0)):
        q = rng.standard_normal(n_head * hd).astype(np.float32) * 3
        k = rng.standard_normal(n_kv_head * hd).astype(np.float32) * 3
        v = rng.standard_normal(n_kv_head * hd).astype(np.float32)
        kc, vc = kc0.copy(), vc0.copy()
        dev = {n: capi.DeviceBuffer.from_array(a) for n, a in
               dict(q=q, k=k, v=v, kc=kc, vc=vc, cs=cs, sn=sn, qn=qn, kn=kn, step=np.array([0, p], np.int32)).items()}
        dout = capi.DeviceBuffer(n_head * hd * 4)
        dxq = capi.DeviceBuffer(n_head * hd // 256 * 292) if with_q8k else None
        capi.check(L.sdy_attn_decode_split(dev["q"].ptr, dev["k"].ptr, dev["v"].ptr, dev["qn"].ptr if qk_norm else None,
                                           dev["kn"].ptr if qk_norm else None, eps, dev["cs"].ptr, dev["sn"].ptr,
                                           dev["step"].ptr, n_head, n_kv_head, hd, interleaved, dev["kc"].ptr,
                                           dev["vc"].ptr, max_seq * hd, max_seq, part.ptr, count.ptr, dout.ptr,
                                           dxq.ptr if with_q8k else None, None))
        got = dout.to_array(np.float32, n_head * hd)
        qe, ke = q.copy(), k.copy()
        if qk_norm:
            for h in range(n_head):
                O.lib().orc_rmsnorm(ptr(qe) + 4 * h * hd, ptr(qe) + 4 * h * hd, ptr(qn), hd, eps)
            for h in range(n_kv_head):
                O.lib().orc_rmsnorm(ptr(ke) + 4 * h * hd, ptr(ke) + 4 * h * hd, ptr(kn), hd, eps)
        O.lib().orc_rope(ptr(qe), n_head, hd, ptr(cs) + 4 * p * half, ptr(sn) + 4 * p * half, interleaved)
        O.lib().orc_rope(ptr(ke), n_kv_head, hd, ptr(cs) + 4 * p * half, ptr(sn) + 4 * p * half, interleaved)
        kc[:, p] = ke.reshape(n_kv_head, hd)
        vc[:, p] = v.reshape(n_kv_head, hd)
        exp = np.empty(n_head * hd, np.float32)
        scores = np.empty(max_seq, np.float32)
        O.lib().orc_attention(ptr(exp), ptr(qe), ptr(kc), ptr(vc), n_head, n_kv_head, hd, p + 1, max_seq, ptr(scores), 1)
        np.testing.assert_allclose(got, exp, rtol=0, atol=1e-5 * float(np.abs(exp).max()))
        assert np.array_equal(bits(dev["kc"].to_array(np.float32, kc.shape)), bits(kc))
        assert np.array_equal(bits(dev["vc"].to_array(np.float32, vc.shape)), bits(vc))
        if with_q8k:
            assert dxq.to_array(np.uint8, n_head * hd // 256 * 292).tobytes() == O.quantize(got, O.Q8_K).tobytes()
        assert np.all(count.to_array(np.uint32, n_kv_head) == 0)


def _mat_bytes(m):
    L = lib()
    out = np.empty(m.bytes, np.uint8)
    capi.check(L.sdy_d2h(out.ctypes.data, m.base, m.bytes, None))
    capi.check(L.sdy_sync(None))
    return out


@pytest.mark.parametrize("kind,n_in,grp,n_grp,bad_scale", [("Q4_K", 2048, 700, 2, False), ("Q6_K", 1024, 3000, 1, False),
                                                           ("Q6_K", 1024, 900, 3, True), ("Q8_0", 2048, 1200, 1, False)])
def test_pipelined_upload_equals_synchronous(kind, n_in, grp, n_grp, bad_scale):
    """The pipelined uploader (1 MiB pinned/device slots, so a tensor spans several slots; the rows of
    a per-group interleaved map, as the engine's per-expert gate|up, split at group boundaries) leaves
    the same device bytes as the synchronous upload, and the deferred variant check the same
    gemm_ok (a Q6_K block with scale -128 selects the wide variant)."""
    L = lib()
    t = TYPES[kind]
    rng = np.random.default_rng(grp + n_in)
    n = grp * n_grp
    w = [random_blocks(kind, n * n_in // O.QK[t], rng).reshape(n, -1) for _ in range(2)]
    if bad_scale:
        w[1][n - 1].reshape(-1, 210)[0, 192:208] = np.uint8(0x80)
    rows = 2 * n
    mats = [capi.SdyMat(), capi.SdyMat()]
    for m in mats:
        capi.check(L.sdy_mat_alloc(ctypes.byref(m), t, n_in, rows))
    # synchronous: the two sources interleaved per group (step 2, group grp, group stride 2 grp)
    for part in range(2):
        capi.check(L.sdy_mat_upload_map(ctypes.byref(mats[0]), part, n, 2, grp, 2 * grp, w[part].ctypes.data, None))
    up = ctypes.c_void_p()
    capi.check(L.sdy_uploader_new(ctypes.byref(up), 1 << 20, 3, 4, None))
    try:
        for part in range(2):
            capi.check(L.sdy_uploader_rows(up, ctypes.byref(mats[1]), part, n, 2, grp, 2 * grp, w[part].ctypes.data))
        capi.check(L.sdy_uploader_finish(up))
        b = ctypes.c_double()
        L.sdy_uploader_stats(up, ctypes.byref(b), None, None)
        assert b.value == 2 * w[0].nbytes
    finally:
        capi.check(L.sdy_uploader_free(up))
    try:
        assert _mat_bytes(mats[0]).tobytes() == _mat_bytes(mats[1]).tobytes()
        assert mats[0].gemm_ok == mats[1].gemm_ok
        if kind in ("Q4_K", "Q6_K"):
            assert mats[1].gemm_ok == (2 if bad_scale else 1)
    finally:
        for m in mats:
            L.sdy_mat_free(ctypes.byref(m))


@pytest.mark.parametrize("n_tok,k,n_exp,bn", [(1, 1, 1, 32), (3, 2, 8, 32), (512, 8, 128, 32), (700, 6, 60, 32),
                                            (2048, 8, 128, 32), (2100, 8, 512, 16), (333, 4, 512, 64)])
def test_moe_sort_stable_grouping(n_tok, k, n_exp, bn):
    """The expert sort against numpy's stable argsort of the expert ids: rows grouped by expert in
    (token, slot) order, each expert's first row and tile offset (tiles of bn rows), for the
    in-LDS sorting network (up to 16384 pairs) and the segmented counting sort beyond it; skewed
    routings (a few experts take most pairs, some none) included."""
    L = lib()
    rng = np.random.default_rng(n_tok * 31 + n_exp)
    hot = rng.choice(n_exp, max(1, n_exp // 8), replace=False)
    top = np.empty((n_tok, k), np.int32)
    for t in range(n_tok):
        pool = hot if rng.random() < 0.5 and len(hot) >= k else np.arange(n_exp)
        top[t] = rng.choice(pool, k, replace=False) if len(pool) >= k else rng.choice(pool, k)
    n = n_tok * k
    dtop = capi.DeviceBuffer.from_array(top)
    grp_tok, grp_tile = capi.DeviceBuffer(4 * (n_exp + 1)), capi.DeviceBuffer(4 * (n_exp + 1))
    src, orow = capi.DeviceBuffer(4 * n), capi.DeviceBuffer(4 * n)
    capi.check(L.sdy_moe_sort(dtop.ptr, n_tok, k, n_exp, bn, grp_tok.ptr, grp_tile.ptr, src.ptr, orow.ptr, None))
    flat = top.reshape(-1)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=n_exp)
    assert np.array_equal(orow.to_array(np.int32, n), order)
    assert np.array_equal(src.to_array(np.int32, n), order // k)
    assert np.array_equal(grp_tok.to_array(np.int32, n_exp + 1), np.concatenate([[0], np.cumsum(counts)]))
    tiles = (counts + bn - 1) // bn
    assert np.array_equal(grp_tile.to_array(np.int32, n_exp + 1), np.concatenate([[0], np.cumsum(tiles)]))


@pytest.mark.parametrize("kind,n_in,rows,n_exp,n_tok,k", [("Q4_K", 512, 96, 8, 45, 3), ("Q6_K", 768, 64, 16, 70, 4),
                                                           ("Q4_K", 256, 128, 128, 33, 8)])
def test_moe_sort_and_grouped_gemm_equal_per_expert_gemm(kind, n_in, rows, n_exp, n_tok, k):
    """The expert sort (stable: each expert's pairs in (token, slot) order, tile counts per expert)
    and the grouped GEMM over a stacked expert matrix: every routed (token, slot) row has the bits of
    the per-expert GEMM of that token's row, through the SwiGLU epilogue (the gate|up form) and
    through the output-row scatter (the down form). Some experts receive no token."""
    L = lib()
    t = TYPES[kind]
    rng = np.random.default_rng(n_exp * 100 + n_tok)
    w = random_blocks(kind, n_exp * rows * n_in // O.QK[t], rng).reshape(n_exp * rows, -1)
    m = capi.DeviceMatrix(t, n_in, n_exp * rows, w)
    assert L.sdy_gemm_ok(ctypes.byref(m.m), 2)
    top = np.stack([rng.choice(n_exp // 2 + 1, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    x = rng.standard_normal((n_tok, n_in)).astype(np.float32)
    bn = L.sdy_gemm_grouped_tile()
    R = n_tok * k
    D = capi.DeviceBuffer.from_array
    dtop, dx = D(top), D(x)
    grp_tok, grp_tile = capi.DeviceBuffer(4 * (n_exp + 1)), capi.DeviceBuffer(4 * (n_exp + 1))
    src, orow = capi.DeviceBuffer(4 * R), capi.DeviceBuffer(4 * R)
    capi.check(L.sdy_moe_sort(dtop.ptr, n_tok, k, n_exp, bn, grp_tok.ptr, grp_tile.ptr, src.ptr, orow.ptr, None))
    gt = grp_tok.to_array(np.int32, n_exp + 1)
    gl = grp_tile.to_array(np.int32, n_exp + 1)
    s_src, s_orow = src.to_array(np.int32, R), orow.to_array(np.int32, R)
    flat = top.reshape(-1)
    exp_rows = [i for e in range(n_exp) for i in range(R) if flat[i] == e]
    assert list(s_orow) == exp_rows and np.array_equal(s_src, s_orow // k)
    cnt = np.bincount(flat, minlength=n_exp)
    assert np.array_equal(gt, np.concatenate([[0], np.cumsum(cnt)]))
    assert np.array_equal(gl, np.concatenate([[0], np.cumsum((cnt + bn - 1) // bn)]))
    # routed rows, quantised with the GEMM expansion
    xs = capi.DeviceBuffer(4 * R * n_in)
    capi.check(L.sdy_gather_rows(dx.ptr, src.ptr, R, n_in, xs.ptr, None))
    xq = capi.DeviceBuffer(R * O.row_size(O.Q8_K, n_in))
    ws = capi.DeviceBuffer(L.sdy_gemm_ws_bytes(R, n_in))
    capi.check(L.sdy_quantize_gemm(xs.ptr, xq.ptr, n_in, R, ws.ptr, None))
    ref = O.matmul_q(w, t, O.quantize(x, O.Q8_K), n_in)  # [n_tok][n_exp * rows]: every expert's rows
    # plain rows scattered back to (token, slot) order
    out = capi.DeviceBuffer.from_array(np.full((R, rows), np.nan, np.float32))
    a = capi.SdyMvArgs(xq=xq.ptr, n_tok=R, out=out.ptr, out_stride=rows, ws_ready=1)
    capi.check(L.sdy_gemm_grouped(ctypes.byref(m.m), rows, n_exp, grp_tok.ptr, grp_tile.ptr, orow.ptr, None, 0,
                                  ctypes.byref(a), ws.ptr, None))
    got = out.to_array(np.float32, (R, rows))
    exp = np.stack([ref[i // k, flat[i] * rows:(flat[i] + 1) * rows] for i in range(R)])
    assert np.array_equal(bits(got), bits(exp))
    # the same rows read by index from the n_tok token rows, quantised once (no gathered copy)
    xq1 = capi.DeviceBuffer(n_tok * O.row_size(O.Q8_K, n_in))
    ws1 = capi.DeviceBuffer(L.sdy_gemm_ws_bytes(n_tok, n_in))
    capi.check(L.sdy_quantize_gemm(dx.ptr, xq1.ptr, n_in, n_tok, ws1.ptr, None))
    out1 = capi.DeviceBuffer.from_array(np.full((R, rows), np.nan, np.float32))
    a1 = capi.SdyMvArgs(xq=xq1.ptr, n_tok=R, out=out1.ptr, out_stride=rows, ws_ready=1)
    capi.check(L.sdy_gemm_grouped(ctypes.byref(m.m), rows, n_exp, grp_tok.ptr, grp_tile.ptr, orow.ptr, src.ptr, n_tok,
                                  ctypes.byref(a1), ws1.ptr, None))
    assert np.array_equal(bits(out1.to_array(np.float32, (R, rows))), bits(exp))
    a1.ws_ready = 0  # an index needs the caller's expansion
    assert L.sdy_gemm_grouped(ctypes.byref(m.m), rows, n_exp, grp_tok.ptr, grp_tile.ptr, orow.ptr, src.ptr, n_tok,
                              ctypes.byref(a1), ws1.ptr, None) != 0
    # SwiGLU pairs (rows 2i, 2i+1 of each expert), outputs in sorted order
    sw = capi.DeviceBuffer.from_array(np.full((R, rows // 2), np.nan, np.float32))
    a = capi.SdyMvArgs(xq=xq.ptr, n_tok=R, out=sw.ptr, out_stride=rows // 2, ws_ready=1, epilogue=capi.EPI_SWIGLU)
    capi.check(L.sdy_gemm_grouped(ctypes.byref(m.m), rows, n_exp, grp_tok.ptr, grp_tile.ptr, None, None, 0,
                                  ctypes.byref(a), ws.ptr, None))
    got = sw.to_array(np.float32, (R, rows // 2))
    srt = exp[s_orow]
    g, u = srt[:, 0::2].copy(), srt[:, 1::2].copy()
    lib().op_silu_mul(ptr(g), ptr(u), g.size)
    assert np.array_equal(bits(got), bits(g))


@pytest.mark.parametrize("mode", [0, 1, 2], ids=["flat", "two_level", "two_level_fenced"])
def test_grid_barrier_probe_publishes_every_value(mode):
    """The persistent-kernel barrier measurement (sdy_grid_barrier_probe): over 300 rounds of a
    256-workgroup co-resident grid, every workgroup reads back another's data of that round, with and
    without the other waves streaming HBM meanwhile; no value is stale and no bounded wait gives up."""
    L = capi.lib()
    capi.check(L.sdy_init())
    for stream_mb in (0, 256):
        st = capi.SdyBarrierStats()
        capi.check(L.sdy_grid_barrier_probe(256, 300, mode, stream_mb, ctypes.byref(st)))
        assert st.timeouts == 0 and st.mismatches == 0, (stream_mb, st.timeouts, st.mismatches)
        assert st.rounds_done == 300 and 0 < st.us_median < 100
    ug, ue = ctypes.c_float(), ctypes.c_float()
    capi.check(L.sdy_kernel_boundary_us(200, ctypes.byref(ug), ctypes.byref(ue)))
    assert 0 < ug.value < 50 and 0 < ue.value < 50

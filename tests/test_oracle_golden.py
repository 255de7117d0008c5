"""CPU pinning of the oracle (oracle/pih_oracle.c) before it is trusted as
the GPU parity checker:
  1. the reference's own known-answer tests (tests/cpp/model/*_test.cpp),
     restated as values;
  2. the committed golden vectors tests/golden/ref_vectors.npz, produced by
     the reference's oracle sources compiled in place (oracle/_ref), and the
     live oracle/_ref library itself where it was built;
  3. closed forms and invariants for what neither covers (BASELINE-only
     formats): reductions to a pinned function, float64 brute force on
     exactly-representable inputs, exhaustive codec sweeps.
"""
import os

import numpy as np
import pytest

import oracle
from pih_amd import synth

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN, allow_pickle=False)


def f32(bits):
    return oracle.bf16_bits_to_f32(bits)


# --------------------------------------------------------------- codecs
def test_e4m3_reference_kats():
    # deepseek_fp8_activation_codec_test.cpp:11-26
    assert oracle.e4m3_encode(0.0) == 0x00
    assert oracle.e4m3_encode(-0.0) == 0x80
    assert oracle.e4m3_encode(1.0) == 0x38
    assert oracle.e4m3_encode(448.0) == 0x7E
    assert oracle.e4m3_decode(0x7E) == 448.0
    assert oracle.e4m3_decode(0x7F) is None
    assert oracle.e4m3_encode(1.0625) == 0x38
    assert oracle.e4m3_encode(1.1875) == 0x3A


def test_e4m3_exhaustive_against_brute_force():
    """Every finite code decodes to the closed-form value and re-encodes to
    itself; every midpoint between neighbours rounds to the even code; a
    float64 nearest search agrees on a dense sweep."""
    t = oracle.e4m3_table()
    for b in range(256):
        e, m = (b >> 3) & 15, b & 7
        if e == 15 and m == 7:
            assert np.isnan(t[b])
            continue
        mag = m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
        assert t[b] == (-mag if b & 0x80 else mag)
        assert oracle.e4m3_encode(float(t[b])) == b or (t[b] == 0 and b in (0, 0x80))
    pos = np.array(sorted({float(t[b]) for b in range(0x7F) if not np.isnan(t[b])}))
    for lo, hi in zip(pos[:-1], pos[1:]):
        mid = (lo + hi) / 2
        c = oracle.e4m3_encode(mid)
        want = oracle.e4m3_encode(lo) if (oracle.e4m3_encode(lo) & 1) == 0 else oracle.e4m3_encode(hi)
        assert c == want, (lo, hi)
    xs = np.linspace(-448, 448, 20001).astype(np.float32)
    codes = np.array([oracle.e4m3_encode(float(x)) for x in xs])
    finite = np.array([b for b in range(256) if not np.isnan(t[b])])
    vals = t[finite].astype(np.float64)
    for x, c in zip(xs[::7], codes[::7]):
        d = np.abs(vals - float(x))
        assert abs(float(t[c]) - float(x)) == d.min()


def test_e4m3_encode_matches_reference_vectors(gold):
    codes = np.array([oracle.e4m3_encode(float(v)) for v in gold["e4m3_in"]], np.uint8)
    np.testing.assert_array_equal(codes, gold["e4m3_codes"])


def test_bf16_and_f16_rounding_closed_form():
    raw = synth.splitmix64(5, 200000).astype(np.uint32) & np.uint32(0xFFFFFFFF)
    x = raw.view(np.float32)
    x = x[np.isfinite(x)]
    got = np.array([oracle.lib().po_bf16_from_f32(float(v)) for v in x[:20000]], np.uint16)
    np.testing.assert_array_equal(got, oracle.f32_to_bf16_bits(x[:20000]))
    y = (synth.normal(6, 20000) * 1000).astype(np.float32)
    y = np.concatenate([y, np.array([65504, 65520, 6e-8, 3e-8, -0.0, 1e-5], np.float32)])
    h = np.array([oracle.lib().po_f16_from_f32(float(v)) for v in y], np.uint16)
    np.testing.assert_array_equal(h, y.astype(np.float16).view(np.uint16))  # IEEE RNE in numpy
    back = np.array([oracle.lib().po_f16_to_f32(int(b)) for b in h], np.float32)
    np.testing.assert_array_equal(back, h.view(np.float16).astype(np.float32))


def test_mxfp4_reference_kats(gold):
    # deepseek_mxfp4_codec_test.cpp:12-64
    d = oracle.C.c_double()
    expected = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    for b in range(16):
        assert oracle.lib().po_mxfp4_decode_scalar(b, 127, oracle.C.byref(d)) == 0
        assert d.value == expected[b] and np.signbit(d.value) == np.signbit(expected[b])
    for s, v in ((126, 0.5), (127, 1.0), (128, 2.0)):
        oracle.lib().po_mxfp4_decode_scalar(2, s, oracle.C.byref(d))
        assert d.value == v
    assert oracle.lib().po_mxfp4_decode_scalar(2, 0xFF, oracle.C.byref(d)) != 0
    row = oracle.mxfp4_decode_row(np.array([0x21, 0xC7], np.uint8), np.array([127], np.uint8), 4)
    assert list(row) == [0.5, 1.0, 6.0, -2.0]
    row = oracle.mxfp4_decode_row(np.full(17, 0x22, np.uint8), np.array([127, 128], np.uint8), 33)
    assert row[31] == 1.0 and row[32] == 2.0
    with pytest.raises(oracle.OracleError):
        oracle.mxfp4_decode_row(np.array([0x77], np.uint8), np.array([254], np.uint8), 2)
    got = oracle.mxfp4_decode_row(gold["mx_packed"], gold["mx_scales"], 256)
    np.testing.assert_array_equal(got.view(np.uint32), gold["mx_out"].view(np.uint32))


# ------------------------------------------------------ activation quant
def test_fp8_quant_reference_kats(gold):
    # deepseek_fp8_activation_codec_test.cpp:28-46
    x = np.zeros((1, 256), np.float32)
    x[0, 0] = 448.0
    x[0, 128] = 1.0
    q, s = oracle.fp8_quant_ue8m0(x)
    assert list(s[0]) == [127, 119]
    assert q[0, 0] == 0x7E and q[0, 128] == 0x78
    q, s = oracle.fp8_quant_ue8m0(np.zeros((1, 128), np.float32))
    assert list(s[0]) == [105]
    with pytest.raises(oracle.OracleError):
        bad = np.zeros((1, 128), np.float32)
        bad[0, -1] = np.inf
        oracle.fp8_quant_ue8m0(bad)
    q, s = oracle.fp8_quant_ue8m0(gold["quant_x"])
    np.testing.assert_array_equal(q, gold["quant_codes"])
    np.testing.assert_array_equal(s, gold["quant_scales"])


def test_fp8_quant_f32_closed_form():
    """BASELINE fp32-scale quant (no reference counterpart): s = max(amax,
    1e-4)/448 exactly as fp32 division, every code is the e4m3 encode of
    clamp(x/s) (codes pinned above), and the group max lands on +-448."""
    x = (synth.normal(9, 8 * 1024) * np.repeat(np.logspace(-6, 3, 8), 1024)).astype(np.float32).reshape(8, 1024)
    q, s = oracle.fp8_quant_f32(x)
    g = x.reshape(8, 8, 128)
    amax = np.maximum(np.abs(g).max(axis=2), np.float32(1e-4))
    np.testing.assert_array_equal(s, (amax / np.float32(448.0)).astype(np.float32))
    scaled = np.clip(g / s[:, :, None], -448, 448).astype(np.float32).reshape(-1)
    want = synth.e4m3_encode(scaled).reshape(8, 1024)
    np.testing.assert_array_equal(q, want)


# ------------------------------------------------------------------ GEMMs
def test_fp8_gemm_reference_kats(gold):
    # deepseek_fp8_gemm_test.cpp:8-53
    a = np.full((1, 256), 0x38, np.uint8)
    sa = np.array([[127, 127]], np.uint8)
    w = np.full((128, 256), 0x38, np.uint8)
    sw = np.array([[127, 128]], np.uint8)
    out = oracle.fp8_gemm_ue8m0(a, sa, w, sw)
    assert out[0, 0] == 384.0 and out[0, 127] == 384.0
    with pytest.raises(oracle.OracleError):
        oracle.fp8_gemm_ue8m0(a[:, :128], sa[:, :1], w[:, :128].copy(), np.array([[0xFF]], np.uint8))
    a2 = np.full((1, 128), 0x38, np.uint8)
    a2[0, 0] = 0x7F
    with pytest.raises(oracle.OracleError):
        oracle.fp8_gemm_ue8m0(a2, sa[:, :1], w[:, :128].copy(), np.array([[127]], np.uint8))
    out = oracle.fp8_gemm_ue8m0(gold["fp8_a"], gold["fp8_sa"], gold["fp8_w"], gold["fp8_sw"])
    np.testing.assert_array_equal(out.view(np.uint32), gold["fp8_out"].view(np.uint32))


def test_fp8_gemm_f32_reduces_to_ue8m0_form():
    """With power-of-two fp32 scales the fp32-scale GEMM must equal the
    pinned UE8M0 GEMM bit for bit (same nesting, exact scale products)."""
    m, n, k = 5, 256, 512
    a = synth.e4m3_encode((synth.normal(31, m * k) * 60).clip(-448, 448).astype(np.float32)).reshape(m, k)
    w = synth.e4m3_encode((synth.normal(32, n * k) * 60).clip(-448, 448).astype(np.float32)).reshape(n, k)
    sa = (118 + synth.splitmix64(33, m * 4) % np.uint64(12)).astype(np.uint8).reshape(m, 4)
    sw = (118 + synth.splitmix64(34, 2 * 4) % np.uint64(12)).astype(np.uint8).reshape(2, 4)
    ref = oracle.fp8_gemm_ue8m0(a, sa, w, sw)
    got = oracle.fp8_gemm_f32(a, np.ldexp(1.0, sa.astype(np.int32) - 127).astype(np.float32), w,
                              np.ldexp(1.0, sw.astype(np.int32) - 127).astype(np.float32))
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    # and with arbitrary scales it stays within fp32 rounding of float64
    fa = (0.001 + synth.uniform(35, m * 4)).astype(np.float32).reshape(m, 4)
    fw = (0.001 + synth.uniform(36, 8)).astype(np.float32).reshape(2, 4)
    got = oracle.fp8_gemm_f32(a, fa, w, fw)
    t = oracle.e4m3_table().astype(np.float64)
    A = t[a].reshape(m, 4, 128)
    W = t[w].reshape(n, 4, 128)
    exact = np.einsum("mbi,nbi,mb,nb->mn", A, W, fa.astype(np.float64), np.repeat(fw, 128, axis=0).astype(np.float64))
    assert np.abs(got - exact).max() <= 1e-5 * np.abs(exact).max()


def test_fp4_gemm_reference_kats(gold):
    # deepseek_fp4_gemm_oracle_test.cpp:11-42
    q, s = oracle.fp8_quant_ue8m0(np.ones((1, 128), np.float32))
    w = np.full((2, 64), 0x22, np.uint8)
    sw = np.full((2, 4), 127, np.uint8)
    sw[1] = 128
    out = oracle.fp4_gemm(q, s, w, sw)
    assert out[0, 0] == 128.0 and out[0, 1] == 256.0
    x = np.zeros((1, 128), np.float32)
    x[0, 0], x[0, 1] = 1.0, 2.0
    q, s = oracle.fp8_quant_ue8m0(x)
    w = np.zeros((1, 64), np.uint8)
    w[0, 0] = 0xA2
    out = oracle.fp4_gemm(q, s, w, np.full((1, 4), 127, np.uint8))
    assert out[0, 0] == -1.0
    out = oracle.fp4_gemm(gold["fp4_a"], gold["fp4_sa"], gold["fp4_w"], gold["fp4_sw"])
    np.testing.assert_array_equal(out.view(np.uint32), gold["fp4_out"].view(np.uint32))


def test_mxfp4_bf16_gemm_closed_form():
    """bf16 activations x MXFP4 weights (BASELINE cfg5 variant): exact in
    float64 for small-integer activations, and equal to a dense GEMM over
    the pinned MXFP4 decode."""
    m, n, k = 3, 16, 128
    xi = (synth.splitmix64(40, m * k) % np.uint64(7)).astype(np.float32).reshape(m, k) - 3
    xb = oracle.f32_to_bf16_bits(xi)
    p, s = synth.mxfp4_weight(41, n, k)
    dec = np.stack([oracle.mxfp4_decode_row(p[r], s[r], k) for r in range(n)]).astype(np.float64)
    exact = xi.astype(np.float64) @ dec.T
    got = oracle.mxfp4_bf16_gemm(xb, p, s)
    np.testing.assert_allclose(got, exact, rtol=0, atol=1e-6 * np.abs(exact).max())


def test_w4a16_symmetric_reference_fixture():
    """Nibble order and sign decode of the reference format: the reference
    quantizer packs {-7,-6,-1,0,1,6,7} as a9 0f 61 07
    (qwen3_int4_reference_quantizer_test.cpp:29-40); a one-hot activation
    reads each weight back as q * scale."""
    k = 128
    packed = np.zeros((1, k // 2), np.uint8)
    packed[0, :4] = [0xA9, 0x0F, 0x61, 0x07]
    scale = np.array([[0x3C00]], np.uint16)  # 1.0
    want = [-7, -6, -1, 0, 1, 6, 7, 0]
    for j, v in enumerate(want):
        x = np.zeros((1, k), np.float32)
        x[0, j] = 1.0
        out = oracle.w4a16_sym(oracle.f32_to_bf16_bits(x), packed, scale)
        assert f32(out)[0, 0] == v
    bad = packed.copy()
    bad[0, 5] = 0x80
    with pytest.raises(oracle.OracleError) as e:
        oracle.w4a16_sym(oracle.f32_to_bf16_bits(np.ones((1, k), np.float32)), bad, scale)
    assert e.value.code == 12


def test_w4a16_asymmetric_reduces_to_symmetric():
    """BASELINE asymmetric format, zero point 8 and power-of-two scales
    (exact in both bf16 and fp16): must equal the pinned symmetric form bit
    for bit, since w = (q - 8) * s is then the same product."""
    n, k, m = 16, 1024, 3
    v = (synth.splitmix64(50, n * k) % np.uint64(15)).astype(np.int32).reshape(n, k) - 7  # [-7, 7]
    qa = (v + 8).astype(np.uint32).reshape(n, k // 8, 8)
    qweight = np.zeros((n, k // 8), np.uint32)
    for j in range(8):
        qweight |= qa[:, :, j] << np.uint32(4 * j)
    zeros = np.full((n, 1), 0x88888888, np.uint32)
    e = (synth.splitmix64(51, n * 8) % np.uint64(6)).astype(np.int32).reshape(n, 8) - 9
    s_bf16 = oracle.f32_to_bf16_bits(np.ldexp(1.0, e).astype(np.float32))
    s_f16 = np.ldexp(1.0, e).astype(np.float16).view(np.uint16)
    nib = (v & 0xF).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    x = synth.bf16_normal(52, (m, k))
    a = oracle.w4a16_asym(x, qweight, s_bf16, zeros)
    b = oracle.w4a16_sym(x, packed, s_f16)
    np.testing.assert_array_equal(a, b)
    w = oracle.w4a16_asym_dequant(qweight, s_bf16, zeros, k)
    np.testing.assert_array_equal(w, (v * np.repeat(np.ldexp(1.0, e), 128, axis=1)).astype(np.float32))


def test_bf16_gemm_exact_on_small_integers():
    m, n, k = 4, 8, 256
    a = (synth.splitmix64(60, m * k) % np.uint64(9)).astype(np.float32).reshape(m, k) - 4
    w = (synth.splitmix64(61, n * k) % np.uint64(9)).astype(np.float32).reshape(n, k) - 4
    got = oracle.bf16_gemm(oracle.f32_to_bf16_bits(a), oracle.f32_to_bf16_bits(w))
    np.testing.assert_array_equal(got, (a.astype(np.float64) @ w.T.astype(np.float64)).astype(np.float32))


# ------------------------------------------------------------ elementwise
def test_swiglu_reference_kats(gold):
    # deepseek_expert_swiglu_oracle_test.cpp:12-33
    silu = lambda v: np.float32(v) / (np.float32(1) + np.exp(np.float32(-v)))
    out = oracle.swiglu(np.array([-20, 20, -2], np.float32), np.array([-20, 20, 3], np.float32), 10.0)
    np.testing.assert_allclose(out, [silu(-20) * -10, silu(10) * 10, silu(-2) * 3], rtol=1e-6)
    out = oracle.swiglu(np.array([4], np.float32), np.array([-4], np.float32), 2.0)
    np.testing.assert_allclose(out, [silu(2) * -2], rtol=1e-6)
    out = oracle.swiglu(gold["swiglu_g"], gold["swiglu_u"], 10.0)
    np.testing.assert_array_equal(out.view(np.uint32), gold["swiglu_out"].view(np.uint32))


def test_silu_mul_reference(gold):
    # qwen3_cpu_oracle_test.cpp:40-52 (round only at output) + golden vectors
    out = oracle.silu_mul(gold["silu_g"], gold["silu_u"])
    np.testing.assert_array_equal(out, gold["silu_out"])


# -------------------------------------------------------------------- MoE
def test_route_plan_reference_kat_and_golden(gold):
    # deepseek_expert_subwave_plan_test.cpp:12-39 (expert, token, ordinal, w)
    routes = [(9, 1, 2, .12), (3, 0, 5, .15), (7, 1, 0, .10), (1, 0, 2, .20), (5, 1, 4, .11), (9, 0, 0, .25),
              (2, 1, 5, .13), (5, 0, 1, .10), (1, 1, 3, .30), (7, 0, 4, .12), (3, 1, 1, .24), (2, 0, 3, .18)]
    ids = np.zeros((2, 6), np.uint32)
    wts = np.zeros((2, 6), np.float32)
    for e, t, o, w in routes:
        ids[t, o], wts[t, o] = e, w
    off, rt, rw, tr = oracle.route_plan(ids, wts, 256)
    assert (off[0], off[1], off[2], off[3], off[10], off[256]) == (0, 0, 2, 4, 12, 12)
    keys = sorted((e, t, o) for e, t, o, _ in routes)
    assert list(rt) == [t for _, t, _ in keys]
    for i, (e, t, o) in enumerate(keys):
        assert tr[t, o] == i
    off, rt, rw, tr = oracle.route_plan(gold["plan_ids"], gold["plan_weights"], 256)
    np.testing.assert_array_equal(off, gold["plan_offsets"])
    np.testing.assert_array_equal(rt, gold["plan_token"])
    np.testing.assert_array_equal(rw, gold["plan_weight_sorted"])


def test_route_plan_against_lexsort():
    ids, wts = synth.zipf_router(70, 333, 64, 5)
    off, rt, rw, tr = oracle.route_plan(ids, wts, 64)
    e = ids.ravel()
    t = np.repeat(np.arange(333), 5)
    o = np.tile(np.arange(5), 333)
    order = np.lexsort((o, t, e))
    np.testing.assert_array_equal(rt, t[order])
    np.testing.assert_array_equal(rw, wts.ravel()[order])
    np.testing.assert_array_equal(off, np.concatenate([[0], np.cumsum(np.bincount(e, minlength=64))]))


def test_ordered_accumulate_reference_kats(gold):
    # deepseek_expert_accumulator_oracle_test.cpp:16-39
    rows = np.array([[0.5] * 4096, [1.0] * 4096, [3.0] * 4096], np.float32)
    acc = oracle.ordered_accumulate(oracle.f32_to_bf16_bits(rows), np.array([0, 1, 0], np.uint32), 2)
    fin = acc + 1.0
    assert fin[0, 0] == 4.5 and fin[1, 0] == 2.0
    acc = oracle.ordered_accumulate(oracle.f32_to_bf16_bits(np.full((1, 4096), 2.0, np.float32)),
                                    np.array([0], np.uint32), 1)
    assert acc[0, 0] + 1.0 == 3.0
    # golden: reference accumulator (experts ascending) + shared
    acc = oracle.ordered_accumulate(gold["acc_rows"], gold["plan_token"], 2)
    np.testing.assert_array_equal((acc + f32(gold["acc_shared"])).view(np.uint32), gold["acc_out"].view(np.uint32))


def test_routed_expert_reference_kat_and_golden(gold):
    # deepseek_routed_expert_oracle_test.cpp:25-45: identity-like first
    # column weights, all outputs bf16(0.75)
    w = 128
    packed = np.zeros((w, w // 2), np.uint8)
    packed[:, 0] = 0x02
    scales = np.full((w, w // 32), 127, np.uint8)
    x = np.zeros((1, w), np.float32)
    x[0, 0] = 1.0
    out = oracle.routed_expert_fp4(oracle.f32_to_bf16_bits(x), np.array([1.0], np.float32), w, w,
                                   packed, scales, packed, scales, packed, scales)
    assert np.all(out == oracle.f32_to_bf16_bits(np.array([0.75], np.float32))[0])
    out = oracle.routed_expert_fp4(gold["re_x"], gold["re_w"], 128, 128, gold["re_w1p"], gold["re_w1s"],
                                   gold["re_w2p"], gold["re_w2s"], gold["re_w3p"], gold["re_w3s"])
    np.testing.assert_array_equal(out, gold["re_out"])


# --------------------------------------------- live reference (optional)
@pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref not built (needs the reference checkout)")
def test_against_live_reference_library():
    R = oracle.ref()
    P = oracle.P
    x = (synth.normal(80, 16 * 1024) * 7).astype(np.float32).reshape(16, 1024)
    q1, s1 = oracle.fp8_quant_ue8m0(x)
    q2 = np.empty_like(q1)
    s2 = np.empty_like(s1)
    assert R.pr_fp8_quant(x.ctypes.data_as(P), 16, 1024, q2.ctypes.data_as(P), s2.ctypes.data_as(P)) == 0
    np.testing.assert_array_equal(q1, q2)
    np.testing.assert_array_equal(s1, s2)
    w = synth.e4m3_encode((synth.normal(81, 256 * 1024) * 30).clip(-448, 448).astype(np.float32)).reshape(256, 1024)
    sw = (120 + synth.splitmix64(82, 16) % np.uint64(5)).astype(np.uint8).reshape(2, 8)
    o1 = oracle.fp8_gemm_ue8m0(q1, s1, w, sw)
    o2 = np.empty_like(o1)
    assert R.pr_fp8_gemm(q1.ctypes.data_as(P), s1.ctypes.data_as(P), w.ctypes.data_as(P), sw.ctypes.data_as(P),
                         16, 256, 1024, o2.ctypes.data_as(P)) == 0
    np.testing.assert_array_equal(o1.view(np.uint32), o2.view(np.uint32))
    p, ps = synth.mxfp4_weight(83, 128, 1024)
    o1 = oracle.fp4_gemm(q1, s1, p, ps)
    o2 = np.empty_like(o1)
    assert R.pr_fp4_gemm(q1.ctypes.data_as(P), s1.ctypes.data_as(P), p.ctypes.data_as(P), ps.ctypes.data_as(P),
                         16, 128, 1024, o2.ctypes.data_as(P)) == 0
    np.testing.assert_array_equal(o1.view(np.uint32), o2.view(np.uint32))

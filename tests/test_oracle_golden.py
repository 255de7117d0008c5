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


def _pack_nibbles_u32(vals: np.ndarray) -> np.ndarray:
    """[rows, 8 j] nibbles -> u32 words, value 8 w + i in nibble i of word w
    (bits 4i .. 4i + 3): the BASELINE layout the test declares."""
    rows, cnt = vals.shape
    v = np.zeros((rows, -(-cnt // 8) * 8), np.uint32)
    v[:, :cnt] = vals
    v = v.reshape(rows, -1, 8)
    out = np.zeros(v.shape[:2], np.uint32)
    for i in range(8):
        out |= v[:, :, i] << np.uint32(4 * i)
    return out


def test_w4a16_asymmetric_distinct_zero_points():
    """Asymmetric INT4 with a different zero point in every group, over two
    zero-point words (16 groups at K = 2048), packed here from unpacked
    values by the declared layout (weight k in nibble k % 8 of word k / 8,
    zero point of group g in nibble g % 8 of zero word g / 8): the dequant
    must return (q - z) * s exactly, and a one-hot activation e_k must read
    bf16((q[n, k] - z[n, k / 128]) * s[n, k / 128]) back through the GEMV.
    A nibble order reversed in either word, or a zero point indexed by k / 8
    or g / 16, changes the answer (checked on the same data)."""
    n, k = 6, 2048
    groups = k // 128
    q = (synth.splitmix64(80, n * k) % np.uint64(16)).astype(np.int64).reshape(n, k)
    z = ((np.arange(groups)[None, :] * 5 + 3 * np.arange(n)[:, None] + 1) % 16).astype(np.int64)
    assert len(np.unique(z[0])) == groups  # every group of a row has its own zero point
    # bf16 scales with few mantissa bits: (q - z) * s is exact in fp32 and bf16
    s = (np.ldexp(1.0, -(synth.splitmix64(81, n * groups) % np.uint64(6)).astype(np.int64) - 6) *
         (1.0 + (synth.splitmix64(82, n * groups) % np.uint64(4)).astype(np.float64) / 4)).reshape(n, groups)
    s_bits = oracle.f32_to_bf16_bits(s.astype(np.float32))
    assert (oracle.bf16_bits_to_f32(s_bits) == s).all()
    qweight = _pack_nibbles_u32(q.astype(np.uint32))
    zeros = _pack_nibbles_u32(z.astype(np.uint32))
    assert qweight.shape == (n, k // 8) and zeros.shape == (n, 2)
    want = ((q - np.repeat(z, 128, 1)) * np.repeat(s, 128, 1)).astype(np.float32)
    got = oracle.w4a16_asym_dequant(qweight, s_bits, zeros, k)
    np.testing.assert_array_equal(got, want)
    # one-hot activations through the GEMV, one per position class: every
    # nibble slot of a weight word, every group of both zero words
    ks = np.array(sorted({g * 128 + (g * 37) % 128 for g in range(groups)} | set(range(8)) |
                         {8 * 129 + j for j in range(8)}))
    x = np.zeros((ks.size, k), np.float32)
    x[np.arange(ks.size), ks] = 1.0
    out = oracle.w4a16_asym(oracle.f32_to_bf16_bits(x), qweight, s_bits, zeros)
    np.testing.assert_array_equal(out, oracle.f32_to_bf16_bits(want[:, ks].T.copy()))
    # the same data read with a reversed zero-point nibble order or the
    # zero point of word k / 8 gives other weights: the check discriminates
    z_rev = np.concatenate([z[:, 7::-1], z[:, 15:7:-1]], 1)
    assert (np.repeat(z_rev, 128, 1) != np.repeat(z, 128, 1)).any()
    assert ((q - np.repeat(z_rev, 128, 1)) * np.repeat(s, 128, 1) != want).any()


def test_qwen_mlp_small_integer_composition():
    """cfg1's checker: gate and up through the BF16 linear (bf16 RNE at the
    output), SiLU-mul in fp32 rounded once, then down.  Integer inputs make
    both first GEMMs exact; their sums exceed 256, so the bf16 rounding of
    gate and up changes them.  A composition that rounds gate and up to
    bf16, takes SiLU-mul in fp32 (numpy; its exp may differ from the C
    library's in the last bit, so no SiLU product of a gate with |g| < 24
    may lie within 4e-6 relative of a bf16 tie, asserted below), rounds
    it, and sums the down GEMM in float64 (no output closer to a tie than
    the fp32 accumulation's error bound) must agree exactly; the compositions with gate and up swapped or
    without rounding gate and up must not."""
    m, hdim, idim = 2, 128, 32
    rng = np.random.default_rng(17)
    x = rng.integers(-8, 9, (m, hdim)).astype(np.float32)
    wg = rng.integers(-8, 9, (idim, hdim)).astype(np.float32)
    wu = rng.integers(-8, 9, (idim, hdim)).astype(np.float32)
    b = oracle.f32_to_bf16_bits
    wd = oracle.bf16_bits_to_f32(b(rng.normal(0.0, 0.05, (hdim, idim)).astype(np.float32)))
    got = oracle.bf16_bits_to_f32(oracle.qwen_mlp(b(x), b(wg), b(wu), b(wd))).astype(np.float64)

    rnd = lambda v: oracle.bf16_bits_to_f32(b(np.asarray(v, np.float32))).astype(np.float64)

    def near_tie(v, tol):
        # within tol of a bf16 rounding midpoint
        v = np.abs(np.asarray(v, np.float64))
        q = np.ldexp(1.0, (np.floor(np.log2(v + 1e-300)) - 7).astype(int))
        frac = v / q - np.floor(v / q)
        return (v > 0) & (np.abs(frac - 0.5) * q <= tol)

    X = x.astype(np.float64)
    g_raw, u_raw = X @ wg.T.astype(np.float64), X @ wu.T.astype(np.float64)
    assert (np.abs(g_raw) > 256).any() and (rnd(g_raw) != g_raw).any()  # the rounding bites

    def chain(g, u, premise=True):
        g32, u32 = g.astype(np.float32), u.astype(np.float32)
        with np.errstate(over="ignore"):
            h = (g32 / (np.float32(1.0) + np.exp(-g32))) * u32
        assert not premise or not (near_tie(h, 4e-6 * np.abs(h)) & (np.abs(g32) < 24)).any()
        y = rnd(h) @ wd.T.astype(np.float64)
        # fp32 strict-k accumulation error bound: k * 2^-24 * sum |terms|
        assert not premise or not near_tie(y, idim * 2.0 ** -24 * (np.abs(rnd(h)) @ np.abs(wd.T.astype(np.float64)))).any()
        return rnd(y)

    want = chain(rnd(g_raw), rnd(u_raw))
    np.testing.assert_array_equal(got, want)
    assert (chain(rnd(u_raw), rnd(g_raw), False) != got).any()  # gate/up swapped
    assert (chain(g_raw, u_raw, False) != got).any()  # gate/up not rounded to bf16


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


def test_finalize_with_shared_rows(gold):
    """po_finalize with a shared-expert row: the reference's finalize
    (deepseek_expert_accumulator_oracle.cpp:69-85) returns acc + shared in
    fp32 (the golden acc_out, written by the compiled reference), and the
    device entry stores it as bf16 (deepseek_expert_accumulate.cu:41-56):
    the oracle must give bf16(acc_out) bit for bit; without the shared row
    it gives bf16(acc); a non-finite sum is an error."""
    acc = oracle.ordered_accumulate(gold["acc_rows"], gold["plan_token"], 2)
    got = oracle.finalize(acc, np.ascontiguousarray(gold["acc_shared"]))
    np.testing.assert_array_equal(got, oracle.f32_to_bf16_bits(gold["acc_out"]))
    assert (got != oracle.finalize(acc)).any()  # the shared rows change the result
    np.testing.assert_array_equal(oracle.finalize(acc), oracle.f32_to_bf16_bits(acc))
    big = np.full((1, 4), 3.0e38, np.float32)
    with pytest.raises(oracle.OracleError):
        oracle.finalize(big, oracle.f32_to_bf16_bits(big))


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


# ----------------------------------------------------------- router top-k
def _v4_route(raw, bias=None):
    return oracle.router_topk(np.asarray(raw, np.float32).reshape(-1, 256), 6, oracle.ROUTER_SQRT_SOFTPLUS, 1.5,
                              np.zeros(256, np.float32) if bias is None else bias)


def test_router_sqrt_softplus_reference_kats():
    # deepseek_learned_router_test.cpp:26-40: top-6 of raw = expert id, sum 1.5
    raw = np.full(256, -10.0, np.float32)
    raw[:8] = np.arange(8)
    ids, w = _v4_route(raw)
    assert list(ids[0]) == [7, 6, 5, 4, 3, 2]
    assert abs(float(w.sum()) - 1.5) <= 1e-6
    # :42-55: a bias of 100 promotes expert 9 to rank 0 with a smaller weight
    raw = np.full(256, -20.0, np.float32)
    raw[:6] = 2.0
    raw[9] = -2.0
    bias = np.zeros(256, np.float32)
    bias[9] = 100.0
    ids, w = _v4_route(raw, bias)
    assert ids[0, 0] == 9 and w[0, 0] < w[0, 1]
    # :57-66: exact ties prefer the smaller id
    ids, _ = _v4_route(np.zeros(256, np.float32))
    assert list(ids[0]) == [0, 1, 2, 3, 4, 5]
    # :68-86: ungrouped selection across the legacy 32-expert groups
    raw = np.full(256, -20.0, np.float32)
    for o, e in enumerate((0, 32, 64, 96, 128, 160)):
        raw[e] = 16.0 - o
    ids, _ = _v4_route(raw)
    assert list(ids[0]) == [0, 32, 64, 96, 128, 160]
    # :88-99: tokens routed independently
    raw = np.full(512, -10.0, np.float32)
    for e in range(6):
        raw[e] = raw[256 + 100 + e] = 10.0 - e
    ids, _ = _v4_route(raw)
    assert ids[0, 0] == 0 and ids[1, 0] == 100
    # :101-109: non-finite scores or bias are rejected
    raw = np.zeros(256, np.float32)
    raw[17] = np.nan
    with pytest.raises(oracle.OracleError):
        _v4_route(raw)
    bias = np.zeros(256, np.float32)
    bias[3] = np.inf
    with pytest.raises(oracle.OracleError):
        _v4_route(np.zeros(256, np.float32), bias)


def test_router_sqrt_softplus_golden(gold):
    ids, w = _v4_route(gold["router_raw"], gold["router_bias"])
    np.testing.assert_array_equal(ids, gold["router_ids"])
    np.testing.assert_array_equal(w.view(np.uint32), gold["router_weights"].view(np.uint32))


def test_router_softmax_closed_form():
    """BASELINE softmax top-k (no reference counterpart): the ids are the
    top-k of the float64 softmax probabilities (stable order, ties to the
    smaller id) and the weights their renormalised values to fp32 rounding;
    a token whose logits tie keeps the smaller ids."""
    t, e, k = 200, 256, 8
    ids64, w64 = synth.zipf_router(synth.config_seed(4, 91), t, e, k)
    logits = (synth.normal(synth.config_seed(4, 91), t * e).reshape(t, e))
    rank = np.empty(e, np.int64)
    rank[np.argsort(synth.splitmix64(synth.config_seed(4, 91) ^ 0xA11CE, e), kind="stable")] = np.arange(e)
    z = (logits - 1.1 * np.log1p(rank)[None, :]).astype(np.float32)
    z[7] = 0.5  # an all-tie token
    ids, w = oracle.router_topk(z, k, oracle.ROUTER_SOFTMAX, 1.0)
    p = np.exp(z.astype(np.float64) - z.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    want = np.argsort(-p, axis=1, kind="stable")[:, :k]
    np.testing.assert_array_equal(ids, want)
    sel = np.take_along_axis(p, want, axis=1)
    np.testing.assert_allclose(w, sel / sel.sum(axis=1, keepdims=True), rtol=2e-6, atol=0)
    assert list(ids[7]) == list(range(k))
    # away from the all-tie row, the float32 logits route like the synthetic
    # float64 router they were rounded from
    keep = np.ones(t, bool)
    keep[7] = False
    assert (ids[keep] == ids64[keep]).mean() > 0.99


# ------------------------------------------ FP8 expert chain (BASELINE cfg4)
def _e4m3_codes(values):
    codes = [oracle.e4m3_encode(float(v)) for v in np.ravel(values)]
    assert all(c is not None for c in codes)
    return np.array(codes, np.uint8).reshape(np.shape(values))


def _kat_expert(route_weight):
    """H = I = 128.  x = [0.875, 5*2^-9, 0, ...]: one 128-group with amax
    0.875 = 448 * 2^-9, so the fp32 activation scale is exactly 2^-9 and the
    codes are 448 and 5 (exact).
    gate rows c < 64:  w[c,0] = -2.5,  w[c,1] = 1.875  (block scale 1.0)
    gate rows c >= 64: w[c,0] = 1.75,  w[c,1] = 1.125
    up rows c < 64:    w[c,0] = 2.75,  w[c,1] = 3.25   (block scale 0.5)
    up rows c >= 64:   w[c,0] = -6.0,  w[c,1] = 2.75
    down: w2[h, (h+1) % 128] = 1.0, block scale 2.0 (y[h] = mid[h+1], so a
    transposed W2 would read mid[h-1] instead)."""
    h = i = 128
    x = np.zeros((1, h), np.float32)
    x[0, 0], x[0, 1] = 0.875, 5 * 2.0 ** -9
    w13v = np.zeros((2 * i, h), np.float32)
    w13v[:64, 0], w13v[:64, 1], w13v[64:i, 0], w13v[64:i, 1] = -2.5, 1.875, 1.75, 1.125
    w13v[i:i + 64, 0], w13v[i:i + 64, 1], w13v[i + 64:, 0], w13v[i + 64:, 1] = 2.75, 3.25, -6.0, 2.75
    w2v = np.zeros((h, i), np.float32)
    w2v[np.arange(h), (np.arange(h) + 1) % i] = 1.0
    s13 = np.array([[1.0], [0.5]], np.float32)  # [2I/128, H/128]: gate block, up block
    s2 = np.array([[2.0]], np.float32)
    return (oracle.f32_to_bf16_bits(x), np.array([route_weight], np.float32), h, i,
            _e4m3_codes(w13v), s13, _e4m3_codes(w2v), s2)


def test_expert_fp8_known_answer():
    """Hand-derived answer of the cfg4 expert chain (po_expert_fp8), every
    rounding point at least 0.2 bf16 ulp from a tie:
      gate_lo = (448*-2.5 + 5*1.875) * 2^-9 * 1.0 = -2.169189453125 -> bf16 -2.171875
      up_lo   = (448*2.75 + 5*3.25) * 2^-9 * 0.5  =  1.218994140625 -> bf16  1.21875
      gate_hi = (448*1.75 + 5*1.125) * 2^-9       =  1.542236328125 -> bf16  1.5390625
      up_hi   = (448*-6 + 5*2.75) * 2^-9 * 0.5    = -2.611572265625 -> bf16 -2.609375
      mid_lo  = silu(-2.171875) * 1.21875 * 0.8 = -0.2222 * 1.21875 * 0.8
              = -0.216638 -> bf16 -0.216796875
      mid_hi  = silu(1.5390625) * -2.609375 * 0.8 = 1.267154 * -2.609375 * 0.8
              = -2.645184 -> bf16 -2.640625
      quant:  s = 2.640625 / 448; mid_hi -> code -448, mid_lo / s = -36.78
              -> e4m3 -36
      down:   y_lo = -36 * s * 2.0 = -0.4243862 -> bf16 -0.423828125
              y_hi = -448 * s * 2.0 = -5.28125
    and y[h] reads mid[h+1]: h in 0..62 and 127 -> y_lo, h in 63..126 -> y_hi.
    The mistakes this pins, each giving another output: gate and up halves
    swapped; gate/up not rounded to bf16; the route weight applied after the
    intermediate's bf16 rounding, or after the down GEMM; the intermediate
    not rounded to bf16 or not quantised; the up block read with the gate
    block's scale; W2 read transposed."""
    out = oracle.expert_fp8(*_kat_expert(0.8))
    lo, hi = oracle.f32_to_bf16_bits(np.array([-0.423828125, -5.28125], np.float32))
    want = np.full(128, lo, np.uint16)
    want[63:127] = hi
    np.testing.assert_array_equal(out[0], want)


def test_expert_fp8_route_weight_and_clamp():
    """Route weight 0.2 in the same derivation: mid_hi = -2.645184 * 0.25 =
    -0.661296 -> bf16 -0.66015625, mid_lo = -0.0541596 -> bf16
    -0.05419921875, mid_lo / s = -36.76 -> e4m3 -36 with s = 0.66015625/448,
    so y_hi = -1.3203125 and y_lo = bf16(-36 * s * 2).  The clamp (limit
    1.0) caps the gate at 1.0 and the up at +-1.0; a zero route weight gives
    an all-zero output (amax floor 1e-4, codes 0)."""
    out = oracle.bf16_bits_to_f32(oracle.expert_fp8(*_kat_expert(0.2)))[0]
    s = np.float32(0.66015625) / np.float32(448.0)
    lo = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(np.array([-36 * s * 2], np.float32)))[0]
    assert out[0] == lo and out[63] == np.float32(-1.3203125)
    args = list(_kat_expert(0.8))
    clamped = oracle.bf16_bits_to_f32(oracle.expert_fp8(*args, limit=1.0))[0]
    # gate_lo -2.171875 (not clamped from below), up_lo 1.21875 -> 1.0;
    # gate_hi 1.5390625 -> 1.0, up_hi -2.609375 -> -1.0
    silu = lambda g: np.float32(g) / (np.float32(1) + np.exp(np.float32(-g)))
    m_lo = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(np.array([silu(-2.171875) * 1.0 * 0.8], np.float32)))[0]
    m_hi = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(np.array([silu(1.0) * -1.0 * np.float32(0.8)], np.float32)))[0]
    assert (m_lo, m_hi) == (np.float32(-0.177734375), np.float32(-0.5859375))
    assert clamped[63] == np.float32(2 * m_hi)
    assert abs(clamped[0] - 2 * m_lo) <= abs(2 * m_lo) / 16  # e4m3 rounding of the lo lane only
    args[1] = np.array([0.0], np.float32)
    assert np.all(oracle.bf16_bits_to_f32(oracle.expert_fp8(*args)) == 0)


def test_expert_fp8_float64_brute_force():
    """A tiny expert with exactly representable inputs (activation groups
    with amax 448 * 2^k, integer e4m3 weight codes, power-of-two block
    scales), so both GEMMs are exact in float64 and fp32 alike.  The float64
    chain (gate/up rows split as [gate; up], SwiGLU, x route weight, the
    pinned bf16 rounding and fp32-scale quant at the same points) must agree
    with po_expert_fp8 to one bf16 ulp everywhere, and exactly on >= 95 % of
    outputs (the fp32 vs float64 SiLU may flip a rounding)."""
    t, h, i = 3, 256, 256
    rng = np.random.default_rng(7)
    ints = np.array([-8, -6, -5, -4, -3, -2, -1, 0, 1, 2, 3, 4, 5, 6, 8], np.float32)
    x = rng.choice(ints, (t, h)).astype(np.float32)
    x[:, ::128] = 448.0  # group amax 448 -> activation scale exactly 1
    w13 = _e4m3_codes(rng.choice(ints, (2 * i, h)))
    w2 = _e4m3_codes(rng.choice(ints, (h, i)))
    # gate/up values of order 1 (SiLU well away from its linear range)
    s13 = np.ldexp(1.0, rng.integers(-11, -8, (2 * i // 128, h // 128))).astype(np.float32)
    s2 = np.ldexp(1.0, rng.integers(-6, -3, (h // 128, i // 128))).astype(np.float32)
    rw = np.array([0.7, 0.25, 1.0], np.float32)
    xb = oracle.f32_to_bf16_bits(x)
    got = oracle.bf16_bits_to_f32(oracle.expert_fp8(xb, rw, h, i, w13, s13, w2, s2)).astype(np.float64)

    tab = oracle.e4m3_table().astype(np.float64)
    rnd = lambda v: oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(np.asarray(v, np.float32))).astype(np.float64)
    W13 = tab[w13] * np.repeat(np.repeat(s13, 128, 0), 128, 1)
    W2 = tab[w2] * np.repeat(np.repeat(s2, 128, 0), 128, 1)
    gu = x.astype(np.float64) @ W13.T  # exact: integer products, power-of-two scales
    g, u = rnd(gu[:, :i]), rnd(gu[:, i:])
    mid = rnd(g / (1.0 + np.exp(-g)) * u * rw[:, None].astype(np.float64))
    mq, ms = oracle.fp8_quant_f32(mid.astype(np.float32))
    mdq = tab[mq] * np.repeat(ms.astype(np.float64), 128, 1)
    want = rnd(mdq @ W2.T)
    ulp = np.abs(got - want) / np.maximum(np.ldexp(1.0, np.floor(np.log2(np.abs(want) + 1e-300)).astype(int) - 7), 1e-300)
    assert ulp.max() <= 1.0 + 1e-9
    assert (got == want).mean() >= 0.95
    # the same float64 chain with the gate/up halves swapped is far outside
    # that band, so the band tells the split apart
    g2, u2 = rnd(gu[:, i:]), rnd(gu[:, :i])
    mid2 = rnd(g2 / (1.0 + np.exp(-g2)) * u2 * rw[:, None].astype(np.float64))
    q2, s2q = oracle.fp8_quant_f32(mid2.astype(np.float32))
    other = rnd((tab[q2] * np.repeat(s2q.astype(np.float64), 128, 1)) @ W2.T)
    assert np.abs(other - got).max() > 0.1 * np.abs(got).max()


def test_moe_fp8_forward_known_answer():
    """Layer level (moe_fp8_forward): one token routed to experts [1, 0]
    with weights [0.2, 0.8].  Expert 0 is the KAT expert, expert 1 has
    all-zero weights (its rows are exactly 0).  The output must be the KAT
    expert's answer at route weight 0.8; pairing the weights with the wrong
    expert gives the 0.2 answer instead."""
    xb, _, h, i, w13, s13, w2, s2 = _kat_expert(0.8)
    W13 = np.stack([w13, np.zeros_like(w13)])
    S13 = np.stack([s13, s13])
    W2 = np.stack([w2, np.zeros_like(w2)])
    S2 = np.stack([s2, s2])
    out, y, _ = oracle.moe_fp8_forward(xb, np.array([[1, 0]], np.uint32), np.array([[0.2, 0.8]], np.float32),
                                       2, h, i, W13, S13, W2, S2)
    np.testing.assert_array_equal(out[0], oracle.expert_fp8(*_kat_expert(0.8))[0])
    assert not np.array_equal(out[0], oracle.expert_fp8(*_kat_expert(0.2))[0])
    assert not y[1].any()


def test_moe_fp8_forward_matches_token_major_composition():
    """moe_fp8_forward works expert-major (route plan, per-expert chains over
    gathered rows, ordered accumulate).  Restated token-major from the pinned
    per-row chain: each token's routes, experts ascending, fp32 sum of the
    bf16 expert rows, one bf16 rounding; must agree bit for bit (the chain is
    row-independent and the accumulate order is experts ascending)."""
    tokens, experts, topk, hidden, inter = 19, 6, 3, 256, 128
    ids, wts = synth.zipf_router(synth.config_seed(4, 77), tokens, experts, topk)
    x = synth.bf16_normal(synth.config_seed(4, 78), (tokens, hidden))
    w13 = np.empty((experts, 2 * inter, hidden), np.uint8)
    s13 = np.empty((experts, 2 * inter // 128, hidden // 128), np.float32)
    w2 = np.empty((experts, hidden, inter), np.uint8)
    s2 = np.empty((experts, hidden // 128, inter // 128), np.float32)
    for e in range(experts):
        w13[e], s13[e] = synth.fp8_block_weight(synth.config_seed(4, 80 + e), 2 * inter, hidden)
        w2[e], s2[e] = synth.fp8_block_weight(synth.config_seed(4, 90 + e), hidden, inter)
    got, _, _ = oracle.moe_fp8_forward(x, ids, wts, experts, hidden, inter, w13, s13, w2, s2)
    want = np.empty_like(got)
    for t in range(tokens):
        acc = np.zeros(hidden, np.float32)
        for j in np.argsort(ids[t], kind="stable"):
            e = int(ids[t, j])
            row = oracle.expert_fp8(x[t:t + 1], wts[t, j:j + 1], hidden, inter, w13[e], s13[e], w2[e], s2[e])
            acc = (acc + oracle.bf16_bits_to_f32(row[0])).astype(np.float32)
        want[t] = oracle.f32_to_bf16_bits(acc)
    np.testing.assert_array_equal(got, want)


# ------------------------------------------------------------ LM head
def _bf(values):
    return (np.asarray(values, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_lm_head_integer_brute_force():
    """Small-integer operands: every order of the fp32 sum is exact, so the
    logits equal the float64 product x . W^T (pins row/word indexing and
    the transposed weight)."""
    rng = np.random.default_rng(41)
    x = rng.integers(-6, 7, (3, 4096))
    w = rng.integers(-6, 7, (29, 4096))
    got, err = oracle.lm_head(_bf(x), _bf(w))
    assert err == 0
    np.testing.assert_array_equal(got, (x.astype(np.float64) @ w.T.astype(np.float64)).astype(np.float32))


def test_lm_head_reference_reduction_order():
    """x = 1 at h = 0..254 and 2^24 at h = 255, W = 1.  In the reference's
    block order (thread t holds h = t; tree halving 128 .. 1) the first level
    adds 1 to 2^24, which rounds to even and loses it; every later level adds
    an even partial sum exactly: 2^24 + 2 + 4 + ... + 128 = 2^24 + 254.  A
    sequential sum would give 2^24 + 256 and the exact value is 2^24 + 255."""
    x = np.zeros((1, 4096), np.float32)
    x[0, :255] = 1.0
    x[0, 255] = 2.0 ** 24
    w = np.ones((2, 4096), np.float32)
    got, err = oracle.lm_head(_bf(x), _bf(w))
    assert err == 0
    assert got[0, 0] == 2.0 ** 24 + 254 and got[0, 1] == 2.0 ** 24 + 254


def test_lm_head_error_bits():
    rng = np.random.default_rng(42)
    x = _bf(rng.integers(-3, 4, (2, 4096)))
    w = _bf(rng.integers(-3, 4, (5, 4096)))
    w_inf = w.copy()
    w_inf[3, 1000] = 0x7F80  # +inf in one weight row: that word's logits, bits 64 | 128
    got, err = oracle.lm_head(x, w_inf)
    assert err == 64 | 128
    assert not np.isfinite(got[:, 3]).any() and np.isfinite(np.delete(got, 3, axis=1)).all()
    # finite operands whose products overflow fp32: bit 128 only
    xo = _bf(np.full((1, 4096), 2.0 ** 70, np.float32))
    wo = _bf(np.full((1, 4096), 2.0 ** 70, np.float32))
    got, err = oracle.lm_head(xo, wo)
    assert err == 128 and np.isinf(got[0, 0])


# --------------------------------------------- live reference (optional)
@pytest.mark.skipif(not os.path.exists(oracle._REF_PATH),
                    reason="oracle/_ref not built (needs the reference checkout)")
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
    raw = (synth.normal(84, 300 * 256) * 4).astype(np.float32).reshape(300, 256)
    raw[100:150] = np.round(raw[100:150] * 2) / 2  # exact ties
    bias = (synth.normal(85, 256) * 0.3).astype(np.float32)
    ids1, w1 = _v4_route(raw, bias)
    ids2 = np.empty_like(ids1)
    w2 = np.empty_like(w1)
    assert R.pr_learned_router(raw.ctypes.data_as(P), 300, bias.ctypes.data_as(P), ids2.ctypes.data_as(P),
                               w2.ctypes.data_as(P)) == 0
    np.testing.assert_array_equal(ids1, ids2)
    np.testing.assert_array_equal(w1.view(np.uint32), w2.view(np.uint32))


# --------------------------------------------------- V4.1 32-block formats
def test_v41_fp4_to_fp8_reference_vectors(gold):
    """ConvertExpertFp4Block of the reference (compiled from its sources):
    narrow and 12-wide row-scale bands, a maximum of exactly 6, all 127."""
    for b in range(gold["v41_fp4_packed"].shape[0]):
        w, s, st = oracle.v41_fp4_block_to_fp8(gold["v41_fp4_packed"][b], gold["v41_fp4_scales"][b])
        assert st == 0 and s == gold["v41_fp8_scale"][b]
        np.testing.assert_array_equal(w.ravel(), gold["v41_fp8_weight"][b])


def test_v41_fp4_to_fp8_tensor_tiling(gold):
    """The tensor form (weight_expert_convert.cpp:64-100) on a 64 x 128
    tensor: 2 x 4 blocks of 32 x 32, block (br, bc) taken from golden block
    (4 br + bc) % 6 of the compiled reference's ConvertExpertFp4Block
    (packed rows of 64 bytes, row scales [64, 4]).  Every output block and
    its shared scale must equal that golden block's, so a transposed block
    grid, a wrong packed-row stride or a wrong scale index fails."""
    rows, cols = 64, 128
    packed = np.zeros((rows, cols // 2), np.uint8)
    scales = np.zeros((rows, cols // 32), np.uint8)
    src = lambda br, bc: (4 * br + bc) % gold["v41_fp4_packed"].shape[0]
    for br in range(2):
        for bc in range(4):
            b = src(br, bc)
            packed[32 * br:32 * br + 32, 16 * bc:16 * bc + 16] = gold["v41_fp4_packed"][b].reshape(32, 16)
            scales[32 * br:32 * br + 32, bc] = gold["v41_fp4_scales"][b]
    w, s = oracle.v41_fp4_to_fp8(packed, scales)
    assert w.shape == (rows, cols) and s.shape == (2, 4)
    for br in range(2):
        for bc in range(4):
            b = src(br, bc)
            assert s[br, bc] == gold["v41_fp8_scale"][b]
            np.testing.assert_array_equal(w[32 * br:32 * br + 32, 32 * bc:32 * bc + 32].ravel(),
                                          gold["v41_fp8_weight"][b])
            wb, sb, st = oracle.v41_fp4_block_to_fp8(gold["v41_fp4_packed"][b], gold["v41_fp4_scales"][b])
            assert st == 0 and sb == s[br, bc]
    # the golden blocks differ, so a swapped block placement is visible
    assert len({gold["v41_fp8_weight"][src(br, bc)].tobytes() for br in range(2) for bc in range(4)}) > 1


def test_v41_fp4_to_fp8_closed_forms():
    """All row scales equal: shift = 6, every e2m1 magnitude m becomes
    m * 64 (exact in e4m3: 32, 64, 96, 128, 192, 256, 384); the negative zero
    nibble gives +0; a row 7 below the maximum (shift -1) maps 0.5 to 0.25
    and 6 to 3; one 12 below (shift -6) maps 0.5 to the subnormal 2^-7 (code
    4) and 6 to 0.09375 (code 0x1C); shared scale = max - 6; errors for 255
    and max < 6."""
    nib = np.arange(16, dtype=np.uint8)
    row = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)  # 16 nibbles 0..15 then again
    packed = np.tile(np.concatenate([row, row]), 32)
    scales = np.full(32, 120, np.uint8)
    w, s, st = oracle.v41_fp4_block_to_fp8(packed, scales)
    assert st == 0 and s == 114
    vals = [oracle.e4m3_decode(int(c)) for c in w[0, :16]]
    assert vals == [0.0, 32.0, 64.0, 96.0, 128.0, 192.0, 256.0, 384.0,
                    0.0, -32.0, -64.0, -96.0, -128.0, -192.0, -256.0, -384.0]
    assert w[0, 8] == 0x00  # e2m1 -0 -> +0
    scales[5], scales[6] = 113, 108
    w, s, st = oracle.v41_fp4_block_to_fp8(packed, scales)
    assert st == 0 and s == 114
    assert oracle.e4m3_decode(int(w[5, 1])) == 0.25 and oracle.e4m3_decode(int(w[5, 7])) == 3.0
    assert w[6, 1] == 0x04 and w[6, 7] == 0x1C and w[6, 9] == 0x84
    bad = scales.copy()
    bad[9] = 255
    assert oracle.v41_fp4_block_to_fp8(packed, bad)[2] == 1
    assert oracle.v41_fp4_block_to_fp8(packed, np.full(32, 5, np.uint8))[2] == 2


def test_v41_dequant_reference_vectors(gold):
    for blk in (32, 128):
        out, st = oracle.v41_dequant_block(gold[f"v41_woa{blk}_src"], gold[f"v41_woa{blk}_scale"][0], blk)
        assert st == 0
        np.testing.assert_array_equal(out, gold[f"v41_woa{blk}_bf16"])
    src = np.full(32 * 32, 0x38, np.uint8)  # 1.0
    out, st = oracle.v41_dequant_block(src, 0.375, 32)
    assert st == 0 and (out == 0x3EC0).all()  # bf16(0.375)
    src[7] = 0x7F
    assert oracle.v41_dequant_block(src, 0.375, 32)[1] == 2
    assert oracle.v41_dequant_block(np.full(1024, 0x7E, np.uint8), 2.0 ** 120, 32)[1] == 3  # 448 * 2^120
    assert oracle.v41_dequant_block(src, 0.0, 32)[1] == 1


def test_v41_quant32_closed_forms():
    """1/448 lies in [2^-9, 2^-8), so a group with amax 1 takes e = -8 (byte
    119) and 1.0 encodes as 256 = 0x78; an all-zero group uses the 1e-4 floor:
    1e-4/448 in [2^-23, 2^-22) -> byte 105; non-finite inputs raise bit 1,
    encode 0 and do not enter the maximum."""
    x = np.zeros((2, 64), np.float32)
    x[0, :32] = 1.0
    x[0, 32:] = 0.0
    x[1, :32] = -1.0
    x[1, 3] = np.inf
    x[1, 32:] = np.linspace(-3.0, 3.0, 32, dtype=np.float32)
    codes, scales, err = oracle.v41_quant32(oracle.f32_to_bf16_bits(x))
    assert scales[0].tolist() == [119, 105] and (codes[0, :32] == 0x78).all() and (codes[0, 32:] == 0).all()
    assert err == 1 and codes[1, 3] == 0 and scales[1, 0] == 119 and codes[1, 0] == 0xF8
    # 3/448 in [2^-8, 2^-7): e = -7, 3.0 * 128 = 384 = 0x7C
    assert scales[1, 1] == 120 and codes[1, 63] == 0x7C and codes[1, 32] == 0xFC


def _v41_operands(seed, rows, n, k, fp4):
    rng = np.random.default_rng(seed)
    a_int = rng.integers(-4, 5, (rows, k))
    a = np.array([oracle.e4m3_encode(float(v)) for v in a_int.ravel()], np.uint8).reshape(rows, k)
    sa = rng.integers(124, 131, (rows, k // 32)).astype(np.uint8)
    if fp4:
        codes = rng.integers(0, 16, (n, k)).astype(np.uint8)
        w = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
        table = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, 0, -.5, -1, -1.5, -2, -3, -4, -6])
        wv = table[codes]
        sw = rng.integers(124, 131, (n, k // 32)).astype(np.uint8)
        sw_full = np.repeat(sw, 32, axis=1)
    else:
        w_int = rng.integers(-4, 5, (n, k))
        w = np.array([oracle.e4m3_encode(float(v)) for v in w_int.ravel()], np.uint8).reshape(n, k)
        wv = w_int.astype(np.float64)
        sw = rng.integers(124, 131, (n // 32, k // 32)).astype(np.uint8)
        sw_full = np.repeat(np.repeat(sw, 32, axis=0), 32, axis=1)
    return a, sa, w, sw, a_int.astype(np.float64), wv, sw_full


@pytest.mark.parametrize("fp4", [False, True])
def test_v41_linear_float64_brute_force(fp4):
    """Small integers / e2m1 values with power-of-two scales: every term and
    partial sum is exact in fp32, so the output is the float64 sum
    sum_k a x 2^(sa-127) x w x 2^(sw-127) rounded once to bf16; the scale of
    W element (n, k) comes from block (n/32, k/32) (FP8) or row n (FP4)."""
    rows, n, k = 3, 64, 128
    a, sa, w, sw, af, wf, swf = _v41_operands(77 + fp4, rows, n, k, fp4)
    got, err = oracle.v41_linear(a, sa, w, sw, n, fp4)
    assert err == 0
    ascale = np.exp2(np.repeat(sa, 32, axis=1).astype(np.float64) - 127)
    wscale = np.exp2(swf.astype(np.float64) - 127)
    want = (af * ascale) @ (wf * wscale).T
    np.testing.assert_array_equal(got, oracle.f32_to_bf16_bits(want.astype(np.float32)))


def test_v41_linear_error_bits():
    rows, n, k = 2, 32, 64
    a, sa, w, sw, *_ = _v41_operands(90, rows, n, k, False)
    a2 = a.copy()
    a2[1, 5] = 0x7F  # NaN code: bit 1, the output row is NaN (bit 2)
    out, err = oracle.v41_linear(a2, sa, w, sw, n, False)
    assert err == 3 and np.isnan(oracle.bf16_bits_to_f32(out[1])).all()
    sa2 = sa.copy()
    sa2[0, 1] = 255  # NaN scale: bit 1 and an infinite term
    assert oracle.v41_linear(a, sa2, w, sw, n, False)[1] == 3
    sa3 = np.full_like(sa, 254)  # finite operands, terms overflow: bit 2 only
    assert oracle.v41_linear(a, sa3, w, np.full_like(sw, 254), n, False)[1] == 2


# ------------------------------------------------ reference INT4 fixture
@pytest.mark.parametrize("m,n,k,seed", [(3, 1024, 1024, 0), (1, 2048, 1024, 0x51A7), (2, 1024, 1024, 0x62B8),
                                        (3, 1024, 2048, 0x73C9), (7, 3072, 1024, 0x84DA),
                                        (17, 1024, 3072, 0x95EB)])
def test_w4a16_sym_reference_fixture(m, n, k, seed):
    """The reference's closed-form INT4 fixture
    (src/backend/cuda/qwen_int4_cuda_fixture.cpp:87-140,291,296-302):
    po_w4a16_sym equals its expected bf16 outputs bit for bit."""
    from tests import qwen_int4_fixture as fx

    x, packed, scales, expected = fx.case(m, n, k, seed)
    np.testing.assert_array_equal(oracle.w4a16_sym(x, packed, scales), expected)

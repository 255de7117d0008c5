"""GPU parity for the rest of the linear path: BF16 GEMM (prefill MFMA) and
GEMV (decode), W4A16 GEMV in both INT4 formats plus their exact dequant,
FP4 x FP8 GEMM (reference format, DeepSeek table), MXFP4 MoE grouped GEMM
(fp8 and bf16 activations), and the elementwise / MoE glue entries of the
DeepSeek table.  All calls go through the packs' C ABI; every result is
checked against the CPU oracle on the same seeded inputs (bit-exact for
integer/byte/dequant outputs, max_rel <= 1e-2 and cos >= 0.9999 otherwise).
"""
import numpy as np
import pytest

import oracle
from pih_amd import abi, synth
from tests.helpers import assert_close, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    import torch

    from pih_amd.device import engine_stream

    with engine_stream() as s:
        yield s
        torch.cuda.synchronize()


def _sync():
    import torch

    torch.cuda.current_stream().synchronize()


def _flag(t):
    return int(t.item()) & 0xFFFFFFFF


def _zeros(nbytes):
    import torch

    return torch.zeros(max(int(nbytes), 1), dtype=torch.uint8, device="cuda")


def _query(kind, m, n, k):
    out = (abi.C.c_uint64 * 1)()
    q = abi.request(abi.LN["workspace_query"], kind=kind, m=m, n=n, k=k, bytes_u64=abi.C.addressof(out))
    st = abi.linear_pack().call("query_workspace", q)
    assert st.code == abi.OK, st
    return int(out[0])


# ------------------------------------------------------------ BF16 GEMM
def _bf16_gemm(a, w, out_type, use_ws=True):
    import torch

    from pih_amd.device import ptr, stream_handle

    m, k = a.shape
    n = w.shape[0]
    ws_bytes = _query(abi.WORKSPACE_BF16_GEMM, m, n, k) if use_ws else 0
    ws = _zeros(ws_bytes) if ws_bytes else None
    out = torch.empty(m, n, dtype=torch.bfloat16 if out_type == abi.OUTPUT_BF16 else torch.float32, device="cuda")
    ad, wd = to_dev(a), to_dev(w)
    r = abi.request(abi.LN["bf16_gemm"], a_bf16=ptr(ad), w_bf16=ptr(wd), output=ptr(out), workspace=ptr(ws),
                    workspace_bytes=ws_bytes, stream=stream_handle(), m=m, n=n, k=k, output_type=out_type)
    st = abi.linear_pack().call("launch_bf16_gemm", r)
    assert st.code == abi.OK, st
    _sync()
    got = to_host(out)
    return oracle.bf16_bits_to_f32(got) if out_type == abi.OUTPUT_BF16 else got


@pytest.mark.parametrize("m,n,k", [(65, 128, 64), (130, 256, 512), (256, 1024, 4096), (200, 384, 12288)])
@pytest.mark.parametrize("out_type", [abi.OUTPUT_BF16, abi.OUTPUT_F32])
def test_bf16_gemm_prefill(eng, m, n, k, out_type):
    a = synth.bf16_normal(synth.config_seed(2, 10 + m), (m, k))
    w = synth.bf16_normal(synth.config_seed(2, 20 + n), (n, k), std=0.02)
    ref = oracle.bf16_gemm(a, w)
    assert_close(_bf16_gemm(a, w, out_type), ref, f"bf16 gemm {m}x{n}x{k}")


@pytest.mark.parametrize("m", [1, 8, 64])
@pytest.mark.parametrize("n,k", [(1024, 4096), (4096, 12288), (256, 1024)])
def test_bf16_gemv_decode(eng, m, n, k):
    a = synth.bf16_normal(synth.config_seed(2, 30 + m), (m, k))
    w = synth.bf16_normal(synth.config_seed(2, 40 + n), (n, k), std=0.02)
    # the largest case (64 x 4096 x 12288) is checked on every 4th output
    # column plus both ends of each 16-row weight block, to bound oracle time
    cols = np.arange(n) if m * n * k < 2 ** 31 else np.unique(
        np.concatenate([np.arange(0, n, 4), np.arange(15, n, 16)]))
    ref = oracle.bf16_gemm(a, np.ascontiguousarray(w[cols]))
    assert_close(_bf16_gemm(a, w, abi.OUTPUT_BF16)[:, cols], ref, f"bf16 gemv {m}x{n}x{k}")
    assert_close(_bf16_gemm(a, w, abi.OUTPUT_F32, use_ws=False)[:, cols], ref, f"bf16 gemv no-ws {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(5, 1024, 4096), (20, 1024, 4096), (40, 256, 1024), (64, 8192, 1024),
                                   (16, 8192, 1024), (64, 1024, 4096), (24, 256, 1152)])
def test_bf16_gemv_mid_m(eng, m, n, k):
    """4 < M <= 64: every configuration of the line-loading mid-M kernel
    (M tiles 1-4; 8192 rows take the 4-W-block and 4-wave variants) and, at
    K = 1152 (36 steps, no even split over 8 waves with 4-step batches),
    the gemv_kernel fallback."""
    a = synth.bf16_normal(synth.config_seed(2, 60 + m), (m, k))
    w = synth.bf16_normal(synth.config_seed(2, 70 + n), (n, k), std=0.02)
    ref = oracle.bf16_gemm(a, w)
    assert_close(_bf16_gemm(a, w, abi.OUTPUT_BF16), ref, f"bf16 gemv {m}x{n}x{k}")
    assert_close(_bf16_gemm(a, w, abi.OUTPUT_F32, use_ws=False), ref, f"bf16 gemv no-ws {m}x{n}x{k}")


# ----------------------------------------------------------------- W4A16
def _w4a16(x, q, s, z, fmt, m, n, k):
    import torch

    from pih_amd.device import ptr, stream_handle

    ws_bytes = _query(abi.WORKSPACE_W4A16, m, n, k)
    ws = _zeros(ws_bytes) if ws_bytes else None
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    xd, qd, sd = to_dev(x), to_dev(q), to_dev(s)
    zd = to_dev(z) if z is not None else None
    r = abi.request(abi.LN["w4a16"], input_bf16=ptr(xd), qweight=ptr(qd), scales=ptr(sd), zeros=ptr(zd),
                    output_bf16=ptr(out), workspace=ptr(ws), workspace_bytes=ws_bytes, error_flag_u32=ptr(flag),
                    stream=stream_handle(), m=m, n=n, k=k, format=fmt)
    st = abi.linear_pack().call("launch_w4a16_gemm", r)
    assert st.code == abi.OK, st
    _sync()
    return to_host(out), _flag(flag)


def _dequant(q, s, z, fmt, n, k):
    import torch

    from pih_amd.device import ptr, stream_handle

    out = torch.empty(n, k, dtype=torch.float32, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    qd, sd = to_dev(q), to_dev(s)
    zd = to_dev(z) if z is not None else None
    r = abi.request(abi.LN["w4a16_dequant"], qweight=ptr(qd), scales=ptr(sd), zeros=ptr(zd), output_f32=ptr(out),
                    error_flag_u32=ptr(flag), stream=stream_handle(), n=n, k=k, format=fmt)
    st = abi.linear_pack().call("launch_w4a16_dequant", r)
    assert st.code == abi.OK, st
    _sync()
    return to_host(out), _flag(flag)


QWEN8B = [(4096, 4096), (1024, 4096), (12288, 4096), (4096, 12288)]


@pytest.mark.parametrize("m", [1, 4, 16])
@pytest.mark.parametrize("n,k", QWEN8B)
def test_w4a16_asym(eng, m, n, k):
    q, s, z = synth.int4_asym_weight(synth.config_seed(3, n + k), n, k)
    x = synth.bf16_normal(synth.config_seed(3, 7 + m), (m, k))
    got, flag = _w4a16(x, q, s, z, abi.W4A16_ASYMMETRIC, m, n, k)
    assert flag == 0
    ref = oracle.w4a16_asym(x, q, s, z)
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref), f"w4a16 asym {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(5, 1024, 4096), (20, 1024, 4096), (32, 8192, 1024), (9, 8192, 1024),
                                   (9, 256, 1152)])
def test_w4a16_asym_mid_m(eng, m, n, k):
    """4 < M <= 32 on the mid-M kernel (one and two M tiles, 8 and 4 waves);
    K = 1152 (9 groups) does not split over its waves and takes
    gemv_kernel."""
    q, s, z = synth.int4_asym_weight(synth.config_seed(3, 4000 + n + k), n, k)
    x = synth.bf16_normal(synth.config_seed(3, 4100 + m), (m, k))
    got, flag = _w4a16(x, q, s, z, abi.W4A16_ASYMMETRIC, m, n, k)
    assert flag == 0
    ref = oracle.w4a16_asym(x, q, s, z)
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref), f"w4a16 asym {m}x{n}x{k}")


@pytest.mark.parametrize("m", [9, 20])
def test_w4a16_symmetric_mid_m_and_errors(eng, m):
    """Reference format on the mid-M kernel: results against the oracle, then
    a reserved nibble raises code 12 and a negative scale code 13."""
    n, k = 1024, 2048
    q, s = synth.int4_sym_weight(synth.config_seed(3, 4200 + m), n, k)
    x = synth.bf16_normal(synth.config_seed(3, 4300 + m), (m, k))
    got, flag = _w4a16(x, q, s, None, abi.W4A16_SYMMETRIC, m, n, k)
    assert flag == 0
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(oracle.w4a16_sym(x, q, s)), f"sym {m}")
    q2 = q.copy()
    q2[517, 300] = (q2[517, 300] & 0x0F) | 0x80  # reserved nibble (high half)
    _, flag = _w4a16(x, q2, s, None, abi.W4A16_SYMMETRIC, m, n, k)
    assert flag == 12
    s2 = s.copy()
    s2[1000, 15] = 0xBC00  # -1.0
    _, flag = _w4a16(x, q, s2, None, abi.W4A16_SYMMETRIC, m, n, k)
    assert flag == 13


def _w4a16_grouped(xs, weights, fmt, m, k):
    """weights: list of (q, s, z, n); xs: list of bf16 inputs [m, k]."""
    import torch

    from pih_amd.device import ptr, stream_handle

    keep, outs = [], []
    probs = (abi.W4A16_PROBLEM * len(weights))()
    for i, ((q, s, z, n), x) in enumerate(zip(weights, xs)):
        xd, qd, sd = to_dev(x), to_dev(q), to_dev(s)
        zd = to_dev(z) if z is not None else None
        out = torch.full((m, n), 0x7E7E, dtype=torch.int16, device="cuda").view(torch.bfloat16)
        keep += [xd, qd, sd, zd]
        outs.append(out)
        probs[i].input_bf16, probs[i].qweight, probs[i].scales = ptr(xd), ptr(qd), ptr(sd)
        probs[i].zeros, probs[i].output_bf16, probs[i].n = ptr(zd), ptr(out), n
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    r = abi.request(abi.LN["w4a16_grouped"], problems=abi.C.addressof(probs), error_flag_u32=ptr(flag),
                    stream=stream_handle(), problem_count=len(weights), m=m, k=k, format=fmt)
    st = abi.linear_pack().call("launch_w4a16_grouped", r)
    assert st.code == abi.OK, st
    _sync()
    return [to_host(o) for o in outs], _flag(flag)


@pytest.mark.parametrize("m", [1, 4, 16])
def test_w4a16_grouped_qkv_and_gate_up(eng, m):
    """q/k/v and gate/up of Qwen3-8B as two grouped launches (one input per
    problem); each output against the oracle's strict-k sum.  m = 1 and 4
    run the small-M kernel, m = 16 the mid-M kernel, one launch per group."""
    k = 4096
    for ns in ((4096, 1024, 1024), (12288, 12288)):
        weights = [synth.int4_asym_weight(synth.config_seed(3, 3000 + i + n), n, k) + (n,) for i, n in enumerate(ns)]
        xs = [synth.bf16_normal(synth.config_seed(3, 3100 + i + m), (m, k)) for i in range(len(ns))]
        got, flag = _w4a16_grouped(xs, weights, abi.W4A16_ASYMMETRIC, m, k)
        assert flag == 0
        for (q, s, z, n), x, g in zip(weights, xs, got):
            ref = oracle.w4a16_asym(x, q, s, z)
            assert_close(oracle.bf16_bits_to_f32(g), oracle.bf16_bits_to_f32(ref), f"grouped w4a16 {m}x{n}x{k}")


def test_w4a16_grouped_symmetric_and_errors(eng):
    """Reference format in a group of three; a bad scale in the last problem
    raises code 13 while the other problems still match the oracle."""
    m, k = 1, 2048
    ns = (1024, 2048, 256)
    weights = [synth.int4_sym_weight(synth.config_seed(3, 3200 + n), n, k) + (None, n) for n in ns]
    xs = [synth.bf16_normal(synth.config_seed(3, 3300 + i), (m, k)) for i in range(3)]
    got, flag = _w4a16_grouped(xs, weights, abi.W4A16_SYMMETRIC, m, k)
    assert flag == 0
    for (q, s, _, n), x, g in zip(weights, xs, got):
        assert_close(oracle.bf16_bits_to_f32(g), oracle.bf16_bits_to_f32(oracle.w4a16_sym(x, q, s)), "grouped sym")
    q, s, z, n = weights[2]
    s = s.copy()
    s[7, 3] = 0xBC00  # -1.0
    weights[2] = (q, s, z, n)
    got, flag = _w4a16_grouped(xs, weights, abi.W4A16_SYMMETRIC, m, k)
    assert flag == 13
    for (q, s, _, n), x, g in list(zip(weights, xs, got))[:2]:
        assert_close(oracle.bf16_bits_to_f32(g), oracle.bf16_bits_to_f32(oracle.w4a16_sym(x, q, s)), "grouped sym")


@pytest.mark.parametrize("n,k", [(1024, 4096), (256, 1024)])
def test_w4a16_asym_dequant_bit_exact(eng, n, k):
    q, s, z = synth.int4_asym_weight(synth.config_seed(3, 99 + n), n, k)
    got, flag = _dequant(q, s, z, abi.W4A16_ASYMMETRIC, n, k)
    assert flag == 0
    ref = oracle.w4a16_asym_dequant(q, s, z, k)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


QWEN06B = [(2048, 1024), (1024, 1024), (1024, 2048), (3072, 1024), (1024, 3072)]


@pytest.mark.parametrize("m", [1, 37])
@pytest.mark.parametrize("n,k", QWEN06B)
def test_w4a16_symmetric_reference_format(eng, m, n, k):
    q, s = synth.int4_sym_weight(synth.config_seed(3, 500 + n + k), n, k)
    x = synth.bf16_normal(synth.config_seed(3, 600 + m), (m, k))
    got, flag = _w4a16(x, q, s, None, abi.W4A16_SYMMETRIC, m, n, k)
    assert flag == 0
    ref = oracle.w4a16_sym(x, q, s)
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref), f"w4a16 sym {m}x{n}x{k}")


def test_w4a16_symmetric_dequant_bit_exact_and_reserved_nibble(eng):
    n, k = 64, 1024
    q, s = synth.int4_sym_weight(synth.config_seed(3, 777), n, k)
    got, flag = _dequant(q, s, None, abi.W4A16_SYMMETRIC, n, k)
    assert flag == 0
    nib = np.stack([q & 0xF, q >> 4], axis=-1).reshape(n, k).astype(np.int32)
    val = np.where(nib < 8, nib, nib - 16).astype(np.float32)
    sc = np.repeat(s.view(np.float16).astype(np.float32), 128, axis=1)
    np.testing.assert_array_equal(got.view(np.uint32), (val * sc).astype(np.float32).view(np.uint32))
    q2 = q.copy()
    q2[3, 17] = (q2[3, 17] & 0xF0) | 0x08  # reserved nibble
    _, flag = _dequant(q2, s, None, abi.W4A16_SYMMETRIC, n, k)
    assert flag == 12
    x = synth.bf16_normal(1, (1, k))
    _, flag = _w4a16(x, q2, s, None, abi.W4A16_SYMMETRIC, 1, n, k)
    assert flag == 12


# ------------------------------------------------------- FP4 x FP8 GEMM
def _fp4_inputs(seed, m, n, k):
    x = synth.bf16_normal(seed, (m, k))
    a, sa = oracle.fp8_quant_ue8m0(oracle.bf16_bits_to_f32(x))
    packed, sw = synth.mxfp4_weight(seed + 1, n, k)
    return a, sa, packed, sw


@pytest.mark.parametrize("m,n,k", [(1, 2048, 4096), (33, 4096, 2048), (130, 2048, 4096), (300, 2048, 4096),
                                   (256, 4096, 7168)])
def test_fp4_gemm_deepseek_table(eng, m, n, k):
    """M 1-130: the small-M kernel; M 300 (above 256 rows) and M 256 at
    7168 -> 4096 (four 64-row chunks would stream 4 x 15.6 MB of weights):
    the dense big tiles with the FP4 W operand."""
    import torch

    from pih_amd.device import ptr, stream_handle

    a, sa, packed, sw = _fp4_inputs(synth.config_seed(5, m), m, n, k)
    ref = oracle.fp4_gemm(a, sa, packed, sw)
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ad, sad, pd, swd = to_dev(a), to_dev(sa), to_dev(packed), to_dev(sw)
    r = abi.request(abi.DS["fp4_gemm"], activation_e4m3=ptr(ad), activation_scale_bits=ptr(sad),
                    packed_weight=ptr(pd), weight_scale_bits=ptr(swd), output_bf16=ptr(out), error_flag=ptr(flag),
                    stream=stream_handle(), m=m, n=n, k=k)
    st = abi.deepseek_pack().call("launch_fp4_gemm", r)
    assert st.code == abi.OK, st
    _sync()
    assert _flag(flag) == 0
    assert_close(oracle.bf16_bits_to_f32(to_host(out)), ref, f"fp4 gemm {m}x{n}x{k}")


def test_fp4_gemm_big_tiles_nan_code(eng):
    """The dense big-tile FP4 route (M 512) with an e4m3 NaN code in A: the
    scan raises bit 1, the big tiles exit, and the checking 128 x 128 kernel
    computes the result with the code as 0 (deepseek_fp4_gemm.cu decodes it
    so)."""
    import torch

    from pih_amd.device import ptr, stream_handle

    m, n, k = 512, 2048, 4096
    a, sa, packed, sw = _fp4_inputs(synth.config_seed(5, 777), m, n, k)
    a0 = a.copy()
    a[200, 1000] = 0x7F
    a0[200, 1000] = 0  # the code decodes as 0
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ad, sad, pd, swd = to_dev(a), to_dev(sa), to_dev(packed), to_dev(sw)
    r = abi.request(abi.DS["fp4_gemm"], activation_e4m3=ptr(ad), activation_scale_bits=ptr(sad),
                    packed_weight=ptr(pd), weight_scale_bits=ptr(swd), output_bf16=ptr(out), error_flag=ptr(flag),
                    stream=stream_handle(), m=m, n=n, k=k)
    st = abi.deepseek_pack().call("launch_fp4_gemm", r)
    assert st.code == abi.OK, st
    _sync()
    assert _flag(flag) == 1
    rows = np.array([0, 199, 200, 201, m - 1])
    ref = oracle.fp4_gemm(np.ascontiguousarray(a0[rows]), np.ascontiguousarray(sa[rows]), packed, sw)
    got = oracle.bf16_bits_to_f32(to_host(out))
    assert np.isfinite(got).all()
    assert_close(got[rows], ref, "fp4 big tiles nan code")


def _mx_moe_weights(experts, n, k, seed):
    p = np.empty((experts, n, k // 2), np.uint8)
    s = np.empty((experts, n, k // 32), np.uint8)
    for e in range(experts):
        p[e], s[e] = synth.mxfp4_weight(seed + e, n, k)
    return p, s


@pytest.mark.parametrize("act", [abi.ACTIVATION_E4M3, abi.ACTIVATION_BF16])
@pytest.mark.parametrize("tokens,experts,topk", [(64, 8, 2), (5, 16, 4), (200, 8, 2)])
def test_moe_mxfp4_gemm_swiglu(eng, act, tokens, experts, topk):
    """Light experts (<= 64 rows with e4m3, <= 32 with bf16 activations) go
    to the weight-streaming kernel, the others to the 128-row tiles; the
    200-token case has experts on both sides of both limits."""
    from pih_amd import linear

    hidden, inter = 512, 256
    ids, wts = synth.zipf_router(synth.config_seed(5, 800 + tokens), tokens, experts, topk)
    x = synth.bf16_normal(synth.config_seed(5, 801), (tokens, hidden))
    w13, s13 = _mx_moe_weights(experts, 2 * inter, hidden, synth.config_seed(5, 900))
    off, rt, rw, tr = oracle.route_plan(ids, wts, experts)
    xq, xs = oracle.fp8_quant_ue8m0(oracle.bf16_bits_to_f32(x))
    rows = tokens * topk
    ref = np.zeros((rows, inter), np.uint16)
    for e in range(experts):
        b, en = int(off[e]), int(off[e + 1])
        if b == en:
            continue
        if act == abi.ACTIVATION_E4M3:
            gu = oracle.fp4_gemm(np.ascontiguousarray(xq[rt[b:en]]), np.ascontiguousarray(xs[rt[b:en]]), w13[e], s13[e])
        else:
            gu = oracle.mxfp4_bf16_gemm(np.ascontiguousarray(x[rt[b:en]]), w13[e], s13[e])
        g = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(gu[:, :inter]))
        u = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(gu[:, inter:]))
        mid = oracle.swiglu(g, u, 0.0) * rw[b:en, None]
        ref[b:en] = oracle.f32_to_bf16_bits(mid.astype(np.float32))
    if act == abi.ACTIVATION_E4M3:
        a_d, as_d = to_dev(xq), to_dev(xs)
    else:
        a_d, as_d = to_dev(x), None
    out, flag = linear.moe_mxfp4_gemm(a_d, as_d, to_dev(rt), to_dev(w13), to_dev(s13), to_dev(off), rows, act,
                                      abi.OUTPUT_SWIGLU_BF16, row_weight=to_dev(rw))
    _sync()
    assert _flag(flag) == 0
    n_rows = int(off[-1])
    assert_close(oracle.bf16_bits_to_f32(to_host(out)[:n_rows]), oracle.bf16_bits_to_f32(ref[:n_rows]),
                 "mxfp4 moe swiglu")


@pytest.mark.parametrize("act", [abi.ACTIVATION_E4M3, abi.ACTIVATION_BF16])
def test_moe_mxfp4_gemm_down_bf16_out(eng, act):
    from pih_amd import linear

    tokens, experts, topk, hidden, inter = 40, 8, 2, 256, 512
    ids, wts = synth.zipf_router(synth.config_seed(5, 1200), tokens, experts, topk)
    off, rt, rw, tr = oracle.route_plan(ids, wts, experts)
    rows = tokens * topk
    mid = synth.bf16_normal(synth.config_seed(5, 1201), (rows, inter))
    w2, s2 = _mx_moe_weights(experts, hidden, inter, synth.config_seed(5, 1300))
    mq, ms = oracle.fp8_quant_ue8m0(oracle.bf16_bits_to_f32(mid))
    ref = np.zeros((rows, hidden), np.float32)
    for e in range(experts):
        b, en = int(off[e]), int(off[e + 1])
        if b == en:
            continue
        if act == abi.ACTIVATION_E4M3:
            ref[b:en] = oracle.fp4_gemm(np.ascontiguousarray(mq[b:en]), np.ascontiguousarray(ms[b:en]), w2[e], s2[e])
        else:
            ref[b:en] = oracle.mxfp4_bf16_gemm(np.ascontiguousarray(mid[b:en]), w2[e], s2[e])
    a_d, as_d = (to_dev(mq), to_dev(ms)) if act == abi.ACTIVATION_E4M3 else (to_dev(mid), None)
    out, flag = linear.moe_mxfp4_gemm(a_d, as_d, None, to_dev(w2), to_dev(s2), to_dev(off), rows, act,
                                      abi.OUTPUT_BF16)
    _sync()
    assert _flag(flag) == 0
    assert_close(oracle.bf16_bits_to_f32(to_host(out)), ref, "mxfp4 moe down")


def test_moe_mxfp4_gemm_forked_stream_threads_and_graph(eng):
    """The tiled experts of an MXFP4 MoE launch run on an auxiliary stream
    forked from the caller's (the weight-streaming experts on the caller's)
    and joined before the entry returns.  Two host threads calling at once on
    two streams, and a captured graph (capture keeps both launches on the
    capturing stream) replayed three times with eager work between the
    replays, give the bits of one plain call."""
    import threading

    import torch

    from pih_amd import linear

    tokens, experts, topk, hidden, inter = 200, 8, 2, 512, 256
    ids, wts = synth.zipf_router(synth.config_seed(5, 800 + tokens), tokens, experts, topk)
    x = synth.bf16_normal(synth.config_seed(5, 801), (tokens, hidden))
    w13, s13 = _mx_moe_weights(experts, 2 * inter, hidden, synth.config_seed(5, 900))
    off, rt, rw, _ = oracle.route_plan(ids, wts, experts)
    counts = np.diff(off.astype(np.int64))
    assert (counts > 64).any() and ((counts > 0) & (counts <= 64)).any()  # both kernels run
    xq, xs = oracle.fp8_quant_ue8m0(oracle.bf16_bits_to_f32(x))
    rows = tokens * topk
    dev = [to_dev(t) for t in (xq, xs, rt, w13, s13, off, rw)]

    def call(out=None, flag=None):
        return linear.moe_mxfp4_gemm(dev[0], dev[1], dev[2], dev[3], dev[4], dev[5], rows, abi.ACTIVATION_E4M3,
                                     abi.OUTPUT_SWIGLU_BF16, row_weight=dev[6], out=out, flag=flag)

    ref, flag = call()
    _sync()
    assert _flag(flag) == 0
    n_rows = int(off[-1])
    want = to_host(ref)[:n_rows]

    results, errors = {}, []

    def worker(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                outs = [call() for _ in range(8)]
            s.synchronize()
            results[i] = [(to_host(o)[:n_rows], _flag(f)) for o, f in outs]
        except Exception as e:  # reported below, on the test's thread
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i in range(2):
        for got, f in results[i]:
            assert f == 0
            np.testing.assert_array_equal(got, want)

    out = torch.empty_like(ref)
    gflag = torch.zeros(1, dtype=torch.int32, device="cuda")
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=side):
        gflag.zero_()
        call(out=out, flag=gflag)
    torch.cuda.synchronize()
    for _ in range(3):
        out.fill_(0)
        _ = call()  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert _flag(gflag) == 0
        np.testing.assert_array_equal(to_host(out)[:n_rows], want)


# ---------------------------------------------------------- elementwise
def test_mxfp4_decode_bit_exact(eng):
    import torch

    from pih_amd.device import ptr, stream_handle

    rows, k = 9, 4096
    packed, scales = synth.mxfp4_weight(synth.config_seed(5, 3), rows, k)
    scales[0, :4] = [0, 1, 126, 250]
    ref = np.stack([oracle.mxfp4_decode_row(packed[r], scales[r], k) for r in range(rows)])
    out = torch.empty(rows, k, dtype=torch.bfloat16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    pd, sd = to_dev(packed), to_dev(scales)
    r = abi.request(abi.LN["mxfp4_decode"], packed=ptr(pd), scales_ue8m0=ptr(sd), output_bf16=ptr(out),
                    error_flag_u32=ptr(flag), stream=stream_handle(), rows=rows, k=k)
    assert abi.linear_pack().call("launch_mxfp4_decode", r).code == abi.OK
    _sync()
    assert _flag(flag) == 0
    got = oracle.bf16_bits_to_f32(to_host(out))
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_silu_mul(eng):
    import torch

    from pih_amd.device import ptr, stream_handle

    g = synth.bf16_normal(synth.config_seed(1, 1), (16, 3072), std=2.0)
    u = synth.bf16_normal(synth.config_seed(1, 2), (16, 3072))
    ref = oracle.silu_mul(g, u)
    out = torch.empty(16, 3072, dtype=torch.bfloat16, device="cuda")
    gd, ud = to_dev(g), to_dev(u)
    r = abi.request(abi.LN["silu_mul"], gate_bf16=ptr(gd), up_bf16=ptr(ud), output_bf16=ptr(out),
                    stream=stream_handle(), count=g.size)
    assert abi.linear_pack().call("launch_silu_mul", r).code == abi.OK
    _sync()
    got = to_host(out)
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref), "silu_mul")
    # bf16 rounding of the same fp32 value: at most one ulp apart
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1


def test_deepseek_expert_and_shared_swiglu(eng):
    import torch

    from pih_amd.device import ptr, stream_handle

    t = 37
    g = synth.bf16_normal(synth.config_seed(1, 3), (t, 2048), std=6.0)
    u = synth.bf16_normal(synth.config_seed(1, 4), (t, 2048), std=6.0)
    w = (0.1 + synth.uniform(5, t)).astype(np.float32)
    sw = oracle.swiglu(oracle.bf16_bits_to_f32(g), oracle.bf16_bits_to_f32(u), 10.0)
    ref_shared = oracle.f32_to_bf16_bits(sw)
    ref_expert = oracle.f32_to_bf16_bits((sw * w[:, None]).astype(np.float32))
    gd, ud, wd = to_dev(g), to_dev(u), to_dev(w)
    out = torch.empty(t, 2048, dtype=torch.bfloat16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    r = abi.request(abi.DS["expert_swiglu"], gate_bf16=ptr(gd), up_bf16=ptr(ud), route_weights_f32=ptr(wd),
                    output_bf16=ptr(out), error_flag=ptr(flag), stream=stream_handle(), token_count=t)
    assert abi.deepseek_pack().call("launch_expert_swiglu", r).code == abi.OK
    _sync()
    assert _flag(flag) == 0
    assert_close(oracle.bf16_bits_to_f32(to_host(out)), oracle.bf16_bits_to_f32(ref_expert), "expert swiglu")
    r = abi.request(abi.DS["shared_swiglu"], gate_bf16=ptr(gd), up_bf16=ptr(ud), output_bf16=ptr(out),
                    error_flag=ptr(flag), stream=stream_handle(), token_count=t)
    assert abi.deepseek_pack().call("launch_shared_swiglu", r).code == abi.OK
    _sync()
    assert_close(oracle.bf16_bits_to_f32(to_host(out)), oracle.bf16_bits_to_f32(ref_shared), "shared swiglu")


def test_deepseek_gather_accumulate_finalize_bit_exact(eng):
    import torch

    from pih_amd.device import ptr, stream_handle

    tokens, hidden = 50, 4096
    src = synth.bf16_normal(synth.config_seed(1, 10), (tokens, hidden))
    idx = np.array([1, 4, 5, 9, 20, 33, 49], np.uint32)
    routes = idx.size
    gathered = torch.empty(routes, hidden, dtype=torch.bfloat16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    sd, idd = to_dev(src), to_dev(idx)
    r = abi.request(abi.DS["route_gather"], source_hidden_bf16=ptr(sd), token_indices_u32=ptr(idd),
                    route_hidden_bf16=ptr(gathered), error_flag=ptr(flag), stream=stream_handle(),
                    route_count=routes, packed_token_count=tokens)
    assert abi.deepseek_pack().call("launch_route_gather", r).code == abi.OK
    _sync()
    np.testing.assert_array_equal(to_host(gathered), src[idx])
    y = synth.bf16_normal(synth.config_seed(1, 11), (routes, hidden))
    acc0 = synth.normal(synth.config_seed(1, 12), tokens * hidden).astype(np.float32).reshape(tokens, hidden)
    acc_ref = acc0.copy()
    for j, t in enumerate(idx):
        acc_ref[t] += oracle.bf16_bits_to_f32(y[j])
    acc = to_dev(acc0)
    yd = to_dev(y)
    r = abi.request(abi.DS["expert_accumulate"], expert_output_bf16=ptr(yd), token_indices=ptr(idd),
                    accumulator_f32=ptr(acc), error_flag=ptr(flag), stream=stream_handle(), route_count=routes,
                    token_count=tokens)
    assert abi.deepseek_pack().call("launch_expert_accumulate", r).code == abi.OK
    _sync()
    assert _flag(flag) == 0
    np.testing.assert_array_equal(to_host(acc).view(np.uint32), acc_ref.view(np.uint32))
    shared = synth.bf16_normal(synth.config_seed(1, 13), (tokens, hidden))
    fin_ref = oracle.finalize(acc_ref, shared)
    out = torch.empty(tokens, hidden, dtype=torch.bfloat16, device="cuda")
    shd = to_dev(shared)
    r = abi.request(abi.DS["expert_finalize"], accumulator_f32=ptr(acc), shared_output_bf16=ptr(shd),
                    output_bf16=ptr(out), error_flag=ptr(flag), stream=stream_handle(), token_count=tokens)
    assert abi.deepseek_pack().call("launch_expert_finalize", r).code == abi.OK
    _sync()
    assert _flag(flag) == 0
    np.testing.assert_array_equal(to_host(out), fin_ref)
    # tokens not strictly increasing -> error bit 1
    bad = to_dev(np.array([3, 3], np.uint32))
    r = abi.request(abi.DS["expert_accumulate"], expert_output_bf16=ptr(yd), token_indices=ptr(bad),
                    accumulator_f32=ptr(acc), error_flag=ptr(flag), stream=stream_handle(), route_count=2,
                    token_count=tokens)
    assert abi.deepseek_pack().call("launch_expert_accumulate", r).code == abi.OK
    _sync()
    assert _flag(flag) & 1


@pytest.mark.parametrize("tokens", [3, 200])
def test_deepseek_router_gemm(eng, tokens):
    import torch

    from pih_amd.device import ptr, stream_handle

    x = synth.bf16_normal(synth.config_seed(1, 20), (tokens, 4096))
    w = synth.bf16_normal(synth.config_seed(1, 21), (256, 4096), std=0.02)
    ref = oracle.bf16_gemm(x, w)
    out = torch.empty(tokens, 256, dtype=torch.float32, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    xd, wd = to_dev(x), to_dev(w)
    r = abi.request(abi.DS["router_gemm"], input_bf16=ptr(xd), weight_bf16=ptr(wd), scores_f32=ptr(out),
                    error_flag_u32=ptr(flag), stream=stream_handle(), token_count=tokens, expert_count=256,
                    hidden_size=4096)
    st = abi.deepseek_pack().call("launch_router_gemm", r)
    assert st.code == abi.OK, st
    _sync()
    assert_close(to_host(out), ref, "router gemm")

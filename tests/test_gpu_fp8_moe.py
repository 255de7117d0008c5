"""GPU parity: FP8 quant, block-scaled FP8 GEMM (dense, grouped, MoE), the
device route plan, combine and the whole FP8 MoE expert layer, each called
through the C ABI of the gfx950 packs and checked against the CPU oracle on
the same seeded inputs.

Bars: integer/byte/index outputs bit-exact; floating outputs max_rel <= 1e-2
(normwise, max|g-r|/max|r|) and cosine >= 0.9999 against the fp32-accumulate
oracle (tests/helpers.py)."""
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


def _codes(seed, shape):
    """Random e4m3 codes without the two NaN codes."""
    c = (synth.splitmix64(seed, int(np.prod(shape))) % np.uint64(254)).astype(np.uint8)
    c = np.where(c >= 0x7F, c + 1, c).astype(np.uint8)  # skip 0x7F
    return c.reshape(shape)


# ----------------------------------------------------------- FP8 quant
@pytest.mark.parametrize("rows,k", [(1, 128), (37, 1024), (64, 7168), (5, 2048)])
def test_fp8_quant_ue8m0_bit_exact(eng, rows, k):
    from pih_amd import linear

    x = synth.bf16_normal(synth.config_seed(4, 1000 + k), (rows, k))
    x[0, :7] = np.array([0x0000, 0x8000, 0x3F80, 0x43E0, 0xC3E0, 0x0001, 0x7F7F], np.uint16)[: min(7, k)]
    q_ref, s_ref = oracle.fp8_quant_ue8m0(oracle.bf16_bits_to_f32(x))
    q, s, flag = linear.fp8_quant(to_dev(x), abi.SCALE_UE8M0)
    _sync()
    assert _flag(flag) == 0
    np.testing.assert_array_equal(to_host(s), s_ref)
    np.testing.assert_array_equal(to_host(q), q_ref)


@pytest.mark.parametrize("rows,k", [(3, 128), (64, 7168), (33, 2048)])
def test_fp8_quant_f32_bit_exact(eng, rows, k):
    from pih_amd import linear

    x = synth.bf16_normal(synth.config_seed(4, 2000 + k), (rows, k), std=3.0)
    q_ref, s_ref = oracle.fp8_quant_f32(oracle.bf16_bits_to_f32(x))
    q, s, flag = linear.fp8_quant(to_dev(x), abi.SCALE_F32)
    _sync()
    assert _flag(flag) == 0
    np.testing.assert_array_equal(to_host(s), s_ref)
    np.testing.assert_array_equal(to_host(q), q_ref)


def test_fp8_quant_gather_rows(eng):
    from pih_amd import linear

    x = synth.bf16_normal(synth.config_seed(4, 3000), (16, 256))
    rows = np.array([5, 0, 15, 5, 3], np.uint32)
    q_ref, s_ref = oracle.fp8_quant_f32(oracle.bf16_bits_to_f32(x[rows]))
    q, s, flag = linear.fp8_quant(to_dev(x), abi.SCALE_F32, rows=to_dev(rows))
    _sync()
    assert _flag(flag) == 0
    np.testing.assert_array_equal(to_host(q), q_ref)
    np.testing.assert_array_equal(to_host(s), s_ref)


def test_fp8_quant_through_deepseek_table(eng):
    import torch

    from pih_amd.device import ptr, stream_handle

    x = synth.bf16_normal(synth.config_seed(4, 3100), (9, 4096))
    q_ref, s_ref = oracle.fp8_quant_ue8m0(oracle.bf16_bits_to_f32(x))
    xd = to_dev(x)
    q = torch.empty(9, 4096, dtype=torch.uint8, device="cuda")
    s = torch.empty(9, 32, dtype=torch.uint8, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    r = abi.request(abi.DS["fp8_activation_quant"], input_bf16=ptr(xd), output_e4m3=ptr(q), scale_bits=ptr(s),
                    error_flag=ptr(flag), stream=stream_handle(), token_count=9, logical_k=4096)
    st = abi.deepseek_pack().call("launch_fp8_activation_quant", r)
    assert st.code == abi.OK, st
    _sync()
    assert _flag(flag) == 0
    np.testing.assert_array_equal(to_host(q), q_ref)
    np.testing.assert_array_equal(to_host(s), s_ref)


# ----------------------------------------------------- dense FP8 GEMM
@pytest.mark.parametrize("m,n,k", [(1, 128, 128), (37, 256, 512), (130, 384, 1024), (256, 128, 7168)])
@pytest.mark.parametrize("out_type", [1, 2])
def test_fp8_gemm_ue8m0_deepseek_table(eng, m, n, k, out_type):
    import torch

    from pih_amd.device import ptr, stream_handle

    a = _codes(synth.config_seed(4, 4000 + m), (m, k))
    w = _codes(synth.config_seed(4, 4100 + n), (n, k))
    sa = (120 + synth.splitmix64(7 + m, m * (k // 128)) % np.uint64(10)).astype(np.uint8).reshape(m, k // 128)
    sw = (118 + synth.splitmix64(9 + n, (n // 128) * (k // 128)) % np.uint64(6)).astype(np.uint8)
    sw = sw.reshape(n // 128, k // 128)
    ref = oracle.fp8_gemm_ue8m0(a, sa, w, sw)
    out = torch.empty(m, n, dtype=torch.bfloat16 if out_type == 1 else torch.float32, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ad, sad, wd, swd = to_dev(a), to_dev(sa), to_dev(w), to_dev(sw)
    r = abi.request(abi.DS["fp8_gemm"], activation_e4m3=ptr(ad), activation_scale_bits=ptr(sad),
                    weight_e4m3=ptr(wd), weight_scale_bits=ptr(swd), output=ptr(out), error_flag=ptr(flag),
                    stream=stream_handle(), m=m, n=n, k=k, output_type=out_type)
    st = abi.deepseek_pack().call("launch_fp8_gemm", r)
    assert st.code == abi.OK, st
    _sync()
    assert _flag(flag) == 0
    got = to_host(out)
    got = oracle.bf16_bits_to_f32(got) if out_type == 1 else got
    assert_close(got, ref, f"fp8_gemm ue8m0 {m}x{n}x{k}")


def test_fp8_gemm_rejects_nan_code_and_ff_scale(eng):
    import torch

    from pih_amd.device import ptr, stream_handle

    m, n, k = 4, 128, 256
    a = _codes(1, (m, k))
    w = _codes(2, (n, k))
    sa = np.full((m, k // 128), 127, np.uint8)
    sw = np.full((n // 128, k // 128), 127, np.uint8)
    a[1, 5] = 0x7F
    sw[0, 1] = 0xFF
    out = torch.empty(m, n, dtype=torch.float32, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ad, sad, wd, swd = to_dev(a), to_dev(sa), to_dev(w), to_dev(sw)
    r = abi.request(abi.DS["fp8_gemm"], activation_e4m3=ptr(ad), activation_scale_bits=ptr(sad),
                    weight_e4m3=ptr(wd), weight_scale_bits=ptr(swd), output=ptr(out), error_flag=ptr(flag),
                    stream=stream_handle(), m=m, n=n, k=k, output_type=2)
    assert abi.deepseek_pack().call("launch_fp8_gemm", r).code == abi.OK
    _sync()
    assert _flag(flag) & 1 and _flag(flag) & 2


@pytest.mark.parametrize("m,n,k", [(1, 128, 128), (77, 256, 1024), (200, 512, 7168)])
def test_fp8_gemm_f32_scales(eng, m, n, k):
    from pih_amd import linear

    x = synth.bf16_normal(synth.config_seed(4, 5000 + m), (m, k))
    xq, xs = oracle.fp8_quant_f32(oracle.bf16_bits_to_f32(x))
    w, ws = synth.fp8_block_weight(synth.config_seed(4, 5100 + n), n, k)
    ref = oracle.fp8_gemm_f32(xq, xs, w, ws)
    out, flag = linear.fp8_gemm(to_dev(xq), to_dev(xs), to_dev(w), to_dev(ws), abi.SCALE_F32, abi.OUTPUT_F32)
    _sync()
    assert _flag(flag) == 0
    assert_close(to_host(out), ref, f"fp8_gemm f32 {m}x{n}x{k}")


def test_grouped_fp8_gemm_deepseek_table(eng):
    import torch

    from pih_amd.device import ptr, stream_handle

    t, g, ng, kg = 5, 8, 128, 512
    x = synth.bf16_normal(synth.config_seed(4, 6000), (t * g, kg))
    w = _codes(synth.config_seed(4, 6001), (g * ng, kg))
    sw = (117 + synth.splitmix64(6002, g * (ng // 128) * (kg // 128)) % np.uint64(8)).astype(np.uint8)
    sw = sw.reshape(g * ng // 128, kg // 128)
    xq, xs = oracle.fp8_quant_ue8m0(oracle.bf16_bits_to_f32(x))
    ref = np.empty((t, g * ng), np.float32)
    for gi in range(g):
        rows = np.arange(t) * g + gi
        ref[:, gi * ng:(gi + 1) * ng] = oracle.fp8_gemm_ue8m0(
            np.ascontiguousarray(xq[rows]), np.ascontiguousarray(xs[rows]),
            np.ascontiguousarray(w[gi * ng:(gi + 1) * ng]), np.ascontiguousarray(sw[gi * ng // 128:(gi + 1) * ng // 128]))
    xd, wd, swd = to_dev(x), to_dev(w), to_dev(sw)
    aq = torch.empty(t * g, kg, dtype=torch.uint8, device="cuda")
    asb = torch.empty(t * g, kg // 128, dtype=torch.uint8, device="cuda")
    out = torch.empty(t, g * ng, dtype=torch.bfloat16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    r = abi.request(abi.DS["grouped_fp8_gemm"], input_bf16=ptr(xd), activation_e4m3=ptr(aq),
                    activation_scale_bits=ptr(asb), weight_e4m3=ptr(wd), weight_scale_bits=ptr(swd),
                    output_bf16=ptr(out), error_flag_u32=ptr(flag), stream=stream_handle(), token_count=t,
                    group_count=g, output_per_group=ng, input_per_group=kg)
    st = abi.deepseek_pack().call("launch_grouped_fp8_gemm", r)
    assert st.code == abi.OK, st
    _sync()
    assert _flag(flag) == 0
    np.testing.assert_array_equal(to_host(aq), xq)
    assert_close(oracle.bf16_bits_to_f32(to_host(out)), ref, "grouped fp8")


# ---------------------------------------------------------- route plan
@pytest.mark.parametrize("tokens,experts,topk", [(1, 8, 2), (64, 1024, 8), (33, 256, 6), (64, 256, 32), (65, 16, 4),
                                                 (4096, 256, 8), (300, 1024, 6)])
def test_route_plan_bit_exact(eng, tokens, experts, topk):
    """The device route plan against the oracle, bit for bit: up to 64 tokens
    the one-launch plan (one chunk: masks, offsets and rows in one block),
    above it the three-launch plan."""
    from pih_amd import linear

    ids, wts = synth.zipf_router(synth.config_seed(4, 7000 + tokens), tokens, experts, topk)
    o_ref, rt_ref, rw_ref, tr_ref = oracle.route_plan(ids, wts, experts)
    o, rt, rw, tr, flag = linear.route_plan(to_dev(ids), to_dev(wts), experts)
    _sync()
    assert _flag(flag) == 0
    np.testing.assert_array_equal(to_host(o), o_ref)
    np.testing.assert_array_equal(to_host(rt), rt_ref)
    np.testing.assert_array_equal(to_host(rw), rw_ref)
    np.testing.assert_array_equal(to_host(tr), tr_ref)


def test_route_plan_flags_bad_routes(eng):
    from pih_amd import linear

    ids = np.array([[0, 1], [2, 2], [9, 0], [3, 1]], np.uint32)
    wts = np.array([[0.5, 0.5], [0.5, 0.5], [0.5, 0.5], [np.nan, 0.5]], np.float32)
    o, rt, rw, tr, flag = linear.route_plan(to_dev(ids), to_dev(wts), 8)
    _sync()
    assert _flag(flag) == 7
    tr = to_host(tr)
    assert tr[1, 1] == 0xFFFFFFFF and tr[2, 0] == 0xFFFFFFFF and tr[3, 0] == 0xFFFFFFFF
    assert to_host(o)[-1] == 5  # five valid routes


# -------------------------------------------------------------- combine
@pytest.mark.parametrize("tokens,hidden", [(200, 512), (64, 7168), (3, 4104), (1, 7168)])
def test_combine_bit_exact(eng, tokens, hidden):
    """The ordered combine + shared add, bit-exact against the oracle; below
    256 tokens a token's row is split over several blocks (64 tokens x 7168:
    4 parts; 3 x 4104: 8 ragged parts of 65 / 58 chunks; 1 token: 14)."""
    from pih_amd import linear

    experts, topk = 32, 4
    ids, wts = synth.zipf_router(synth.config_seed(4, 8000), tokens, experts, topk)
    o, rt, rw, tr = oracle.route_plan(ids, wts, experts)
    y = synth.bf16_normal(synth.config_seed(4, 8001), (tokens * topk, hidden))
    shared = synth.bf16_normal(synth.config_seed(4, 8002), (tokens, hidden))
    ref = oracle.finalize(oracle.ordered_accumulate(y, rt, tokens), shared)
    out, flag = linear.moe_combine(to_dev(y), to_dev(tr), shared=to_dev(shared))
    _sync()
    assert _flag(flag) == 0
    np.testing.assert_array_equal(to_host(out), ref)


# ------------------------------------------------------------- MoE GEMMs
def _moe_weights(experts, hidden, inter, base):
    w13 = np.empty((experts, 2 * inter, hidden), np.uint8)
    s13 = np.empty((experts, 2 * inter // 128, hidden // 128), np.float32)
    w2 = np.empty((experts, hidden, inter), np.uint8)
    s2 = np.empty((experts, hidden // 128, inter // 128), np.float32)
    for e in range(experts):
        w13[e], s13[e] = synth.fp8_block_weight(synth.config_seed(4, base + e), 2 * inter, hidden)
        w2[e], s2[e] = synth.fp8_block_weight(synth.config_seed(4, base + 500 + e), hidden, inter)
    return w13, s13, w2, s2


@pytest.mark.parametrize("tokens,experts,topk,hidden,inter,limit",
                         [(64, 8, 2, 256, 256, 0.0), (300, 16, 4, 512, 256, 10.0), (1, 4, 2, 256, 128, 0.0)])
def test_moe_fp8_layer(eng, tokens, experts, topk, hidden, inter, limit):
    from pih_amd.linear import MoeFp8Layer

    ids, wts = synth.zipf_router(synth.config_seed(4, 9000 + tokens), tokens, experts, topk)
    x = synth.bf16_normal(synth.config_seed(4, 9001), (tokens, hidden))
    w13, s13, w2, s2 = _moe_weights(experts, hidden, inter, 9100)
    ref, y_ref, _ = oracle.moe_fp8_forward(x, ids, wts, experts, hidden, inter, w13, s13, w2, s2, limit)
    layer = MoeFp8Layer(to_dev(w13), to_dev(s13), to_dev(w2), to_dev(s2), tokens, topk, swiglu_limit=limit)
    out = layer.forward(to_dev(x), to_dev(ids), to_dev(wts))
    _sync()
    assert _flag(layer.flag) == 0
    assert_close(oracle.bf16_bits_to_f32(to_host(layer.y)), oracle.bf16_bits_to_f32(y_ref), "expert rows")
    assert_close(oracle.bf16_bits_to_f32(to_host(out)), oracle.bf16_bits_to_f32(ref), "moe layer")


def test_moe_fp8_layer_full_shape_cold_experts(eng):
    """BASELINE cfg4 geometry (T=4096, E=256, top-8, H=7168, I=2048): the
    route plan is checked bit-exact in full, the expert rows of the coldest
    touched experts against the oracle chain, and 48 sampled rows of each of
    the two hottest experts (3997 and 3612 rows: the multi-tile path with
    its 256-row tiles, rows on both sides of tile boundaries and the last
    partial tile) against the same chain."""
    import torch

    from pih_amd.linear import MoeFp8Layer

    tokens, experts, topk, hidden, inter = 4096, 256, 8, 7168, 2048
    ids, wts = synth.zipf_router(synth.config_seed(4, 0), tokens, experts, topk)
    x = synth.bf16_normal(synth.config_seed(4, 1), (tokens, hidden))
    o_ref, rt_ref, rw_ref, tr_ref = oracle.route_plan(ids, wts, experts)
    counts = np.diff(o_ref.astype(np.int64))
    cold = [int(e) for e in np.argsort(counts, kind="stable") if counts[e] > 0][:3]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)
    # random codes for the experts not checked, exact synth weights for the checked ones
    w13 = torch.randint(0, 0x7E, (experts, 2 * inter, hidden), dtype=torch.uint8, device="cuda", generator=gen)
    w2 = torch.randint(0, 0x7E, (experts, hidden, inter), dtype=torch.uint8, device="cuda", generator=gen)
    s13 = torch.full((experts, 2 * inter // 128, hidden // 128), 1e-3, dtype=torch.float32, device="cuda")
    s2 = torch.full((experts, hidden // 128, inter // 128), 1e-3, dtype=torch.float32, device="cuda")
    host = {}
    for e in cold:
        a, sa = synth.fp8_block_weight(synth.config_seed(4, 20 + e), 2 * inter, hidden)
        b, sb = synth.fp8_block_weight(synth.config_seed(4, 600 + e), hidden, inter)
        host[e] = (a, sa, b, sb)
        w13[e].copy_(torch.from_numpy(a))
        s13[e].copy_(torch.from_numpy(sa))
        w2[e].copy_(torch.from_numpy(b))
        s2[e].copy_(torch.from_numpy(sb))
    layer = MoeFp8Layer(w13, s13, w2, s2, tokens, topk)
    layer.forward(to_dev(x), to_dev(ids), to_dev(wts))
    _sync()
    assert _flag(layer.flag) == 0
    np.testing.assert_array_equal(to_host(layer.offsets), o_ref)
    np.testing.assert_array_equal(to_host(layer.row_token), rt_ref)
    np.testing.assert_array_equal(to_host(layer.token_rows), tr_ref)
    y = to_host(layer.y)
    for e in cold:
        b, en = int(o_ref[e]), int(o_ref[e + 1])
        a, sa, bw, sb = host[e]
        ref = oracle.expert_fp8(np.ascontiguousarray(x[rt_ref[b:en]]), rw_ref[b:en], hidden, inter, a, sa, bw, sb)
        assert_close(oracle.bf16_bits_to_f32(y[b:en]), oracle.bf16_bits_to_f32(ref), f"expert {e} rows")
    hot = [int(e) for e in np.argsort(-counts, kind="stable")[:2]]
    for e in hot:
        b, en = int(o_ref[e]), int(o_ref[e + 1])
        n = en - b
        edges = [j for t in range(256, n, 256) for j in (t - 1, t)]
        pick = np.unique(np.concatenate([[0, 1, n - 2, n - 1], edges[:: max(1, len(edges) // 24)][:30],
                                         np.linspace(0, n - 1, 14).astype(np.int64)]))[:48]
        rows = b + pick
        hw = [t[e].cpu().numpy() for t in (w13, s13, w2, s2)]
        ref = oracle.expert_fp8(np.ascontiguousarray(x[rt_ref[rows]]), rw_ref[rows], hidden, inter, *hw)
        assert_close(oracle.bf16_bits_to_f32(y[rows]), oracle.bf16_bits_to_f32(ref), f"hot expert {e} sampled rows")


def test_moe_gemm_plain_output_forms_and_bad_segment(eng):
    """The plain-output MoE GEMM without a row gather (the down projection's
    form, one block per CU walking its XCD's tiles) and with an identity
    gather (one block per tile) give the same bits on the same segments:
    empty experts, a one-row expert, 8 x 16 tiles more than the GPU has CUs.
    Sampled rows of every segment match the oracle.  Offsets whose segment
    ends past the row capacity (its tile count runs to 2^25) raise bit 1,
    the rows outside the valid segment stay unwritten and the walk ends at
    the one-block-per-tile grid; a valid call afterwards gives the first
    result again."""
    import torch

    from pih_amd import linear

    experts, n, k, cap = 8, 4096, 1024, 4000
    counts = np.array([0, 900, 1, 0, 1300, 129, 700, 960], np.int64)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.uint32)
    assert off[-1] <= cap
    a = _codes(synth.config_seed(4, 9500), (cap, k))
    w = _codes(synth.config_seed(4, 9501), (experts, n, k))
    rng = np.random.default_rng(9502)
    sa = (rng.uniform(0.5, 2.0, (cap, k // 128)) / 448).astype(np.float32)
    sw = (rng.uniform(0.5, 2.0, (experts, n // 128, k // 128)) / 448).astype(np.float32)
    ad, sad, wd, swd = to_dev(a), to_dev(sa), to_dev(w), to_dev(sw)
    ident = to_dev(np.arange(cap, dtype=np.uint32))
    sentinel = 0x7FC1

    def call(offsets, gather):
        out = torch.full((cap + 64, n), sentinel, dtype=torch.int16, device="cuda")
        view = out[:cap].view(torch.bfloat16)
        _, flag = linear.moe_fp8_gemm(ad, sad, ident if gather else None, wd, swd, to_dev(offsets), cap,
                                      abi.SCALE_F32, abi.OUTPUT_BF16, out=view)
        _sync()
        return to_host(out).view(np.uint16), _flag(flag)

    walk, f_walk = call(off, False)
    tiled, f_tiled = call(off, True)
    assert f_walk == 0 and f_tiled == 0
    np.testing.assert_array_equal(walk, tiled)
    assert np.all(walk[off[-1]:] == sentinel)
    for e in range(experts):
        lo, hi = int(off[e]), int(off[e + 1])
        if hi == lo:
            continue
        rows = np.unique(np.array([lo, lo + 1, (lo + hi) // 2, hi - 2, hi - 1]).clip(lo, hi - 1))
        ref = oracle.fp8_gemm_f32(np.ascontiguousarray(a[rows]), np.ascontiguousarray(sa[rows]), w[e], sw[e])
        assert_close(oracle.bf16_bits_to_f32(walk[rows]), ref, f"expert {e} rows {lo}..{hi}")

    bad = off.copy()  # expert 1 keeps rows 0..900, expert 2 runs from 900 to 0xFFFF0000
    bad[3:] = 0xFFFF0000
    bad[-1] = cap
    for gather in (False, True):
        got, flag = call(bad, gather)
        assert flag & 1, (gather, flag)
        assert np.all(got[int(off[2]):] == sentinel), gather
        written = got[: int(off[2])]
        assert np.all((written == sentinel) | (written == walk[: int(off[2])])), gather

    again, f_again = call(off, False)
    assert f_again == 0
    np.testing.assert_array_equal(again, walk)

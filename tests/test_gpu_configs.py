"""GPU parity of every BASELINE configuration at its own shapes, through the
entries the bench times and a drop-in caller would call.

* the Qwen3-0.6B MLP block (x [16, 1024], gate/up [3072, 1024],
  down [1024, 3072]) against the reference's CPU composition, in full.
* Qwen3-8B BF16 prefill at M = 2048 on all seven projections
  (sampled rows against the oracle, every row through a row-sum checksum
  computed in float64 on the host), and decode M = 64 on the K = 12288 down
  projection (a column subset against the oracle).
* configs[3] and [4]: the whole MoE layer through launch_moe_layer at
  E = 256, top-8, H = 7168, I = 2048 (FP8 at T = 4096; MXFP4 at T = 64 and
  512 with e4m3 and bf16 activations).  Every expert outside a checked set
  has all-zero weights, so its rows are exactly zero while every kernel
  still runs over the full routed geometry; the layer's whole output is
  then the ordered sum of the checked experts' rows and is compared with
  the oracle chain over those experts.  The checked sets cover every kernel
  bucket: experts with <= 16 rows and 17-64 rows (MXFP4: the streaming
  kernel, fully unrolled at K = 7168 and 2048) and larger ones (the tiled
  kernels).
* Reference call geometries of the DeepSeek table: launch_fp8_gemm at
  1024 -> 32768 and 8192 -> 4096, launch_grouped_fp8_gemm at G = 8,
  N_g = 1024, K_g = 4096 (deepseek_attention_dense_primitives_test.cpp:
  93-106), including its store of a non-finite result.

Tolerance: max_rel <= 1e-2 (normwise) and cosine >= 0.9999 against the
fp32-accumulate oracle (tests/helpers.py); route plans and zero rows exact.
"""
import numpy as np
import pytest

import oracle
from pih_amd import abi, synth
from tests.helpers import assert_close, to_dev, to_host

pytestmark = pytest.mark.gpu

E, TOPK, H, I = 256, 8, 7168, 2048


@pytest.fixture(scope="module")
def eng():
    import torch

    from pih_amd.device import engine_stream

    oracle.set_threads(min(16, __import__("os").cpu_count() or 1))
    with engine_stream() as s:
        yield s
        torch.cuda.synchronize()


def _sync():
    import torch

    torch.cuda.synchronize()


def _flag(t) -> int:
    return int(t.item()) & 0xFFFFFFFF


def _pick(counts, lo, hi, n):
    """Up to n experts whose row count is in [lo, hi]: the smallest, the
    largest and evenly spaced ones between."""
    cand = [int(e) for e in np.argsort(counts, kind="stable") if lo <= counts[e] <= hi]
    if len(cand) <= n or n == 1:
        return cand[:n]
    return [cand[int(round(j * (len(cand) - 1) / (n - 1)))] for j in range(n)]


# ------------------------------------------------------------- configs[0]
def test_cfg1_qwen_mlp_block(eng):
    from pih_amd.linear import QwenMlpBlock

    m, hidden, inter = 16, 1024, 3072
    x = synth.bf16_normal(synth.config_seed(1, 0), (m, hidden))
    wg = synth.bf16_normal(synth.config_seed(1, 1), (inter, hidden), std=0.02)
    wu = synth.bf16_normal(synth.config_seed(1, 2), (inter, hidden), std=0.02)
    wd = synth.bf16_normal(synth.config_seed(1, 3), (hidden, inter), std=0.02)
    ref = oracle.qwen_mlp(x, wg, wu, wd)
    block = QwenMlpBlock(to_dev(wg), to_dev(wu), to_dev(wd), m)
    got = to_host(block.forward(to_dev(x)))
    _sync()
    # the intermediate h is bf16 in both; compare it too (one rounding apart
    # at most where the fp32 dots differ in their last bit)
    h_ref = oracle.silu_mul(oracle.f32_to_bf16_bits(oracle.bf16_gemm(x, wg)),
                            oracle.f32_to_bf16_bits(oracle.bf16_gemm(x, wu)))
    assert_close(oracle.bf16_bits_to_f32(to_host(block.h)), oracle.bf16_bits_to_f32(h_ref), "cfg1 silu_mul out")
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref), "cfg1 mlp block")


# ------------------------------------------------------------- configs[1]
QWEN8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
          ("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]


@pytest.mark.parametrize("name,n,k", QWEN8B)
def test_cfg2_prefill_m2048(eng, name, n, k):
    """M = 2048 (the MFMA GEMM): 48 rows spread over M against the oracle;
    all 2048 rows through sum_n C[m, n] = A[m, :] . (sum_n W[n, :]) in
    float64 (a plausible tile-indexing mistake moves whole rows or columns
    and shows in the checksum)."""
    from pih_amd.linear import bf16_gemm

    m = 2048
    a = synth.bf16_normal(synth.config_seed(2, 100 + n + k), (m, k))
    w = synth.bf16_normal(synth.config_seed(2, 200 + n + k), (n, k), std=0.02)
    got = oracle.bf16_bits_to_f32(to_host(bf16_gemm(to_dev(a), to_dev(w))))
    _sync()
    rows = np.unique(np.concatenate([np.arange(0, m, 47), [m - 1, 127, 128, 255, 256]]))
    ref = oracle.bf16_gemm(np.ascontiguousarray(a[rows]), w)
    assert_close(got[rows], ref, f"prefill {name} sampled rows")
    colsum = oracle.bf16_bits_to_f32(w).astype(np.float64).sum(axis=0)
    want = oracle.bf16_bits_to_f32(a).astype(np.float64) @ colsum
    have = got.astype(np.float64).sum(axis=1)
    # each output carries a bf16 rounding (2^-9 relative); their sum's error
    # is bounded by the sum of magnitudes times that
    bound = np.abs(got).astype(np.float64).sum(axis=1) * 2.0 ** -8 + 1e-3
    assert np.all(np.abs(have - want) <= bound), f"prefill {name} row checksums"


def test_cfg2_decode_m64_down_k12288(eng):
    """Decode M = 64 on the down projection (K = 12288): 512 output columns
    (a spread of weight rows incl. both ends of every 16-row block group)
    against the oracle, which takes seconds for the full 4096."""
    from pih_amd.linear import bf16_gemm

    m, n, k = 64, 4096, 12288
    a = synth.bf16_normal(synth.config_seed(2, 300), (m, k))
    w = synth.bf16_normal(synth.config_seed(2, 301), (n, k), std=0.02)
    got = oracle.bf16_bits_to_f32(to_host(bf16_gemm(to_dev(a), to_dev(w))))
    _sync()
    cols = np.unique(np.concatenate([np.arange(0, n, 9), np.arange(0, n, 256), np.arange(255, n, 256)]))[:512]
    ref = oracle.bf16_gemm(a, np.ascontiguousarray(w[cols]))
    assert_close(got[:, cols], ref, "decode m64 down")


# ------------------------------------------------------- configs[3] (FP8)
def _fp8_device_expert(torch, gen, rows, cols):
    """One expert's e4m3 weight from N(0, 0.02) quantised per 128x128 block
    with an fp32 scale amax/448, made on the device (as bench.py does)."""
    v = torch.randn(rows, cols, device="cuda", generator=gen) * 0.02
    blk = v.view(rows // 128, 128, cols // 128, 128)
    sc = blk.abs().amax(dim=(1, 3)).clamp_min(1e-12) / 448.0
    q = (blk / sc[:, None, :, None]).clamp(-448.0, 448.0).view(rows, cols)
    return q.to(torch.float8_e4m3fn).view(torch.uint8), sc


def test_cfg4_fp8_layer_full_shape(eng):
    """The bench's own entry (MoeLayer -> launch_moe_layer) at T = 4096 with
    the bench's routing: route plan bit-exact through the stage entry, the
    whole output against the oracle over 7 checked experts (1, 2-64 and
    128-700 rows: streaming tiles, single M tiles, multi-tile experts)."""
    import torch

    from pih_amd.linear import MoeLayer, route_plan

    T = 4096
    ids, wts = synth.zipf_router(synth.config_seed(4, 0), T, E, TOPK)
    x = synth.bf16_normal(synth.config_seed(4, 1), (T, H))
    o_ref, rt_ref, rw_ref, tr_ref = oracle.route_plan(ids, wts, E)
    counts = np.diff(o_ref.astype(np.int64))
    checked = _pick(counts, 1, 1, 1) + _pick(counts, 2, 64, 3) + _pick(counts, 128, 700, 3)
    assert len(checked) == 7
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4104)
    w13 = torch.zeros(E, 2 * I, H, dtype=torch.uint8, device="cuda")
    s13 = torch.ones(E, 2 * I // 128, H // 128, dtype=torch.float32, device="cuda")
    w2 = torch.zeros(E, H, I, dtype=torch.uint8, device="cuda")
    s2 = torch.ones(E, H // 128, I // 128, dtype=torch.float32, device="cuda")
    for e in checked:
        w13[e], s13[e] = _fp8_device_expert(torch, gen, 2 * I, H)
        w2[e], s2[e] = _fp8_device_expert(torch, gen, H, I)
    xd, idd, wtd = to_dev(x), to_dev(ids), to_dev(wts)
    o, rt, rw, tr, pflag = route_plan(idd, wtd, E)
    layer = MoeLayer(w13, s13, w2, s2, T, TOPK, scale_format=abi.SCALE_F32)
    got = to_host(layer.forward(xd, idd, wtd))
    _sync()
    assert _flag(layer.flag) == 0 and _flag(pflag) == 0
    np.testing.assert_array_equal(to_host(o), o_ref)
    np.testing.assert_array_equal(to_host(rt), rt_ref)
    np.testing.assert_array_equal(to_host(tr), tr_ref)
    y = np.zeros((T * TOPK, H), np.uint16)
    for e in checked:
        b, en = int(o_ref[e]), int(o_ref[e + 1])
        hw = [to_host(t[e]) for t in (w13, s13, w2, s2)]
        y[b:en] = oracle.expert_fp8(np.ascontiguousarray(x[rt_ref[b:en]]), rw_ref[b:en], H, I, *hw)
    ref = oracle.finalize(oracle.ordered_accumulate(y, rt_ref, T))
    touched = np.isin(ids, checked).any(axis=1)
    assert np.all(oracle.bf16_bits_to_f32(got[~touched]) == 0), "unchecked experts not zero"
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref), "cfg4 layer (checked experts)")


# ----------------------------------------------------- configs[4] (MXFP4)
@pytest.fixture(scope="module")
def mxfp4_zero_layer(eng):
    import torch

    w13 = torch.zeros(E, 2 * I, H // 2, dtype=torch.uint8, device="cuda")
    s13 = torch.full((E, 2 * I, H // 32), 127, dtype=torch.uint8, device="cuda")
    w2 = torch.zeros(E, H, I // 2, dtype=torch.uint8, device="cuda")
    s2 = torch.full((E, H, I // 32), 127, dtype=torch.uint8, device="cuda")
    yield w13, s13, w2, s2
    del w13, s13, w2, s2
    torch.cuda.empty_cache()


def _mx_ref_rows(act, xs, rw, w13p, w13s, w2p, w2s):
    if act == "e4m3":
        # the reference's routed-expert chain (clamp 10), W1 = gate rows, W3 = up rows
        return oracle.routed_expert_fp4(xs, rw, H, I, np.ascontiguousarray(w13p[:I]),
                                        np.ascontiguousarray(w13s[:I]), w2p, w2s,
                                        np.ascontiguousarray(w13p[I:]), np.ascontiguousarray(w13s[I:]))
    gu = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(oracle.mxfp4_bf16_gemm(xs, w13p, w13s)))
    act_v = oracle.swiglu(gu[:, :I], gu[:, I:], 0.0) * rw[:, None]
    mid = oracle.f32_to_bf16_bits(act_v.astype(np.float32))
    return oracle.f32_to_bf16_bits(oracle.mxfp4_bf16_gemm(np.ascontiguousarray(mid), w2p, w2s))


@pytest.mark.parametrize("tokens", [64, 512])
def test_cfg5_mxfp4_layer_full_shape(eng, mxfp4_zero_layer, tokens):
    """MoeLayer with MXFP4 weights at the bench's routing:
    e4m3 activations with the reference chain (clamp 10) and bf16
    activations with plain SiLU-mul.  Checked experts: <= 16 rows (the
    one-fragment streaming path), 17-64 rows (two 32-row chunks for bf16,
    full 64-row fragments for e4m3) and, at 512 tokens, > 64 rows (the tiled
    kernels)."""
    import torch

    from pih_amd.linear import MoeLayer

    w13, s13, w2, s2 = mxfp4_zero_layer
    ids, wts = synth.zipf_router(synth.config_seed(5, tokens), tokens, E, TOPK)
    x = synth.bf16_normal(synth.config_seed(5, tokens + 1), (tokens, H))
    o_ref, rt_ref, rw_ref, _ = oracle.route_plan(ids, wts, E)
    counts = np.diff(o_ref.astype(np.int64))
    checked = _pick(counts, 1, 16, 3) + _pick(counts, 17, 64, 3) + _pick(counts, 65, 200, 1)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5000 + tokens)
    host = {}
    for e in checked:
        w13[e] = torch.randint(0, 256, (2 * I, H // 2), dtype=torch.uint8, device="cuda", generator=gen)
        s13[e] = torch.randint(118, 125, (2 * I, H // 32), dtype=torch.uint8, device="cuda", generator=gen)
        w2[e] = torch.randint(0, 256, (H, I // 2), dtype=torch.uint8, device="cuda", generator=gen)
        s2[e] = torch.randint(118, 125, (H, I // 32), dtype=torch.uint8, device="cuda", generator=gen)
        host[e] = [to_host(t[e]) for t in (w13, s13, w2, s2)]
    xd, idd, wtd = to_dev(x), to_dev(ids), to_dev(wts)
    touched = np.isin(ids, checked).any(axis=1)
    try:
        for act, code, limit in (("e4m3", abi.ACTIVATION_E4M3, 10.0), ("bf16", abi.ACTIVATION_BF16, 0.0)):
            layer = MoeLayer(w13, s13, w2, s2, tokens, TOPK, weight_format=abi.WEIGHT_MXFP4,
                             activation_type=code, swiglu_limit=limit)
            got = to_host(layer.forward(xd, idd, wtd))
            _sync()
            assert _flag(layer.flag) == 0
            y = np.zeros((tokens * TOPK, H), np.uint16)
            for e in checked:
                b, en = int(o_ref[e]), int(o_ref[e + 1])
                y[b:en] = _mx_ref_rows(act, np.ascontiguousarray(x[rt_ref[b:en]]), rw_ref[b:en], *host[e])
            ref = oracle.finalize(oracle.ordered_accumulate(y, rt_ref, tokens))
            assert np.all(oracle.bf16_bits_to_f32(got[~touched]) == 0), f"{act}: unchecked experts not zero"
            assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref),
                         f"cfg5 T={tokens} {act} (experts {[(e, int(counts[e])) for e in checked]})")
            del layer
    finally:
        for e in checked:  # back to zero for the next parametrisation
            w13[e].zero_()
            w2[e].zero_()


# ----------------------------------------- reference call geometries (DeepSeek table)
def _codes(seed, shape):
    c = (synth.splitmix64(seed, int(np.prod(shape))) % np.uint64(254)).astype(np.uint8)
    return np.where(c >= 0x7F, c + 1, c).astype(np.uint8).reshape(shape)


@pytest.mark.parametrize("m,n,k", [(64, 32768, 1024), (512, 4096, 8192), (4096, 1024, 4096)])
def test_fp8_gemm_reference_call_shapes(eng, m, n, k):
    """launch_fp8_gemm (UE8M0) at call shapes of the reference's DeepSeek
    model (deepseek_fp8_gemm.cpp:5-20 validator; 1024 -> 32768,
    8192 -> 4096, 4096 -> 1024 at M up to 4096): 40 sampled rows against
    the oracle."""
    import torch

    from pih_amd.device import ptr, stream_handle

    a = _codes(synth.config_seed(4, 11000 + n), (m, k))
    w = _codes(synth.config_seed(4, 11100 + k), (n, k))
    sa = (118 + synth.splitmix64(11200 + m, m * (k // 128)) % np.uint64(6)).astype(np.uint8).reshape(m, k // 128)
    sw = (112 + synth.splitmix64(11300 + n, (n // 128) * (k // 128)) % np.uint64(6)).astype(np.uint8)
    sw = sw.reshape(n // 128, k // 128)
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ad, sad, wd, swd = to_dev(a), to_dev(sa), to_dev(w), to_dev(sw)
    r = abi.request(abi.DS["fp8_gemm"], activation_e4m3=ptr(ad), activation_scale_bits=ptr(sad),
                    weight_e4m3=ptr(wd), weight_scale_bits=ptr(swd), output=ptr(out), error_flag=ptr(flag),
                    stream=stream_handle(), m=m, n=n, k=k, output_type=1)
    st = abi.deepseek_pack().call("launch_fp8_gemm", r)
    assert st.code == abi.OK, st
    _sync()
    assert _flag(flag) == 0
    rows = np.unique(np.linspace(0, m - 1, 40).astype(np.int64))
    ref = oracle.fp8_gemm_ue8m0(np.ascontiguousarray(a[rows]), np.ascontiguousarray(sa[rows]), w, sw)
    got = oracle.bf16_bits_to_f32(to_host(out))[rows]
    assert_close(got, ref, f"fp8_gemm {m}x{n}x{k}")


def _grouped(x, w, sw, t, g, ng, kg):
    import torch

    from pih_amd.device import ptr, stream_handle

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
    return to_host(aq), to_host(out), _flag(flag)


@pytest.mark.parametrize("t", [64, 512])
def test_grouped_fp8_gemm_reference_geometry(eng, t):
    """The attention wo_a geometry of the reference (G = 8, N_g = 1024,
    K_g = 4096; deepseek_attention_dense_primitives_test.cpp:93-106) at 64
    tokens (the 128 x 128 kernel) and 512 (the big-tile kernel's strided
    problems): quantised activations bit-exact, the outputs of every token
    (64) or of 24 sampled tokens (512) against the oracle."""
    g, ng, kg = 8, 1024, 4096
    x = synth.bf16_normal(synth.config_seed(4, 12000), (t * g, kg))
    w = _codes(synth.config_seed(4, 12001), (g * ng, kg))
    sw = (112 + synth.splitmix64(12002, g * (ng // 128) * (kg // 128)) % np.uint64(6)).astype(np.uint8)
    sw = sw.reshape(g * ng // 128, kg // 128)
    aq, out, flag = _grouped(x, w, sw, t, g, ng, kg)
    assert flag == 0
    xq, xs = oracle.fp8_quant_ue8m0(oracle.bf16_bits_to_f32(x))
    np.testing.assert_array_equal(aq, xq)
    toks = np.arange(t) if t <= 64 else np.unique(np.linspace(0, t - 1, 24).astype(np.int64))
    ref = np.empty((len(toks), g * ng), np.float32)
    for gi in range(g):
        rows = toks * g + gi
        ref[:, gi * ng:(gi + 1) * ng] = oracle.fp8_gemm_ue8m0(
            np.ascontiguousarray(xq[rows]), np.ascontiguousarray(xs[rows]),
            np.ascontiguousarray(w[gi * ng:(gi + 1) * ng]), np.ascontiguousarray(sw[gi * ng // 128:(gi + 1) * ng // 128]))
    assert_close(oracle.bf16_bits_to_f32(out)[toks], ref, f"grouped fp8 8/1024/4096 at {t} tokens")


@pytest.mark.parametrize("t,ng", [(2, 128), (256, 1024)])
def test_grouped_fp8_gemm_stores_nonfinite(eng, t, ng):
    """As the reference's grouped kernel does (deepseek_attention_dense_
    primitives.cu:247-249): a non-finite sum raises 2048 and its bf16 value
    is stored; finite elements are untouched by it (small-M kernel at 2
    tokens, big-tile kernel at 256 tokens x 1024 columns)."""
    g, kg = 8, 128
    x = synth.bf16_normal(synth.config_seed(4, 12100), (t * g, kg))
    x[:, 0] = 0x4380  # 256.0 in every row: group amax >= 256
    w = np.zeros((g * ng, kg), np.uint8)
    w[:, 0] = 0x7E  # 448
    sw = np.full((g * ng // 128, kg // 128), 127, np.uint8)
    sw[3 * ng // 128:4 * ng // 128, 0] = 254  # group 3: 2^127 scale, the sum overflows
    _, out, flag = _grouped(x, w, sw, t, g, ng, kg)
    assert flag == 2048
    vals = oracle.bf16_bits_to_f32(out).reshape(t, g, ng)
    assert np.all(np.isinf(vals[:, 3])) and np.all(np.isfinite(np.delete(vals, 3, axis=1)))


# ------------------------------- DeepSeek-V4-Flash geometry (the reference's own)
V4_H, V4_I, V4_TOPK = 4096, 2048, 6


@pytest.fixture(scope="module")
def v4_zero_layer(eng):
    import torch

    w13 = torch.zeros(E, 2 * V4_I, V4_H // 2, dtype=torch.uint8, device="cuda")
    s13 = torch.full((E, 2 * V4_I, V4_H // 32), 127, dtype=torch.uint8, device="cuda")
    w2 = torch.zeros(E, V4_H, V4_I // 2, dtype=torch.uint8, device="cuda")
    s2 = torch.full((E, V4_H, V4_I // 32), 127, dtype=torch.uint8, device="cuda")
    yield w13, s13, w2, s2
    del w13, s13, w2, s2
    torch.cuda.empty_cache()


def v4_router_inputs(tokens: int):
    """Router logits ~N(0, 1) and a selection bias that sends most tokens
    to a few experts (so one layer holds light and multi-tile experts)."""
    raw = synth.normal(synth.config_seed(6, tokens), tokens * E).astype(np.float32).reshape(tokens, E)
    bias = (0.05 * synth.normal(synth.config_seed(6, 1), E)).astype(np.float32)
    bias[[3, 77, 140]] += np.float32(1.5)
    return raw, bias


@pytest.mark.parametrize("tokens", [64, 512])
def test_v4_flash_mxfp4_layer(eng, v4_zero_layer, tokens):
    """The reference's production MoE geometry (include/pih/model/
    deepseek_v4_config.h:22-27: hidden 4096, 256 routed experts, 6 active;
    expert intermediate 2048): the device V4 router (sqrt-softplus + bias
    selection, weights x 1.5, learned_router.cpp:21-105) feeds the layer
    entry with MXFP4 experts and e4m3 activations, at decode batches of 64
    and 512 tokens.  The router's ids equal the oracle's and its weights
    agree to rtol 1e-5 (device expf / log1pf / sqrtf against the host's, as
    in tests/test_gpu_router.py); the chain below takes the device's
    weights.  Every expert outside a checked set has zero weights, and the
    layer's output equals the reference's routed-expert chain (clamp 10)
    over the checked experts, which cover <= 16 rows, 17-64 rows (the
    streaming kernel, fully unrolled at K = 4096 and 2048) and, at 512
    tokens, a multi-tile expert."""
    import torch

    from pih_amd.linear import MoeLayer, router_topk

    H, I = V4_H, V4_I
    w13, s13, w2, s2 = v4_zero_layer
    raw, bias = v4_router_inputs(tokens)
    ids_d, wts_d, rflag = router_topk(to_dev(raw), V4_TOPK, abi.ROUTER_SQRT_SOFTPLUS, 1.5, to_dev(bias))
    _sync()
    ids, wts = to_host(ids_d).view(np.uint32), to_host(wts_d)
    rid, rw = oracle.router_topk(raw, V4_TOPK, oracle.ROUTER_SQRT_SOFTPLUS, 1.5, bias)
    assert _flag(rflag) == 0
    np.testing.assert_array_equal(ids, rid)
    np.testing.assert_allclose(wts, rw, rtol=1e-5, atol=0)
    x = synth.bf16_normal(synth.config_seed(6, tokens + 1), (tokens, H))
    o_ref, rt_ref, rw_ref, _ = oracle.route_plan(rid, wts, E)
    counts = np.diff(o_ref.astype(np.int64))
    checked = _pick(counts, 1, 16, 3) + _pick(counts, 17, 64, 2) + _pick(counts, 65, 4096, 1)
    if tokens >= 512:
        assert any(counts[e] > 64 for e in checked), counts.max()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(6000 + tokens)
    host = {}
    for e in checked:
        w13[e] = torch.randint(0, 256, (2 * I, H // 2), dtype=torch.uint8, device="cuda", generator=gen)
        s13[e] = torch.randint(118, 125, (2 * I, H // 32), dtype=torch.uint8, device="cuda", generator=gen)
        w2[e] = torch.randint(0, 256, (H, I // 2), dtype=torch.uint8, device="cuda", generator=gen)
        s2[e] = torch.randint(118, 125, (H, I // 32), dtype=torch.uint8, device="cuda", generator=gen)
        host[e] = [to_host(t[e]) for t in (w13, s13, w2, s2)]
    try:
        layer = MoeLayer(w13, s13, w2, s2, tokens, V4_TOPK, weight_format=abi.WEIGHT_MXFP4,
                         activation_type=abi.ACTIVATION_E4M3, swiglu_limit=10.0)
        got = to_host(layer.forward(to_dev(x), ids_d, wts_d))
        _sync()
        assert _flag(layer.flag) == 0
        y = np.zeros((tokens * V4_TOPK, H), np.uint16)
        for e in checked:
            b, en = int(o_ref[e]), int(o_ref[e + 1])
            w13p, w13s, w2p, w2s = host[e]
            y[b:en] = oracle.routed_expert_fp4(np.ascontiguousarray(x[rt_ref[b:en]]), rw_ref[b:en], H, I,
                                               np.ascontiguousarray(w13p[:I]), np.ascontiguousarray(w13s[:I]), w2p,
                                               w2s, np.ascontiguousarray(w13p[I:]), np.ascontiguousarray(w13s[I:]))
        ref = oracle.finalize(oracle.ordered_accumulate(y, rt_ref, tokens))
        touched = np.isin(rid, checked).any(axis=1)
        assert np.all(oracle.bf16_bits_to_f32(got[~touched]) == 0), "unchecked experts not zero"
        assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref),
                     f"V4-Flash T={tokens} (experts {[(e, int(counts[e])) for e in checked]})")
    finally:
        for e in checked:
            w13[e].zero_()
            w2[e].zero_()

"""The whole MoE expert layer through the pack's C++ layer entry
(`launch_moe_layer`), FP8 and MXFP4 weights.

* FP8: the native layer must equal the six stage entries launched one by one
  (MoeFp8Layer) bit for bit, and the CPU oracle within tolerance.
* MXFP4 with e4m3 activations: each routed expert follows the reference's
  routed-expert chain (src/model/deepseek_routed_expert_oracle.cpp:50-95:
  UE8M0 quant -> FP4 GEMM W1/W3 -> bf16 -> SwiGLU clamp 10 -> x route weight
  -> bf16 -> quant -> FP4 GEMM W2 -> bf16), restated as
  oracle.routed_expert_fp4, then the ordered accumulate of
  deepseek_expert_accumulator_oracle.cpp: the composed per-expert pipeline
  of the reference's DeepSeekExpertCudaBackend, in one call.
* MXFP4 with bf16 activations: the same chain with exact MXFP4 decode x bf16
  GEMMs (oracle.mxfp4_bf16_gemm) and no quant stages.
Tolerance: max_rel <= 1e-2 normwise and cosine >= 0.9999 (tests/helpers.py).
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

    torch.cuda.synchronize()


def _flag(t) -> int:
    return int(t.item()) & 0xFFFFFFFF


def _fp8_weights(experts, hidden, inter, base, ue8m0=False):
    make = synth.ue8m0_block_weight if ue8m0 else synth.fp8_block_weight
    sdt = np.uint8 if ue8m0 else np.float32
    w13 = np.empty((experts, 2 * inter, hidden), np.uint8)
    s13 = np.empty((experts, 2 * inter // 128, hidden // 128), sdt)
    w2 = np.empty((experts, hidden, inter), np.uint8)
    s2 = np.empty((experts, hidden // 128, inter // 128), sdt)
    for e in range(experts):
        w13[e], s13[e] = make(synth.config_seed(4, base + e), 2 * inter, hidden)
        w2[e], s2[e] = make(synth.config_seed(4, base + 500 + e), hidden, inter)
    return w13, s13, w2, s2


@pytest.mark.parametrize("tokens,experts,topk,hidden,inter,limit,ue8m0",
                         [(64, 8, 2, 256, 256, 0.0, False), (300, 16, 4, 512, 256, 10.0, False),
                          (130, 8, 3, 384, 256, 0.0, True)])
def test_native_fp8_layer_equals_stages(eng, tokens, experts, topk, hidden, inter, limit, ue8m0):
    from pih_amd.linear import MoeFp8Layer, MoeLayer

    fmt = abi.SCALE_UE8M0 if ue8m0 else abi.SCALE_F32
    ids, wts = synth.zipf_router(synth.config_seed(4, 9500 + tokens), tokens, experts, topk)
    x = synth.bf16_normal(synth.config_seed(4, 9501), (tokens, hidden))
    shared = synth.bf16_normal(synth.config_seed(4, 9502), (tokens, hidden))
    w13, s13, w2, s2 = [to_dev(t) for t in _fp8_weights(experts, hidden, inter, 9600, ue8m0)]
    xd, idd, wtd, shd = to_dev(x), to_dev(ids), to_dev(wts), to_dev(shared)
    staged = MoeFp8Layer(w13, s13, w2, s2, tokens, topk, swiglu_limit=limit, scale_format=fmt)
    ref = to_host(staged.forward(xd, idd, wtd, shared=shd)).copy()
    native = MoeLayer(w13, s13, w2, s2, tokens, topk, scale_format=fmt, swiglu_limit=limit)
    got = to_host(native.forward(xd, idd, wtd, shared=shd))
    _sync()
    assert _flag(staged.flag) == 0 and _flag(native.flag) == 0
    np.testing.assert_array_equal(got, ref)
    if not ue8m0:
        hw = [to_host(t) for t in (w13, s13, w2, s2)]
        o_ref, _, _ = oracle.moe_fp8_forward(x, ids, wts, experts, hidden, inter, *hw, limit)
        acc = oracle.bf16_bits_to_f32(o_ref) + oracle.bf16_bits_to_f32(shared)
        assert_close(oracle.bf16_bits_to_f32(got), acc, "native fp8 layer vs oracle (+shared)")


def _mxfp4_weights(experts, hidden, inter, base):
    w1 = [synth.mxfp4_weight(synth.config_seed(5, base + e), inter, hidden) for e in range(experts)]
    w3 = [synth.mxfp4_weight(synth.config_seed(5, base + 300 + e), inter, hidden) for e in range(experts)]
    w2 = [synth.mxfp4_weight(synth.config_seed(5, base + 600 + e), hidden, inter) for e in range(experts)]
    w13p = np.stack([np.concatenate([a[0], b[0]]) for a, b in zip(w1, w3)])
    w13s = np.stack([np.concatenate([a[1], b[1]]) for a, b in zip(w1, w3)])
    w2p = np.stack([p for p, _ in w2])
    w2s = np.stack([s for _, s in w2])
    return w1, w3, w2, (w13p, w13s, w2p, w2s)


def _combine(y, row_token, tokens):
    return oracle.finalize(oracle.ordered_accumulate(y, row_token, tokens))


def test_native_mxfp4_layer_e4m3_follows_reference_expert_chain(eng):
    from pih_amd.linear import MoeLayer

    tokens, experts, topk, hidden, inter = 48, 8, 2, 256, 256
    ids, wts = synth.zipf_router(synth.config_seed(5, 9700), tokens, experts, topk)
    x = synth.bf16_normal(synth.config_seed(5, 9701), (tokens, hidden))
    w1, w3, w2, fused = _mxfp4_weights(experts, hidden, inter, 9800)
    layer = MoeLayer(*[to_dev(t) for t in fused], tokens, topk, weight_format=abi.WEIGHT_MXFP4,
                     activation_type=abi.ACTIVATION_E4M3, swiglu_limit=10.0)
    got = to_host(layer.forward(to_dev(x), to_dev(ids), to_dev(wts)))
    _sync()
    assert _flag(layer.flag) == 0
    offsets, row_token, row_weight, _ = oracle.route_plan(ids, wts, experts)
    y = np.zeros((tokens * topk, hidden), np.uint16)
    for e in range(experts):
        b, en = int(offsets[e]), int(offsets[e + 1])
        if b == en:
            continue
        y[b:en] = oracle.routed_expert_fp4(np.ascontiguousarray(x[row_token[b:en]]), row_weight[b:en], hidden, inter,
                                           w1[e][0], w1[e][1], w2[e][0], w2[e][1], w3[e][0], w3[e][1])
    ref = _combine(y, row_token, tokens)
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref), "mxfp4 e4m3 layer vs expert chain")


def test_native_mxfp4_layer_bf16_activations(eng):
    from pih_amd.linear import MoeLayer

    tokens, experts, topk, hidden, inter = 40, 6, 2, 256, 128
    ids, wts = synth.zipf_router(synth.config_seed(5, 9900), tokens, experts, topk)
    x = synth.bf16_normal(synth.config_seed(5, 9901), (tokens, hidden))
    _, _, _, fused = _mxfp4_weights(experts, hidden, inter, 9950)
    w13p, w13s, w2p, w2s = fused
    layer = MoeLayer(*[to_dev(t) for t in fused], tokens, topk, weight_format=abi.WEIGHT_MXFP4,
                     activation_type=abi.ACTIVATION_BF16, swiglu_limit=0.0)
    got = to_host(layer.forward(to_dev(x), to_dev(ids), to_dev(wts)))
    _sync()
    assert _flag(layer.flag) == 0
    offsets, row_token, row_weight, _ = oracle.route_plan(ids, wts, experts)
    y = np.zeros((tokens * topk, hidden), np.uint16)
    for e in range(experts):
        b, en = int(offsets[e]), int(offsets[e + 1])
        if b == en:
            continue
        xs = np.ascontiguousarray(x[row_token[b:en]])
        gu = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(oracle.mxfp4_bf16_gemm(xs, w13p[e], w13s[e])))
        act = oracle.swiglu(gu[:, :inter], gu[:, inter:], 0.0) * row_weight[b:en, None]
        mid = oracle.f32_to_bf16_bits(act.astype(np.float32))
        y[b:en] = oracle.f32_to_bf16_bits(oracle.mxfp4_bf16_gemm(np.ascontiguousarray(mid), w2p[e], w2s[e]))
    ref = _combine(y, row_token, tokens)
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref), "mxfp4 bf16 layer")


def test_layer_query_and_request_checks(eng):
    """Workspace query, a too-small workspace and bad shapes are refused
    before anything is enqueued."""
    import torch

    from pih_amd.device import ptr, stream_handle
    L = abi.linear_pack()
    need = (abi.C.c_uint64 * 1)()
    q = abi.request(abi.LN["moe_layer"], required_bytes_u64=abi.C.addressof(need), token_count=64, top_k=2,
                    expert_count=8, hidden_size=256, intermediate_size=256, weight_format=abi.WEIGHT_FP8,
                    scale_format=abi.SCALE_F32, activation_type=0)
    assert L.call("query_moe_layer_workspace", q).code == abi.OK and need[0] > 0
    q.hidden_size = 200
    assert L.call("query_moe_layer_workspace", q).code == abi.INVALID_ARGUMENT
    buf = torch.zeros(16, dtype=torch.uint8, device="cuda")
    r = abi.request(abi.LN["moe_layer"], input_bf16=ptr(buf), topk_ids_u32=ptr(buf), topk_weights_f32=ptr(buf),
                    w13=ptr(buf), w13_scale=ptr(buf), w2=ptr(buf), w2_scale=ptr(buf), output_bf16=ptr(buf),
                    workspace=ptr(buf), workspace_bytes=16, error_flag_u32=ptr(buf), stream=stream_handle(),
                    token_count=64, top_k=2, expert_count=8, hidden_size=256, intermediate_size=256,
                    weight_format=abi.WEIGHT_FP8, scale_format=abi.SCALE_F32)
    assert L.call("launch_moe_layer", r).code == abi.INVALID_ARGUMENT  # workspace too small
    r.weight_format = 9
    assert L.call("launch_moe_layer", r).code == abi.INVALID_ARGUMENT


@pytest.mark.parametrize("tokens,experts,topk,limit,ue8m0",
                         [(200, 8, 2, 0.0, False), (300, 16, 4, 10.0, False), (130, 8, 3, 0.0, True)])
def test_swiglu_e4m3_output_equals_bf16_then_quant(eng, tokens, experts, topk, limit, ue8m0):
    """The gate/up GEMM's quantising epilogue (OUTPUT_SWIGLU_E4M3) writes the
    codes and scales the quant entry produces from its bf16 SwiGLU output,
    bit for bit (routed rows only; rows past offsets[E] are not written)."""
    from pih_amd import linear

    hidden, inter = 512, 256
    fmt = abi.SCALE_UE8M0 if ue8m0 else abi.SCALE_F32
    ids, wts = synth.zipf_router(synth.config_seed(4, 9700 + tokens), tokens, experts, topk)
    x = synth.bf16_normal(synth.config_seed(4, 9701), (tokens, hidden))
    w13, s13, _, _ = [to_dev(t) for t in _fp8_weights(experts, hidden, inter, 9800, ue8m0)]
    off, rt, rw, _ = oracle.route_plan(ids, wts, experts)
    rows = tokens * topk
    xq, xs, flag0 = linear.fp8_quant(to_dev(x), fmt)
    args = (xq, xs, to_dev(rt), w13, s13, to_dev(off), rows, fmt)
    mid, flag1 = linear.moe_fp8_gemm(*args, abi.OUTPUT_SWIGLU_BF16, row_weight=to_dev(rw), swiglu_limit=limit)
    q_ref, s_ref, flag2 = linear.fp8_quant(mid, fmt)
    (q, s), flag3 = linear.moe_fp8_gemm(*args, abi.OUTPUT_SWIGLU_E4M3, row_weight=to_dev(rw), swiglu_limit=limit)
    _sync()
    assert [_flag(f) for f in (flag0, flag1, flag2, flag3)] == [0, 0, 0, 0]
    n = int(off[-1])
    np.testing.assert_array_equal(to_host(q)[:n], to_host(q_ref)[:n])
    np.testing.assert_array_equal(to_host(s)[:n], to_host(s_ref)[:n])


def test_swiglu_e4m3_output_flags_nonfinite(eng):
    """Weight scales that overflow the gate/up products: both SwiGLU output
    kinds raise the non-finite bit (4) and nothing else."""
    from pih_amd import linear

    tokens, experts, topk, hidden, inter = 64, 8, 2, 256, 256
    fmt = abi.SCALE_F32
    ids, wts = synth.zipf_router(synth.config_seed(4, 9900), tokens, experts, topk)
    x = synth.bf16_normal(synth.config_seed(4, 9901), (tokens, hidden))
    w13, s13, _, _ = _fp8_weights(experts, hidden, inter, 9902, False)
    s13 = np.full_like(s13, 3.0e38)
    off, rt, rw, _ = oracle.route_plan(ids, wts, experts)
    xq, xs, _ = linear.fp8_quant(to_dev(x), fmt)
    args = (xq, xs, to_dev(rt), to_dev(w13), to_dev(s13), to_dev(off), tokens * topk, fmt)
    _, f_bf16 = linear.moe_fp8_gemm(*args, abi.OUTPUT_SWIGLU_BF16, row_weight=to_dev(rw))
    _, f_e4m3 = linear.moe_fp8_gemm(*args, abi.OUTPUT_SWIGLU_E4M3, row_weight=to_dev(rw))
    _sync()
    assert _flag(f_bf16) == 4 and _flag(f_e4m3) == 4

"""GPU tests of the on-disk formats feeding the kernels:

* a canonical Qwen3 INT4 artifact (written by tests/artifact_files.py,
  whose metadata is pinned to the reference serialiser) is verified,
  uploaded with one copy and its projections run through the W4A16
  symmetric entry and the Qwen code object's by-name compat kernel, against
  the oracle (po_w4a16_sym) on the same file bytes;
* DeepSeek expert bundles on the device are bound (reference Bind offsets),
  repacked into the grouped MoE weights, checked byte for byte, and the
  MXFP4 MoE layer over them follows the reference's routed-expert chain
  (oracle.routed_expert_fp4 on the bundle's W1/W3/W2 host bytes).
Tolerance: max_rel <= 1e-2, cos >= 0.9999 (tests/helpers.py).
"""
import numpy as np
import pytest

import oracle
from pih_amd import abi, synth
from tests import artifact_files as af
from tests.helpers import assert_close, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    import torch

    from pih_amd.device import engine_stream

    with engine_stream() as s:
        yield s
        torch.cuda.synchronize()


PROJ = {"model.layers.0.mlp.gate_proj.weight": (3072, 1024), "model.layers.13.mlp.down_proj.weight": (1024, 3072),
        "model.layers.27.self_attn.q_proj.weight": (2048, 1024)}


@pytest.fixture(scope="module")
def qwen_file(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("qwen") / "qwen3-0.6b-int4.xing")
    payloads, host = {}, {}
    for seed, (src, (n, k)) in enumerate(PROJ.items()):
        packed, scales = af.int4_linear_payloads(100 + seed, src, n, k)
        payloads[src + ".packed_values"], payloads[src + ".scales"] = packed, scales
        host[src] = (np.frombuffer(packed, np.uint8).reshape(n, k // 2),
                     np.frombuffer(scales, np.uint16).reshape(n, k // 128))
    # any finite bf16 bit pattern (bit 14 clear keeps the exponent below all-ones)
    emb = (np.random.default_rng(7000).integers(0, 1 << 16, size=(151936, 1024)) & 0xBFFF).astype(np.uint16)
    payloads["model.embed_tokens.weight"] = emb.tobytes()
    af.write_qwen_artifact(path, payloads)
    return path, host, emb


def test_qwen_artifact_upload_and_views(eng, qwen_file):
    import torch

    from pih_amd.artifacts import QwenInt4Artifact

    path, host, emb = qwen_file
    art = QwenInt4Artifact(path)
    torch.cuda.synchronize()
    for src, (packed, scales) in host.items():
        q, s = art.linear(src)
        assert np.array_equal(q.cpu().numpy(), packed)
        assert np.array_equal(s.view(torch.int16).cpu().numpy().view(np.uint16), scales)
    head = art.tensor("lm_head.weight")
    assert head.data_ptr() == art.tensor("model.embed_tokens.weight").data_ptr()
    assert np.array_equal(to_host(head[::997]), emb[::997])
    assert not art.tensor("model.norm.weight").view(torch.int16).any()


@pytest.mark.parametrize("m", [1, 4, 16])
def test_qwen_artifact_w4a16_entry(eng, qwen_file, m):
    import torch

    from pih_amd.artifacts import QwenInt4Artifact
    from pih_amd.device import ptr, stream_handle

    path, host, _ = qwen_file
    art = QwenInt4Artifact(path, verify_payloads=False)
    for src, (n, k) in PROJ.items():
        q, s = art.linear(src)
        x = synth.bf16_normal(synth.config_seed(3, 7100 + m + n), (m, k))
        out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        flag = torch.zeros(1, dtype=torch.int32, device="cuda")
        xd = to_dev(x)
        r = abi.request(abi.LN["w4a16"], input_bf16=ptr(xd), qweight=ptr(q), scales=ptr(s), zeros=0,
                        output_bf16=ptr(out), workspace=0, workspace_bytes=0, error_flag_u32=ptr(flag),
                        stream=stream_handle(), m=m, n=n, k=k, format=abi.W4A16_SYMMETRIC)
        assert abi.linear_pack().call("launch_w4a16_gemm", r).code == abi.OK
        torch.cuda.synchronize()
        assert int(flag.item()) == 0
        ref = oracle.w4a16_sym(x, *host[src])
        assert_close(oracle.bf16_bits_to_f32(to_host(out)), oracle.bf16_bits_to_f32(ref), f"artifact {src} m={m}")


def test_qwen_artifact_code_object_compat(eng, qwen_file):
    """The model's by-name kernel (pih_qwen_w4a16_gemm_compat_v1) over the
    artifact's device views, at the 0.6B shapes."""
    import torch

    from pih_amd.artifacts import QwenInt4Artifact
    from pih_amd.qwen import QwenCodeObject

    path, host, _ = qwen_file
    art = QwenInt4Artifact(path, verify_payloads=False)
    co = QwenCodeObject()
    s = torch.cuda.current_stream()
    for src, (n, k) in PROJ.items():
        q, sc = art.linear(src)
        x = synth.bf16_normal(synth.config_seed(3, 7200 + n), (2, k))
        xd = to_dev(x)
        out = torch.empty(2, n, dtype=torch.bfloat16, device="cuda")
        flag = torch.zeros(1, dtype=torch.int32, device="cuda")
        co.w4a16_gemm(xd.data_ptr(), q.data_ptr(), sc.data_ptr(), out.data_ptr(), flag.data_ptr(), 2, n, k,
                      s.cuda_stream)
        s.synchronize()
        assert int(flag.item()) == 0
        ref = oracle.w4a16_sym(x, *host[src])
        assert_close(oracle.bf16_bits_to_f32(to_host(out)), oracle.bf16_bits_to_f32(ref), f"compat {src}")


H, I = 4096, 2048


def _bundle(seed):
    """One expert bundle in host memory: the six segments in Bind order
    (W1 packed, W1 scales, W2 packed, W2 scales, W3 packed, W3 scales)."""
    w1p, w1s = synth.mxfp4_weight(synth.config_seed(5, seed), I, H)
    w2p, w2s = synth.mxfp4_weight(synth.config_seed(5, seed + 1), H, I)
    w3p, w3s = synth.mxfp4_weight(synth.config_seed(5, seed + 2), I, H)
    parts = (w1p, w1s, w2p, w2s, w3p, w3s)
    return np.concatenate([np.ascontiguousarray(p).ravel() for p in parts]), parts


def test_expert_bundles_to_moe_layer(eng):
    import torch

    from pih_amd import artifacts
    from pih_amd.linear import MoeLayer

    experts, tokens, topk = 3, 24, 2
    bundles = [_bundle(11000 + 10 * e) for e in range(experts)]
    dev = torch.empty(experts * artifacts.BUNDLE_BYTES, dtype=torch.uint8, device="cuda")
    for e, (flat, _) in enumerate(bundles):
        assert flat.size == artifacts.BUNDLE_BYTES
        dev[e * artifacts.BUNDLE_BYTES:(e + 1) * artifacts.BUNDLE_BYTES] = torch.from_numpy(flat).cuda()
    bases = [dev.data_ptr() + e * artifacts.BUNDLE_BYTES for e in range(experts)]
    for e, (_, parts) in enumerate(bundles):  # Bind spans address the right bytes
        v = artifacts.bind_expert_bundle(bases[e])
        w3s = torch.empty(v.scale_bytes, dtype=torch.uint8, device="cuda")
        w3s.copy_(dev[v.w3_scales - dev.data_ptr():v.w3_scales - dev.data_ptr() + v.scale_bytes])
        assert np.array_equal(w3s.cpu().numpy(), parts[5].ravel())
    w13 = torch.empty(experts, 2 * I, H // 2, dtype=torch.uint8, device="cuda")
    w13s = torch.empty(experts, 2 * I, H // 32, dtype=torch.uint8, device="cuda")
    w2 = torch.empty(experts, H, I // 2, dtype=torch.uint8, device="cuda")
    w2s = torch.empty(experts, H, I // 32, dtype=torch.uint8, device="cuda")
    artifacts.bundles_to_moe(bases, w13, w13s, w2, w2s)
    torch.cuda.synchronize()
    for e, (_, (w1p, w1s_, w2p, w2s_, w3p, w3s_)) in enumerate(bundles):
        assert np.array_equal(w13[e].cpu().numpy(), np.concatenate([w1p, w3p]))
        assert np.array_equal(w13s[e].cpu().numpy(), np.concatenate([w1s_, w3s_]))
        assert np.array_equal(w2[e].cpu().numpy(), w2p) and np.array_equal(w2s[e].cpu().numpy(), w2s_)
    ids, wts = synth.zipf_router(synth.config_seed(5, 11500), tokens, experts, topk)
    x = synth.bf16_normal(synth.config_seed(5, 11501), (tokens, H))
    layer = MoeLayer(w13, w13s, w2, w2s, tokens, topk, weight_format=abi.WEIGHT_MXFP4,
                     activation_type=abi.ACTIVATION_E4M3, swiglu_limit=10.0)
    got = to_host(layer.forward(to_dev(x), to_dev(ids), to_dev(wts)))
    torch.cuda.synchronize()
    assert int(layer.flag.item()) == 0
    offsets, row_token, row_weight, _ = oracle.route_plan(ids, wts, experts)
    y = np.zeros((tokens * topk, H), np.uint16)
    for e, (_, (w1p, w1s_, w2p, w2s_, w3p, w3s_)) in enumerate(bundles):
        b, en = int(offsets[e]), int(offsets[e + 1])
        if b < en:
            y[b:en] = oracle.routed_expert_fp4(np.ascontiguousarray(x[row_token[b:en]]), row_weight[b:en], H, I,
                                               w1p, w1s_, w2p, w2s_, w3p, w3s_)
    ref = oracle.finalize(oracle.ordered_accumulate(y, row_token, tokens))
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref), "bundle MoE layer vs expert chain")

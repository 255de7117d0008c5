"""GPU parity of the small-M GEMM path (gemm_small_m.hip): the dense FP8
GEMM (UE8M0 through the DeepSeek table, fp32 scales through the linear
pack), the FP4 x FP8 GEMM and the grouped FP8 GEMM with at most 64
activation rows, and with up to 256 rows in 64-row chunks where the
128 x 128 tiles would be fewer than 128 (M = 65..256 at N <= 4096), which
stream their weights over 16-row blocks instead of the tiles.  Every output
is checked against the CPU oracle (max_rel <= 1e-2 normwise, cosine >=
0.9999), across the activation-block counts (1, 2 and 4 blocks of 16 rows),
chunk counts 2-4 with a short last chunk, K splits with equal and unequal
runs per wave, runs of several batches (K = 12288 past 16 rows), the tiled
fallback (M = 65..256 at N = 128, K = 12288: one tile), and the error bits
of the reference kernels (NaN code 1, scale 0xFF 2, non-finite
result 4: the element is skipped, as deepseek_fp8_gemm.cu:67-70 skips
it)."""
import numpy as np
import pytest

import oracle
from pih_amd import abi, synth
from tests.helpers import assert_close, to_dev, to_host

pytestmark = pytest.mark.gpu

SENTINEL = 0x7FC1  # a bf16 NaN no kernel writes


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


def _codes(seed, shape):
    c = (synth.splitmix64(seed, int(np.prod(shape))) % np.uint64(254)).astype(np.uint8)
    return np.where(c >= 0x7F, c + 1, c).astype(np.uint8).reshape(shape)


def _ds_fp8(a, sa, w, sw, out_type=1):
    import torch

    from pih_amd.device import ptr, stream_handle

    m, k = a.shape
    n = w.shape[0]
    out = torch.full((m, n), SENTINEL, dtype=torch.int16, device="cuda")
    if out_type == 2:
        out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ad, sad, wd, swd = to_dev(a), to_dev(sa), to_dev(w), to_dev(sw)
    r = abi.request(abi.DS["fp8_gemm"], activation_e4m3=ptr(ad), activation_scale_bits=ptr(sad),
                    weight_e4m3=ptr(wd), weight_scale_bits=ptr(swd), output=ptr(out), error_flag=ptr(flag),
                    stream=stream_handle(), m=m, n=n, k=k, output_type=out_type)
    st = abi.deepseek_pack().call("launch_fp8_gemm", r)
    assert st.code == abi.OK, st
    _sync()
    got = out.cpu().numpy()
    return (got.view(np.uint16) if out_type == 1 else got), int(flag.item()) & 0xFFFFFFFF


def _fp8_inputs(seed, m, n, k):
    a = _codes(seed, (m, k))
    w = _codes(seed + 1, (n, k))
    sa = (118 + synth.splitmix64(seed + 2, m * (k // 128)) % np.uint64(6)).astype(np.uint8).reshape(m, k // 128)
    sw = (110 + synth.splitmix64(seed + 3, (n // 128) * (k // 128)) % np.uint64(6)).astype(np.uint8)
    return a, sa, w, sw.reshape(n // 128, k // 128)


@pytest.mark.parametrize("m", [1, 5, 16, 17, 33, 64, 65, 128, 200])
@pytest.mark.parametrize("n,k", [(1024, 4096), (384, 7168), (256, 1024), (128, 12288)])
def test_fp8_ue8m0_small_m(eng, m, n, k):
    a, sa, w, sw = _fp8_inputs(synth.config_seed(4, 15000 + m + n), m, n, k)
    got, flag = _ds_fp8(a, sa, w, sw)
    assert flag == 0
    assert_close(oracle.bf16_bits_to_f32(got), oracle.fp8_gemm_ue8m0(a, sa, w, sw), f"fp8 small m {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(1, 512, 2048), (16, 256, 7168), (40, 512, 4096), (64, 128, 1024),
                                   (128, 512, 4096), (256, 1024, 2048)])
@pytest.mark.parametrize("out_type", [abi.OUTPUT_BF16, abi.OUTPUT_F32])
def test_fp8_f32_scales_small_m(eng, m, n, k, out_type):
    from pih_amd import linear

    x = synth.bf16_normal(synth.config_seed(4, 15100 + m), (m, k))
    xq, xs = oracle.fp8_quant_f32(oracle.bf16_bits_to_f32(x))
    w, ws = synth.fp8_block_weight(synth.config_seed(4, 15101 + n), n, k)
    out, flag = linear.fp8_gemm(to_dev(xq), to_dev(xs), to_dev(w), to_dev(ws), abi.SCALE_F32, out_type)
    _sync()
    assert int(flag.item()) == 0
    got = to_host(out)
    got = oracle.bf16_bits_to_f32(got) if out_type == abi.OUTPUT_BF16 else got
    assert_close(got, oracle.fp8_gemm_f32(xq, xs, w, ws), f"fp8 f32 small m {m}x{n}x{k}")


@pytest.mark.parametrize("m", [1, 8, 16, 17, 64, 128, 256])
@pytest.mark.parametrize("n,k", [(2048, 4096), (4096, 2048), (256, 7168)])
def test_fp4_small_m(eng, m, n, k):
    import torch

    from pih_amd.device import ptr, stream_handle

    x = synth.bf16_normal(synth.config_seed(5, 15200 + m), (m, k))
    a, sa = oracle.fp8_quant_ue8m0(oracle.bf16_bits_to_f32(x))
    packed, sw = synth.mxfp4_weight(synth.config_seed(5, 15201 + n), n, k)
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ad, sad, pd, swd = to_dev(a), to_dev(sa), to_dev(packed), to_dev(sw)
    r = abi.request(abi.DS["fp4_gemm"], activation_e4m3=ptr(ad), activation_scale_bits=ptr(sad),
                    packed_weight=ptr(pd), weight_scale_bits=ptr(swd), output_bf16=ptr(out), error_flag=ptr(flag),
                    stream=stream_handle(), m=m, n=n, k=k)
    assert abi.deepseek_pack().call("launch_fp4_gemm", r).code == abi.OK
    _sync()
    assert int(flag.item()) == 0
    assert_close(oracle.bf16_bits_to_f32(to_host(out)), oracle.fp4_gemm(a, sa, packed, sw), f"fp4 small m {m}x{n}x{k}")


def test_small_m_error_bits(eng):
    """A NaN code in an activation row and a 0xFF weight scale raise 1 and 2;
    a sum that overflows raises 4 and leaves its element unwritten, as the
    reference's fp8_gemm_kernel skips it."""
    m, n, k = 3, 256, 512
    a, sa, w, sw = _fp8_inputs(synth.config_seed(4, 15300), m, n, k)
    a2 = a.copy()
    a2[1, 77] = 0xFF
    _, flag = _ds_fp8(a2, sa, w, sw)
    assert flag == 1
    sw2 = sw.copy()
    sw2[1, 2] = 0xFF
    _, flag = _ds_fp8(a, sa, w, sw2)
    assert flag == 2
    a3 = np.zeros_like(a)
    a3[:, :128] = 0x7E  # 448
    w3 = np.zeros_like(w)
    w3[:, :128] = 0x7E
    sa3 = np.full_like(sa, 127)
    sw3 = np.full_like(sw, 127)
    sw3[1, 0] = 254  # rows 128..255: 448 * 448 * 128 * 2^127 overflows
    got, flag = _ds_fp8(a3, sa3, w3, sw3)
    assert flag == 4
    assert np.all(got[:, 128:] == SENTINEL)
    np.testing.assert_array_equal(got[:, :128], oracle.f32_to_bf16_bits(np.full((m, 128), 448.0 * 448 * 128,
                                                                                np.float32)))


@pytest.mark.parametrize("t", [1, 3, 16, 100])
def test_grouped_fp8_small_t(eng, t):
    """The attention wo_a geometry (G = 8, 1024, 4096) at decode token
    counts (and at 100, two row chunks): A row t * 8 + g of the quantised
    input feeds group g."""
    import torch

    from pih_amd.device import ptr, stream_handle

    g, ng, kg = 8, 1024, 4096
    x = synth.bf16_normal(synth.config_seed(4, 15400 + t), (t * g, kg))
    w = _codes(synth.config_seed(4, 15401), (g * ng, kg))
    sw = (112 + synth.splitmix64(15402, g * (ng // 128) * (kg // 128)) % np.uint64(6)).astype(np.uint8)
    sw = sw.reshape(g * ng // 128, kg // 128)
    xd, wd, swd = to_dev(x), to_dev(w), to_dev(sw)
    aq = torch.empty(t * g, kg, dtype=torch.uint8, device="cuda")
    asb = torch.empty(t * g, kg // 128, dtype=torch.uint8, device="cuda")
    out = torch.empty(t, g * ng, dtype=torch.bfloat16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    r = abi.request(abi.DS["grouped_fp8_gemm"], input_bf16=ptr(xd), activation_e4m3=ptr(aq),
                    activation_scale_bits=ptr(asb), weight_e4m3=ptr(wd), weight_scale_bits=ptr(swd),
                    output_bf16=ptr(out), error_flag_u32=ptr(flag), stream=stream_handle(), token_count=t,
                    group_count=g, output_per_group=ng, input_per_group=kg)
    assert abi.deepseek_pack().call("launch_grouped_fp8_gemm", r).code == abi.OK
    _sync()
    assert int(flag.item()) == 0
    xq, xs = oracle.fp8_quant_ue8m0(oracle.bf16_bits_to_f32(x))
    ref = np.empty((t, g * ng), np.float32)
    for gi in range(g):
        rows = np.arange(t) * g + gi
        ref[:, gi * ng:(gi + 1) * ng] = oracle.fp8_gemm_ue8m0(
            np.ascontiguousarray(xq[rows]), np.ascontiguousarray(xs[rows]), np.ascontiguousarray(w[gi * ng:(gi + 1) * ng]),
            np.ascontiguousarray(sw[gi * ng // 128:(gi + 1) * ng // 128]))
    assert_close(oracle.bf16_bits_to_f32(to_host(out)), ref, f"grouped fp8 t={t}")

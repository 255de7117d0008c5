"""GPU parity of the DeepSeek V4.1 32-block formats against the oracle
(oracle/pih_oracle.c po_v41_*, pinned to the reference's
weight_expert_convert.cpp / weight_dequantize.cpp by golden vectors and to
linear_fp8.cu by closed forms):

* FP4 -> FP8 32x32 expert conversion at the V4.1 shared-expert shapes
  [2304, 5120] and [5120, 2304]: bit-exact codes and block scales; NaN and
  out-of-range row scales raise bits 1 / 2 and leave the block unwritten;
* wo_a block dequantisation [8192, 4096] with 32- and 128-blocks, UE8M0 and
  fp32 scales: bit-exact bf16; bad codes / scales / overflow flagged;
* the V4.1 linear (``launch_v41_linear``): the per-32 activation quant is
  bit-exact; outputs within max_rel <= 1e-2 and cos >= 0.9999 of the
  oracle's sequential per-group fp32 sums, and each element within
  K * 2^-22 * sum |a w scales| (the MX MFMA sums a 128-deep step in its own
  order); error bits and the reference's request checks.
"""
import numpy as np
import pytest

import oracle
from pih_amd import abi
from tests.helpers import assert_close, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def eng():
    import torch

    from pih_amd.device import engine_stream

    with engine_stream() as s:
        yield s
        torch.cuda.synchronize()


def _sync():
    import torch

    torch.cuda.synchronize()


def _fp4_expert(seed, rows, cols, lo=110, hi=127):
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    scales = rng.integers(lo, hi + 1, (rows, cols // 32), dtype=np.uint8)
    return packed, scales


@pytest.mark.parametrize("rows,cols", [(2304, 5120), (5120, 2304), (64, 96)])
def test_v41_fp4_to_fp8_bit_exact(rows, cols):
    from pih_amd.linear import v41_fp4_to_fp8

    packed, scales = _fp4_expert(rows + cols, rows, cols)
    w, s, flag = v41_fp4_to_fp8(to_dev(packed), to_dev(scales))
    _sync()
    assert int(flag.item()) == 0
    ref_w, ref_s = oracle.v41_fp4_to_fp8(packed, scales)
    np.testing.assert_array_equal(w.cpu().numpy(), ref_w)
    np.testing.assert_array_equal(s.cpu().numpy(), ref_s)


def test_v41_fp4_to_fp8_errors():
    import torch

    from pih_amd.linear import v41_fp4_to_fp8

    packed, scales = _fp4_expert(5, 64, 64)
    bad = scales.copy()
    bad[40, 1] = 255  # block (1, 1): NaN scale
    bad[0:32, 0] = 3  # block (0, 0): shared scale below range
    w, s, flag = v41_fp4_to_fp8(to_dev(packed), to_dev(bad))
    _sync()
    assert int(flag.item()) == 3
    ref_w, ref_s = oracle.v41_fp4_to_fp8(packed, scales)  # the untouched blocks are unchanged
    got = w.cpu().numpy()
    np.testing.assert_array_equal(got[0:32, 32:64], ref_w[0:32, 32:64])
    np.testing.assert_array_equal(got[32:64, 0:32], ref_w[32:64, 0:32])
    assert oracle.v41_fp4_block_to_fp8(packed[0:32, 0:16].ravel(), bad[0:32, 0])[2] == 2
    del torch


def _woa(seed, rows, cols):
    rng = np.random.default_rng(seed)
    src = rng.integers(0, 256, (rows, cols), dtype=np.uint8)
    src[(src & 0x7F) == 0x7F] = 0x42
    return src


@pytest.mark.parametrize("block,f32", [(32, False), (128, False), (128, True), (32, True)])
def test_v41_block_dequant_bit_exact(block, f32):
    from pih_amd.linear import v41_block_dequant

    rows, cols = 8192, 4096
    src = _woa(block + f32, rows, cols)
    rng = np.random.default_rng(7 + block)
    if f32:
        sc = rng.uniform(1e-4, 4e-3, (rows // block, cols // block)).astype(np.float32)
    else:
        sc = rng.integers(110, 125, (rows // block, cols // block), dtype=np.uint8)
    out, flag = v41_block_dequant(to_dev(src), to_dev(sc), block)
    _sync()
    assert int(flag.item()) == 0
    got = to_host(out)
    # the oracle block by block on a sample of blocks (every block is one call)
    for bi in range(0, rows // block, 37):
        for bj in range(0, cols // block, 29):
            blk = src[bi * block:(bi + 1) * block, bj * block:(bj + 1) * block]
            scale = float(sc[bi, bj]) if f32 else 2.0 ** (int(sc[bi, bj]) - 127)
            ref, st = oracle.v41_dequant_block(blk, scale, block)
            assert st == 0
            np.testing.assert_array_equal(got[bi * block:(bi + 1) * block, bj * block:(bj + 1) * block].ravel(), ref)


def test_v41_block_dequant_errors():
    import torch

    from pih_amd.linear import v41_block_dequant

    src = _woa(3, 256, 256)
    sc = np.full((2, 2), 120, np.uint8)
    src[5, 9] = 0x7F
    sc[1, 1] = 255
    out = torch.full((256, 256), 0x1234, dtype=torch.int16, device="cuda").view(torch.bfloat16)
    out, flag = v41_block_dequant(to_dev(src), to_dev(sc), 128, out=out)
    _sync()
    assert int(flag.item()) == 3
    got = to_host(out)
    assert got[5, 9] == 0x1234 and (got[128:, 128:] == 0x1234).all() and got[5, 10] != 0x1234
    big = np.full((128, 128), 0x7E, np.uint8)  # 448 x 2^127 overflows
    out, flag = v41_block_dequant(to_dev(big), to_dev(np.full((1, 1), 254, np.uint8)), 128)
    _sync()
    assert int(flag.item()) == 4


def _v41_case(seed, rows, n, k, fp4):
    rng = np.random.default_rng(seed)
    x = oracle.f32_to_bf16_bits(rng.standard_normal((rows, k)).astype(np.float32))
    if fp4:
        w = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
        sw = rng.integers(118, 125, (n, k // 32), dtype=np.uint8)
    else:
        w = rng.integers(0, 256, (n, k), dtype=np.uint8)
        w[(w & 0x7F) == 0x7F] = 0x30
        sw = rng.integers(112, 120, (n // 32, k // 32), dtype=np.uint8)
    return x, w, sw


def _bound(a, sa, w, sw, fp4):
    """sum over k of |a w| times both scales, in float64."""
    e4m3 = np.abs(np.array([oracle.e4m3_decode(int(c)) or 0.0 for c in range(256)], np.float64))
    at = e4m3[a]
    at *= np.exp2(np.repeat(sa, 32, axis=1).astype(np.float64) - 127)
    if fp4:
        table = np.abs(np.array([0, .5, 1, 1.5, 2, 3, 4, 6] * 2, np.float64))
        wv = np.empty((w.shape[0], w.shape[1] * 2))
        wv[:, 0::2], wv[:, 1::2] = table[w & 15], table[w >> 4]
        wv *= np.exp2(np.repeat(sw, 32, axis=1).astype(np.float64) - 127)
    else:
        wv = e4m3[w]
        wv *= np.exp2(np.repeat(np.repeat(sw, 32, axis=0), 32, axis=1).astype(np.float64) - 127)
    return at @ wv.T


@pytest.mark.parametrize("fp4", [False, True])
@pytest.mark.parametrize("rows,n,k", [(1, 2304, 5120), (7, 5120, 2304), (64, 256, 1024), (300, 384, 2048)])
def test_v41_linear(fp4, rows, n, k):
    from pih_amd.linear import v41_linear

    x, w, sw = _v41_case(rows + n + k + fp4, rows, n, k, fp4)
    fmt = abi.V41_WEIGHT_MXFP4 if fp4 else abi.V41_WEIGHT_FP8_BLOCK32
    out, q, qs, flag = v41_linear(to_dev(x), to_dev(w), to_dev(sw), fmt)
    _sync()
    assert int(flag.item()) == 0
    ref_q, ref_qs, qerr = oracle.v41_quant32(x)
    assert qerr == 0
    np.testing.assert_array_equal(q.cpu().numpy(), ref_q)
    np.testing.assert_array_equal(qs.cpu().numpy(), ref_qs)
    # the oracle on whole 32-row weight blocks: 0, a middle one and the last
    blocks = sorted({0, (n // 32) // 2, n // 32 - 1})
    cols = np.concatenate([np.arange(b * 32, b * 32 + 32) for b in blocks])
    w_sub = w[cols]
    sw_sub = sw[cols] if fp4 else sw[blocks]
    ref, err = oracle.v41_linear(ref_q, ref_qs, w_sub, sw_sub, len(cols), fp4)
    assert err == 0
    got = to_host(out)[:, cols]
    gf, rf = oracle.bf16_bits_to_f32(got).astype(np.float64), oracle.bf16_bits_to_f32(ref).astype(np.float64)
    tol = k * 2.0 ** -22 * _bound(ref_q, ref_qs, w_sub, sw_sub, fp4) + np.abs(rf) * 2.0 ** -7
    assert (np.abs(gf - rf) <= tol).all()
    assert_close(gf, rf, f"v41 linear fp4={fp4} {rows}x{n}x{k}")


def test_v41_linear_errors_and_validation():
    import torch

    from pih_amd.device import ptr, stream_handle
    from pih_amd.linear import KernelError, v41_linear

    rows, n, k = 4, 128, 256
    x, w, sw = _v41_case(11, rows, n, k, False)
    xb = x.copy()
    xb[2, 7] = 0x7F80  # +inf input: bit 1, encoded as 0
    out, q, _, flag = v41_linear(to_dev(xb), to_dev(w), to_dev(sw), abi.V41_WEIGHT_FP8_BLOCK32)
    _sync()
    assert int(flag.item()) == 1 and q.cpu().numpy()[2, 7] == 0
    sw2 = sw.copy()
    sw2[1, 3] = 255  # NaN weight scale: bit 1, and the affected outputs are non-finite (bit 2)
    out, _, _, flag = v41_linear(to_dev(x), to_dev(w), to_dev(sw2), abi.V41_WEIGHT_FP8_BLOCK32)
    _sync()
    assert int(flag.item()) == 3
    assert not np.isfinite(oracle.bf16_bits_to_f32(to_host(out))[:, 32:64]).any()
    # the reference's request checks
    xd, wd, swd = to_dev(x), to_dev(w), to_dev(sw)
    o = torch.empty(rows, n, dtype=torch.bfloat16, device="cuda")
    qd = torch.empty(rows, k, dtype=torch.uint8, device="cuda")
    qsd = torch.empty(rows, k // 32, dtype=torch.uint8, device="cuda")
    f = torch.zeros(1, dtype=torch.int32, device="cuda")
    base = dict(input_bf16=ptr(xd), input_bytes=rows * k * 2, weight=ptr(wd), weight_bytes=n * k,
                weight_scales=ptr(swd), weight_scale_bytes=(n // 32) * (k // 32), quantized_e4m3=ptr(qd),
                quantized_bytes=rows * k, activation_scales=ptr(qsd), activation_scale_bytes=rows * (k // 32),
                output_bf16=ptr(o), output_bytes=rows * n * 2, error_flag_u32=ptr(f), error_flag_bytes=4,
                stream=stream_handle(), rows=rows, in_features=k, out_features=n,
                weight_format=abi.V41_WEIGHT_FP8_BLOCK32)
    L = abi.linear_pack()
    assert L.call("launch_v41_linear", abi.request(abi.LN["v41_linear"], **base)).code == abi.OK
    for bad in (dict(rows=0), dict(rows=4097), dict(in_features=250), dict(out_features=100),
                dict(weight_bytes=n * k - 1), dict(output_bytes=rows * n * 2 + 2), dict(error_flag_bytes=8),
                dict(quantized_e4m3=ptr(xd)), dict(activation_scales=ptr(qd), activation_scale_bytes=rows * (k // 32)),
                dict(weight_format=3), dict(stream=0), dict(in_features=32 * 9, input_bytes=rows * 288 * 2,
                                                            quantized_bytes=rows * 288,
                                                            activation_scale_bytes=rows * 9, weight_bytes=n * 288,
                                                            weight_scale_bytes=(n // 32) * 9)):
        st = L.call("launch_v41_linear", abi.request(abi.LN["v41_linear"], **{**base, **bad}))
        assert st.code == abi.INVALID_ARGUMENT, bad
    _sync()
    del KernelError

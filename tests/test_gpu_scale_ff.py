"""A UE8M0 block scale of 0xFF in the drop-in FP8 / FP4 GEMMs.

The reference's kernels raise bit 2 and skip that scale block
(`continue` in plugins/kernels/deepseek-v4-sm89/native/deepseek_fp8_gemm.cu:48
and deepseek_fp4_gemm.cu:53-56): the other operand's scale must not leak
into the sum.  Each case pairs the 0xFF scale with a large scale on the
other operand in the same k block (228, against 0 on the other rows of that
block, so that every block of the k step contributes 2^-26 times its sum;
228 keeps the oracle's left-to-right product local * 2^101 finite), and
every other block uses scales near 100 (2^-54 times its sum), so a block
that were run with the 0xFF replaced by 2^-127 would add as much as a
valid one.  Expected: the oracle on the same operands with the skipped
block's codes zeroed (and a valid scale in its place).  Cases:

* big-tile kernel (M = 2048, 128 x 256 tiles): a W block scale and an A-row
  scale of 0xFF;
* 128 x 128 kernel (M = 512, N = 1024: fewer than 64 big tiles): the same;
* 128 x 128 FP4 kernel (M = 512): a W row's per-32 scale and an A-row scale;
* small-M kernel (M = 32): the same as the big tile, for the same result at
  every M.

Tolerance: max_rel <= 1e-2 (normwise), cosine >= 0.9999 (tests/helpers.py);
a leaked block changes the affected outputs by as much as their size.
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

    oracle.set_threads(min(16, __import__("os").cpu_count() or 1))
    with engine_stream() as s:
        yield s
        torch.cuda.synchronize()


def _codes(seed, shape):
    """e4m3 codes without NaN codes (0x7F / 0xFF skipped)."""
    c = (synth.splitmix64(seed, int(np.prod(shape))) % np.uint64(254)).astype(np.uint8)
    return np.where(c >= 0x7F, c + 1, c).astype(np.uint8).reshape(shape)


def _fp8_case(m, n, k, seed):
    """Operands with W block (3, 5) and A rows `ff_rows` at k block 2 set to
    0xFF, and the skip-equivalent operands for the oracle."""
    a = _codes(synth.config_seed(5, seed), (m, k))
    w = _codes(synth.config_seed(5, seed + 1), (n, k))
    sa = (100 + synth.splitmix64(seed + 2, m * (k // 128)) % np.uint64(6)).astype(np.uint8).reshape(m, k // 128)
    sw = (100 + synth.splitmix64(seed + 3, (n // 128) * (k // 128)) % np.uint64(6)).astype(np.uint8)
    sw = sw.reshape(n // 128, k // 128)
    ff_rows = np.array([1, 17, m // 2 + 3, m - 1])
    sa[:, 5], sw[:, 5] = 228, 0
    sw[3, 5] = 0xFF
    sw[:, 2], sa[:, 2] = 228, 0
    sa[ff_rows, 2] = 0xFF
    a0, w0, sa0, sw0 = a.copy(), w.copy(), sa.copy(), sw.copy()
    a0[ff_rows, 256:384] = 0
    sa0[ff_rows, 2] = 127
    w0[384:512, 640:768] = 0
    sw0[3, 5] = 127
    rows = np.unique(np.concatenate([ff_rows, ff_rows + 1 - (ff_rows == m - 1) * 2, np.linspace(0, m - 1, 12)
                                     .astype(np.int64)]))
    return (a, sa, w, sw), (a0, sa0, w0, sw0), rows


def _ds_fp8(a, sa, w, sw, m, n, k):
    import torch

    from pih_amd.device import ptr, stream_handle

    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ad, sad, wd, swd = to_dev(a), to_dev(sa), to_dev(w), to_dev(sw)
    r = abi.request(abi.DS["fp8_gemm"], activation_e4m3=ptr(ad), activation_scale_bits=ptr(sad),
                    weight_e4m3=ptr(wd), weight_scale_bits=ptr(swd), output=ptr(out), error_flag=ptr(flag),
                    stream=stream_handle(), m=m, n=n, k=k, output_type=1)
    st = abi.deepseek_pack().call("launch_fp8_gemm", r)
    assert st.code == abi.OK, st
    torch.cuda.synchronize()
    return oracle.bf16_bits_to_f32(to_host(out)), int(flag.item()) & 0xFFFFFFFF


@pytest.mark.parametrize("m,n,k", [(2048, 4096, 1024), (512, 1024, 1024), (32, 1024, 1024)])
def test_fp8_ff_scale_skips_the_block(eng, m, n, k):
    (a, sa, w, sw), (a0, sa0, w0, sw0), rows = _fp8_case(m, n, k, 900 + m)
    got, flag = _ds_fp8(a, sa, w, sw, m, n, k)
    assert flag == 2, flag
    ref = oracle.fp8_gemm_ue8m0(np.ascontiguousarray(a0[rows]), np.ascontiguousarray(sa0[rows]), w0, sw0)
    assert np.isfinite(got[rows]).all()
    assert_close(got[rows], ref, f"0xFF scale fp8 {m}x{n}x{k}")
    # the W block's columns and the A rows are where a leak would show
    assert_close(got[rows][:, 384:512], ref[:, 384:512], "0xFF W block columns")
    sel = np.isin(rows, [1, 17])
    assert_close(got[rows[sel]], ref[sel], "0xFF A rows")


def test_fp4_ff_scale_skips_the_block(eng):
    """128 x 128 FP4 kernel (M = 512, N = 2048, K = 4096): W row 77's scale
    of 32-k block 9 and A rows' scale of 128-k block 1 are 0xFF."""
    import torch

    from pih_amd.device import ptr, stream_handle

    m, n, k = 512, 2048, 4096
    x = synth.bf16_normal(synth.config_seed(5, 950), (m, k))
    a, _ = oracle.fp8_quant_ue8m0(oracle.bf16_bits_to_f32(x))
    packed, _ = synth.mxfp4_weight(synth.config_seed(5, 951), n, k)
    sa = (100 + synth.splitmix64(952, m * (k // 128)) % np.uint64(6)).astype(np.uint8).reshape(m, k // 128)
    sw = (100 + synth.splitmix64(953, n * (k // 32)) % np.uint64(6)).astype(np.uint8).reshape(n, k // 32)
    ff_rows = np.array([2, 300])
    sa[:, 2], sw[:, 8:12] = 228, 0  # 128-k block 2 = 32-k blocks 8..11
    sw[77, 9] = 0xFF
    sw[:, 4:8], sa[:, 1] = 228, 0  # 128-k block 1 = 32-k blocks 4..7
    sa[ff_rows, 1] = 0xFF
    a0, sa0, p0, sw0 = a.copy(), sa.copy(), packed.copy(), sw.copy()
    a0[ff_rows, 128:256] = 0
    sa0[ff_rows, 1] = 127
    p0[77, 9 * 16:10 * 16] = 0
    sw0[77, 9] = 127
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ad, sad, pd, swd = to_dev(a), to_dev(sa), to_dev(packed), to_dev(sw)
    r = abi.request(abi.DS["fp4_gemm"], activation_e4m3=ptr(ad), activation_scale_bits=ptr(sad),
                    packed_weight=ptr(pd), weight_scale_bits=ptr(swd), output_bf16=ptr(out), error_flag=ptr(flag),
                    stream=stream_handle(), m=m, n=n, k=k)
    assert abi.deepseek_pack().call("launch_fp4_gemm", r).code == abi.OK
    torch.cuda.synchronize()
    assert int(flag.item()) == 2
    got = oracle.bf16_bits_to_f32(to_host(out))
    rows = np.array([0, 2, 3, 300, 511])
    ref = oracle.fp4_gemm(np.ascontiguousarray(a0[rows]), np.ascontiguousarray(sa0[rows]), p0, sw0)
    assert np.isfinite(got[rows]).all()
    assert_close(got[rows], ref, "0xFF scale fp4")
    assert_close(got[rows][:, 77], ref[:, 77], "0xFF W row")
    assert_close(got[[2, 300]], ref[[1, 3]], "0xFF A rows")


@pytest.mark.parametrize("gather", [False, True])
def test_moe_fp4_ff_scale_skips_the_block(eng, gather):
    """MXFP4 MoE, e4m3 activations (N = 2048, K = 4096): expert 0 has 300
    rows (the 128 x 256 tiles with the FP4 W operand; persistent without a
    gather, one block per tile with one), expert 1 has 40 (the streaming
    kernel).  Expert 0's W row 77 scale of 32-k block 9 and A rows 2 and 250's
    scale of 128-k block 1 are 0xFF."""
    import torch

    from pih_amd import linear

    n, k, heavy, light = 2048, 4096, 300, 40
    m = heavy + light
    x = synth.bf16_normal(synth.config_seed(5, 960), (m, k))
    a, _ = oracle.fp8_quant_ue8m0(oracle.bf16_bits_to_f32(x))
    packed = np.empty((2, n, k // 2), np.uint8)
    for e in range(2):
        packed[e], _ = synth.mxfp4_weight(synth.config_seed(5, 961 + e), n, k)
    sa = (100 + synth.splitmix64(962, m * (k // 128)) % np.uint64(6)).astype(np.uint8).reshape(m, k // 128)
    sw = (100 + synth.splitmix64(963, 2 * n * (k // 32)) % np.uint64(6)).astype(np.uint8).reshape(2, n, k // 32)
    ff_rows = np.array([2, 250])
    sa[:heavy, 2], sw[0, :, 8:12] = 228, 0
    sw[0, 77, 9] = 0xFF
    sw[0, :, 4:8], sa[:heavy, 1] = 228, 0
    sa[ff_rows, 1] = 0xFF
    a0, sa0, p0, sw0 = a.copy(), sa.copy(), packed[0].copy(), sw[0].copy()
    a0[ff_rows, 128:256] = 0
    sa0[ff_rows, 1] = 127
    p0[77, 9 * 16:10 * 16] = 0
    sw0[77, 9] = 127
    off = np.array([0, heavy, m], np.uint32)
    # the gather reverses each expert's rows (the 0xFF A rows stay in expert 0)
    rt = np.concatenate([np.arange(heavy)[::-1], np.arange(heavy, m)[::-1]]).astype(np.uint32) if gather else None
    src = rt if gather else np.arange(m)
    out, flag = linear.moe_mxfp4_gemm(to_dev(a), to_dev(sa), to_dev(rt) if gather else None, to_dev(packed),
                                      to_dev(sw), to_dev(off), m, abi.ACTIVATION_E4M3, abi.OUTPUT_BF16)
    torch.cuda.synchronize()
    assert int(flag.item()) == 2
    got = oracle.bf16_bits_to_f32(to_host(out))
    assert np.isfinite(got).all()
    rows = np.array([0, 1, 2, 3, 127, 128, 250, 255, 256, 299])
    ref = oracle.fp4_gemm(np.ascontiguousarray(a0[src[rows]]), np.ascontiguousarray(sa0[src[rows]]), p0, sw0)
    assert_close(got[rows], ref, "0xFF scale moe fp4")
    assert_close(got[rows][:, 77], ref[:, 77], "0xFF W row")
    lrows = np.arange(heavy, m, 7)
    ref_l = oracle.fp4_gemm(np.ascontiguousarray(a[src[lrows]]), np.ascontiguousarray(sa[src[lrows]]), packed[1], sw[1])
    assert_close(got[lrows], ref_l, "light expert")


def test_moe_fp4_bf16_ff_weight_scale(eng):
    """MXFP4 MoE with bf16 activations (N = 2048, K = 4096): expert 0 (300
    rows, the 128 x 256 tiles) has W row 77's scale of 32-k block 9 at 0xFF.
    As in the 128 x 128 tile kernel, bf16 activations take the decoded
    weight times 2^(255 - 127): the scale bit and the non-finite bit are
    raised, the non-finite outputs of column 77 are left unwritten, and
    every other output of both experts matches the oracle."""
    import torch

    from pih_amd import linear

    n, k, heavy, light = 2048, 4096, 300, 40
    m = heavy + light
    x = synth.bf16_normal(synth.config_seed(5, 970), (m, k))
    packed = np.empty((2, n, k // 2), np.uint8)
    sw = np.empty((2, n, k // 32), np.uint8)
    for e in range(2):
        packed[e], sw[e] = synth.mxfp4_weight(synth.config_seed(5, 971 + e), n, k)
    sw[0, 77, 9] = 0xFF
    off = np.array([0, heavy, m], np.uint32)
    sentinel = 0x1234
    out = torch.full((m, n), sentinel, dtype=torch.int16, device="cuda").view(torch.bfloat16)
    out, flag = linear.moe_mxfp4_gemm(to_dev(x), None, None, to_dev(packed), to_dev(sw), to_dev(off), m,
                                      abi.ACTIVATION_BF16, abi.OUTPUT_BF16, out=out)
    torch.cuda.synchronize()
    assert int(flag.item()) == 6
    bits = to_host(out).view(np.uint16)
    got = oracle.bf16_bits_to_f32(bits)
    cols = np.r_[0:77, 78:n]
    rows = np.array([0, 1, 127, 128, 255, 256, 299])
    sw0 = sw[0].copy()
    sw0[77, 9] = 127  # the oracle rejects a 0xFF scale; column 77 is not compared
    ref = oracle.mxfp4_bf16_gemm(np.ascontiguousarray(x[rows]), packed[0], sw0)
    assert_close(got[rows][:, cols], ref[:, cols], "bf16 moe fp4, other columns")
    col = bits[:heavy, 77]
    assert ((col == sentinel) | ~np.isfinite(oracle.bf16_bits_to_f32(col))).all()
    lrows = np.arange(heavy, m, 7)
    ref_l = oracle.mxfp4_bf16_gemm(np.ascontiguousarray(x[lrows]), packed[1], sw[1])
    assert_close(got[lrows], ref_l, "light expert")

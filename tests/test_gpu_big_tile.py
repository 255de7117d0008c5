"""Dense GEMMs on the MoE kernel's 128 x 256 tiles (large single problems).

* DeepSeek `launch_fp8_gemm` (UE8M0 scales) and the linear pack's
  `launch_fp8_gemm` (fp32 scales) at shapes whose tile grid fills the GPU:
  sampled rows against the oracle.
* The reference decodes an e4m3 NaN code as 0 and raises bit 1
  (deepseek_fp8_gemm.cu:11-17); the big tiles' MFMAs do not decode codes,
  but a code's NaN reaches every sum over its A or W row, so a persistent
  tile whose block came out non-finite looks for codes in its operand rows
  and, finding one, computes the block again the reference's way.  Checked
  with NaN codes planted in A and in W (the rows they reach against the
  oracle, with the codes zeroed), with UE8M0 and fp32 scales, at 128- and
  32-row M tiles, next to overflowing sums (bit 4, elements unwritten), in
  a block a 0xFF scale skips (bit 2 only: the reference never decodes it),
  and with the bit already set before the call.
* BF16 `launch_bf16_gemm` at M = 1024 and 2048 (prefill sizes) with bf16
  and fp32 output against the fp32-accumulate oracle.

Tolerance: max_rel <= 1e-2 (normwise), cosine >= 0.9999 (tests/helpers.py).
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


def _ds_fp8(a, sa, w, sw, m, n, k, flag_init=0):
    import torch

    from pih_amd.device import ptr, stream_handle

    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    flag = torch.full((1,), flag_init, dtype=torch.int32, device="cuda")
    ad, sad, wd, swd = to_dev(a), to_dev(sa), to_dev(w), to_dev(sw)
    r = abi.request(abi.DS["fp8_gemm"], activation_e4m3=ptr(ad), activation_scale_bits=ptr(sad),
                    weight_e4m3=ptr(wd), weight_scale_bits=ptr(swd), output=ptr(out), error_flag=ptr(flag),
                    stream=stream_handle(), m=m, n=n, k=k, output_type=1)
    st = abi.deepseek_pack().call("launch_fp8_gemm", r)
    assert st.code == abi.OK, st
    torch.cuda.synchronize()
    return oracle.bf16_bits_to_f32(to_host(out)), int(flag.item()) & 0xFFFFFFFF


def _ue8m0_operands(m, n, k, seed):
    a = _codes(synth.config_seed(5, seed), (m, k))
    w = _codes(synth.config_seed(5, seed + 1), (n, k))
    sa = (118 + synth.splitmix64(seed + 2, m * (k // 128)) % np.uint64(6)).astype(np.uint8).reshape(m, k // 128)
    sw = (112 + synth.splitmix64(seed + 3, (n // 128) * (k // 128)) % np.uint64(6)).astype(np.uint8)
    return a, sa, w, sw.reshape(n // 128, k // 128)


@pytest.mark.parametrize("m,n,k", [(2048, 4096, 2048), (2048, 4096, 8192), (4096, 2048, 1024)])
def test_deepseek_fp8_gemm_big_tile(eng, m, n, k):
    a, sa, w, sw = _ue8m0_operands(m, n, k, 100 + k)
    got, flag = _ds_fp8(a, sa, w, sw, m, n, k)
    assert flag == 0
    rows = np.unique(np.linspace(0, m - 1, 24).astype(np.int64))
    ref = oracle.fp8_gemm_ue8m0(np.ascontiguousarray(a[rows]), np.ascontiguousarray(sa[rows]), w, sw)
    assert_close(got[rows], ref, f"big-tile fp8 {m}x{n}x{k}")


def test_nan_codes_in_a_and_w(eng):
    m, n, k = 2048, 4096, 1024
    a, sa, w, sw = _ue8m0_operands(m, n, k, 300)
    a[5, 77] = 0x7F   # NaN code in A (row 5)
    w[1000, 300] = 0xFF  # NaN code in W (column 1000 of every row)
    got, flag = _ds_fp8(a, sa, w, sw, m, n, k)
    assert flag & 1, flag
    rows = np.array([0, 5, 6, 1023, 2047])
    # the oracle rejects NaN codes; the kernel's decode reads them as 0
    a0, w0 = a.copy(), w.copy()
    a0[5, 77] = 0
    w0[1000, 300] = 0
    ref = oracle.fp8_gemm_ue8m0(np.ascontiguousarray(a0[rows]), np.ascontiguousarray(sa[rows]), w0, sw)
    assert np.isfinite(got[rows]).all()
    assert_close(got[rows], ref, "nan codes as zero")


@pytest.mark.parametrize("m,n,k", [(2048, 1024, 4096), (2048, 4096, 1024), (2048, 4096, 384)])
@pytest.mark.parametrize("where", ["a", "w"])
def test_nan_code_found_in_tiles(eng, m, n, k, where):
    """One NaN code in A (last M tile, last K block) or in W: the persistent
    big tiles (32-row M tiles at 2048 x 1024 x 4096) find it in the operand
    rows of the blocks whose sums it turned into NaN, raise bit 1 only and
    compute those blocks again with the code as 0.  K = 384 (three K steps)
    is too short for the persistent tiles: a scan raises the bit, the big
    tiles exit and the checking kernel computes the result."""
    a, sa, w, sw = _ue8m0_operands(m, n, k, 600 + k + (where == "w"))
    a0, w0 = a.copy(), w.copy()
    if where == "a":
        a[m - 3, k - 5] = 0xFF
    else:
        w[n - 7, 1] = 0x7F
    got, flag = _ds_fp8(a, sa, w, sw, m, n, k)
    assert flag == 1, flag
    assert np.isfinite(got).all()
    rows = np.array([0, 31, 32, m // 2, m - 3, m - 1])
    ref = oracle.fp8_gemm_ue8m0(np.ascontiguousarray(a0[rows]), np.ascontiguousarray(sa[rows]), w0, sw)
    assert_close(got[rows], ref, f"nan code in {where} as zero")


def test_nan_code_in_a_skipped_block(eng):
    """A NaN code in a 128-k block whose UE8M0 activation scale is 0xFF: the
    reference skips the block before decoding it, so the flag holds bit 2
    only, and that block adds nothing to its row."""
    m, n, k = 2048, 1024, 4096
    a, sa, w, sw = _ue8m0_operands(m, n, k, 650)
    a[100, 1000] = 0x7F
    sa[100, 1000 // 128] = 0xFF
    got, flag = _ds_fp8(a, sa, w, sw, m, n, k)
    assert flag == 2, flag
    a0, sa0 = a.copy(), sa.copy()
    a0[100, 896:1024] = 0  # the skipped block
    sa0[100, 7] = 127
    rows = np.array([0, 99, 100, 101, m - 1])
    ref = oracle.fp8_gemm_ue8m0(np.ascontiguousarray(a0[rows]), np.ascontiguousarray(sa0[rows]), w, sw)
    assert np.isfinite(got).all()
    assert_close(got[rows], ref, "code in a skipped block")


def test_nan_code_with_overflow_elsewhere(eng):
    """A NaN code in A row 7 and, in other columns, sums that overflow: bit 1
    from the code and bit 4 from the overflow (the overflowing elements are
    left unwritten, as the reference does, row 7's among them); the other
    elements hold the oracle's values with the code as 0."""
    import torch

    from pih_amd.device import ptr, stream_handle

    m, n, k = 2048, 1024, 4096
    a = np.zeros((m, k), np.uint8)
    a[:, :128] = 0x7E  # 448
    w = np.zeros((n, k), np.uint8)
    w[:, :128] = 0x7E
    a[7, 2000] = 0x7F
    sa = np.full((m, k // 128), 127, np.uint8)
    sw = np.full((n // 128, k // 128), 127, np.uint8)
    sw[5, 0] = 254  # W rows 640..767: 448 * 448 * 128 * 2^127 overflows
    sentinel = 0x7FC1
    out = torch.full((m, n), sentinel, dtype=torch.int16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ad, sad, wd, swd = to_dev(a), to_dev(sa), to_dev(w), to_dev(sw)
    r = abi.request(abi.DS["fp8_gemm"], activation_e4m3=ptr(ad), activation_scale_bits=ptr(sad),
                    weight_e4m3=ptr(wd), weight_scale_bits=ptr(swd), output=ptr(out), error_flag=ptr(flag),
                    stream=stream_handle(), m=m, n=n, k=k, output_type=1)
    st = abi.deepseek_pack().call("launch_fp8_gemm", r)
    assert st.code == abi.OK, st
    torch.cuda.synchronize()
    assert int(flag.item()) == 5
    got = to_host(out).view(np.uint16)
    assert np.all(got[:, 640:768] == sentinel)
    want = oracle.f32_to_bf16_bits(np.float32(448.0 * 448 * 128))
    assert np.all(got[:, :640] == want) and np.all(got[:, 768:] == want)


@pytest.mark.parametrize("out_type", [1, 2])
def test_linear_fp8_gemm_nan_code_f32_scales(eng, out_type):
    """The linear pack's fp32-scale entry on the persistent big tiles, bf16
    and fp32 output: a NaN code in W raises bit 1 and the result has it as
    0."""
    import torch

    from pih_amd.device import ptr, stream_handle

    m, n, k = 2048, 1024, 4096
    a = _codes(synth.config_seed(5, 700), (m, k))
    w = _codes(synth.config_seed(5, 701), (n, k))
    w0 = w.copy()
    w[300, 4000] = 0xFF
    rng = np.random.default_rng(702)
    sa = (rng.uniform(0.5, 2.0, (m, k // 128)) / 448).astype(np.float32)
    sw = (rng.uniform(0.5, 2.0, (n // 128, k // 128)) / 448).astype(np.float32)
    dt = torch.bfloat16 if out_type == abi.OUTPUT_BF16 else torch.float32
    out = torch.empty(m, n, dtype=dt, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ad, sad, wd, swd = to_dev(a), to_dev(sa), to_dev(w), to_dev(sw)
    r = abi.request(abi.LN["fp8_gemm"], activation_e4m3=ptr(ad), activation_scale=ptr(sad), weight_e4m3=ptr(wd),
                    weight_scale=ptr(swd), output=ptr(out), error_flag_u32=ptr(flag), stream=stream_handle(),
                    m=m, n=n, k=k, scale_format=abi.SCALE_F32, output_type=out_type)
    st = abi.linear_pack().call("launch_fp8_gemm", r)
    assert st.code == abi.OK, st
    torch.cuda.synchronize()
    assert int(flag.item()) == 1
    host = to_host(out)
    got = oracle.bf16_bits_to_f32(host) if out_type == abi.OUTPUT_BF16 else host
    assert np.isfinite(got).all()
    rows = np.unique(np.linspace(0, m - 1, 16).astype(np.int64))
    ref = oracle.fp8_gemm_f32(np.ascontiguousarray(a[rows]), np.ascontiguousarray(sa[rows]), w0, sw)
    assert_close(got[rows], ref, "f32-scale nan code as zero")


def test_code_bit_already_set(eng):
    """A flag that already holds bit 1 (a poisoned lane) before the call:
    the bit stays, and the result is the same."""
    m, n, k = 2048, 4096, 1024
    a, sa, w, sw = _ue8m0_operands(m, n, k, 400)
    clean, flag0 = _ds_fp8(a, sa, w, sw, m, n, k)
    assert flag0 == 0
    again, flag1 = _ds_fp8(a, sa, w, sw, m, n, k, flag_init=1)
    assert flag1 == 1
    rows = np.unique(np.linspace(0, m - 1, 16).astype(np.int64))
    ref = oracle.fp8_gemm_ue8m0(np.ascontiguousarray(a[rows]), np.ascontiguousarray(sa[rows]), w, sw)
    assert_close(again[rows], ref, "bit set before the call")
    assert_close(clean[rows], ref, "big-tile kernel")


@pytest.mark.parametrize("out_type", [1, 2])
def test_linear_fp8_gemm_big_tile_f32_scales(eng, out_type):
    import torch

    from pih_amd.device import ptr, stream_handle

    m, n, k = 2048, 4096, 2048
    a = _codes(synth.config_seed(5, 500), (m, k))
    w = _codes(synth.config_seed(5, 501), (n, k))
    rng = np.random.default_rng(502)
    sa = (rng.uniform(0.5, 2.0, (m, k // 128)) / 448).astype(np.float32)
    sw = (rng.uniform(0.5, 2.0, (n // 128, k // 128)) / 448).astype(np.float32)
    dt = torch.bfloat16 if out_type == abi.OUTPUT_BF16 else torch.float32
    out = torch.empty(m, n, dtype=dt, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ad, sad, wd, swd = to_dev(a), to_dev(sa), to_dev(w), to_dev(sw)
    r = abi.request(abi.LN["fp8_gemm"], activation_e4m3=ptr(ad), activation_scale=ptr(sad), weight_e4m3=ptr(wd),
                    weight_scale=ptr(swd), output=ptr(out), error_flag_u32=ptr(flag), stream=stream_handle(),
                    m=m, n=n, k=k, scale_format=abi.SCALE_F32, output_type=out_type)
    st = abi.linear_pack().call("launch_fp8_gemm", r)
    assert st.code == abi.OK, st
    torch.cuda.synchronize()
    assert int(flag.item()) == 0
    host = to_host(out)
    got = oracle.bf16_bits_to_f32(host) if out_type == abi.OUTPUT_BF16 else host
    rows = np.unique(np.linspace(0, m - 1, 24).astype(np.int64))
    ref = oracle.fp8_gemm_f32(np.ascontiguousarray(a[rows]), np.ascontiguousarray(sa[rows]), w, sw)
    assert_close(got[rows], ref, f"big-tile fp8 f32-scale out {out_type}")


@pytest.mark.parametrize("m,n,k,out_type", [(1024, 8192, 1024, 1), (2048, 4096, 1536, 2)])
def test_bf16_gemm_big_tile(eng, m, n, k, out_type):
    import torch

    from pih_amd.device import ptr, stream_handle

    x = synth.bf16_normal(synth.config_seed(5, 600 + m), (m, k))
    w = synth.bf16_normal(synth.config_seed(5, 601 + n), (n, k), std=0.02)
    dt = torch.bfloat16 if out_type == abi.OUTPUT_BF16 else torch.float32
    out = torch.empty(m, n, dtype=dt, device="cuda")
    xd, wd = to_dev(x), to_dev(w)
    r = abi.request(abi.LN["bf16_gemm"], a_bf16=ptr(xd), w_bf16=ptr(wd), output=ptr(out), workspace=0,
                    workspace_bytes=0, stream=stream_handle(), m=m, n=n, k=k, output_type=out_type)
    st = abi.linear_pack().call("launch_bf16_gemm", r)
    assert st.code == abi.OK, st
    torch.cuda.synchronize()
    host = to_host(out)
    got = oracle.bf16_bits_to_f32(host) if out_type == abi.OUTPUT_BF16 else host
    rows = np.unique(np.linspace(0, m - 1, 24).astype(np.int64))
    ref = oracle.bf16_gemm(np.ascontiguousarray(x[rows]), w)
    assert_close(got[rows], ref, f"big-tile bf16 {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(2048, 1024, 4096), (1000, 2048, 4096), (2048, 1280, 4608), (128, 4096, 12288),
                                   (96, 1024, 4096)])
@pytest.mark.parametrize("out_type", [abi.OUTPUT_BF16, abi.OUTPUT_F32])
def test_bf16_gemm_k_split(eng, m, n, k, out_type):
    """launch_bf16_gemm with the queried workspace at shapes with fewer big
    tiles than CUs (the Qwen3-8B k/v projections at M 2048: 4 K splits; M
    1000: a partial M tile; 4608 -> 1280: 3 splits; batches of 96 and 128
    rows: 8 splits, one partial M tile; without the workspace they run
    unsplit on 32-row M tiles): the fp32 partial sums go to the
    workspace (filled with NaN bytes first, so an element no split writes
    would show) and are summed in split order.  Sampled rows against the
    oracle, every row's sum against a float64 checksum, and the whole output
    against the unsplit launch (workspace 0) within the fp32 reordering of
    the K sum (bf16: one unit in the last place)."""
    import torch

    from pih_amd.device import ptr, stream_handle

    x = synth.bf16_normal(synth.config_seed(5, 700 + m), (m, k))
    w = synth.bf16_normal(synth.config_seed(5, 701 + n), (n, k), std=0.02)
    xd, wd = to_dev(x), to_dev(w)
    cnt = (abi.C.c_uint64 * 1)()
    qr = abi.request(abi.LN["workspace_query"], kind=abi.WORKSPACE_BF16_GEMM, m=m, n=n, k=k,
                     bytes_u64=abi.C.addressof(cnt))
    assert abi.linear_pack().call("query_workspace", qr).code == abi.OK
    wsb = int(cnt[0])
    assert wsb > 0 and wsb % (m * n * 4) == 0
    ws = torch.full((wsb,), 0xFF, dtype=torch.uint8, device="cuda")
    dt = torch.bfloat16 if out_type == abi.OUTPUT_BF16 else torch.float32

    def run(use_ws):
        out = torch.empty(m, n, dtype=dt, device="cuda")
        r = abi.request(abi.LN["bf16_gemm"], a_bf16=ptr(xd), w_bf16=ptr(wd), output=ptr(out),
                        workspace=ptr(ws) if use_ws else 0, workspace_bytes=wsb if use_ws else 0,
                        stream=stream_handle(), m=m, n=n, k=k, output_type=out_type)
        st = abi.linear_pack().call("launch_bf16_gemm", r)
        assert st.code == abi.OK, st
        torch.cuda.synchronize()
        host = to_host(out)
        return oracle.bf16_bits_to_f32(host) if out_type == abi.OUTPUT_BF16 else host

    split, whole = run(True), run(False)
    assert np.all(np.isfinite(split))
    rows = np.unique(np.concatenate([np.linspace(0, m - 1, 24).astype(np.int64), [127, 128, m - 1]]))
    rows = rows[rows < m]
    ref = oracle.bf16_gemm(np.ascontiguousarray(x[rows]), w)
    assert_close(split[rows], ref, f"k-split bf16 {m}x{n}x{k}")
    colsum = oracle.bf16_bits_to_f32(w).astype(np.float64).sum(axis=0)
    want = oracle.bf16_bits_to_f32(x).astype(np.float64) @ colsum
    have = split.astype(np.float64).sum(axis=1)
    bound = np.abs(split).astype(np.float64).sum(axis=1) * 2.0 ** -8 + 1e-3
    assert np.all(np.abs(have - want) <= bound), "k-split row checksums"
    if out_type == abi.OUTPUT_F32:
        # fp32 sums of the same products in two orders (outputs ~1.3 rms)
        assert np.all(np.abs(split - whole) <= 2e-5 + np.abs(whole) * 1e-5)
    else:
        # one bf16 rounding each of two fp32 sums that differ in the order of
        # their K parts (~1e-6 here): one unit in the last place, plus slack
        # for results that cancel to near zero
        ulp = np.maximum(np.abs(whole), np.abs(split)) * 2.0 ** -7 + 1e-4
        assert np.all(np.abs(split - whole) <= ulp)


def test_big_tile_nonfinite_results_skipped(eng):
    """Sums that overflow (UE8M0 weight scale 2^127 on one 128-row block)
    raise bit 4 and leave their elements unwritten, as the reference's
    fp8_gemm_kernel skips them (deepseek_fp8_gemm.cu:67-70); the other
    columns hold the oracle's values.  M = 2048 runs the persistent big-tile
    kernel, whose waves with such an element store per element."""
    import torch

    from pih_amd.device import ptr, stream_handle

    m, n, k = 2048, 4096, 1024
    a = np.zeros((m, k), np.uint8)
    a[:, :128] = 0x7E  # 448
    w = np.zeros((n, k), np.uint8)
    w[:, :128] = 0x7E
    sa = np.full((m, k // 128), 127, np.uint8)
    sw = np.full((n // 128, k // 128), 127, np.uint8)
    sw[3, 0] = 254  # W rows 384..511: 448 * 448 * 128 * 2^127 overflows
    sentinel = 0x7FC1
    out = torch.full((m, n), sentinel, dtype=torch.int16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    ad, sad, wd, swd = to_dev(a), to_dev(sa), to_dev(w), to_dev(sw)
    r = abi.request(abi.DS["fp8_gemm"], activation_e4m3=ptr(ad), activation_scale_bits=ptr(sad),
                    weight_e4m3=ptr(wd), weight_scale_bits=ptr(swd), output=ptr(out), error_flag=ptr(flag),
                    stream=stream_handle(), m=m, n=n, k=k, output_type=1)
    st = abi.deepseek_pack().call("launch_fp8_gemm", r)
    assert st.code == abi.OK, st
    torch.cuda.synchronize()
    assert int(flag.item()) == 4
    got = to_host(out).view(np.uint16)
    assert np.all(got[:, 384:512] == sentinel)
    want = oracle.f32_to_bf16_bits(np.float32(448.0 * 448 * 128))
    assert np.all(got[:, :384] == want) and np.all(got[:, 512:] == want)

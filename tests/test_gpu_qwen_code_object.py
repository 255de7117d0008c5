"""GPU parity of the gfx950 Qwen code object, launched the way the Qwen model
launches the reference cubin: resolved through the pack's root(), loaded by
the C++ kernel-module driver (libpih_hip_kernel_module.so: manifest, digest
and kernarg-layout checks, hipModuleLoadData, by-name resolution) and
launched by name with the 64-byte packet through its identity-checked submit
entry, with the plan entry's geometry: ceil(m*n/256) blocks of 256 threads
for the compatibility kernel (qwen3_int4_gemm_plan.cpp:55-85), (n/16,
ceil(m/16)) blocks whose waves split K for pih_qwen_w4a16_gemm_gfx950_v1.

W4A16 results are compared with the oracle's po_w4a16_sym (the reference's
strict-k fp32 sum, qwen_bf16_primitives.cu:98-149) at max_rel <= 1e-2 and
cos >= 0.9999; the error protocol (first-wins codes 11-14, failing elements
not written) and SiLU-mul are checked against the same file.
"""
import numpy as np
import pytest

import oracle
from pih_amd import synth
from tests.helpers import assert_close, to_dev, to_host

pytestmark = pytest.mark.gpu

QWEN06B = [(2048, 1024), (1024, 1024), (1024, 2048), (3072, 1024), (1024, 3072)]
SENTINEL = 0x7E7E


@pytest.fixture(scope="module")
def co():
    import torch

    from pih_amd.device import engine_stream
    from pih_amd.qwen import QwenCodeObject

    with engine_stream() as s:
        yield QwenCodeObject(), s
        torch.cuda.synchronize()


def _run_w4a16(co, x, q, s, m, n, k, grid=None, block=None, variant=1):
    import torch

    obj, stream = co
    xd, qd, sd = to_dev(x), to_dev(q), to_dev(s)
    out = torch.full((m, n), SENTINEL, dtype=torch.int16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    if grid is not None and block is None:
        block = 256
    obj.w4a16_gemm(xd.data_ptr(), qd.data_ptr(), sd.data_ptr(), out.data_ptr(), flag.data_ptr(), m, n, k,
                   stream.cuda_stream, grid=grid, block=block, variant=variant)
    stream.synchronize()
    return out.cpu().numpy().view(np.uint16), int(flag.item()) & 0xFFFFFFFF


@pytest.mark.parametrize("m", [1, 4, 16, 17, 48])
@pytest.mark.parametrize("n,k", QWEN06B)
def test_w4a16_compat_qwen06b_shapes(co, m, n, k):
    """m = 16 and 48 take the 16 x 16 tile mapping of the launch's blocks,
    the others the per-x-row mapping."""
    q, s = synth.int4_sym_weight(synth.config_seed(3, 900 + n + k), n, k)
    x = synth.bf16_normal(synth.config_seed(3, 950 + m), (m, k))
    got, flag = _run_w4a16(co, x, q, s, m, n, k)
    assert flag == 0
    ref = oracle.w4a16_sym(x, q, s)
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref), f"compat w4a16 {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (3, 1024, 4096), (1, 12288, 4096), (1, 4096, 12288),
                                   (2, 256, 640)])
def test_w4a16_compat_relaxed_shapes(co, m, n, k):
    """Qwen3-8B projections and a K that is not a multiple of 1024."""
    q, s = synth.int4_sym_weight(synth.config_seed(3, 1900 + n + k), n, k)
    x = synth.bf16_normal(synth.config_seed(3, 1950 + m), (m, k))
    got, flag = _run_w4a16(co, x, q, s, m, n, k)
    assert flag == 0
    ref = oracle.w4a16_sym(x, q, s)
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref), f"compat w4a16 {m}x{n}x{k}")


def test_w4a16_compat_errors(co):
    m, n, k = 2, 1024, 1024
    q, s = synth.int4_sym_weight(synth.config_seed(3, 4242), n, k)
    x = synth.bf16_normal(synth.config_seed(3, 4243), (m, k))
    ref = oracle.w4a16_sym(x, q, s)

    # reserved nibble in W row 5: only column 5 is left unwritten, code 12
    q2 = q.copy()
    q2[5, 300] = (q2[5, 300] & 0x0F) | 0x80
    got, flag = _run_w4a16(co, x, q2, s, m, n, k)
    assert flag == 12
    assert (got[:, 5] == SENTINEL).all()
    keep = np.ones(n, bool)
    keep[5] = False
    assert_close(oracle.bf16_bits_to_f32(got[:, keep]), oracle.bf16_bits_to_f32(ref[:, keep]), "rows kept")

    # a zero, a negative and a NaN fp16 scale: code 13, those columns unwritten
    for bad in (0x0000, 0xBC00, 0x7E00):
        s2 = s.copy()
        s2[700, 3] = bad
        got, flag = _run_w4a16(co, x, q, s2, m, n, k)
        assert flag == 13, hex(bad)
        assert (got[:, 700] == SENTINEL).all()
        assert (got[:, 699] != SENTINEL).all()

    # launch contract: wrong grid, wrong block size, n not a multiple of 256
    for grid, block in (((m * n + 255) // 256 - 1, 256), ((m * n + 255) // 256 + 1, 256), ((m * n + 127) // 128, 128)):
        got, flag = _run_w4a16(co, x, q, s, m, n, k, grid=grid, block=block)
        assert flag == 11
        assert (got == SENTINEL).all()
    # (the plan entry refuses these shapes; the model's own geometry is
    # launched to reach the kernel's check)
    q3, s3 = synth.int4_sym_weight(5, 320, k)
    got, flag = _run_w4a16(co, x, q3, s3, m, 320, k, grid=(m * 320 + 255) // 256)
    assert flag == 11 and (got == SENTINEL).all()
    got, flag = _run_w4a16(co, synth.bf16_normal(1, (4097, 128)), *synth.int4_sym_weight(6, 256, 128), 4097, 256,
                           128, grid=4097)
    assert flag == 11


def test_w4a16_compat_errors_tile_mapping(co):
    """m = 32 (16 x 16 output tiles, K split over the block's waves): a
    reserved nibble in W row 300 leaves that column unwritten in every row
    (code 12); the other columns match the oracle."""
    m, n, k = 32, 1024, 1024
    q, s = synth.int4_sym_weight(synth.config_seed(3, 4300), n, k)
    x = synth.bf16_normal(synth.config_seed(3, 4301), (m, k))
    ref = oracle.w4a16_sym(x, q, s)
    q2 = q.copy()
    q2[300, 400] = (q2[300, 400] & 0xF0) | 0x08
    got, flag = _run_w4a16(co, x, q2, s, m, n, k)
    assert flag == 12
    assert (got[:, 300] == SENTINEL).all()
    keep = np.ones(n, bool)
    keep[300] = False
    assert_close(oracle.bf16_bits_to_f32(got[:, keep]), oracle.bf16_bits_to_f32(ref[:, keep]), "tile rows kept")


def test_w4a16_compat_nonfinite_output(co):
    m, n, k = 1, 256, 128
    q, s = synth.int4_sym_weight(synth.config_seed(3, 31), n, k)
    x = synth.bf16_normal(synth.config_seed(3, 32), (m, k))
    x[0, 7] = 0x7F80  # +inf
    got, flag = _run_w4a16(co, x, q, s, m, n, k)
    assert flag == 14


def test_silu_mul_code_object(co):
    import torch

    obj, stream = co
    count = 3 * 1024 + 17
    g = synth.bf16_normal(synth.config_seed(1, 70), (count,))
    u = synth.bf16_normal(synth.config_seed(1, 71), (count,))
    gd, ud = to_dev(g), to_dev(u)
    out = torch.empty(count, dtype=torch.bfloat16, device="cuda")
    obj.silu_mul(gd.data_ptr(), ud.data_ptr(), out.data_ptr(), count, stream.cuda_stream)
    stream.synchronize()
    got = to_host(out)
    ref = oracle.silu_mul(g, u)
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref), "code-object silu_mul")
    # at most one bf16 ulp from the reference formula
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1


@pytest.mark.parametrize("m,n,k,seed", [(3, 1024, 1024, 0), (1, 2048, 1024, 0x51A7), (2, 1024, 1024, 0x62B8),
                                        (3, 1024, 2048, 0x73C9), (7, 3072, 1024, 0x84DA),
                                        (17, 1024, 3072, 0x95EB)])
def test_w4a16_compat_reference_fixture(co, m, n, k, seed):
    """The reference's own fixture matrix for this kernel
    (src/backend/cuda/qwen_int4_cuda_fixture.cpp:87-140,291,296-302): exact
    sums, so the outputs must equal the expected bf16 values bit for bit
    (exact zero sums as +0, see tests/qwen_int4_fixture.py)."""
    from tests import qwen_int4_fixture as fx

    x, q, s, expected = fx.case(m, n, k, seed)
    got, flag = _run_w4a16(co, x, q, s, m, n, k)
    assert flag == 0
    np.testing.assert_array_equal(got, expected)


@pytest.mark.parametrize("m,n,k,seed", [(3, 1024, 1024, 0), (7, 3072, 1024, 0x84DA), (17, 1024, 3072, 0x95EB)])
def test_w4a16_entry_reference_fixture(co, m, n, k, seed):
    """The same fixture through the linear pack's launch_w4a16_gemm
    (symmetric format)."""
    import torch

    from pih_amd import abi
    from pih_amd.device import ptr
    from tests import qwen_int4_fixture as fx

    _, stream = co
    x, q, s, expected = fx.case(m, n, k, seed)
    xd, qd, sd = to_dev(x), to_dev(q), to_dev(s)
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    r = abi.request(abi.LN["w4a16"], input_bf16=ptr(xd), qweight=ptr(qd), scales=ptr(sd), zeros=0,
                    output_bf16=ptr(out), workspace=0, workspace_bytes=0, error_flag_u32=ptr(flag),
                    stream=stream.cuda_stream, m=m, n=n, k=k, format=abi.W4A16_SYMMETRIC)
    assert abi.linear_pack().call("launch_w4a16_gemm", r).code == abi.OK
    stream.synchronize()
    assert int(flag.item()) == 0
    np.testing.assert_array_equal(to_host(out), expected)


# ------------------------------------------ the gfx950 plan's kernel
GFX950 = 2


@pytest.mark.parametrize("m", [1, 4, 16, 17, 48])
@pytest.mark.parametrize("n,k", QWEN06B)
def test_w4a16_gfx950_qwen06b_shapes(co, m, n, k):
    """pih_qwen_w4a16_gemm_gfx950_v1 with the plan's geometry: ragged m
    (rows past m read row m - 1 and are not stored), 8 to 16 waves per
    block splitting the groups."""
    q, s = synth.int4_sym_weight(synth.config_seed(3, 900 + n + k), n, k)
    x = synth.bf16_normal(synth.config_seed(3, 950 + m), (m, k))
    got, flag = _run_w4a16(co, x, q, s, m, n, k, variant=GFX950)
    assert flag == 0
    ref = oracle.w4a16_sym(x, q, s)
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref), f"gfx950 w4a16 {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (3, 1024, 4096), (1, 12288, 4096), (1, 4096, 12288),
                                   (2, 272, 640), (130, 2048, 1024)])
def test_w4a16_gfx950_relaxed_shapes(co, m, n, k):
    """Qwen3-8B projections, n a multiple of 16 only, a K that is not a
    multiple of 1024, and a prefill-sized m."""
    q, s = synth.int4_sym_weight(synth.config_seed(3, 1900 + n + k), n, k)
    x = synth.bf16_normal(synth.config_seed(3, 1950 + m), (m, k))
    got, flag = _run_w4a16(co, x, q, s, m, n, k, variant=GFX950)
    assert flag == 0
    ref = oracle.w4a16_sym(x, q, s)
    assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(ref), f"gfx950 w4a16 {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k,seed", [(3, 1024, 1024, 0), (1, 2048, 1024, 0x51A7), (7, 3072, 1024, 0x84DA),
                                        (17, 1024, 3072, 0x95EB)])
def test_w4a16_gfx950_reference_fixture(co, m, n, k, seed):
    """The reference's fixture matrix (exact sums): bit for bit."""
    from tests import qwen_int4_fixture as fx

    x, q, s, expected = fx.case(m, n, k, seed)
    got, flag = _run_w4a16(co, x, q, s, m, n, k, variant=GFX950)
    assert flag == 0
    np.testing.assert_array_equal(got, expected)


def test_w4a16_gfx950_errors(co):
    """The error protocol of the compatibility kernel: a reserved nibble
    (12) and a bad scale (13) leave only their column unwritten; a geometry
    other than the plan's, n not a multiple of 16 and m > 4096 publish 11
    and write nothing."""
    m, n, k = 5, 1024, 1024
    q, s = synth.int4_sym_weight(synth.config_seed(3, 4400), n, k)
    x = synth.bf16_normal(synth.config_seed(3, 4401), (m, k))
    ref = oracle.w4a16_sym(x, q, s)
    q2 = q.copy()
    q2[77, 100] = (q2[77, 100] & 0xF0) | 0x08
    got, flag = _run_w4a16(co, x, q2, s, m, n, k, variant=GFX950)
    assert flag == 12 and (got[:, 77] == SENTINEL).all()
    keep = np.ones(n, bool)
    keep[77] = False
    assert_close(oracle.bf16_bits_to_f32(got[:, keep]), oracle.bf16_bits_to_f32(ref[:, keep]), "gfx950 kept")
    s2 = s.copy()
    s2[600, 5] = 0xBC00
    got, flag = _run_w4a16(co, x, q, s2, m, n, k, variant=GFX950)
    assert flag == 13 and (got[:, 600] == SENTINEL).all() and (got[:, 601] != SENTINEL).all()
    for grid, block in (((n // 16 - 1, 1), 512), ((n // 16, 2), 512), ((n // 16, 1), 96)):
        got, flag = _run_w4a16(co, x, q, s, m, n, k, grid=grid, block=block, variant=GFX950)
        assert flag == 11 and (got == SENTINEL).all(), (grid, block)


def test_driver_submit_refusals(co):
    """submit_verified_kernel's refusals on a loaded module
    (verified_kernel_launcher.cpp:36-57, :10-34): stream 0, a packet whose
    logical id or parameter-ABI digest is not the function's, a packet of
    another size, zero or oversized dimensions; each is refused before
    anything is enqueued (the output stays untouched)."""
    import struct

    import torch

    from pih_amd import abi

    obj, stream = co
    m, n, k = 1, 1024, 1024
    out = torch.full((m, n), SENTINEL, dtype=torch.int16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    q, s = synth.int4_sym_weight(3, n, k)
    x = synth.bf16_normal(4, (m, k))
    xd, qd, sd = to_dev(x), to_dev(q), to_dev(s)
    packet = struct.pack("<5Q3Q", xd.data_ptr(), qd.data_ptr(), sd.data_ptr(), out.data_ptr(), flag.data_ptr(), m, n, k)
    lid = "qwen.linear.w4a16.compatibility.v1"
    ok = obj.submit(lid, packet, 4, 256, stream.cuda_stream)
    assert ok.code == abi.OK
    stream.synchronize()
    good = to_host(out.view(torch.bfloat16)).copy()
    out.fill_(SENTINEL)
    torch.cuda.synchronize()
    for what, st in (
            ("stream 0", obj.submit(lid, packet, 4, 256, 0)),
            ("other logical id", obj.submit(lid, packet, 4, 256, stream.cuda_stream,
                                            packet_logical_id="qwen.linear.w4a16.gfx950.v1")),
            ("other abi digest", obj.submit(lid, packet, 4, 256, stream.cuda_stream, abi_digest=b"0" * 64)),
            ("short packet", obj.submit(lid, packet[:56], 4, 256, stream.cuda_stream)),
            ("zero grid", obj.submit(lid, packet, 0, 256, stream.cuda_stream)),
            ("block > 1024", obj.submit(lid, packet, 4, 2048, stream.cuda_stream))):
        assert st.code == abi.INVALID_ARGUMENT, what
    stream.synchronize()
    assert (out.cpu().numpy().view(np.uint16) == SENTINEL).all()
    assert int(flag.item()) == 0
    assert_close(oracle.bf16_bits_to_f32(good), oracle.bf16_bits_to_f32(oracle.w4a16_sym(x, q, s)), "submit ok")


def test_driver_load_unload_cycle():
    """A second module of the same image loads, launches and unloads on its
    own; a refused signature leaves nothing loaded."""
    import ctypes as C

    import torch

    from pih_amd import abi, qwen
    from pih_amd.device import engine_stream

    with engine_stream() as s:
        obj = qwen.QwenCodeObject()
        m, n, k = 4, 2048, 1024
        q, sc = synth.int4_sym_weight(8, n, k)
        x = synth.bf16_normal(9, (m, k))
        got, flag = _run_w4a16((obj, s), x, q, sc, m, n, k, variant=GFX950)
        assert flag == 0
        assert_close(oracle.bf16_bits_to_f32(got), oracle.bf16_bits_to_f32(oracle.w4a16_sym(x, q, sc)), "2nd module")
        obj.unload()
        bad, _ = qwen.w4a16_signature(abi.QWEN_INT4_COMPAT, b"f" * 64)
        handle = C.c_void_p()
        st = abi.kernel_module_lib().pih_hip_kernel_module_load_v1(qwen.image_path(obj.root).encode(), C.byref(bad),
                                                                   1, C.byref(handle))
        assert st.code == abi.INVALID_ARGUMENT and not handle.value
        torch.cuda.synchronize()

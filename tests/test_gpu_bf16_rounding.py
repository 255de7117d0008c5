"""The kernels' fp32 -> bf16 output rounding is the reference's
round-to-nearest-even (include/pih/core/bfloat16.h:13-23, restated by
oracle.f32_to_bf16_bits), bit for bit, on the GEMV (M = 1) and big-tile
(M = 256) paths of launch_bf16_gemm.

Each output column n is made to hold an exact target fp32 value x_n: A's
rows are [1, 1, 1, 0, ...] and W row n holds the three bf16 pieces
h1 + h2 + h3 = x_n (the top, middle and low 8 significand bits), so every
partial sum is exact and the kernel's fp32 result is x_n itself.  The
targets cover every rounding case: exact bf16 values, ties with an even and
with an odd upper half (the tie must go to even), values just above and
below a tie, carries into the exponent, the largest finite values that
round up to infinity, and random bit patterns.
"""
import numpy as np
import pytest

import oracle
from pih_amd import abi
from tests.helpers import to_dev, to_host

pytestmark = pytest.mark.gpu

N, K = 8192, 64


@pytest.fixture(scope="module")
def eng():
    import torch

    from pih_amd.device import engine_stream

    with engine_stream() as s:
        yield s
        torch.cuda.synchronize()


def _targets(rng):
    """fp32 bit patterns with exponent fields in [18, 254] (the low piece
    h3 ~ 2^(e - 16) stays a normal bf16)."""
    hi = rng.integers(0, 1 << 16, N, dtype=np.uint32)
    exp = (hi >> 7) & 0xFF
    hi = np.where((exp < 18) | (exp > 254), (hi & 0x807F) | (0x80 << 7), hi)
    low_cases = np.array([0x0000, 0x8000, 0x7FFF, 0x8001, 0xFFFF, 0x0001, 0x4000, 0xC000], np.uint32)
    low = np.where(np.arange(N) % 2 == 0, low_cases[np.arange(N) // 2 % len(low_cases)],
                   rng.integers(0, 1 << 16, N, dtype=np.uint32))
    raw = (hi << 16) | low
    # the largest finite values: ties and beyond round up to infinity
    raw[:8] = [0x7F7F8000, 0x7F7FFFFF, 0x7F7F7FFF, 0xFF7F8000, 0x7F7E8000, 0x3F7FFFFF, 0x3F7F8000, 0x3F808000]
    return raw.view(np.float32)


def _pieces(x):
    """Three bf16 bit arrays whose exact sum is x (the 8-bit chunks of the
    significand)."""
    raw = x.view(np.uint32)
    h1 = (raw >> 16).astype(np.uint16)
    r1 = (x - oracle.bf16_bits_to_f32(h1)).astype(np.float32)
    h2 = (r1.view(np.uint32) >> 16).astype(np.uint16)
    r2 = (r1 - oracle.bf16_bits_to_f32(h2)).astype(np.float32)
    h3 = (r2.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(oracle.bf16_bits_to_f32(h3), r2), "low piece not a bf16 value"
    return h1, h2, h3


@pytest.mark.parametrize("m", [1, 256])
def test_bf16_output_rounding_is_rne(eng, m):
    import torch

    from pih_amd.device import ptr, stream_handle

    x = _targets(np.random.default_rng(0xB16))
    h1, h2, h3 = _pieces(x)
    w = np.zeros((N, K), np.uint16)
    w[:, 0], w[:, 1], w[:, 2] = h1, h2, h3
    a = np.zeros((m, K), np.uint16)
    a[:, :3] = 0x3F80  # 1.0
    out = torch.empty(m, N, dtype=torch.bfloat16, device="cuda")
    ad, wd = to_dev(a), to_dev(w)
    r = abi.request(abi.LN["bf16_gemm"], a_bf16=ptr(ad), w_bf16=ptr(wd), output=ptr(out), workspace=0,
                    workspace_bytes=0, stream=stream_handle(), m=m, n=N, k=K, output_type=abi.OUTPUT_BF16)
    st = abi.linear_pack().call("launch_bf16_gemm", r)
    assert st.code == abi.OK, st
    torch.cuda.synchronize()
    got = to_host(out).view(np.uint16)
    want = oracle.f32_to_bf16_bits(x)
    for row in (0, m - 1):
        bad = np.nonzero(got[row] != want)[0]
        assert bad.size == 0, [(hex(int(x.view(np.uint32)[i])), hex(int(got[row, i])), hex(int(want[i])))
                               for i in bad[:5]]

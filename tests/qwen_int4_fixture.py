"""The reference's closed-form INT4 GEMM fixture, restated as test data
(src/backend/cuda/qwen_int4_cuda_fixture.cpp:87-140 builds the inputs and
expected outputs; :296-302 lists the (m, n, k, seed) matrix; :291 the
seed-0 positional case).

Input rows are constants from a 7-value pattern, symmetric INT4 weights
either at six fixed positions (seed 0, scales 1.0 / 0.5 by group parity) or
from a 64-bit mix of (seed, output, k) (scales 0.25 / 0.5 / 1 / 2 by
group + output + seed); expected[row, n] = bf16(x_row * sum_k q * s).  Every
term and partial sum is a multiple of 1/16 below 2^17, so any summation
order is exact and the expected values are bit-exact targets -- with one
correction: where a sum cancels to exactly zero and x_row is negative the
fixture's bf16(x * 0) is -0, while the kernel it checks accumulates
x * (q * s) from +0 in k order (kernels/cuda/qwen_bf16_primitives.cu:
132-146), and a round-to-nearest sum that cancels is +0; ``case`` returns
the kernel's +0 there (``fixture_expected`` keeps the fixture's own bits).
"""
import numpy as np

ROW_PATTERN = np.array([1.0, -0.5, 2.0, -1.5, 0.25, 0.75, -2.0], np.float32)
SHAPE_MATRIX = ((1, 2048, 1024, 0x51A7), (2, 1024, 1024, 0x62B8), (3, 1024, 2048, 0x73C9),
                (7, 3072, 1024, 0x84DA), (17, 1024, 3072, 0x95EB))
POSITIONAL_CASE = (3, 1024, 1024, 0)


def _bf16(x: np.ndarray) -> np.ndarray:
    raw = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((raw + 0x7FFF + ((raw >> 16) & 1)) >> 16).astype(np.uint16)


def case(m: int, n: int, k: int, seed: int):
    """(x bf16 [m, k], packed u8 [n, k/2], scales fp16 bits [n, k/128],
    expected bf16 [m, n] with exact zero sums as +0)."""
    groups = k // 128
    x = np.repeat(_bf16(ROW_PATTERN[np.arange(m) % 7])[:, None], k, axis=1)
    out_idx = np.arange(n, dtype=np.uint64)
    grp = np.arange(groups, dtype=np.uint64)
    q = np.zeros((n, k), np.int64)
    if seed == 0:
        scale = np.where(grp % 2 == 0, 1.0, 0.5)[None, :].repeat(n, 0)
        direction = np.where(out_idx % 2 == 0, 1, -1)[:, None]
        positions = [0, 1, 127, 128, 129, k - 1]
        values = np.array([-7, -1, 1, 7, -7, 1])
        q[:, positions] = values[None, :] * direction
    else:
        table = np.array([0.25, 0.5, 1.0, 2.0])
        scale = table[(grp[None, :] + out_idx[:, None] + np.uint64(seed)) & np.uint64(3)]
        with np.errstate(over="ignore"):
            o1 = (out_idx + np.uint64(1)) * np.uint64(0x9E3779B97F4A7C15)
            i1 = (np.arange(k, dtype=np.uint64) + np.uint64(1)) * np.uint64(0xBF58476D1CE4E5B9)
            mixed = np.uint64(seed) ^ o1[:, None]
            mixed = mixed ^ i1[None, :]
            mixed ^= mixed >> np.uint64(30)
            mixed = mixed * np.uint64(0xBF58476D1CE4E5B9)
            mixed ^= mixed >> np.uint64(27)
        q = (mixed % np.uint64(15)).astype(np.int64) - 7
    nib = (q & 0xF).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    scales = scale.astype(np.float16).view(np.uint16)
    sums = (q.astype(np.float64) * np.repeat(scale, 128, axis=1)).sum(axis=1)
    expected = fixture_expected = _bf16(
        (ROW_PATTERN[np.arange(m) % 7][:, None].astype(np.float64) * sums[None, :]).astype(np.float32))
    expected = np.where(fixture_expected == 0x8000, np.uint16(0), fixture_expected)
    return x, packed, scales, expected

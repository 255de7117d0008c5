"""Seeded synthetic inputs for the five BASELINE configurations.

SplitMix64 streams (one per (config, tensor) seed), Box-Muller normals in
float64 rounded to bf16 with round-to-nearest-even, uniforms for INT4 codes,
scales and zero points.  Everything here is host-side numpy and is used for
the sizes that fit comfortably in host memory; the full-size cfg4/cfg5 expert
weights are generated on the device by the pack's own fill kernels.
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)


def config_seed(cfg: int, tensor: int) -> int:
    """seed = 0x504948_00 + cfg, combined with a per-tensor index."""
    return ((0x50494800 + cfg) << 16) ^ (tensor * 0x9E37)


def splitmix64(seed: int, count: int) -> np.ndarray:
    i = np.arange(1, count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform(seed: int, count: int) -> np.ndarray:
    """float64 in [0, 1) from the top 53 bits."""
    return (splitmix64(seed, count) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, count: int, std: float = 1.0) -> np.ndarray:
    n2 = (count + 1) // 2
    u = uniform(seed, 2 * n2)
    u1 = np.maximum(u[0::2], 1e-300)
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * n2)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return z[:count] * std


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    raw = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (raw & 0x7FFFFFFF) > 0x7F800000
    rounded = ((raw + 0x7FFF + ((raw >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((raw >> 16) | 0x0040).astype(np.uint16), rounded)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_normal(seed: int, shape, std: float = 1.0) -> np.ndarray:
    count = int(np.prod(shape))
    return f32_to_bf16_bits(normal(seed, count, std).astype(np.float32)).reshape(shape)


# ------------------------------------------------------------------- fp8
def e4m3_encode(v: np.ndarray) -> np.ndarray:
    """Nearest finite e4m3fn code, ties to even; |v| <= 448 (vectorised form of
    the reference's exhaustive search in deepseek_fp8_activation_codec.cpp:27-51)."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    sign = (np.signbit(v).astype(np.uint32) << 7)
    mag = np.abs(v)
    raw = mag.view(np.uint32)
    exp = ((raw >> 23) & 0xFF).astype(np.int32) - 127
    sub = np.rint(mag.astype(np.float64) * 512.0).astype(np.uint32)
    mant = raw & 0x7FFFFF
    q = mant >> 20
    rem = mant & 0xFFFFF
    up = (rem > 0x80000) | ((rem == 0x80000) & ((q & 1) == 1))
    q = q + up.astype(np.uint32)
    e = exp + (q == 8)
    q = np.where(q == 8, 0, q)
    normal_code = (np.clip(e + 7, 0, 15).astype(np.uint32) << 3) | q
    code = np.where(exp < -6, sub, normal_code)
    code = np.where(mag == 0, 0, code)
    return (code | sign).astype(np.uint8)


def e4m3_decode_table() -> np.ndarray:
    t = np.zeros(256, np.float32)
    for b in range(256):
        e, m = (b >> 3) & 15, b & 7
        if e == 15 and m == 7:
            t[b] = np.nan
            continue
        mag = np.ldexp(m, -9) if e == 0 else np.ldexp(1.0 + m / 8.0, e - 7)
        t[b] = -mag if b & 0x80 else mag
    return t


def fp8_block_weight(seed: int, rows: int, cols: int, std: float = 0.02):
    """W ~ N(0, std) quantised per 128x128 block with an fp32 scale
    s = amax / 448 (DeepSeek-V3 style); returns (codes [rows, cols] u8,
    scales [rows/128, cols/128] f32)."""
    w = normal(seed, rows * cols, std).astype(np.float32).reshape(rows // 128, 128, cols // 128, 128)
    amax = np.abs(w).max(axis=(1, 3))
    s = (np.maximum(amax, 1e-12) / 448.0).astype(np.float32)
    q = np.clip(w / s[:, None, :, None], -448.0, 448.0)
    codes = e4m3_encode(q.reshape(-1)).reshape(rows // 128, 128, cols // 128, 128)
    return codes.reshape(rows, cols), s


def ue8m0_block_weight(seed: int, rows: int, cols: int, std: float = 0.02):
    """Reference-format FP8 weight: power-of-two UE8M0 scale per 128x128 block
    (scale = 2^ceil(log2(amax/448)))."""
    w = normal(seed, rows * cols, std).astype(np.float32).reshape(rows // 128, 128, cols // 128, 128)
    amax = np.maximum(np.abs(w).max(axis=(1, 3)), 1e-4)
    e = np.ceil(np.log2(amax.astype(np.float64) / 448.0)).astype(np.int32)
    q = np.clip(w / np.ldexp(1.0, e)[:, None, :, None], -448.0, 448.0)
    codes = e4m3_encode(q.reshape(-1).astype(np.float32)).reshape(rows // 128, 128, cols // 128, 128)
    return codes.reshape(rows, cols), (e + 127).astype(np.uint8)


# ------------------------------------------------------------------ MXFP4
def mxfp4_weight(seed: int, rows: int, cols: int):
    """e2m1 codes packed two per byte (low nibble = even k) with an e8m0 scale
    per (row, 32 columns).  Codes uniform over the 15 non-negative-zero
    values, scale bytes uniform in [118, 124] (magnitudes ~2^-9..2^-3 x 6)."""
    u = splitmix64(seed, rows * cols)
    nib = (u % np.uint64(16)).astype(np.uint8).reshape(rows, cols)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    su = splitmix64(seed ^ 0x5CA1E, rows * (cols // 32))
    scales = (118 + (su % np.uint64(7))).astype(np.uint8).reshape(rows, cols // 32)
    return packed, scales


# ------------------------------------------------------------------- INT4
def int4_asym_weight(seed: int, n: int, k: int):
    """BASELINE cfg3 weight: q uniform in [0,15] packed 8 per u32 along k (low
    nibble = lowest k), bf16 scale ~U(0.001, 0.02) per (n, 128 k), int4 zero
    point per (n, group) packed 8 per u32 along the group axis."""
    q = (splitmix64(seed, n * k) % np.uint64(16)).astype(np.uint32).reshape(n, k // 8, 8)
    qweight = np.zeros((n, k // 8), np.uint32)
    for j in range(8):
        qweight |= q[:, :, j] << np.uint32(4 * j)
    groups = k // 128
    s = 0.001 + 0.019 * uniform(seed ^ 0x5CA1E, n * groups)
    scales = f32_to_bf16_bits(s.astype(np.float32)).reshape(n, groups)
    zw = (groups + 7) // 8
    z = (splitmix64(seed ^ 0x2E60, n * zw * 8) % np.uint64(16)).astype(np.uint32).reshape(n, zw, 8)
    zeros = np.zeros((n, zw), np.uint32)
    for j in range(8):
        zeros |= z[:, :, j] << np.uint32(4 * j)
    return qweight, scales, zeros


def int4_sym_weight(seed: int, n: int, k: int):
    """Reference-format (xing-w4a16-sym-g128-v1) weight: signed codes in
    [-7, 7] (nibble 8 never produced), low nibble = even k, fp16 scale per
    (n, 128 k) drawn from powers of two and ~U(0.001, 0.02)."""
    v = (splitmix64(seed, n * k) % np.uint64(15)).astype(np.int32).reshape(n, k) - 7
    nib = (v & 0xF).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    s = (0.001 + 0.019 * uniform(seed ^ 0x5CA1E, n * (k // 128))).astype(np.float16)
    return packed, s.view(np.uint16).reshape(n, k // 128)


# ----------------------------------------------------------------- router
def zipf_router(seed: int, tokens: int, experts: int, topk: int, alpha: float = 1.1):
    """Router logits ~N(0,1) plus a log-Zipf(alpha) bias over a seeded expert
    permutation; softmax; top-k (ties -> lower expert id); weights
    renormalised to sum 1.  Returns (ids u32 [T,k], weights f32 [T,k])."""
    logits = normal(seed, tokens * experts).reshape(tokens, experts)
    perm = np.argsort(splitmix64(seed ^ 0xA11CE, experts), kind="stable")
    rank = np.empty(experts, np.int64)
    rank[perm] = np.arange(experts)
    bias = -alpha * np.log1p(rank.astype(np.float64))
    z = logits + bias[None, :]
    z = z - z.max(axis=1, keepdims=True)
    p = np.exp(z)
    p = p / p.sum(axis=1, keepdims=True)
    order = np.argsort(-p, axis=1, kind="stable")[:, :topk]
    w = np.take_along_axis(p, order, axis=1)
    w = w / w.sum(axis=1, keepdims=True)
    return order.astype(np.uint32), w.astype(np.float32)

"""CPU oracle for the linear-layer hot path — TEST INFRASTRUCTURE ONLY.

Python bindings over ``oracle/_build/libpih_oracle.so`` (the C restatement in
``oracle/pih_oracle.c``) and, where it was built, ``oracle/_ref/libpih_ref.so``
(the reference's own CPU oracle sources compiled in place, see
``oracle/Makefile``).  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or the timed CPU baseline; the product packs never call it.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libpih_oracle.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libpih_ref.so")

_lib: Optional[C.CDLL] = None
_ref: Optional[C.CDLL] = None

P = C.c_void_p
U32 = C.c_uint32
U64 = C.c_uint64
F32 = C.c_float


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(P)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle not built: {_LIB_PATH} (run __graft_entry__.build())")
        L = C.CDLL(_LIB_PATH)
        sigs = {
            "po_set_threads": (None, [C.c_int]),
            "po_get_threads": (C.c_int, []),
            "po_bf16_from_f32": (C.c_uint16, [F32]),
            "po_bf16_to_f32": (F32, [C.c_uint16]),
            "po_f16_from_f32": (C.c_uint16, [F32]),
            "po_f16_to_f32": (F32, [C.c_uint16]),
            "po_e4m3_decode": (C.c_int, [C.c_uint8, C.POINTER(F32)]),
            "po_e4m3_encode": (C.c_int, [F32, C.POINTER(C.c_uint8)]),
            "po_mxfp4_decode_scalar": (C.c_int, [C.c_uint8, C.c_uint8, C.POINTER(C.c_double)]),
            "po_mxfp4_decode_row": (C.c_int, [P, P, U32, P]),
            "po_fp8_quant_ue8m0": (C.c_int, [P, U32, U32, P, P]),
            "po_fp8_quant_f32": (C.c_int, [P, U32, U32, P, P]),
            "po_fp8_gemm_ue8m0": (C.c_int, [P, P, P, P, U32, U32, U32, P]),
            "po_fp8_gemm_f32": (C.c_int, [P, P, P, P, U32, U32, U32, P]),
            "po_fp4_gemm": (C.c_int, [P, P, P, P, U32, U32, U32, P]),
            "po_mxfp4_bf16_gemm": (C.c_int, [P, P, P, U32, U32, U32, P]),
            "po_w4a16_sym": (C.c_int, [P, P, P, U32, U32, U32, P]),
            "po_w4a16_asym": (C.c_int, [P, P, P, P, U32, U32, U32, P]),
            "po_w4a16_asym_dequant": (C.c_int, [P, P, P, U32, U32, P]),
            "po_bf16_gemm": (None, [P, P, U32, U32, U32, P]),
            "po_lm_head": (U32, [P, P, U32, U32, U32, P]),
            "po_v41_fp4_block_to_fp8": (C.c_int, [P, P, P, P]),
            "po_v41_fp4_to_fp8": (C.c_int, [P, P, U32, U32, P, P]),
            "po_v41_dequant_block": (C.c_int, [P, F32, U32, P]),
            "po_v41_quant32": (U32, [P, U32, U32, P, P]),
            "po_v41_linear": (U32, [P, P, P, P, U32, U32, U32, C.c_int, P]),
            "po_silu_mul": (None, [P, P, C.c_size_t, P]),
            "po_swiglu": (C.c_int, [P, P, C.c_size_t, F32, P]),
            "po_route_plan": (C.c_int, [P, P, U32, U32, U32, P, P, P, P]),
            "po_ordered_accumulate": (C.c_int, [P, P, U32, U32, U32, P]),
            "po_finalize": (C.c_int, [P, P, C.c_size_t, P]),
            "po_routed_expert_fp4": (C.c_int, [P, P, U32, U32, U32, P, P, P, P, P, P, P]),
            "po_expert_fp8": (C.c_int, [P, P, U32, U32, U32, P, P, P, P, F32, P]),
            "po_router_topk": (C.c_int, [P, P, U32, U32, U32, U32, F32, P, P]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def ref() -> Optional[C.CDLL]:
    """The reference's own oracles, or None where oracle/_ref was not built."""
    global _ref
    if _ref is None and os.path.exists(_REF_PATH):
        R = C.CDLL(_REF_PATH)
        sigs = {
            "pr_bf16_from_f32": (C.c_uint16, [F32]),
            "pr_f16_from_f32": (C.c_uint16, [F32]),
            "pr_f16_to_f32": (F32, [C.c_uint16]),
            "pr_e4m3_decode": (C.c_int, [C.c_uint8, C.POINTER(F32)]),
            "pr_e4m3_encode": (C.c_int, [F32, C.POINTER(C.c_uint8)]),
            "pr_fp8_quant": (C.c_int, [P, U32, U32, P, P]),
            "pr_fp8_gemm": (C.c_int, [P, P, P, P, U32, U32, U32, P]),
            "pr_fp4_gemm": (C.c_int, [P, P, P, P, U32, U32, U32, P]),
            "pr_mxfp4_decode_row": (C.c_int, [P, P, U32, P]),
            "pr_swiglu": (C.c_int, [P, P, U32, U32, F32, P]),
            "pr_silu_mul": (C.c_int, [P, P, C.c_size_t, P]),
            "pr_subwave_plan": (C.c_int, [P, P, P, P, U32, P, P, P, P, P]),
            "pr_accumulate": (C.c_int, [P, U32, P, P, U32, P, P]),
            "pr_routed_expert": (C.c_int, [P, P, U32, U32, U32, P, P, P, P, P, P, P]),
            "pr_int4_quantize": (C.c_int, [P, U64, U64, P, P]),
            "pr_learned_router": (C.c_int, [P, U32, P, P, P]),
            "pr_qwen_int4_metadata": (C.c_int, [P, P, P, P]),
            "pr_qwen_int4_parse": (C.c_int, [P]),
            "pr_v41_fp4_block_to_fp8": (C.c_int, [P, P, P, P]),
            "pr_v41_dequant_block": (C.c_int, [P, F32, U32, P]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(R, name)
            fn.restype = res
            fn.argtypes = args
        _ref = R
    return _ref


def set_threads(n: int) -> None:
    lib().po_set_threads(int(n))


class OracleError(RuntimeError):
    def __init__(self, fn: str, code: int):
        super().__init__(f"{fn} rejected its input (code {code})")
        self.code = code


def _check(fn: str, code: int) -> None:
    if code:
        raise OracleError(fn, code)


# ------------------------------------------------------------------ codecs
def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """include/pih/core/bfloat16.h:13-23, vectorised (identical bits)."""
    raw = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (raw & 0x7FFFFFFF) > 0x7F800000
    rounded = ((raw + 0x7FFF + ((raw >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((raw >> 16) | 0x0040).astype(np.uint16), rounded)


def e4m3_decode(bits: int):
    v = F32()
    bad = lib().po_e4m3_decode(int(bits), C.byref(v))
    return None if bad else v.value


def e4m3_table() -> np.ndarray:
    """float32[256]; NaN for the two NaN codes."""
    t = np.empty(256, np.float32)
    for b in range(256):
        v = e4m3_decode(b)
        t[b] = np.nan if v is None else v
    return t


def e4m3_encode(value: float):
    b = C.c_uint8()
    bad = lib().po_e4m3_encode(float(value), C.byref(b))
    return None if bad else b.value


def mxfp4_decode_row(packed: np.ndarray, scales: np.ndarray, k: int) -> np.ndarray:
    out = np.empty(k, np.float32)
    _check("po_mxfp4_decode_row",
           lib().po_mxfp4_decode_row(_ptr(packed), _ptr(scales), k, _ptr(out)))
    return out


# ------------------------------------------------------- activation quant
def fp8_quant_ue8m0(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    t, k = x.shape
    q = np.empty((t, k), np.uint8)
    s = np.empty((t, k // 128), np.uint8)
    _check("po_fp8_quant_ue8m0", lib().po_fp8_quant_ue8m0(_ptr(x), t, k, _ptr(q), _ptr(s)))
    return q, s


def fp8_quant_f32(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    t, k = x.shape
    q = np.empty((t, k), np.uint8)
    s = np.empty((t, k // 128), np.float32)
    _check("po_fp8_quant_f32", lib().po_fp8_quant_f32(_ptr(x), t, k, _ptr(q), _ptr(s)))
    return q, s


# ------------------------------------------------------------------ GEMMs
def fp8_gemm_ue8m0(a, sa, w, sw) -> np.ndarray:
    m, k = a.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float32)
    _check("po_fp8_gemm_ue8m0", lib().po_fp8_gemm_ue8m0(
        _ptr(a), _ptr(sa), _ptr(w), _ptr(sw), m, n, k, _ptr(out)))
    return out


def fp8_gemm_f32(a, sa, w, sw) -> np.ndarray:
    m, k = a.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float32)
    _check("po_fp8_gemm_f32", lib().po_fp8_gemm_f32(
        _ptr(a), _ptr(np.ascontiguousarray(sa, np.float32)), _ptr(w),
        _ptr(np.ascontiguousarray(sw, np.float32)), m, n, k, _ptr(out)))
    return out


def fp4_gemm(a, sa, packed, sw) -> np.ndarray:
    m, k = a.shape
    n = packed.shape[0]
    out = np.empty((m, n), np.float32)
    _check("po_fp4_gemm", lib().po_fp4_gemm(
        _ptr(a), _ptr(sa), _ptr(packed), _ptr(sw), m, n, k, _ptr(out)))
    return out


def mxfp4_bf16_gemm(x_bits, packed, sw) -> np.ndarray:
    m, k = x_bits.shape
    n = packed.shape[0]
    out = np.empty((m, n), np.float32)
    _check("po_mxfp4_bf16_gemm", lib().po_mxfp4_bf16_gemm(
        _ptr(x_bits), _ptr(packed), _ptr(sw), m, n, k, _ptr(out)))
    return out


def w4a16_sym(x_bits, packed, scales_f16) -> np.ndarray:
    m, k = x_bits.shape
    n = packed.shape[0]
    out = np.empty((m, n), np.uint16)
    _check("po_w4a16_sym", lib().po_w4a16_sym(
        _ptr(x_bits), _ptr(packed), _ptr(scales_f16), m, n, k, _ptr(out)))
    return out


def w4a16_asym(x_bits, qweight, scales_bf16, zeros) -> np.ndarray:
    m, k = x_bits.shape
    n = qweight.shape[0]
    out = np.empty((m, n), np.uint16)
    _check("po_w4a16_asym", lib().po_w4a16_asym(
        _ptr(x_bits), _ptr(qweight), _ptr(scales_bf16), _ptr(zeros), m, n, k, _ptr(out)))
    return out


def w4a16_asym_dequant(qweight, scales_bf16, zeros, k: int) -> np.ndarray:
    n = qweight.shape[0]
    w = np.empty((n, k), np.float32)
    _check("po_w4a16_asym_dequant", lib().po_w4a16_asym_dequant(
        _ptr(qweight), _ptr(scales_bf16), _ptr(zeros), n, k, _ptr(w)))
    return w


def bf16_gemm(a_bits, w_bits) -> np.ndarray:
    m, k = a_bits.shape
    n = w_bits.shape[0]
    out = np.empty((m, n), np.float32)
    lib().po_bf16_gemm(_ptr(a_bits), _ptr(w_bits), m, n, k, _ptr(out))
    return out


def lm_head(x_bits, w_bits):
    """DeepSeek LM head logits (fp32, the reference kernel's 256-way strided
    partial sums and tree) and its error bits (64 non-finite operand, 128
    non-finite logit)."""
    rows, hidden = x_bits.shape
    vocab = w_bits.shape[0]
    out = np.empty((rows, vocab), np.float32)
    err = lib().po_lm_head(_ptr(np.ascontiguousarray(x_bits)), _ptr(np.ascontiguousarray(w_bits)), rows, vocab,
                           hidden, _ptr(out))
    return out, int(err)


# ------------------------------------------------ DeepSeek V4.1 32-blocks
def v41_fp4_block_to_fp8(packed, scales):
    """One 32x32 block: (e4m3 [32, 32], shared UE8M0, status code)."""
    w = np.empty(1024, np.uint8)
    s = np.zeros(1, np.uint8)
    st = lib().po_v41_fp4_block_to_fp8(_ptr(np.ascontiguousarray(packed, np.uint8)),
                                       _ptr(np.ascontiguousarray(scales, np.uint8)), _ptr(w), _ptr(s))
    return w.reshape(32, 32), int(s[0]), int(st)


def v41_fp4_to_fp8(packed, scales):
    rows, half = packed.shape
    cols = half * 2
    w = np.empty((rows, cols), np.uint8)
    s = np.empty((rows // 32, cols // 32), np.uint8)
    _check("po_v41_fp4_to_fp8", lib().po_v41_fp4_to_fp8(_ptr(np.ascontiguousarray(packed)),
                                                        _ptr(np.ascontiguousarray(scales)), rows, cols, _ptr(w),
                                                        _ptr(s)))
    return w, s


def v41_dequant_block(src, scale, block):
    out = np.empty(block * block, np.uint16)
    st = lib().po_v41_dequant_block(_ptr(np.ascontiguousarray(src, np.uint8)), float(np.float32(scale)), block,
                                    _ptr(out))
    return out, int(st)


def v41_quant32(x_bits):
    rows, k = x_bits.shape
    codes = np.empty((rows, k), np.uint8)
    scales = np.empty((rows, k // 32), np.uint8)
    err = lib().po_v41_quant32(_ptr(np.ascontiguousarray(x_bits)), rows, k, _ptr(codes), _ptr(scales))
    return codes, scales, int(err)


def v41_linear(a, sa, w, sw, n, fp4):
    """bf16 [rows, n] and error bits of the V4.1 projection."""
    rows, k = a.shape
    out = np.empty((rows, n), np.uint16)
    err = lib().po_v41_linear(_ptr(np.ascontiguousarray(a)), _ptr(np.ascontiguousarray(sa)),
                              _ptr(np.ascontiguousarray(w)), _ptr(np.ascontiguousarray(sw)), rows, n, k,
                              1 if fp4 else 0, _ptr(out))
    return out, int(err)


# ------------------------------------------------------------ elementwise
def silu_mul(g_bits, u_bits) -> np.ndarray:
    out = np.empty_like(g_bits)
    lib().po_silu_mul(_ptr(g_bits), _ptr(u_bits), g_bits.size, _ptr(out))
    return out


def swiglu(g, u, limit: float) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    _check("po_swiglu", lib().po_swiglu(_ptr(g), _ptr(u), g.size, float(limit), _ptr(out)))
    return out


# -------------------------------------------------------------------- MoE
def route_plan(topk_ids: np.ndarray, topk_weights: np.ndarray, experts: int):
    ids = np.ascontiguousarray(topk_ids, np.uint32)
    w = np.ascontiguousarray(topk_weights, np.float32)
    t, k = ids.shape
    offsets = np.empty(experts + 1, np.uint32)
    row_token = np.empty(t * k, np.uint32)
    row_weight = np.empty(t * k, np.float32)
    token_rows = np.empty((t, k), np.uint32)
    _check("po_route_plan", lib().po_route_plan(
        _ptr(ids), _ptr(w), t, k, experts, _ptr(offsets), _ptr(row_token),
        _ptr(row_weight), _ptr(token_rows)))
    return offsets, row_token, row_weight, token_rows


def ordered_accumulate(expert_out_bits, row_token, tokens: int) -> np.ndarray:
    rows, hidden = expert_out_bits.shape
    acc = np.zeros((tokens, hidden), np.float32)
    _check("po_ordered_accumulate", lib().po_ordered_accumulate(
        _ptr(expert_out_bits), _ptr(np.ascontiguousarray(row_token, np.uint32)),
        rows, tokens, hidden, _ptr(acc)))
    return acc


def finalize(acc, shared_bits=None) -> np.ndarray:
    out = np.empty(acc.shape, np.uint16)
    _check("po_finalize", lib().po_finalize(
        _ptr(acc), None if shared_bits is None else _ptr(shared_bits), acc.size, _ptr(out)))
    return out


def routed_expert_fp4(x_bits, route_weights, hidden, inter, w1p, w1s, w2p, w2s, w3p, w3s):
    t = x_bits.shape[0]
    out = np.empty((t, hidden), np.uint16)
    _check("po_routed_expert_fp4", lib().po_routed_expert_fp4(
        _ptr(x_bits), _ptr(np.ascontiguousarray(route_weights, np.float32)), t, hidden,
        inter, _ptr(w1p), _ptr(w1s), _ptr(w2p), _ptr(w2s), _ptr(w3p), _ptr(w3s), _ptr(out)))
    return out


def expert_fp8(x_bits, route_weights, hidden, inter, w13, w13s, w2, w2s, limit=0.0):
    t = x_bits.shape[0]
    out = np.empty((t, hidden), np.uint16)
    _check("po_expert_fp8", lib().po_expert_fp8(
        _ptr(x_bits), _ptr(np.ascontiguousarray(route_weights, np.float32)), t, hidden,
        inter, _ptr(w13), _ptr(np.ascontiguousarray(w13s, np.float32)), _ptr(w2),
        _ptr(np.ascontiguousarray(w2s, np.float32)), float(limit), _ptr(out)))
    return out


def moe_fp8_forward(x_bits, topk_ids, topk_weights, experts, hidden, inter,
                    w13, w13s, w2, w2s, limit=0.0, expert_subset=None):
    """Whole cfg4 MoE on the CPU: route plan -> per-expert chain
    (po_expert_fp8) -> ordered accumulate -> bf16.  Returns (out_bits,
    per-row expert outputs, plan).  ``expert_subset`` restricts the work to the
    listed experts (rows of other experts are left zero and the combined
    output is then only meaningful for tokens routed solely into the subset).
    """
    t = x_bits.shape[0]
    offsets, row_token, row_weight, token_rows = route_plan(topk_ids, topk_weights, experts)
    y = np.zeros((row_token.size, hidden), np.uint16)
    todo = range(experts) if expert_subset is None else expert_subset
    for e in todo:
        b, en = int(offsets[e]), int(offsets[e + 1])
        if b == en:
            continue
        xs = np.ascontiguousarray(x_bits[row_token[b:en]])
        y[b:en] = expert_fp8(xs, row_weight[b:en], hidden, inter, w13[e], w13s[e], w2[e], w2s[e], limit)
    acc = ordered_accumulate(y, row_token, t)
    return finalize(acc), y, (offsets, row_token, row_weight, token_rows)


def qwen_mlp(x_bits, wg_bits, wu_bits, wd_bits):
    """Qwen3 MLP block as the reference computes it:
    gate and up through the BF16 linear (fp32 strict-k dot, bf16 RNE out,
    GemmPlan at src/backend/cuda/gemm_plan.cpp:169-198), SiLU-mul with one
    rounding at its output (plugins/model-qwen3/qwen3_cpu_oracle.cpp:114-126),
    then the down linear.  Returns the bf16 bits [M, hidden]."""
    gate = f32_to_bf16_bits(bf16_gemm(x_bits, wg_bits))
    up = f32_to_bf16_bits(bf16_gemm(x_bits, wu_bits))
    h = silu_mul(gate, up)
    return f32_to_bf16_bits(bf16_gemm(h, wd_bits))


ROUTER_SOFTMAX, ROUTER_SQRT_SOFTPLUS = 1, 2


def router_topk(scores, topk: int, mode: int, scale: float = 1.0, bias=None):
    """po_router_topk: (ids u32 [T, k], weights f32 [T, k]) in rank order."""
    s = np.ascontiguousarray(scores, np.float32)
    t, e = s.shape
    ids = np.empty((t, topk), np.uint32)
    w = np.empty((t, topk), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    _check("po_router_topk", lib().po_router_topk(
        _ptr(s), None if b is None else _ptr(b), t, e, topk, mode, float(scale), _ptr(ids), _ptr(w)))
    return ids, w

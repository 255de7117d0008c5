"""Python-side callers of the gfx950 pack tables (torch tensors in, torch
tensors out).  Every function goes through the C ABI of the built packs
(``pih_amd.abi``); there is no fallback: a missing pack or a non-OK status
raises.

Layouts (row-major):
  e4m3 codes   uint8 [rows, K], scales fp32 or uint8 (UE8M0) [rows, K/128]
  FP8 weights  uint8 [E, N, K], scales [E, N/128, K/128]
  MXFP4        uint8 [E, N, K/2] (low nibble = even k), UE8M0 [E, N, K/32]
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import abi
from .device import error_flag, ptr, stream_handle


class KernelError(RuntimeError):
    pass


def _check(status: abi.Status, what: str) -> None:
    if status.code != abi.OK:
        raise KernelError(f"{what}: {status!r}")


def _ln():
    return abi.linear_pack()


def _ds():
    return abi.deepseek_pack()


# ------------------------------------------------------------ route plan
def route_plan_workspace(tokens: int, topk: int, experts: int) -> int:
    out = (abi.C.c_uint64 * 1)()
    q = abi.request(abi.LN["workspace_query"], kind=abi.WORKSPACE_ROUTE_PLAN, m=tokens, n=topk, k=experts,
                    bytes_u64=abi.C.addressof(out))
    _check(_ln().call("query_workspace", q), "query_workspace")
    return int(out[0])


def bf16_gemm_workspace(m: int, n: int, k: int) -> int:
    """Scratch bytes launch_bf16_gemm can use at this shape (query_workspace;
    0: none)."""
    out = (abi.C.c_uint64 * 1)()
    q = abi.request(abi.LN["workspace_query"], kind=abi.WORKSPACE_BF16_GEMM, m=m, n=n, k=k,
                    bytes_u64=abi.C.addressof(out))
    _check(_ln().call("query_workspace", q), "query_workspace")
    return int(out[0])


def route_plan(topk_ids: torch.Tensor, topk_weights: torch.Tensor, experts: int,
               flag: Optional[torch.Tensor] = None):
    """Returns (expert_offsets [E+1], row_token [R], row_weight [R],
    token_rows [T, k], flag)."""
    tokens, topk = topk_ids.shape
    dev = topk_ids.device
    ws = torch.empty(route_plan_workspace(tokens, topk, experts), dtype=torch.uint8, device=dev)
    offsets = torch.empty(experts + 1, dtype=torch.int32, device=dev)
    row_token = torch.empty(tokens * topk, dtype=torch.int32, device=dev)
    row_weight = torch.empty(tokens * topk, dtype=torch.float32, device=dev)
    token_rows = torch.empty(tokens, topk, dtype=torch.int32, device=dev)
    flag = error_flag() if flag is None else flag
    r = abi.request(abi.LN["route_plan"], topk_ids_u32=ptr(topk_ids), topk_weights_f32=ptr(topk_weights),
                    expert_offsets_u32=ptr(offsets), row_token_u32=ptr(row_token),
                    row_weight_f32=ptr(row_weight), token_rows_u32=ptr(token_rows), workspace=ptr(ws),
                    workspace_bytes=ws.numel(), error_flag_u32=ptr(flag), stream=stream_handle(),
                    token_count=tokens, top_k=topk, expert_count=experts)
    _check(_ln().call("launch_route_plan", r), "route_plan")
    return offsets, row_token, row_weight, token_rows, flag


def router_topk(scores: torch.Tensor, topk: int, mode: int, route_scale: float = 1.0,
                bias: Optional[torch.Tensor] = None, flag: Optional[torch.Tensor] = None,
                out: Optional[Tuple[torch.Tensor, torch.Tensor]] = None):
    """Raw router scores f32 [T, E] -> (topk_ids int32 [T, k], topk_weights
    f32 [T, k], flag) on the device (``launch_router_topk``): softmax top-k
    renormalised (abi.ROUTER_SOFTMAX) or the V4 learned router's
    sqrt-softplus + bias selection (abi.ROUTER_SQRT_SOFTPLUS)."""
    tokens, experts = scores.shape
    if out is None:
        out = (torch.empty(tokens, topk, dtype=torch.int32, device=scores.device),
               torch.empty(tokens, topk, dtype=torch.float32, device=scores.device))
    ids, wts = out
    flag = error_flag() if flag is None else flag
    r = abi.request(abi.LN["router_topk"], scores_f32=ptr(scores), bias_f32=ptr(bias), topk_ids_u32=ptr(ids),
                    topk_weights_f32=ptr(wts), error_flag_u32=ptr(flag), stream=stream_handle(),
                    token_count=tokens, expert_count=experts, top_k=topk, mode=mode, route_scale=route_scale)
    _check(_ln().call("launch_router_topk", r), "router_topk")
    return ids, wts, flag


# ------------------------------------------------------------- FP8 quant
def fp8_quant(x: torch.Tensor, scale_format: int, rows: Optional[torch.Tensor] = None,
              flag: Optional[torch.Tensor] = None):
    """bf16 [R, K] (or gathered via rows) -> (codes uint8, scales, flag)."""
    n_out = x.shape[0] if rows is None else rows.numel()
    k = x.shape[1]
    codes = torch.empty(n_out, k, dtype=torch.uint8, device=x.device)
    sdt = torch.float32 if scale_format == abi.SCALE_F32 else torch.uint8
    scales = torch.empty(n_out, k // 128, dtype=sdt, device=x.device)
    flag = error_flag() if flag is None else flag
    r = abi.request(abi.LN["fp8_quant"], input_bf16=ptr(x), row_index_u32=ptr(rows), output_e4m3=ptr(codes),
                    scale=ptr(scales), error_flag_u32=ptr(flag), stream=stream_handle(), row_count=n_out,
                    logical_k=k, input_rows=x.shape[0], scale_format=scale_format)
    _check(_ln().call("launch_fp8_quant", r), "fp8_quant")
    return codes, scales, flag


def fp8_gemm(a, a_scale, w, w_scale, scale_format: int, output_type: int = abi.OUTPUT_BF16,
             flag: Optional[torch.Tensor] = None):
    m, k = a.shape
    n = w.shape[0]
    out = torch.empty(m, n, dtype=torch.bfloat16 if output_type == abi.OUTPUT_BF16 else torch.float32,
                      device=a.device)
    flag = error_flag() if flag is None else flag
    r = abi.request(abi.LN["fp8_gemm"], activation_e4m3=ptr(a), activation_scale=ptr(a_scale),
                    weight_e4m3=ptr(w), weight_scale=ptr(w_scale), output=ptr(out), error_flag_u32=ptr(flag),
                    stream=stream_handle(), m=m, n=n, k=k, scale_format=scale_format, output_type=output_type)
    _check(_ln().call("launch_fp8_gemm", r), "fp8_gemm")
    return out, flag


def moe_fp8_gemm(a, a_scale, row_token, w, w_scale, offsets, rows: int, scale_format: int,
                 output_type: int, row_weight=None, swiglu_limit: float = 0.0,
                 flag: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
    """Returns (out, flag); OUTPUT_SWIGLU_E4M3 returns ((codes, scales), flag)."""
    experts, n, k = w.shape
    e4m3 = output_type == abi.OUTPUT_SWIGLU_E4M3
    ncols = n // 2 if output_type in (abi.OUTPUT_SWIGLU_BF16, abi.OUTPUT_SWIGLU_E4M3) else n
    scales = None
    if e4m3:
        out = torch.empty(rows, ncols, dtype=torch.uint8, device=a.device) if out is None else out
        sdt = torch.float32 if scale_format == abi.SCALE_F32 else torch.uint8
        scales = torch.empty(rows, ncols // 128, dtype=sdt, device=a.device)
    elif out is None:
        out = torch.empty(rows, ncols, dtype=torch.float32 if output_type == abi.OUTPUT_F32 else torch.bfloat16,
                          device=a.device)
    flag = error_flag() if flag is None else flag
    r = abi.request(abi.LN["moe_fp8_gemm"], activation_e4m3=ptr(a), activation_scale=ptr(a_scale),
                    row_token_u32=ptr(row_token), weight_e4m3=ptr(w), weight_scale=ptr(w_scale),
                    expert_offsets_u32=ptr(offsets), row_weight_f32=ptr(row_weight), output=ptr(out),
                    error_flag_u32=ptr(flag), stream=stream_handle(), row_capacity=rows, expert_count=experts,
                    n=n, k=k, activation_rows=a.shape[0], scale_format=scale_format, output_type=output_type,
                    swiglu_limit=swiglu_limit, output_scale=ptr(scales))
    _check(_ln().call("launch_moe_fp8_gemm", r), "moe_fp8_gemm")
    return ((out, scales) if e4m3 else out), flag


def moe_mxfp4_gemm(a, a_scale, row_token, w_packed, w_scale, offsets, rows: int, activation_type: int,
                   output_type: int, row_weight=None, swiglu_limit: float = 0.0,
                   flag: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
    experts, n, k2 = w_packed.shape
    k = 2 * k2
    ncols = n // 2 if output_type == abi.OUTPUT_SWIGLU_BF16 else n
    if out is None:
        out = torch.empty(rows, ncols, dtype=torch.float32 if output_type == abi.OUTPUT_F32 else torch.bfloat16,
                          device=w_packed.device)
    flag = error_flag() if flag is None else flag
    r = abi.request(abi.LN["moe_mxfp4_gemm"], activation=ptr(a), activation_scale_ue8m0=ptr(a_scale),
                    row_token_u32=ptr(row_token), packed_weight=ptr(w_packed), weight_scale_ue8m0=ptr(w_scale),
                    expert_offsets_u32=ptr(offsets), row_weight_f32=ptr(row_weight), output=ptr(out),
                    error_flag_u32=ptr(flag), stream=stream_handle(), row_capacity=rows, expert_count=experts,
                    n=n, k=k, activation_rows=a.shape[0], activation_type=activation_type,
                    output_type=output_type, swiglu_limit=swiglu_limit)
    _check(_ln().call("launch_moe_mxfp4_gemm", r), "moe_mxfp4_gemm")
    return out, flag


def moe_combine(expert_out, token_rows, shared=None, flag: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None):
    rows, hidden = expert_out.shape
    tokens, topk = token_rows.shape
    if out is None:
        out = torch.empty(tokens, hidden, dtype=torch.bfloat16, device=expert_out.device)
    flag = error_flag() if flag is None else flag
    r = abi.request(abi.LN["moe_combine"], expert_output_bf16=ptr(expert_out), token_rows_u32=ptr(token_rows),
                    shared_bf16=ptr(shared), output_bf16=ptr(out), error_flag_u32=ptr(flag),
                    stream=stream_handle(), token_count=tokens, top_k=topk, hidden_size=hidden, row_count=rows)
    _check(_ln().call("launch_moe_combine", r), "moe_combine")
    return out, flag


def bf16_gemm(a: torch.Tensor, w: torch.Tensor, output_type: int = abi.OUTPUT_BF16,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """C[m, n] = A[m, k] . W[n, k]^T through ``launch_bf16_gemm`` (the
    GemmPlan::execute replacement, src/backend/cuda/gemm_plan.cpp:169-198):
    bf16 in, fp32 accumulate, bf16 or fp32 out."""
    m, k = a.shape
    n = w.shape[0]
    if out is None:
        out = torch.empty(m, n, dtype=torch.bfloat16 if output_type == abi.OUTPUT_BF16 else torch.float32,
                          device=a.device)
    wsb = bf16_gemm_workspace(m, n, k)
    ws = torch.empty(wsb, dtype=torch.uint8, device=a.device) if wsb else None
    r = abi.request(abi.LN["bf16_gemm"], a_bf16=ptr(a), w_bf16=ptr(w), output=ptr(out),
                    workspace=ptr(ws) if ws is not None else 0, workspace_bytes=wsb, stream=stream_handle(),
                    m=m, n=n, k=k, output_type=output_type)
    _check(_ln().call("launch_bf16_gemm", r), "bf16_gemm")
    return out


def silu_mul(gate: torch.Tensor, up: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16(silu(g) * u) elementwise (pih_qwen_silu_mul_bf16_v1)."""
    if out is None:
        out = torch.empty_like(gate)
    r = abi.request(abi.LN["silu_mul"], gate_bf16=ptr(gate), up_bf16=ptr(up), output_bf16=ptr(out),
                    stream=stream_handle(), count=gate.numel())
    _check(_ln().call("launch_silu_mul", r), "silu_mul")
    return out


class QwenMlpBlock:
    """The Qwen3 MLP block as the reference's model issues it per layer:
    gate = x.Wg^T and up = x.Wu^T (GemmPlan, bf16 out;
    plugins/model-qwen3/qwen3_bf16_execution_schedule.cpp:34-37), then
    silu_mul (qwen3_cpu_oracle.cpp:114-126 semantics), then down = h.Wd^T.
    Buffers and the workspace are allocated at construction and the four
    requests are built once per (input, stream), as a native host holds its
    GemmPlans, so ``forward`` only enqueues."""

    def __init__(self, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor, tokens: int):
        self.wg, self.wu, self.wd = w_gate, w_up, w_down
        inter, hidden = w_gate.shape
        dev = w_gate.device
        self.tokens, self.inter, self.hidden = tokens, inter, hidden
        self.gate = torch.empty(tokens, inter, dtype=torch.bfloat16, device=dev)
        self.up = torch.empty(tokens, inter, dtype=torch.bfloat16, device=dev)
        self.h = torch.empty(tokens, inter, dtype=torch.bfloat16, device=dev)
        self.out = torch.empty(tokens, hidden, dtype=torch.bfloat16, device=dev)
        self.ws_gu = bf16_gemm_workspace(tokens, inter, hidden)
        self.ws_d = bf16_gemm_workspace(tokens, hidden, inter)
        wsb = max(self.ws_gu, self.ws_d)
        self.ws = torch.empty(wsb, dtype=torch.uint8, device=dev) if wsb else None
        self._key = None
        self._reqs = None

    def _gemm(self, a, w, out, m, n, k, wsb, s):
        return abi.request(abi.LN["bf16_gemm"], a_bf16=ptr(a), w_bf16=ptr(w), output=ptr(out),
                           workspace=ptr(self.ws) if wsb else 0, workspace_bytes=wsb, stream=s, m=m, n=n, k=k,
                           output_type=abi.OUTPUT_BF16)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape != (self.tokens, self.hidden) or x.dtype != torch.bfloat16:
            raise ValueError("Qwen MLP block input shape is invalid")
        s = stream_handle()
        key = (ptr(x), s)
        if key != self._key:
            t, i, h = self.tokens, self.inter, self.hidden
            self._reqs = (
                self._gemm(x, self.wg, self.gate, t, i, h, self.ws_gu, s),
                self._gemm(x, self.wu, self.up, t, i, h, self.ws_gu, s),
                abi.request(abi.LN["silu_mul"], gate_bf16=ptr(self.gate), up_bf16=ptr(self.up),
                            output_bf16=ptr(self.h), stream=s, count=t * i),
                self._gemm(self.h, self.wd, self.out, t, h, i, self.ws_d, s),
            )
            self._key = key
        ln = _ln()
        g, u, sm, d = self._reqs
        _check(ln.call("launch_bf16_gemm", g), "bf16_gemm")
        _check(ln.call("launch_bf16_gemm", u), "bf16_gemm")
        _check(ln.call("launch_silu_mul", sm), "silu_mul")
        _check(ln.call("launch_bf16_gemm", d), "bf16_gemm")
        return self.out


QWEN_VOCAB, QWEN_HIDDEN = 151936, 1024


class QwenLmHead:
    """The Qwen3-0.6B LM head as the reference's INT4 execution driver runs
    it (plugins/model-qwen3/nvidia_qwen3_int4_execution_driver.cpp:16-67): a
    bank of GemmPlans for 1..maximum_rows rows (at most 32) over the tied
    [151936, 1024] bf16 weight with fp32 logits; ``execute`` rejects a row
    count outside the bank.  Here every row count is the same
    ``launch_bf16_gemm`` call (the weight-streaming GEMV, no workspace)."""

    def __init__(self, maximum_rows: int):
        if not 1 <= maximum_rows <= 32:
            raise ValueError("NVIDIA Qwen INT4 workspace identity is invalid")
        self.maximum_rows = maximum_rows

    def execute(self, x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        if x.dim() != 2 or x.shape[0] == 0 or x.shape[0] > self.maximum_rows:
            raise ValueError("NVIDIA Qwen INT4 LM head row count is invalid")
        if tuple(weight.shape) != (QWEN_VOCAB, QWEN_HIDDEN) or x.shape[1] != QWEN_HIDDEN:
            raise ValueError("Qwen LM head shape is invalid")
        return bf16_gemm(x, weight, abi.OUTPUT_F32, out=out)


def deepseek_lm_head(x: torch.Tensor, weight: torch.Tensor, out: Optional[torch.Tensor] = None,
                     flag: Optional[torch.Tensor] = None):
    """logits f32 [rows, 129280] through the DeepSeek table's
    ``launch_lm_head`` (plugins/kernels/deepseek-v4-sm89/native/
    deepseek_endpoint.cu:94-115,484-497): bit 128 of the flag for a
    non-finite logit, bit 64 for a non-finite x or W element."""
    rows, hidden = x.shape
    vocab = weight.shape[0]
    if out is None:
        out = torch.empty(rows, vocab, dtype=torch.float32, device=x.device)
    flag = error_flag() if flag is None else flag
    r = abi.request(abi.DS["lm_head"], input_bf16=ptr(x), weight_bf16=ptr(weight), logits_f32=ptr(out),
                    error_flag_u32=ptr(flag), stream=stream_handle(), output_rows=rows, vocab_size=vocab,
                    hidden_size=hidden)
    _check(abi.deepseek_pack().call("launch_lm_head", r), "lm_head")
    return out, flag


class MoeFp8Layer:
    """The BASELINE FP8 MoE expert layer on device, one launch per stage:
    route plan -> FP8 quant of the token rows -> grouped gate/up GEMM with
    the fused SwiGLU * route-weight epilogue that also quantises the
    intermediate to FP8 (as the quant entry would quantise its bf16 values)
    -> grouped down GEMM -> ordered combine.

    Buffers are allocated once at construction for ``tokens`` x ``topk``
    routes, so ``forward`` allocates nothing and can be timed or replayed.
    The stage order and rounding points are those of the reference's
    routed-expert chain (src/model/deepseek_routed_expert_oracle.cpp:50-95)
    with fp32 scales and a fused [2I, H] gate/up weight."""

    def __init__(self, w13, w13_scale, w2, w2_scale, tokens: int, topk: int, swiglu_limit: float = 0.0,
                 scale_format: int = abi.SCALE_F32):
        self.w13, self.w13_scale, self.w2, self.w2_scale = w13, w13_scale, w2, w2_scale
        self.experts, n13, self.hidden = w13.shape
        self.inter = n13 // 2
        self.tokens, self.topk = tokens, topk
        self.rows = tokens * topk
        self.limit = swiglu_limit
        self.fmt = scale_format
        dev = w13.device
        sdt = torch.float32 if scale_format == abi.SCALE_F32 else torch.uint8
        self.ws = torch.empty(route_plan_workspace(tokens, topk, self.experts), dtype=torch.uint8, device=dev)
        self.offsets = torch.empty(self.experts + 1, dtype=torch.int32, device=dev)
        self.row_token = torch.empty(self.rows, dtype=torch.int32, device=dev)
        self.row_weight = torch.empty(self.rows, dtype=torch.float32, device=dev)
        self.token_rows = torch.empty(tokens, topk, dtype=torch.int32, device=dev)
        self.xq = torch.empty(tokens, self.hidden, dtype=torch.uint8, device=dev)
        self.xs = torch.empty(tokens, self.hidden // 128, dtype=sdt, device=dev)
        self.mq = torch.empty(self.rows, self.inter, dtype=torch.uint8, device=dev)
        self.ms = torch.empty(self.rows, self.inter // 128, dtype=sdt, device=dev)
        self.y = torch.empty(self.rows, self.hidden, dtype=torch.bfloat16, device=dev)
        self.out = torch.empty(tokens, self.hidden, dtype=torch.bfloat16, device=dev)
        self.flag = error_flag()

    STAGES = ("route_plan", "quant_x", "gate_up", "down", "combine")

    def forward(self, x, topk_ids, topk_weights, shared=None, marks=None):
        """``marks``: optional list of len(STAGES)+1 events recorded on the
        launch stream around the stages (for per-kernel timing)."""
        L = _ln()
        s = stream_handle()
        f = ptr(self.flag)
        mark = (lambda i: marks[i].record()) if marks is not None else (lambda i: None)
        mark(0)
        st = L.call("launch_route_plan", abi.request(
            abi.LN["route_plan"], topk_ids_u32=ptr(topk_ids), topk_weights_f32=ptr(topk_weights),
            expert_offsets_u32=ptr(self.offsets), row_token_u32=ptr(self.row_token),
            row_weight_f32=ptr(self.row_weight), token_rows_u32=ptr(self.token_rows), workspace=ptr(self.ws),
            workspace_bytes=self.ws.numel(), error_flag_u32=f, stream=s, token_count=self.tokens,
            top_k=self.topk, expert_count=self.experts))
        _check(st, "route_plan")
        mark(1)
        st = L.call("launch_fp8_quant", abi.request(
            abi.LN["fp8_quant"], input_bf16=ptr(x), row_index_u32=0, output_e4m3=ptr(self.xq), scale=ptr(self.xs),
            error_flag_u32=f, stream=s, row_count=self.tokens, logical_k=self.hidden, input_rows=self.tokens,
            scale_format=self.fmt))
        _check(st, "fp8_quant(x)")
        mark(2)
        st = L.call("launch_moe_fp8_gemm", abi.request(
            abi.LN["moe_fp8_gemm"], activation_e4m3=ptr(self.xq), activation_scale=ptr(self.xs),
            row_token_u32=ptr(self.row_token), weight_e4m3=ptr(self.w13), weight_scale=ptr(self.w13_scale),
            expert_offsets_u32=ptr(self.offsets), row_weight_f32=ptr(self.row_weight), output=ptr(self.mq),
            output_scale=ptr(self.ms), error_flag_u32=f, stream=s, row_capacity=self.rows,
            expert_count=self.experts, n=2 * self.inter, k=self.hidden, activation_rows=self.tokens,
            scale_format=self.fmt, output_type=abi.OUTPUT_SWIGLU_E4M3, swiglu_limit=self.limit))
        _check(st, "moe_fp8_gemm(gate/up)")
        mark(3)
        st = L.call("launch_moe_fp8_gemm", abi.request(
            abi.LN["moe_fp8_gemm"], activation_e4m3=ptr(self.mq), activation_scale=ptr(self.ms),
            row_token_u32=0, weight_e4m3=ptr(self.w2), weight_scale=ptr(self.w2_scale),
            expert_offsets_u32=ptr(self.offsets), row_weight_f32=0, output=ptr(self.y), error_flag_u32=f,
            stream=s, row_capacity=self.rows, expert_count=self.experts, n=self.hidden, k=self.inter,
            activation_rows=self.rows, scale_format=self.fmt, output_type=abi.OUTPUT_BF16, swiglu_limit=0.0))
        _check(st, "moe_fp8_gemm(down)")
        mark(4)
        st = L.call("launch_moe_combine", abi.request(
            abi.LN["moe_combine"], expert_output_bf16=ptr(self.y), token_rows_u32=ptr(self.token_rows),
            shared_bf16=ptr(shared), output_bf16=ptr(self.out), error_flag_u32=f, stream=s,
            token_count=self.tokens, top_k=self.topk, hidden_size=self.hidden, row_count=self.rows))
        _check(st, "moe_combine")
        mark(5)
        return self.out


class MoeLayer:
    """One MoE expert layer per call through the pack's C++ layer entry
    (``launch_moe_layer``): the six stages of ``MoeFp8Layer`` enqueued by the
    native host code, for FP8 or MXFP4 weights.  Scratch is sized once with
    ``query_moe_layer_workspace`` and allocated at construction."""

    def __init__(self, w13, w13_scale, w2, w2_scale, tokens: int, topk: int, weight_format: int = abi.WEIGHT_FP8,
                 scale_format: int = abi.SCALE_F32, activation_type: int = abi.ACTIVATION_E4M3,
                 swiglu_limit: float = 0.0):
        self.w13, self.w13_scale, self.w2, self.w2_scale = w13, w13_scale, w2, w2_scale
        self.experts, n13, k13 = w13.shape
        self.hidden = k13 if weight_format == abi.WEIGHT_FP8 else 2 * k13
        self.inter = n13 // 2
        self.tokens, self.topk = tokens, topk
        self.fields = dict(token_count=tokens, top_k=topk, expert_count=self.experts, hidden_size=self.hidden,
                           intermediate_size=self.inter, weight_format=weight_format, scale_format=scale_format,
                           activation_type=activation_type, swiglu_limit=swiglu_limit)
        need = (abi.C.c_uint64 * 1)()
        q = abi.request(abi.LN["moe_layer"], required_bytes_u64=abi.C.addressof(need), **self.fields)
        _check(_ln().call("query_moe_layer_workspace", q), "query_moe_layer_workspace")
        self.ws = torch.empty(int(need[0]), dtype=torch.uint8, device=w13.device)
        self.out = torch.empty(tokens, self.hidden, dtype=torch.bfloat16, device=w13.device)
        self.flag = error_flag()

    def forward(self, x, topk_ids, topk_weights, shared=None):
        r = abi.request(abi.LN["moe_layer"], input_bf16=ptr(x), topk_ids_u32=ptr(topk_ids),
                        topk_weights_f32=ptr(topk_weights), w13=ptr(self.w13), w13_scale=ptr(self.w13_scale),
                        w2=ptr(self.w2), w2_scale=ptr(self.w2_scale), shared_bf16=ptr(shared),
                        output_bf16=ptr(self.out), workspace=ptr(self.ws), workspace_bytes=self.ws.numel(),
                        error_flag_u32=ptr(self.flag), stream=stream_handle(), **self.fields)
        _check(_ln().call("launch_moe_layer", r), "moe_layer")
        return self.out


# ------------------------------------------------ DeepSeek V4.1 32-block formats
def v41_linear(x: torch.Tensor, weight: torch.Tensor, weight_scales: torch.Tensor, weight_format: int,
               out: Optional[torch.Tensor] = None, quantized: Optional[torch.Tensor] = None,
               activation_scales: Optional[torch.Tensor] = None, flag: Optional[torch.Tensor] = None):
    """The V4.1 FP8 (32x32 weight blocks) or mixed FP8/FP4 linear
    (plugins/model-deepseek-v41/linear_fp8.cu:82-105) through
    ``launch_v41_linear``: per-32 activation quant into ``quantized`` /
    ``activation_scales`` (allocated when None), then the MX GEMM; returns
    (out bf16 [rows, N], quantized, activation_scales, flag)."""
    rows, k = x.shape
    n = weight.shape[0]
    dev = x.device
    if out is None:
        out = torch.empty(rows, n, dtype=torch.bfloat16, device=dev)
    if quantized is None:
        quantized = torch.empty(rows, k, dtype=torch.uint8, device=dev)
    if activation_scales is None:
        activation_scales = torch.empty(rows, k // 32, dtype=torch.uint8, device=dev)
    flag = error_flag() if flag is None else flag
    nbytes = lambda t: t.numel() * t.element_size()  # noqa: E731
    r = abi.request(abi.LN["v41_linear"], input_bf16=ptr(x), input_bytes=nbytes(x), weight=ptr(weight),
                    weight_bytes=nbytes(weight), weight_scales=ptr(weight_scales),
                    weight_scale_bytes=nbytes(weight_scales), quantized_e4m3=ptr(quantized),
                    quantized_bytes=nbytes(quantized), activation_scales=ptr(activation_scales),
                    activation_scale_bytes=nbytes(activation_scales), output_bf16=ptr(out),
                    output_bytes=nbytes(out), error_flag_u32=ptr(flag), error_flag_bytes=4,
                    stream=stream_handle(), rows=rows, in_features=k, out_features=n, weight_format=weight_format)
    _check(_ln().call("launch_v41_linear", r), "v41_linear")
    return out, quantized, activation_scales, flag


def v41_fp4_to_fp8(packed: torch.Tensor, scales: torch.Tensor, flag: Optional[torch.Tensor] = None):
    """V4.1 expert FP4 -> FP8 32x32 conversion on the device
    (weight_expert_convert.cpp:33-100): (e4m3 [rows, cols], UE8M0 [rows/32,
    cols/32], flag)."""
    rows, half = packed.shape
    cols = half * 2
    w = torch.empty(rows, cols, dtype=torch.uint8, device=packed.device)
    s = torch.empty(rows // 32, cols // 32, dtype=torch.uint8, device=packed.device)
    flag = error_flag() if flag is None else flag
    r = abi.request(abi.LN["v41_fp4_to_fp8"], packed=ptr(packed), scales=ptr(scales), weight_e4m3=ptr(w),
                    weight_scales=ptr(s), error_flag_u32=ptr(flag), stream=stream_handle(), rows=rows, columns=cols)
    _check(_ln().call("launch_v41_fp4_to_fp8", r), "v41_fp4_to_fp8")
    return w, s, flag


def v41_block_dequant(source: torch.Tensor, scales: torch.Tensor, block: int, out: Optional[torch.Tensor] = None,
                      flag: Optional[torch.Tensor] = None):
    """e4m3 [rows, cols] x per-block scale (uint8 UE8M0 or float32 tensor)
    -> bf16 (weight_dequantize.cpp:17-50, DequantizeWoATensor)."""
    rows, cols = source.shape
    if out is None:
        out = torch.empty(rows, cols, dtype=torch.bfloat16, device=source.device)
    flag = error_flag() if flag is None else flag
    storage = abi.V41_SCALE_F32 if scales.dtype == torch.float32 else abi.V41_SCALE_E8M0
    r = abi.request(abi.LN["v41_block_dequant"], source_e4m3=ptr(source), scales=ptr(scales), output_bf16=ptr(out),
                    error_flag_u32=ptr(flag), stream=stream_handle(), rows=rows, columns=cols, block=block,
                    scale_storage=storage)
    _check(_ln().call("launch_v41_block_dequant", r), "v41_block_dequant")
    return out, flag

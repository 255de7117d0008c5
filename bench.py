"""Benchmark of the north-star path on one MI355X.

Workload: DeepSeek-style FP8 MoE expert layer,
T=4096 tokens, E=256 experts, top-8 routing (Zipf(1.1) skew, softmax,
renormalised), hidden 7168, expert intermediate 2048, fused gate/up
7168->4096, SiLU-mul, down 2048->7168; e4m3 weights with fp32 128x128 block
scales, e4m3 activations with fp32 per-token per-128 scales.  One step is
one pass of the whole expert layer through the gfx950 packs: device route
plan -> activation quant -> grouped gate/up GEMM (+SwiGLU*w epilogue that
quantises the intermediate to e4m3) -> grouped down GEMM -> ordered combine.  Inputs are resident in HBM
before timing starts.

A timed step is one call of the linear pack's C++ layer entry
(``launch_moe_layer``), which enqueues the five grouped launches; a staged
copy of the same layer launched stage by stage gives the per-kernel times.

Prints one JSON line.  ``value`` is the layer's TFLOP/s (2*R*(2I*H + H*I)
FLOP per step, R = T*top_k).  ``roofline`` covers the dominant kernel (the
grouped gate/up GEMM), timed with HIP events on its launch stream.  Side
measurements: ``moe_mxfp4_decode`` (configs[4], MXFP4 experts at 64 and 512
tokens) and ``decode_gemv`` (configs[1] and [2] decode, BF16 prefill).
``cpu_baseline`` times the C restatement of the reference's CPU oracle
(oracle/pih_oracle.c, po_expert_fp8: the per-expert chain) on a bounded
sample of the same routed rows.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "TFLOP/s + %MFMA peak, FP8 MoE grouped GEMM; decode GEMV HBM GB/s"
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5033.2  # 256 CU x 2.4 GHz x 8192 dense FP8 FLOP/clk/CU

T, E, TOPK, H, I = 4096, 256, 8, 7168, 2048


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_inputs(torch):
    from pih_amd import synth

    ids, wts = synth.zipf_router(synth.config_seed(4, 0), T, E, TOPK)
    x = synth.bf16_normal(synth.config_seed(4, 1), (T, H))
    dev = torch.device("cuda")
    # Expert weights: e4m3 codes of N(0, 0.02) values quantised per 128x128
    # block with fp32 scale amax/448.  Generated on the device (11.3 GB) with
    # a seeded torch generator: same distribution as synth.fp8_block_weight.
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x50494804)

    def block_weight(rows, cols):
        w = torch.empty(E, rows, cols, dtype=torch.uint8, device=dev)
        s = torch.empty(E, rows // 128, cols // 128, dtype=torch.float32, device=dev)
        for e in range(E):
            v = torch.randn(rows, cols, device=dev, generator=gen) * 0.02
            blk = v.view(rows // 128, 128, cols // 128, 128)
            amax = blk.abs().amax(dim=(1, 3)).clamp_min(1e-12)
            sc = amax / 448.0
            q = (blk / sc[:, None, :, None]).clamp(-448.0, 448.0)
            w[e] = q.view(rows, cols).to(torch.float8_e4m3fn).view(torch.uint8)
            s[e] = sc
        return w, s

    w13, s13 = block_weight(2 * I, H)
    w2, s2 = block_weight(H, I)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return ids, wts, x, t(ids.view(np.int32)), t(wts), t(x.view(np.int16)).view(torch.bfloat16), w13, s13, w2, s2


def cpu_baseline(ids, wts, x_bits, budget_s: float = 12.0):
    """Time po_expert_fp8 (the reference's per-expert CPU chain, restated) on
    a bounded sample: routed rows of the hottest expert, grown until the
    sample takes about ``budget_s``.  Returns the CPU TFLOP/s."""
    import oracle
    from pih_amd import synth

    threads = int(os.environ.get("PIH_CPU_THREADS", min(16, os.cpu_count() or 1)))
    oracle.set_threads(threads)
    offsets, row_token, row_weight, _ = oracle.route_plan(ids, wts, E)
    counts = np.diff(offsets.astype(np.int64))
    e = int(np.argmax(counts))
    b = int(offsets[e])
    w13, s13 = synth.fp8_block_weight(synth.config_seed(4, 20 + e), 2 * I, H)
    w2, s2 = synth.fp8_block_weight(synth.config_seed(4, 600 + e), H, I)
    flop_per_row = 2.0 * (2 * I * H + H * I)
    rows, elapsed = threads, 0.0
    while True:
        xs = np.ascontiguousarray(x_bits[row_token[b:b + rows]])
        t0 = time.perf_counter()
        oracle.expert_fp8(xs, row_weight[b:b + rows], H, I, w13, s13, w2, s2)
        elapsed = time.perf_counter() - t0
        if elapsed * 2 > budget_s or rows * 2 > int(counts[e]):
            break
        rows *= 2
    return {"value": flop_per_row * rows / elapsed / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"po_expert_fp8 on {rows} routed rows of expert {e} (gate/up+SiLU-mul+down, fp32 scales), "
                      f"{elapsed:.2f} s"}


QWEN8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
          ("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]


def _timed(torch, fn, iters: int):
    """Mean ms per call of fn(i) measured with HIP events on the launch stream."""
    s = torch.cuda.current_stream()
    fn(0)
    s.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(s)
    for i in range(iters):
        fn(i)
    ev1.record(s)
    ev1.synchronize()
    return ev0.elapsed_time(ev1) / iters


def _graphed(torch, make_calls, nsets: int, iters: int):
    """Mean ms per pass with each weight set's pass captured once in a HIP
    graph (torch.cuda.CUDAGraph) and replayed; the launches inside are the
    same C-ABI calls, captured on the graph's stream."""
    from pih_amd.device import stream_handle

    graphs = []
    for j in range(nsets):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            keep = make_calls(j, stream_handle())
        graphs.append((g, keep))
    torch.cuda.synchronize()
    return _timed(torch, lambda i: graphs[i % nsets][0].replay(), iters)


def _decode_line(ms: float, ms_graph: float, algo: int, nsets: int, launches: int = 7) -> dict:
    gbs = algo / (ms * 1e-3) / 1e9
    gbs_graph = algo / (ms_graph * 1e-3) / 1e9
    return {"us_per_pass": round(ms * 1e3, 2), "gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "us_per_pass_graph": round(ms_graph * 1e3, 2), "gbs_graph": round(gbs_graph, 1),
            "frac_hbm_graph": round(gbs_graph / HBM_PEAK_GBS, 4), "launches": launches,
            "algorithmic_bytes": algo, "weight_sets": nsets}


def bench_decode(torch, iters: int):
    """BASELINE configs[1] decode (bf16, M=1, 8, 64) and configs[2] (W4A16
    asymmetric, M=1, 4, 16): one pass = the 7 Qwen3-8B projections; weight
    sets rotate through > 512 MB so HBM, not the 256 MB Infinity Cache,
    serves them.  Each pass is timed twice: eager launches through the C-ABI
    (host launch cost included) and replayed from a captured HIP graph."""
    from pih_amd import abi
    from pih_amd.device import ptr, stream_handle

    L = abi.linear_pack()
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x50494802)
    out = {}

    def query(kind, m, n, k):
        b = (abi.C.c_uint64 * 1)()
        L.call("query_workspace", abi.request(abi.LN["workspace_query"], kind=kind, m=m, n=n, k=k,
                                              bytes_u64=abi.C.addressof(b)))
        return int(b[0])

    # ---- W4A16 asymmetric, M = 1, 4, 16
    set_bytes = sum(n * k // 2 + (n * k // 128) * 2 + n * ((k // 128 + 7) // 8) * 4 for _, n, k in QWEN8B)
    nsets = max(2, -(-600_000_000 // set_bytes))
    sets = []
    for _ in range(nsets):
        layer = []
        for _, n, k in QWEN8B:
            q = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), dtype=torch.int32, device=dev, generator=gen)
            s = (torch.rand(n, k // 128, device=dev, generator=gen) * 0.019 + 0.001).to(torch.bfloat16)
            z = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, (k // 128 + 7) // 8), dtype=torch.int32, device=dev,
                              generator=gen)
            layer.append((q, s, z))
        sets.append(layer)
    for m in (1, 4, 16):
        xs = {k: torch.randn(m, k, device=dev, generator=gen).to(torch.bfloat16) for k in (4096, 12288)}
        ys = [torch.empty(m, n, dtype=torch.bfloat16, device=dev) for _, n, _ in QWEN8B]
        ws = [torch.zeros(max(1, query(abi.WORKSPACE_W4A16, m, n, k)), dtype=torch.uint8, device=dev)
              for _, n, k in QWEN8B]
        flag = torch.zeros(1, dtype=torch.int32, device=dev)

        def calls(i, stream, m=m, xs=xs, ys=ys, ws=ws, flag=flag):
            rs = []
            for j, (_, n, k) in enumerate(QWEN8B):
                q, s, z = sets[i][j]
                r = abi.request(abi.LN["w4a16"], input_bf16=ptr(xs[k]), qweight=ptr(q), scales=ptr(s),
                                zeros=ptr(z), output_bf16=ptr(ys[j]), workspace=ptr(ws[j]),
                                workspace_bytes=ws[j].numel(), error_flag_u32=ptr(flag), stream=stream,
                                m=m, n=n, k=k, format=abi.W4A16_ASYMMETRIC)
                st = L.call("launch_w4a16_gemm", r)
                if st.code != abi.OK:
                    raise RuntimeError(f"w4a16 launch: {st}")
                rs.append(r)
            return rs

        # the same pass as a decode step can issue it with the grouped entry:
        # [q, k, v] (one input), o, [gate, up] (one input), down
        groups = [[0, 1, 2], [3], [4, 5], [6]]

        def grouped_calls(i, stream, m=m, xs=xs, ys=ys, flag=flag):
            keep = []
            for g in groups:
                k = QWEN8B[g[0]][2]
                probs = (abi.W4A16_PROBLEM * len(g))()
                for slot, j in enumerate(g):
                    q, s, z = sets[i][j]
                    pr = probs[slot]
                    pr.input_bf16, pr.qweight, pr.scales, pr.zeros = ptr(xs[k]), ptr(q), ptr(s), ptr(z)
                    pr.output_bf16, pr.n = ptr(ys[j]), QWEN8B[j][1]
                r = abi.request(abi.LN["w4a16_grouped"], problems=abi.C.addressof(probs), error_flag_u32=ptr(flag),
                                stream=stream, problem_count=len(g), m=m, k=k, format=abi.W4A16_ASYMMETRIC)
                st = L.call("launch_w4a16_grouped", r)
                if st.code != abi.OK:
                    raise RuntimeError(f"w4a16 grouped launch: {st}")
                keep.append((probs, r))
            return keep

        reqs = [calls(i, stream_handle()) for i in range(nsets)]  # also the warm pass
        ms = _timed(torch, lambda i: [L.call("launch_w4a16_gemm", r) for r in reqs[i % nsets]], iters)
        ms_graph = _graphed(torch, calls, nsets, iters)
        gkeep = [grouped_calls(i, stream_handle()) for i in range(nsets)]
        ms_grp = _timed(torch, lambda i: [L.call("launch_w4a16_grouped", r) for _, r in gkeep[i % nsets]], iters)
        ms_grp_graph = _graphed(torch, grouped_calls, nsets, iters)
        if int(flag.item()):
            raise RuntimeError(f"w4a16 error flag {int(flag.item())}")
        algo = set_bytes + sum(m * k * 2 + m * n * 2 for _, n, k in QWEN8B)
        out[f"w4a16_m{m}"] = _decode_line(ms, ms_graph, algo, nsets)
        out[f"w4a16_m{m}_grouped"] = _decode_line(ms_grp, ms_grp_graph, algo, nsets, launches=len(groups))
    del sets
    # ---- BF16 decode, M = 1, 8, 64
    set_bytes = sum(n * k * 2 for _, n, k in QWEN8B)
    nsets = max(2, -(-600_000_000 // set_bytes))
    wsets = [[(torch.randn(n, k, device=dev, generator=gen) * 0.02).to(torch.bfloat16) for _, n, k in QWEN8B]
             for _ in range(nsets)]
    for m in (1, 8, 64):
        xs = {k: torch.randn(m, k, device=dev, generator=gen).to(torch.bfloat16) for k in (4096, 12288)}
        ys = [torch.empty(m, n, dtype=torch.bfloat16, device=dev) for _, n, _ in QWEN8B]
        ws = [torch.zeros(max(1, query(abi.WORKSPACE_BF16_GEMM, m, n, k)), dtype=torch.uint8, device=dev)
              for _, n, k in QWEN8B]

        def calls(i, stream, m=m, xs=xs, ys=ys, ws=ws):
            rs = []
            for j, (_, n, k) in enumerate(QWEN8B):
                r = abi.request(abi.LN["bf16_gemm"], a_bf16=ptr(xs[k]), w_bf16=ptr(wsets[i][j]), output=ptr(ys[j]),
                                workspace=ptr(ws[j]), workspace_bytes=ws[j].numel(), stream=stream,
                                m=m, n=n, k=k, output_type=abi.OUTPUT_BF16)
                st = L.call("launch_bf16_gemm", r)
                if st.code != abi.OK:
                    raise RuntimeError(f"bf16 launch: {st}")
                rs.append(r)
            return rs

        reqs = [calls(i, stream_handle()) for i in range(nsets)]
        ms = _timed(torch, lambda i: [L.call("launch_bf16_gemm", r) for r in reqs[i % nsets]], iters)
        ms_graph = _graphed(torch, calls, nsets, iters)
        algo = set_bytes + sum(m * k * 2 + m * n * 2 for _, n, k in QWEN8B)
        out[f"bf16_m{m}"] = _decode_line(ms, ms_graph, algo, nsets)
    # ---- BF16 prefill, M = 2048
    m = 2048
    xs = {k: torch.randn(m, k, device=dev, generator=gen).to(torch.bfloat16) for k in (4096, 12288)}
    ys = [torch.empty(m, n, dtype=torch.bfloat16, device=dev) for _, n, _ in QWEN8B]
    reqs = [abi.request(abi.LN["bf16_gemm"], a_bf16=ptr(xs[k]), w_bf16=ptr(wsets[0][j]), output=ptr(ys[j]),
                        workspace=0, workspace_bytes=0, stream=stream_handle(), m=m, n=n, k=k,
                        output_type=abi.OUTPUT_BF16) for j, (_, n, k) in enumerate(QWEN8B)]

    def run_prefill(i):
        for r in reqs:
            L.call("launch_bf16_gemm", r)

    ms = _timed(torch, run_prefill, max(3, iters // 4))
    flop = sum(2.0 * m * n * k for _, n, k in QWEN8B)
    out["bf16_prefill_m2048"] = {"ms_per_pass": round(ms, 4), "tflops": round(flop / (ms * 1e-3) / 1e12, 1),
                                 "frac_mfma": round(flop / (ms * 1e-3) / 1e12 / 2516.6, 4)}
    return out


def bench_mxfp4(torch, iters: int):
    """the cfg4 MoE shapes (E=256, top-8, H=7168,
    I=2048) with MXFP4 experts (e2m1 two per byte + UE8M0 per 32 k) at decode
    batches of 64 and 512 tokens, bf16 and e4m3 (UE8M0 per 128) activations,
    through the pack's layer entry.  Memory-bound: bytes = touched experts x
    23,396,352 (weights + scales) + token activations in and out."""
    from pih_amd import abi, synth
    from pih_amd.linear import MoeLayer

    dev = torch.device("cuda")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x50494805)
    # any byte is two valid e2m1 codes; UE8M0 scales 2^-9 .. 2^-1
    w13 = torch.randint(0, 256, (E, 2 * I, H // 2), dtype=torch.uint8, device=dev, generator=gen)
    s13 = torch.randint(118, 127, (E, 2 * I, H // 32), dtype=torch.uint8, device=dev, generator=gen)
    w2 = torch.randint(0, 256, (E, H, I // 2), dtype=torch.uint8, device=dev, generator=gen)
    s2 = torch.randint(118, 127, (E, H, I // 32), dtype=torch.uint8, device=dev, generator=gen)
    per_expert = 2 * I * H // 2 + H * I // 2 + 2 * I * H // 32 + H * I // 32
    out = {}
    for tokens in (64, 512):
        ids, wts = synth.zipf_router(synth.config_seed(5, tokens), tokens, E, TOPK)
        touched = int((np.bincount(ids.ravel(), minlength=E) > 0).sum())
        x = torch.from_numpy(synth.bf16_normal(synth.config_seed(5, tokens + 1), (tokens, H)).view(np.int16))
        x = x.to(dev).view(torch.bfloat16)
        ids_d = torch.from_numpy(ids.view(np.int32)).to(dev)
        wts_d = torch.from_numpy(wts).to(dev)
        for act, name in ((abi.ACTIVATION_BF16, "bf16"), (abi.ACTIVATION_E4M3, "e4m3")):
            layer = MoeLayer(w13, s13, w2, s2, tokens, TOPK, weight_format=abi.WEIGHT_MXFP4, activation_type=act)
            ms = _timed(torch, lambda i: layer.forward(x, ids_d, wts_d), iters)
            if int(layer.flag.item()):
                raise RuntimeError(f"mxfp4 layer error flag {int(layer.flag.item())}")
            algo = touched * per_expert + tokens * H * 2 * 2
            flop = 2.0 * tokens * TOPK * (2 * I * H + H * I)
            gbs = algo / (ms * 1e-3) / 1e9
            out[f"t{tokens}_{name}"] = {"us_per_layer": round(ms * 1e3, 1), "gbs": round(gbs, 1),
                                        "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                        "tflops": round(flop / (ms * 1e-3) / 1e12, 2),
                                        "touched_experts": touched, "algorithmic_bytes": algo}
            del layer
    return out


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "moe_fp8_cfg4_hbm_traffic.md")


def profiled_traffic():
    """HBM bytes per launch of the gate/up kernel, from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE summary (its ``traffic_bytes_per_launch``
    line); None when that summary is absent."""
    import re

    try:
        with open(TRAFFIC_PROFILE) as f:
            m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", f.read())
    except OSError:
        return None
    return int(m.group(1)) if m else None


def copy_calibration(nbytes: int = 1 << 30, reps: int = 3) -> int:
    """Three D2D copies of exactly ``nbytes``: under rocprofv3 --pmc their
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch) give the factors that turn
    those counters into bytes for the path's kernels."""
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copied {nbytes} bytes x {reps}")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode GEMV / prefill side measurements")
    ap.add_argument("--no-mxfp4", action="store_true", help="skip the MXFP4 MoE decode side measurement")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 1 GiB device-to-device copies (the reference kernel for scaling the "
                         "FETCH_SIZE / WRITE_SIZE counters to bytes) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU (the north-star path is a single-GPU kernel "
              "pack); --gpus must be 1", file=sys.stderr)
        return 2

    import torch

    from pih_amd import abi
    from pih_amd.device import engine_stream, flag_value
    from pih_amd.linear import MoeFp8Layer, MoeLayer

    log("generating inputs")
    ids, wts, x_bits, ids_d, wts_d, x_d, w13, s13, w2, s2 = build_inputs(torch)
    counts = np.bincount(ids.ravel(), minlength=E)
    touched = int((counts > 0).sum())
    R = T * TOPK
    flop = 2.0 * R * (2 * I * H + H * I)
    flop_gu = 2.0 * R * 2 * I * H
    # algorithmic bytes of the gate/up kernel: weights + scales of touched
    # experts, fp8 activations + scales of all tokens, bf16 mid out
    # weights + fp32 block scales of the touched experts, e4m3 tokens + scales,
    # e4m3 SwiGLU output + fp32 per-128 scales (the epilogue quantises it)
    bytes_gu = (touched * (2 * I * H + (2 * I // 128) * (H // 128) * 4) + T * H + T * (H // 128) * 4
                + R * I + R * (I // 128) * 4)
    bytes_layer = (touched * (3 * I * H + ((2 * I // 128) * (H // 128) + (H // 128) * (I // 128)) * 4)
                   + T * H * 2 + T * H * 2)

    with engine_stream() as s:
        # the timed step: one call of the pack's C++ layer entry (six grouped
        # launches); the staged copy below times each launch on its own
        layer = MoeLayer(w13, s13, w2, s2, T, TOPK, scale_format=abi.SCALE_F32)
        staged = MoeFp8Layer(w13, s13, w2, s2, T, TOPK, scale_format=abi.SCALE_F32)
        log("warmup")
        for _ in range(args.warmup):
            layer.forward(x_d, ids_d, wts_d)
            staged.forward(x_d, ids_d, wts_d)
        s.synchronize()
        if flag_value(layer.flag) or flag_value(staged.flag):
            log(f"device error flag {flag_value(layer.flag):#x} {flag_value(staged.flag):#x}")
            return 1
        log(f"timing {args.steps} steps")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            layer.forward(x_d, ids_d, wts_d)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        n_marks = len(MoeFp8Layer.STAGES) + 1
        marks = [[torch.cuda.Event(enable_timing=True) for _ in range(n_marks)] for _ in range(args.steps)]
        for i in range(args.steps):
            staged.forward(x_d, ids_d, wts_d, marks=marks[i])
        torch.cuda.synchronize()
        stage_ms = {name: float(np.median([m[j].elapsed_time(m[j + 1]) for m in marks]))
                    for j, name in enumerate(MoeFp8Layer.STAGES)}
        if flag_value(layer.flag) or flag_value(staged.flag):
            log(f"device error flag {flag_value(layer.flag):#x} {flag_value(staged.flag):#x}")
            return 1
    ms = wall * 1000.0 / args.steps
    tflops = flop / (ms * 1e-3) / 1e12
    gu_ms = stage_ms["gate_up"]
    gu_gbs = bytes_gu / (gu_ms * 1e-3) / 1e9
    log("stage ms: " + ", ".join(f"{k}={v:.3f}" for k, v in stage_ms.items()))

    del layer, staged, w13, w2
    torch.cuda.empty_cache()
    mxfp4 = None
    if not args.no_mxfp4:
        log("MXFP4 MoE decode (configs[4])")
        with engine_stream():
            mxfp4 = bench_mxfp4(torch, iters=max(10, args.steps))
        torch.cuda.empty_cache()
        log("mxfp4: " + json.dumps(mxfp4))

    decode = None
    if not args.no_decode:
        log("decode GEMV / prefill side measurements")
        with engine_stream():
            decode = bench_decode(torch, iters=max(10, args.steps))
        log("decode: " + json.dumps(decode))

    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(ids, wts, x_bits)

    line = {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (fp32 acc, fp32 block scales)",
        "data": "synthetic (seeded router/activations; random-init e4m3 expert weights)",
        "config": {"workload": "cfg4 FP8 MoE expert layer", "tokens": T, "experts": E, "top_k": TOPK,
                   "hidden": H, "intermediate": I, "routed_rows": R, "touched_experts": touched,
                   "parallelism": "single GPU"},
        "mfma_frac": round(tflops / FP8_PEAK_TFLOPS, 4),
        "layer_hbm_gbs": round(bytes_layer / (ms * 1e-3) / 1e9, 1),
        "stage_ms": {k: round(v, 4) for k, v in stage_ms.items()},
        "roofline": {"kernel": "fp8_moe_gemm_kernel<1, 4> (MoE gate/up, SwiGLU + e4m3 requant epilogue)",
                     "bound": "hbm",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(),
                     "algorithmic_bytes": int(bytes_gu), "flop": flop_gu, "ms": round(gu_ms, 4),
                     "mfma_tflops": round(flop_gu / (gu_ms * 1e-3) / 1e12, 1),
                     "mfma_frac": round(flop_gu / (gu_ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4)},
        "moe_mxfp4_decode": mxfp4,
        "decode_gemv": decode,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

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
import gc
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


def cpu_threads_available() -> int:
    """Threads the CPU baseline may use: the cores this job is allowed to
    run on, at most 16 (a one-GPU box's CPU share), or PIH_CPU_THREADS."""
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        allowed = os.cpu_count() or 1
    return int(os.environ.get("PIH_CPU_THREADS", min(16, allowed)))


def _grow(run, start: int, limit: int, budget_s: float):
    """Doubles the sample size from ``start`` until one run takes about
    ``budget_s`` / 2 or the sample reaches ``limit``; returns (size, s)."""
    size = max(1, min(start, limit))
    while True:
        t0 = time.perf_counter()
        run(size)
        elapsed = time.perf_counter() - t0
        if elapsed * 2 > budget_s or size * 2 > limit:
            return size, elapsed
        size *= 2


def cpu_baselines(ids, wts, x_bits):
    """The reference's CPU arithmetic (the C restatement oracle/pih_oracle.c,
    built -O2 without fast-math) timed on this host, single-threaded and on
    every thread the job may use (OpenMP over output elements; per-element
    arithmetic and results are identical for any thread count).  Each line
    times the same work its GPU counterpart measures, in that line's unit:
      cfg4  po_expert_fp8 (quant, gate/up, SiLU-mul x w, requant, down) on
            routed rows of the hottest expert, TFLOP/s (the headline's unit);
      cfg1  the Qwen3-0.6B MLP block in full, GB/s of its weights;
      cfg2  the seven Qwen3-8B BF16 projections at M = 1 in full, GB/s;
      cfg3  the seven W4A16 projections at M = 1 in full, GB/s;
      cfg5  the MXFP4 routed-expert chain (e4m3 activations) on the rows of
            one expert of the 64-token decode batch, GB/s of its weights."""
    import oracle
    from pih_amd import synth

    t_all = cpu_threads_available()
    lines = {}

    def line(name, unit, work, run, start, limit, budget, what):
        out = {}
        for label, th in (("threads_1", 1), ("threads_all", t_all)):
            oracle.set_threads(th)
            size, sec = _grow(run, start if th == 1 else start * th, limit, budget)
            out[label] = {"value": round(work(size) / sec, 4), "unit": unit, "threads": th,
                          "seconds": round(sec, 3), "sample": what(size)}
        lines[name] = out

    # cfg4: the headline's expert chain
    offsets = np.concatenate([[0], np.cumsum(np.bincount(ids.ravel(), minlength=E))])
    order = np.lexsort((np.tile(np.arange(TOPK), T), np.repeat(np.arange(T), TOPK), ids.ravel()))
    row_token = np.repeat(np.arange(T), TOPK)[order]
    row_weight = wts.ravel()[order].astype(np.float32)
    counts = np.diff(offsets)
    e = int(np.argmax(counts))
    b = int(offsets[e])
    w13, s13 = synth.fp8_block_weight(synth.config_seed(4, 20 + e), 2 * I, H)
    w2, s2 = synth.fp8_block_weight(synth.config_seed(4, 600 + e), H, I)
    flop_row = 2.0 * (2 * I * H + H * I)
    line("cfg4_fp8_expert", "TFLOP/s", lambda r: flop_row * r / 1e12,
         lambda r: oracle.expert_fp8(np.ascontiguousarray(x_bits[row_token[b:b + r]]), row_weight[b:b + r], H, I,
                                     w13, s13, w2, s2), 2, int(counts[e]), 5.0,
         lambda r: f"po_expert_fp8 on {r} routed rows of expert {e} (fp32 scales)")
    # cfg1: Qwen3-0.6B MLP block, x [16, 1024]
    xq = synth.bf16_normal(synth.config_seed(1, 0), (16, 1024))
    wg = synth.bf16_normal(synth.config_seed(1, 1), (3072, 1024), std=0.02)
    wu = synth.bf16_normal(synth.config_seed(1, 2), (3072, 1024), std=0.02)
    wd = synth.bf16_normal(synth.config_seed(1, 3), (1024, 3072), std=0.02)
    mlp_bytes = 3 * 3072 * 1024 * 2
    line("cfg1_qwen_mlp_m16", "GB/s", lambda r: mlp_bytes * r / 1e9,
         lambda r: [oracle.qwen_mlp(xq, wg, wu, wd) for _ in range(r)], 1, 64, 2.0,
         lambda r: f"{r} x the full MLP block (x [16,1024], gate/up [3072,1024], down [1024,3072])")
    # cfg2 / cfg3: the seven Qwen3-8B projections at M = 1
    xs = {k: synth.bf16_normal(synth.config_seed(2, 500 + k), (1, k)) for k in (4096, 12288)}
    # weight values do not change the CPU's time; draw them fast: bf16 bits
    # with magnitudes below 2^-5 and random signs; INT4 codes, zeros and
    # scales in their valid ranges
    rng = np.random.default_rng(synth.config_seed(2, 510))
    bw = [((rng.integers(0, 1 << 16, (n, k), dtype=np.uint16) & np.uint16(0x3CFF)) | np.uint16(0x8000)
           * rng.integers(0, 2, (n, k), dtype=np.uint16)).astype(np.uint16) for _, n, k in QWEN8B]
    b_bytes = sum(n * k * 2 for _, n, k in QWEN8B)
    line("cfg2_bf16_decode_m1", "GB/s", lambda r: b_bytes * r / 1e9,
         lambda r: [[oracle.bf16_gemm(xs[k], w) for (_, _, k), w in zip(QWEN8B, bw)] for _ in range(r)], 1, 16, 2.0,
         lambda r: f"{r} x the 7 projections (bf16 weights, M = 1)")
    del bw
    iw = [(rng.integers(0, 1 << 32, (n, k // 8), dtype=np.uint32),
           oracle.f32_to_bf16_bits(rng.uniform(0.001, 0.02, (n, k // 128)).astype(np.float32)),
           rng.integers(0, 1 << 32, (n, (k // 128 + 7) // 8), dtype=np.uint32)) for _, n, k in QWEN8B]
    i_bytes = sum(n * k // 2 + (n * k // 128) * 2 + n * ((k // 128 + 7) // 8) * 4 for _, n, k in QWEN8B)
    line("cfg3_w4a16_decode_m1", "GB/s", lambda r: i_bytes * r / 1e9,
         lambda r: [[oracle.w4a16_asym(xs[k], *w) for (_, _, k), w in zip(QWEN8B, iw)] for _ in range(r)], 1, 16,
         3.0, lambda r: f"{r} x the 7 projections (asymmetric INT4, M = 1)")
    del iw
    # cfg5: one expert of the 64-token MXFP4 decode batch
    ids5, wts5 = synth.zipf_router(synth.config_seed(5, 64), 64, E, TOPK)
    e5 = int(np.argmax(np.bincount(ids5.ravel(), minlength=E)))
    tok5 = np.nonzero((ids5 == e5).any(axis=1))[0]
    rw5 = wts5[ids5 == e5].astype(np.float32)
    x5 = synth.bf16_normal(synth.config_seed(5, 65), (64, H))
    w1p, w1s = synth.mxfp4_weight(synth.config_seed(5, 700), I, H)
    w3p, w3s = synth.mxfp4_weight(synth.config_seed(5, 701), I, H)
    w2p, w2s = synth.mxfp4_weight(synth.config_seed(5, 702), H, I)
    mx_bytes = 3 * I * H // 2 + 3 * I * H // 32
    line("cfg5_mxfp4_expert_t64", "GB/s", lambda r: mx_bytes / 1e9,
         lambda r: oracle.routed_expert_fp4(np.ascontiguousarray(x5[tok5[:r]]), rw5[:r], H, I, w1p, w1s, w2p, w2s,
                                            w3p, w3s), len(tok5), len(tok5), 4.0,
         lambda r: f"po_routed_expert_fp4 on all {r} rows of expert {e5} (one pass over its weights)")
    head = lines["cfg4_fp8_expert"]["threads_all"]
    return {"value": head["value"], "unit": "TFLOP/s", "cores": head["threads"], "kind": "port",
            "sample": head["sample"] + f", {head['seconds']} s", "host_nproc": os.cpu_count(),
            "threads_available": t_all, "lines": lines}


QWEN8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
          ("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]


def _timed(torch, fn, iters: int):
    """Mean ms per call of fn(i) measured with HIP events on the launch stream.
    The Python garbage collector is off meanwhile: the eager decode loops
    launch from Python, and a collection pass inside the timed region
    (measured: one ~50 ms stall in 30 passes) idles the GPU."""
    s = torch.cuda.current_stream()
    fn(0)
    s.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    gc_was_on = gc.isenabled()
    gc.collect()
    gc.disable()
    try:
        ev0.record(s)
        for i in range(iters):
            fn(i)
        ev1.record(s)
        ev1.synchronize()
    finally:
        if gc_was_on:
            gc.enable()
    return ev0.elapsed_time(ev1) / iters


def _graphed(torch, make_calls, nsets: int, iters: int):
    """Mean ms per pass with the passes over all ``nsets`` weight sets
    captured back to back in one HIP graph (torch.cuda.CUDAGraph), as a
    captured decode loop would hold them, and the graph replayed; the
    launches inside are the same C-ABI calls, captured on the graph's stream.
    (A graph per pass pays one graph launch per pass; replaying such
    per-pass graphs measured slower than the eager launches.)"""
    from pih_amd.device import stream_handle

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        keep = [make_calls(j, stream_handle()) for j in range(nsets)]
    torch.cuda.synchronize()
    reps = max(2, iters // nsets)
    ms = _timed(torch, lambda i: g.replay(), reps)
    del keep
    return ms / nsets


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
    from pih_amd.linear import bf16_gemm_workspace

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
    # ---- BF16 decode, M = 1, 8, 64, and a 128-row batch (the big tiles with
    # the K split into each projection's queried workspace)
    set_bytes = sum(n * k * 2 for _, n, k in QWEN8B)
    nsets = max(2, -(-600_000_000 // set_bytes))
    wsets = [[(torch.randn(n, k, device=dev, generator=gen) * 0.02).to(torch.bfloat16) for _, n, k in QWEN8B]
             for _ in range(nsets)]
    for m in (1, 8, 64, 128):
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
    # the workspace each projection queries (a K split of the projections
    # with fewer tiles than CUs), allocated once like a caller's scratch
    wsb = [bf16_gemm_workspace(m, n, k) for _, n, k in QWEN8B]
    scratch = torch.empty(max(wsb) or 1, dtype=torch.uint8, device=dev)
    reqs = [abi.request(abi.LN["bf16_gemm"], a_bf16=ptr(xs[k]), w_bf16=ptr(wsets[0][j]), output=ptr(ys[j]),
                        workspace=ptr(scratch) if wsb[j] else 0, workspace_bytes=wsb[j], stream=stream_handle(),
                        m=m, n=n, k=k, output_type=abi.OUTPUT_BF16) for j, (_, n, k) in enumerate(QWEN8B)]

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


V4_H, V4_I, V4_TOPK = 4096, 2048, 6


def v4_router_inputs(tokens: int):
    """Router logits ~N(0, 1) and a selection bias (N(0, 0.05) with +1.5 on
    three experts, so a batch holds both light and multi-tile experts)."""
    from pih_amd import synth

    raw = synth.normal(synth.config_seed(6, tokens), tokens * E).astype(np.float32).reshape(tokens, E)
    bias = (0.05 * synth.normal(synth.config_seed(6, 1), E)).astype(np.float32)
    bias[[3, 77, 140]] += np.float32(1.5)
    return raw, bias


def bench_v4flash(torch, iters: int):
    """The reference's production MoE geometry, DeepSeek-V4-Flash
    (include/pih/model/deepseek_v4_config.h:22-27: hidden 4096, 256 routed
    experts, 6 active; intermediate 2048; MXFP4 experts x e4m3 activations):
    the device router (sqrt-softplus + bias, weights x 1.5) and the layer
    entry at decode batches of 64 and 512 tokens.  HBM-bound: bytes =
    touched experts x 13,369,344 (the reference's expert bundle: W1/W3/W2
    e2m1 + UE8M0) + token activations in and out; the router is timed on
    its own (it reads the f32 logits)."""
    from pih_amd import abi, synth
    from pih_amd.linear import MoeLayer, router_topk

    H4, I4, K6 = V4_H, V4_I, V4_TOPK
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x50494806)
    w13 = torch.randint(0, 256, (E, 2 * I4, H4 // 2), dtype=torch.uint8, device=dev, generator=gen)
    s13 = torch.randint(118, 127, (E, 2 * I4, H4 // 32), dtype=torch.uint8, device=dev, generator=gen)
    w2 = torch.randint(0, 256, (E, H4, I4 // 2), dtype=torch.uint8, device=dev, generator=gen)
    s2 = torch.randint(118, 127, (E, H4, I4 // 32), dtype=torch.uint8, device=dev, generator=gen)
    per_expert = 3 * I4 * H4 // 2 + 3 * I4 * H4 // 32
    out = {}
    for tokens in (64, 512):
        raw, bias = v4_router_inputs(tokens)
        raw_d = torch.from_numpy(raw).to(dev)
        bias_d = torch.from_numpy(bias).to(dev)
        ids_d, wts_d, rflag = router_topk(raw_d, K6, abi.ROUTER_SQRT_SOFTPLUS, 1.5, bias_d)
        router_ms = _timed(torch, lambda i: router_topk(raw_d, K6, abi.ROUTER_SQRT_SOFTPLUS, 1.5, bias_d,
                                                         flag=rflag, out=(ids_d, wts_d)), iters)
        ids = ids_d.cpu().numpy()
        touched = int((np.bincount(ids.ravel(), minlength=E) > 0).sum())
        x = torch.from_numpy(synth.bf16_normal(synth.config_seed(6, tokens + 1), (tokens, H4)).view(np.int16))
        x = x.to(dev).view(torch.bfloat16)
        layer = MoeLayer(w13, s13, w2, s2, tokens, K6, weight_format=abi.WEIGHT_MXFP4,
                         activation_type=abi.ACTIVATION_E4M3, swiglu_limit=10.0)
        ms = _timed(torch, lambda i: layer.forward(x, ids_d, wts_d), iters)
        if int(layer.flag.item()) or int(rflag.item()):
            raise RuntimeError(f"v4-flash error flags {int(layer.flag.item())} {int(rflag.item())}")
        algo = touched * per_expert + tokens * H4 * 2 * 2
        flop = 2.0 * tokens * K6 * 3 * I4 * H4
        gbs = algo / (ms * 1e-3) / 1e9
        out[f"t{tokens}_e4m3"] = {"us_per_layer": round(ms * 1e3, 1), "gbs": round(gbs, 1),
                                  "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                  "tflops": round(flop / (ms * 1e-3) / 1e12, 2), "touched_experts": touched,
                                  "algorithmic_bytes": algo, "router_us": round(router_ms * 1e3, 1)}
        del layer
    return out


def _rotation(torch, gen, per_bytes: int, min_total: int = 600_000_000):
    """One uint8 buffer of random bytes holding enough weight sets of
    ``per_bytes`` (each 256-byte aligned) that cycling through them exceeds
    the 256 MB Infinity Cache; returns (buffer, set stride, set count)."""
    stride = (per_bytes + 255) // 256 * 256
    nsets = max(2, -(-min_total // stride))
    buf = torch.randint(0, 256, (nsets * stride,), dtype=torch.uint8, device="cuda", generator=gen)
    return buf, stride, nsets


def _line(ms: float, algo: int, flop: float, peak_tflops: float) -> dict:
    gbs = algo / (ms * 1e-3) / 1e9
    tf = flop / (ms * 1e-3) / 1e12
    bound = "hbm" if algo / (HBM_PEAK_GBS * 1e9) >= flop / (peak_tflops * 1e12) else "mfma"
    return {"us": round(ms * 1e3, 2), "gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "tflops": round(tf, 2), "frac_mfma": round(tf / peak_tflops, 4), "bound": bound,
            "algorithmic_bytes": int(algo)}


def bench_dropin(torch, iters: int):
    """The entries an unchanged reference model calls, one launch each, at
    the reference's call shapes, weights rotated through > 512 MB:
      DeepSeek table  launch_fp4_gemm per routed expert (V4 Flash W1/W3
                      4096 -> 2048, W2 2048 -> 4096) at 8 and 128 rows;
                      launch_fp8_gemm at the model's dense call shapes at
                      M = 4 (decode) and 2048 (prefill);
                      launch_grouped_fp8_gemm at G = 8, 1024, 4096 (wo_a);
      Qwen model      pih_qwen_w4a16_gemm_compat_v1 launched by name from the
                      code object with the model plan's geometry at the
                      Qwen3-0.6B shapes, M = 1; the BF16 MLP block of
                      configs[0] (x [16, 1024]);
      LM heads        DeepSeek launch_lm_head at 1, 64 and 512 rows and the
                      Qwen3-0.6B 1..32-row plan bank at 1 and 32 rows;
      router          launch_router_topk (softmax top-8 of 256) and
                      launch_route_plan at 4096 tokens."""
    from pih_amd import abi
    from pih_amd.device import ptr, stream_handle
    from pih_amd.linear import QwenMlpBlock, route_plan, route_plan_workspace, router_topk
    from pih_amd.qwen import QwenCodeObject

    dev = torch.device("cuda")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x50494806)
    D = abi.deepseek_pack()
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    out = {}

    def codes(shape):  # e4m3 codes without the two NaN codes
        c = torch.randint(0, 0x7E, shape, dtype=torch.uint8, device=dev, generator=gen)
        return c | (torch.randint(0, 2, shape, dtype=torch.uint8, device=dev, generator=gen) << 7)

    def scales(shape, lo, hi):
        return torch.randint(lo, hi, shape, dtype=torch.uint8, device=dev, generator=gen)

    # ---- launch_fp4_gemm per expert
    for n, k in ((2048, 4096), (4096, 2048)):
        wb, ws = n * k // 2, n * k // 32
        buf, stride, nsets = _rotation(torch, gen, wb + ws)
        buf.view(nsets, stride)[:, wb:wb + ws] = scales((nsets, ws), 118, 125)
        for m in (8, 128, 512):
            a, sa = codes((m, k)), scales((m, k // 128), 118, 125)
            o = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            reqs = [abi.request(abi.DS["fp4_gemm"], activation_e4m3=ptr(a), activation_scale_bits=ptr(sa),
                                packed_weight=ptr(buf) + j * stride, weight_scale_bits=ptr(buf) + j * stride + wb,
                                output_bf16=ptr(o), error_flag=ptr(flag), stream=stream_handle(), m=m, n=n, k=k)
                    for j in range(nsets)]
            ms = _timed(torch, lambda i: D.call("launch_fp4_gemm", reqs[i % nsets]), iters)
            out[f"ds_fp4_gemm_m{m}_{k}to{n}"] = _line(ms, wb + ws + m * k + m * k // 128 + m * n * 2,
                                                     2.0 * m * n * k, FP8_PEAK_TFLOPS)
        del buf
    # ---- launch_fp8_gemm (UE8M0) at the dense call shapes (K -> N)
    for k, n in ((4096, 1024), (1024, 32768), (8192, 4096), (4096, 2048), (2048, 4096)):
        wb, ws = n * k, (n // 128) * (k // 128)
        buf, stride, nsets = _rotation(torch, gen, wb + ws)
        buf.view(nsets, stride)[:, wb:wb + ws] = scales((nsets, ws), 112, 118)
        buf.view(nsets, stride)[:, :wb] = codes((nsets, wb))
        for m in (4, 256, 2048):
            a, sa = codes((m, k)), scales((m, k // 128), 118, 124)
            o = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            reqs = [abi.request(abi.DS["fp8_gemm"], activation_e4m3=ptr(a), activation_scale_bits=ptr(sa),
                                weight_e4m3=ptr(buf) + j * stride, weight_scale_bits=ptr(buf) + j * stride + wb,
                                output=ptr(o), error_flag=ptr(flag), stream=stream_handle(), m=m, n=n, k=k,
                                output_type=1) for j in range(nsets)]
            ms = _timed(torch, lambda i: D.call("launch_fp8_gemm", reqs[i % nsets]), iters)
            out[f"ds_fp8_gemm_m{m}_{k}to{n}"] = _line(ms, wb + ws + m * k + m * (k // 128) + m * n * 2,
                                                     2.0 * m * n * k, FP8_PEAK_TFLOPS)
        del buf
    # ---- launch_grouped_fp8_gemm, G = 8, N_g = 1024, K_g = 4096
    g, ng, kg = 8, 1024, 4096
    wb, ws = g * ng * kg, g * (ng // 128) * (kg // 128)
    buf, stride, nsets = _rotation(torch, gen, wb + ws)
    buf.view(nsets, stride)[:, wb:wb + ws] = scales((nsets, ws), 112, 118)
    buf.view(nsets, stride)[:, :wb] = codes((nsets, wb))
    for t in (4, 2048):
        x = (torch.randn(t * g, kg, device=dev, generator=gen)).to(torch.bfloat16)
        aq = torch.empty(t * g, kg, dtype=torch.uint8, device=dev)
        asb = torch.empty(t * g, kg // 128, dtype=torch.uint8, device=dev)
        o = torch.empty(t, g * ng, dtype=torch.bfloat16, device=dev)
        reqs = [abi.request(abi.DS["grouped_fp8_gemm"], input_bf16=ptr(x), activation_e4m3=ptr(aq),
                            activation_scale_bits=ptr(asb), weight_e4m3=ptr(buf) + j * stride,
                            weight_scale_bits=ptr(buf) + j * stride + wb, output_bf16=ptr(o),
                            error_flag_u32=ptr(flag), stream=stream_handle(), token_count=t, group_count=g,
                            output_per_group=ng, input_per_group=kg) for j in range(nsets)]
        ms = _timed(torch, lambda i: D.call("launch_grouped_fp8_gemm", reqs[i % nsets]), iters)
        out[f"ds_grouped_fp8_t{t}_8x1024x4096"] = _line(ms, wb + ws + t * g * kg * 2 + t * g * ng * 2,
                                                       2.0 * t * g * ng * kg, FP8_PEAK_TFLOPS)
    del buf
    # ---- Qwen code object by name through the C++ kernel-module driver,
    # Qwen3-0.6B shapes, M = 1: the compatibility kernel in the reference's
    # geometry and the gfx950 plan's kernel (launches prepared once, as a
    # model's decode loop holds them)
    co = QwenCodeObject()
    for n, k in ((2048, 1024), (1024, 1024), (1024, 2048), (3072, 1024), (1024, 3072)):
        wb, ws = n * k // 2, (n * k // 128) * 2
        buf, stride, nsets = _rotation(torch, gen, wb + ws)
        buf.view(nsets, stride)[:, :wb] &= 0x77  # nibbles in [0, 7]: no reserved 8
        buf.view(nsets, stride)[:, wb:wb + ws] = torch.tensor([0x00, 0x20], dtype=torch.uint8,  # fp16 0.0078125
                                                              device=dev).repeat(nsets * ws // 2).view(nsets, ws)
        x = torch.randn(1, k, device=dev, generator=gen).to(torch.bfloat16)
        o = torch.empty(1, n, dtype=torch.bfloat16, device=dev)
        s = stream_handle()
        for variant, name in ((abi.QWEN_INT4_COMPAT, "qwen_compat"), (abi.QWEN_INT4_GFX950, "qwen_gfx950_plan")):
            launches = [co.prepare_w4a16(ptr(x), ptr(buf) + j * stride, ptr(buf) + j * stride + wb, ptr(o), ptr(flag),
                                         1, n, k, s, variant) for j in range(nsets)]
            ms = _timed(torch, lambda i: launches[i % nsets](), iters)
            out[f"{name}_w4a16_m1_{k}to{n}"] = _line(ms, wb + ws + k * 2 + n * 2, 2.0 * n * k, 2516.6)
        del buf, launches
    # ---- configs[0] MLP block (BF16 GemmPlan x3 + SiLU-mul), M = 16
    per = 3 * 3072 * 1024 * 2
    nsets = max(2, -(-600_000_000 // per))
    wv = (torch.randn(nsets, per // 2, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
    blocks = [QwenMlpBlock(wv[j, :3072 * 1024].view(3072, 1024), wv[j, 3072 * 1024:2 * 3072 * 1024].view(3072, 1024),
                           wv[j, 2 * 3072 * 1024:].view(1024, 3072), 16) for j in range(nsets)]
    x = torch.randn(16, 1024, device=dev, generator=gen).to(torch.bfloat16)
    ms = _timed(torch, lambda i: blocks[i % nsets].forward(x), iters)
    out["cfg1_qwen_mlp_m16"] = dict(_line(ms, per + 16 * 1024 * 2 * 2, 2.0 * 16 * 3 * 3072 * 1024, 2516.6),
                                    launches=4)
    del blocks, wv
    # ---- LM heads: DeepSeek launch_lm_head (1.06 GB bf16 weight) and the
    # Qwen3-0.6B tied head (311 MB, two copies rotated), fp32 logits
    from pih_amd.linear import QwenLmHead, deepseek_lm_head
    wd = (torch.randn(129280, 4096, device=dev, generator=gen, dtype=torch.float32) * 0.02).to(torch.bfloat16)
    for m in (1, 64, 512):
        x = torch.randn(m, 4096, device=dev, generator=gen).to(torch.bfloat16)
        lo = torch.empty(m, 129280, dtype=torch.float32, device=dev)
        ms = _timed(torch, lambda i: deepseek_lm_head(x, wd, out=lo, flag=flag), iters)
        out[f"ds_lm_head_m{m}_4096to129280"] = _line(ms, 129280 * 4096 * 2 + m * 4096 * 2 + m * 129280 * 4,
                                                     2.0 * m * 129280 * 4096, 2516.6)
    del wd
    wq = [(torch.randn(151936, 1024, device=dev, generator=gen) * 0.02).to(torch.bfloat16) for _ in range(2)]
    head = QwenLmHead(32)
    for m in (1, 32):
        x = torch.randn(m, 1024, device=dev, generator=gen).to(torch.bfloat16)
        lo = torch.empty(m, 151936, dtype=torch.float32, device=dev)
        ms = _timed(torch, lambda i: head.execute(x, wq[i % 2], lo), iters)
        out[f"qwen_lm_head_m{m}_1024to151936"] = _line(ms, 151936 * 1024 * 2 + m * 1024 * 2 + m * 151936 * 4,
                                                       2.0 * m * 151936 * 1024, 2516.6)
    del wq
    # ---- router top-k and route plan, 4096 tokens x 256 experts
    sc = torch.randn(T, E, device=dev, generator=gen)
    ids, wts, _ = router_topk(sc, TOPK, abi.ROUTER_SOFTMAX, flag=flag)
    ms = _timed(torch, lambda i: router_topk(sc, TOPK, abi.ROUTER_SOFTMAX, flag=flag, out=(ids, wts)), iters)
    out["router_topk_softmax_t4096_e256_k8"] = {"us": round(ms * 1e3, 2)}
    o_off, o_rt, o_rw, o_tr, _ = route_plan(ids, wts, E, flag=flag)
    ws = torch.empty(route_plan_workspace(T, TOPK, E), dtype=torch.uint8, device=dev)
    rp = abi.request(abi.LN["route_plan"], topk_ids_u32=ptr(ids), topk_weights_f32=ptr(wts),
                     expert_offsets_u32=ptr(o_off), row_token_u32=ptr(o_rt), row_weight_f32=ptr(o_rw),
                     token_rows_u32=ptr(o_tr), workspace=ptr(ws), workspace_bytes=ws.numel(),
                     error_flag_u32=ptr(flag), stream=stream_handle(), token_count=T, top_k=TOPK, expert_count=E)
    L = abi.linear_pack()
    ms = _timed(torch, lambda i: L.call("launch_route_plan", rp), iters)
    out["route_plan_t4096_e256_k8"] = {"us": round(ms * 1e3, 2)}
    if int(flag.item()):
        raise RuntimeError(f"drop-in leg error flag {int(flag.item()):#x}")
    return out


def bench_buckets(torch, layer, ids, wts, iters: int):
    """Per-expert-bucket utilisation of the cfg4 gate/up kernel: the same
    launch restricted to the experts with <= 64 routed rows (weight
    streaming, HBM-bound) and to the others (weight reuse, MFMA-bound), each
    over its own contiguous row segments (the plan of the full layer with
    the other bucket's experts emptied)."""
    from pih_amd import abi
    from pih_amd.device import ptr, stream_handle

    L = abi.linear_pack()
    flat = ids.ravel().astype(np.int64)
    tok = np.repeat(np.arange(T), TOPK)
    order = np.lexsort((np.tile(np.arange(TOPK), T), tok, flat))
    e_sorted, t_sorted, w_sorted = flat[order], tok[order], wts.ravel()[order]
    counts = np.bincount(flat, minlength=E)
    out = {}
    for name, sel in (("light_le64_rows", (counts > 0) & (counts <= 64)), ("heavy_gt64_rows", counts > 64)):
        keep = sel[e_sorted]
        offsets = np.concatenate([[0], np.cumsum(np.where(sel, counts, 0))]).astype(np.int32)
        rows = int(keep.sum())
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
        off_d, rt_d = dev(offsets), dev(t_sorted[keep].astype(np.int32))
        rw_d = dev(w_sorted[keep].astype(np.float32))
        mq = torch.empty(rows, I, dtype=torch.uint8, device="cuda")
        ms_ = torch.empty(rows, I // 128, dtype=torch.float32, device="cuda")
        r = abi.request(abi.LN["moe_fp8_gemm"], activation_e4m3=ptr(layer.xq), activation_scale=ptr(layer.xs),
                        row_token_u32=ptr(rt_d), weight_e4m3=ptr(layer.w13), weight_scale=ptr(layer.w13_scale),
                        expert_offsets_u32=ptr(off_d), row_weight_f32=ptr(rw_d), output=ptr(mq),
                        output_scale=ptr(ms_), error_flag_u32=ptr(layer.flag), stream=stream_handle(),
                        row_capacity=rows, expert_count=E, n=2 * I, k=H, activation_rows=T,
                        scale_format=abi.SCALE_F32, output_type=abi.OUTPUT_SWIGLU_E4M3, swiglu_limit=0.0)
        ms = _timed(torch, lambda i: L.call("launch_moe_fp8_gemm", r), iters)
        n_exp = int(sel.sum())
        algo = n_exp * (2 * I * H + (2 * I // 128) * (H // 128) * 4) + rows * (H + H // 32) + rows * (I + I // 32)
        out[name] = dict(_line(ms, algo, 2.0 * rows * 2 * I * H, FP8_PEAK_TFLOPS), experts=n_exp, rows=rows)
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
    ap.add_argument("--legs", default=",".join(LEGS),
                    help="comma-separated legs to run (default all: " + ",".join(LEGS) + "); without moe_fp8 "
                         "the line carries only the side measurements (for profiling one leg)")
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
    legs = {leg for leg in args.legs.split(",") if leg}
    unknown = legs - set(LEGS)
    if unknown:
        print(f"bench.py: unknown legs {sorted(unknown)}", file=sys.stderr)
        return 2
    for flag_name, leg in (("no_cpu", "cpu"), ("no_decode", "decode"), ("no_mxfp4", "mxfp4")):
        if getattr(args, flag_name):
            legs.discard(leg)

    import torch

    from pih_amd import abi
    from pih_amd.device import engine_stream, flag_value
    from pih_amd.linear import MoeFp8Layer, MoeLayer

    if "moe_fp8" not in legs:
        return side_legs_only(torch, legs, args)

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
        buckets = None
        if "buckets" in legs:
            log("gate/up kernel per expert bucket")
            buckets = bench_buckets(torch, staged, ids, wts, iters=max(10, args.steps))
            if flag_value(staged.flag):
                log(f"device error flag {flag_value(staged.flag):#x}")
                return 1
            log("buckets: " + json.dumps(buckets))
    ms = wall * 1000.0 / args.steps
    tflops = flop / (ms * 1e-3) / 1e12
    gu_ms = stage_ms["gate_up"]
    gu_gbs = bytes_gu / (gu_ms * 1e-3) / 1e9
    log("stage ms: " + ", ".join(f"{k}={v:.3f}" for k, v in stage_ms.items()))

    del layer, staged, w13, w2
    torch.cuda.empty_cache()
    side = run_side_legs(torch, legs, args)
    cpu = None
    if "cpu" in legs:
        log("cpu baseline")
        cpu = cpu_baselines(ids, wts, x_bits)

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
        "roofline": {"kernel": "fp8_moe_gemm_kernel<0, 1, 4, false> (MoE gate/up, SwiGLU + e4m3 requant epilogue)",
                     "bound": "hbm",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(),
                     "algorithmic_bytes": int(bytes_gu), "flop": flop_gu, "ms": round(gu_ms, 4),
                     "mfma_tflops": round(flop_gu / (gu_ms * 1e-3) / 1e12, 1),
                     "mfma_frac": round(flop_gu / (gu_ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4)},
        "expert_buckets": buckets,
        "moe_mxfp4_decode": side.get("mxfp4"),
        "moe_mxfp4_v4_flash": side.get("v4flash"),
        "decode_gemv": side.get("decode"),
        "drop_in": side.get("dropin"),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


LEGS = ("moe_fp8", "buckets", "mxfp4", "v4flash", "decode", "dropin", "cpu")


def run_side_legs(torch, legs, args) -> dict:
    """The side measurements, each on the engine stream, freeing device
    memory between legs."""
    from pih_amd.device import engine_stream

    iters = max(10, args.steps)
    out = {}
    for leg, fn, what in (("mxfp4", bench_mxfp4, "MXFP4 MoE decode (configs[4])"),
                          ("v4flash", bench_v4flash, "MXFP4 MoE at the DeepSeek-V4-Flash geometry"),
                          ("decode", bench_decode, "decode GEMV / prefill (configs[1], [2])"),
                          ("dropin", bench_dropin, "drop-in entries at the reference's call shapes")):
        if leg not in legs:
            continue
        log(what)
        with engine_stream():
            out[leg] = fn(torch, iters=iters)
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        log(f"{leg}: " + json.dumps(out[leg]))
    return out


def side_legs_only(torch, legs, args) -> int:
    """A profiling run of chosen side legs: prints their results as one JSON
    line without the headline (``value`` null)."""
    side = run_side_legs(torch, legs, args)
    print(json.dumps({"metric": METRIC, "value": None, "legs": sorted(legs), **side}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

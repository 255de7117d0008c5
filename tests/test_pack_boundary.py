"""CPU tests of the drop-in boundary (no device work):
  - every C struct the packs exchange has the size and field offsets the
    ctypes mirror assumes (headers compiled with gcc);
  - each pack exports exactly the two Kernel Pack symbols and passes the
    reference loader's checks (src/microkernel/kernel_pack_loader.cpp:90-123);
  - request validation: NULL request, wrong struct_size or abi_version give
    INVALID_ARGUMENT; stream 0 and bad shapes are rejected before any
    launch; entries outside the linear path answer UNAVAILABLE.
"""
import ctypes as C
import json
import os
import subprocess
import tempfile

import pytest

from pih_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")

DS_C = {n: f"pih_deepseek_{n}_launch_v1" for n in abi.DS}
LN_C = {n: f"pih_amd_{n}_launch_v1" for n in abi.LN}
LN_C["workspace_query"] = "pih_amd_workspace_query_v1"
LN_C["w4a16"] = "pih_amd_w4a16_launch_v1"


def _layout_program():
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "pih/contracts/deepseek_kernels_v1.h"',
             '#include "pih/contracts/amd_linear_kernels_v1.h"', '#include "pih/contracts/qwen_kernels_v1.h"',
             '#include "pih/backend/hip/kernel_module_v1.h"', '#include "pih/contracts/qwen_int4_plan_gfx950_v1.h"',
             "int main(void) {", 'printf("{");']
    first = True

    def emit(key, ctype, fields):
        nonlocal first
        sep = "" if first else ","
        first = False
        lines.append(f'printf("{sep}\\"{key}\\": [%zu", sizeof({ctype}));')
        for f in fields:
            lines.append(f'printf(", %zu", offsetof({ctype}, {f}));')
        lines.append('printf("]");')

    for n, t in abi.DS.items():
        emit("ds." + n, DS_C[n], [f[0] for f in t._fields_])
    for n, t in abi.LN.items():
        emit("ln." + n, LN_C[n], [f[0] for f in t._fields_])
    emit("status", "pih_status_v1", [f[0] for f in abi.Status._fields_])
    emit("identity", "pih_kernel_pack_identity_v1", [f[0] for f in abi.Identity._fields_])
    emit("api", "pih_kernel_pack_api_v1", [f[0] for f in abi.PackApi._fields_])
    emit("ds_api", "pih_deepseek_kernels_api_v1", [f[0] for f in abi.DS_API._fields_])
    emit("ln_api", "pih_amd_linear_kernels_api_v1", [f[0] for f in abi.LN_API._fields_])
    emit("qwen_api", "pih_qwen_kernels_api_v1", [f[0] for f in abi.QWEN_API._fields_])
    emit("w4a16_problem", "pih_amd_w4a16_problem_v1", [f[0] for f in abi.W4A16_PROBLEM._fields_])
    for key, ctype, t in (("km_parameter", "pih_hip_kernel_parameter_v1", abi.KM_PARAMETER),
                          ("km_signature", "pih_hip_kernel_signature_v1", abi.KM_SIGNATURE),
                          ("km_geometry", "pih_hip_launch_geometry_v1", abi.KM_GEOMETRY),
                          ("km_arguments", "pih_hip_kernel_arguments_v1", abi.KM_ARGUMENTS),
                          ("qwen_int4_plan", "pih_qwen_int4_gemm_plan_v1", abi.QWEN_INT4_PLAN)):
        emit(key, ctype, [f[0] for f in t._fields_])
    lines += ['printf("}\\n");', "return 0; }"]
    return "\n".join(lines)


def test_c_struct_layouts_match_ctypes_mirror():
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "layout.c")
        exe = os.path.join(d, "layout")
        with open(src, "w") as f:
            f.write(_layout_program())
        subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", INCLUDE, src, "-o", exe], check=True)
        got = json.loads(subprocess.run([exe], check=True, capture_output=True, text=True).stdout)

    def mirror(t):
        return [C.sizeof(t)] + [getattr(t, f[0]).offset for f in t._fields_]

    want = {"ds." + n: mirror(t) for n, t in abi.DS.items()}
    want.update({"ln." + n: mirror(t) for n, t in abi.LN.items()})
    want.update(status=mirror(abi.Status), identity=mirror(abi.Identity), api=mirror(abi.PackApi),
                ds_api=mirror(abi.DS_API), ln_api=mirror(abi.LN_API), qwen_api=mirror(abi.QWEN_API),
                w4a16_problem=mirror(abi.W4A16_PROBLEM), km_parameter=mirror(abi.KM_PARAMETER),
                km_signature=mirror(abi.KM_SIGNATURE), km_geometry=mirror(abi.KM_GEOMETRY),
                km_arguments=mirror(abi.KM_ARGUMENTS), qwen_int4_plan=mirror(abi.QWEN_INT4_PLAN))
    assert got == want
    assert got["status"][0] == 268
    assert len(abi.DS_ORDER) == 29


@pytest.mark.parametrize("path", [abi.DEEPSEEK_PACK, abi.LINEAR_PACK, abi.QWEN_PACK])
def test_pack_exports_exactly_two_symbols(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True, text=True).stdout
    syms = sorted(line.split()[-1] for line in out.splitlines() if line.split() and line.split()[-2] in "TtDdBbRr")
    assert syms == ["pih_kernel_pack_api_v1_get", "pih_kernel_pack_identity_v1_get"], syms


def test_packs_pass_reference_loader_checks():
    ds = abi.deepseek_pack()
    assert (ds.pack_id, ds.pack_abi, ds.architecture) == (
        "pih.kernels.deepseek-v4.gfx950", "pih.deepseek-gfx950-kernel-pack.v1", "gfx950")
    ln = abi.linear_pack()
    assert (ln.pack_id, ln.pack_abi, ln.architecture) == (
        "pih.kernels.amd-linear.gfx950", "pih.amd-linear-kernels.v1", "gfx950")
    for name in abi.DS_ORDER:
        assert getattr(ds.table, "launch_" + name), name
    for f, _ in abi.LN_ORDER:
        assert getattr(ln.table, f), f
    # bind_origin: absolute path OK, relative path rejected, no device work
    assert ds.api.bind_origin(b"/opt/pack.so").code == abi.OK
    assert ds.api.bind_origin(b"relative.so").code == abi.INVALID_ARGUMENT
    with pytest.raises(abi.PackError):
        abi.load_pack(abi.LINEAR_PACK, "pih.deepseek-gfx950-kernel-pack.v1")


def test_canonical_id_rules():
    ok = [b"pih.kernels.x", b"a-b.c0"]
    bad = [b"", b".a", b"a.", b"a..b", b"A", b"a_b", b"a b"]
    assert all(abi.valid_canonical_id(v, 64) for v in ok)
    assert not any(abi.valid_canonical_id(v, 64) for v in bad)


def _all_entries():
    for n in abi.DS_ORDER:
        yield "ds", "launch_" + n, abi.DS[n]
    for f, s in abi.LN_ORDER:
        yield "ln", f, abi.LN[s]


@pytest.mark.parametrize("pack,entry,rtype", list(_all_entries()), ids=lambda v: v if isinstance(v, str) else "")
def test_header_validation(pack, entry, rtype):
    p = abi.deepseek_pack() if pack == "ds" else abi.linear_pack()
    fn = getattr(p.table, entry)
    st = fn(None)
    assert st.code == abi.INVALID_ARGUMENT and st.struct_size == 268 and st.abi_version == 1
    r = abi.request(rtype)
    r.struct_size -= 4
    assert fn(C.byref(r)).code == abi.INVALID_ARGUMENT
    r = abi.request(rtype)
    r.abi_version = 2
    assert fn(C.byref(r)).code == abi.INVALID_ARGUMENT


HOT_DS = {"fp8_activation_quant", "fp8_gemm", "grouped_fp8_gemm", "route_gather", "fp4_gemm", "expert_swiglu",
          "expert_accumulate", "router_gemm", "shared_swiglu", "expert_finalize", "lm_head"}


@pytest.mark.parametrize("name", [n for n in abi.DS_ORDER if n not in HOT_DS])
def test_non_linear_entries_unavailable(name):
    st = abi.deepseek_pack().call("launch_" + name, abi.request(abi.DS[name]))
    assert st.code == abi.UNAVAILABLE, st


@pytest.mark.parametrize("name", sorted(HOT_DS))
def test_hot_entries_reject_zero_stream(name):
    r = abi.request(abi.DS[name])
    for f, t in r._fields_:
        if t is abi.UPTR and f != "stream":
            setattr(r, f, 0x1000)
    for f in ("m", "n", "k", "token_count", "route_count", "packed_token_count", "logical_k", "group_count",
              "output_per_group", "input_per_group", "expert_count", "hidden_size"):
        if hasattr(r, f):
            setattr(r, f, 128)
    if hasattr(r, "output_type"):
        r.output_type = 1
    st = abi.deepseek_pack().call("launch_" + name, r)
    assert st.code == abi.INVALID_ARGUMENT, st


def test_linear_entries_reject_bad_requests():
    ln = abi.linear_pack()
    r = abi.request(abi.LN["moe_fp8_gemm"], activation_e4m3=0x1000, activation_scale=0x1000, weight_e4m3=0x1000,
                    weight_scale=0x1000, expert_offsets_u32=0x1000, output=0x1000, error_flag_u32=0x1000, stream=0,
                    row_capacity=128, expert_count=8, n=256, k=128, activation_rows=16, scale_format=1, output_type=1)
    assert ln.call("launch_moe_fp8_gemm", r).code == abi.INVALID_ARGUMENT  # stream 0
    r.stream = 0x2000
    r.k = 100
    assert ln.call("launch_moe_fp8_gemm", r).code == abi.INVALID_ARGUMENT  # k % 128
    r.k = 128
    r.scale_format = 9
    assert ln.call("launch_moe_fp8_gemm", r).code == abi.INVALID_ARGUMENT
    r.scale_format = 1
    r.output_type = 3
    r.n = 128
    assert ln.call("launch_moe_fp8_gemm", r).code == abi.INVALID_ARGUMENT  # SwiGLU needs n % 256
    q = abi.request(abi.LN["route_plan"], topk_ids_u32=1, topk_weights_f32=1, expert_offsets_u32=1, row_token_u32=1,
                    row_weight_f32=1, token_rows_u32=1, workspace=1, workspace_bytes=1, error_flag_u32=1, stream=1,
                    token_count=10, top_k=33, expert_count=8)
    assert ln.call("launch_route_plan", q).code == abi.INVALID_ARGUMENT  # top_k > 32
    q.top_k = 4
    assert ln.call("launch_route_plan", q).code == abi.INVALID_ARGUMENT  # workspace too small
    out = (C.c_uint64 * 1)()
    w = abi.request(abi.LN["workspace_query"], kind=abi.WORKSPACE_ROUTE_PLAN, m=4096, n=8, k=256,
                    bytes_u64=C.addressof(out))
    assert ln.call("query_workspace", w).code == abi.OK and out[0] > 0
    w.kind = 77
    assert ln.call("query_workspace", w).code == abi.INVALID_ARGUMENT


def test_bf16_gemm_workspace_sizes():
    """launch_bf16_gemm's scratch (query_workspace, host only): a K split of
    the big tiles when a GEMM has fewer 128 x 256 tiles than about a round on
    the 256 CUs -- 4 fp32 partial-sum slabs for M 2048, 4096 -> 1024 (64
    tiles, 64 K steps of 64) and M 1000, 4096 -> 2048; 3 for M 2048,
    4608 -> 1280 (80 tiles, 72 K steps); 8 for M 1000, 4096 -> 1024 (32
    tiles) and, the largest count when no count reaches a round, for M 128,
    12288 -> 4096 (16 tiles) -- and none for a full round (4096 -> 4096: 256
    tiles), decode shapes (m <= 64), shapes below the big tiles (K under 512:
    the 128 x 128 kernel) or K too short to split (at least 8 K steps per
    split)."""
    ln = abi.linear_pack()
    out = (C.c_uint64 * 1)()

    def q(m, n, k):
        w = abi.request(abi.LN["workspace_query"], kind=abi.WORKSPACE_BF16_GEMM, m=m, n=n, k=k,
                        bytes_u64=C.addressof(out))
        assert ln.call("query_workspace", w).code == abi.OK
        return int(out[0])

    assert q(2048, 1024, 4096) == 4 * 2048 * 1024 * 4
    assert q(1000, 2048, 4096) == 4 * 1000 * 2048 * 4
    assert q(2048, 1280, 4608) == 3 * 2048 * 1280 * 4
    assert q(2048, 4096, 4096) == 0
    assert q(64, 1024, 4096) == 0
    assert q(1000, 1024, 4096) == 8 * 1000 * 1024 * 4
    assert q(128, 4096, 12288) == 8 * 128 * 4096 * 4
    assert q(65, 128, 64) == 0
    assert q(2048, 1024, 512) == 0


def test_w4a16_grouped_rejects_bad_groups():
    """Group validation happens before any device work: count 0 or above 8,
    a NULL problem array, n not a multiple of 16 or a missing zeros pointer
    in the asymmetric format are INVALID_ARGUMENT."""
    ln = abi.linear_pack()
    probs = (abi.W4A16_PROBLEM * 9)()
    for p in probs:
        p.input_bf16 = p.qweight = p.scales = p.zeros = p.output_bf16 = 0x1000
        p.n = 256
    r = abi.request(abi.LN["w4a16_grouped"], problems=C.addressof(probs), error_flag_u32=0x1000, stream=0x2000,
                    problem_count=0, m=1, k=4096, format=abi.W4A16_ASYMMETRIC)
    assert ln.call("launch_w4a16_grouped", r).code == abi.INVALID_ARGUMENT
    r.problem_count = 9
    assert ln.call("launch_w4a16_grouped", r).code == abi.INVALID_ARGUMENT
    r.problem_count = 3
    r.problems = 0
    assert ln.call("launch_w4a16_grouped", r).code == abi.INVALID_ARGUMENT
    r.problems = C.addressof(probs)
    probs[1].n = 200
    assert ln.call("launch_w4a16_grouped", r).code == abi.INVALID_ARGUMENT
    probs[1].n = 256
    probs[2].zeros = 0
    assert ln.call("launch_w4a16_grouped", r).code == abi.INVALID_ARGUMENT
    r.format = 7
    assert ln.call("launch_w4a16_grouped", r).code == abi.INVALID_ARGUMENT


def test_moe_layer_workspace_carve():
    """query_moe_layer_workspace (host only) returns the exact carve: route
    plan scratch, offsets, row_token / row_weight / token_rows, the quantised
    tokens and intermediate (+ scales) and the bf16 expert rows, each rounded
    up to 256 bytes.  FP8 weights write the e4m3 intermediate straight from
    the gate/up epilogue, so they carry no bf16 intermediate; MXFP4 weights
    do (their intermediate is re-quantised by its own launch)."""
    ln = abi.linear_pack()
    up = lambda b: (b + 255) // 256 * 256
    T, k, E, H, I = 4096, 8, 256, 7168, 2048
    R = T * k
    out = (C.c_uint64 * 1)()
    ln.call("query_workspace", abi.request(abi.LN["workspace_query"], kind=abi.WORKSPACE_ROUTE_PLAN, m=T, n=k,
                                           k=E, bytes_u64=C.addressof(out)))
    plan = up(out[0]) + up((E + 1) * 4) + 3 * up(R * 4)

    def query(fmt, scale_fmt, act):
        need = (C.c_uint64 * 1)()
        q = abi.request(abi.LN["moe_layer"], required_bytes_u64=C.addressof(need), token_count=T, top_k=k,
                        expert_count=E, hidden_size=H, intermediate_size=I, weight_format=fmt,
                        scale_format=scale_fmt, activation_type=act)
        assert ln.call("query_moe_layer_workspace", q).code == abi.OK
        return int(need[0])

    fp8 = plan + up(T * H) + up(T * H // 128 * 4) + up(R * I) + up(R * I // 128 * 4) + up(R * H * 2)
    assert query(abi.WEIGHT_FP8, abi.SCALE_F32, 0) == fp8
    mx_e4m3 = plan + up(T * H) + up(T * H // 128) + up(R * I * 2) + up(R * I) + up(R * I // 128) + up(R * H * 2)
    assert query(abi.WEIGHT_MXFP4, 0, abi.ACTIVATION_E4M3) == mx_e4m3
    assert query(abi.WEIGHT_MXFP4, 0, abi.ACTIVATION_BF16) == plan + up(R * I * 2) + up(R * H * 2)

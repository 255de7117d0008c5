"""The backend-amd-hip plugin without a GPU.

Checks, against the reference backend's behaviour
(plugins/backend-nvidia-cuda/entrypoint.cpp and manifest.json):
  - the plugin ABI and device-contract structs have the same size and field
    offsets in include/ as the ctypes mirror (and, where the reference tree
    is present, as the reference's own headers);
  - the library exports only pih_plugin_entry_v1;
  - entry validation (host table, plugin table, one binding per process);
  - the lifecycle order register -> configure -> start -> ready -> drain ->
    stop -> dispose, with out-of-order calls answering FAILED_PRECONDITION;
  - the four capabilities it registers match its manifest, it resolves
    platform.linux.v1 in configure and calls validate_runtime once at start;
  - device calls before ready, with a foreign context or with malformed
    arguments are refused before any HIP call.
Each scenario runs in a fresh process: the plugin's binding is process state.
"""
import ctypes as C
import json
import os
import subprocess
import sys
import tempfile
import textwrap

import pytest

from pih_amd import backend as B
from pih_amd.abi import FAILED_PRECONDITION, INVALID_ARGUMENT, OK

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INCLUDE = "/root/reference/include"

STRUCTS = [("pih_capability_v1", B.Capability), ("pih_plugin_lifecycle_v1", B.Lifecycle),
           ("pih_host_api_v1", B.HostApi), ("pih_plugin_api_v1", B.PluginApi),
           ("pih_cuda_allocation_v1", B.Allocation), ("pih_nvidia_cuda_api_v1", B.RuntimeApi),
           ("pih_nvidia_cuda_memory_api_v1", B.MemoryApi), ("pih_nvidia_cuda_resources_api_v1", B.ResourcesApi),
           ("pih_nvidia_cuda_async_api_v1", B.AsyncApi), ("pih_platform_linux_api_v1", B.PlatformApi)]


def _layouts(include, headers):
    lines = ["#include <stdio.h>", "#include <stddef.h>"] + [f'#include "{h}"' for h in headers]
    lines += ["int main(void) {", 'printf("{");']
    for i, (ctype, t) in enumerate(STRUCTS):
        lines.append(f'printf("{"," if i else ""}\\"{ctype}\\": [%zu", sizeof({ctype}));')
        for f in t._fields_:
            lines.append(f'printf(", %zu", offsetof({ctype}, {f[0]}));')
        lines.append('printf("]");')
    lines += ['printf("}\\n");', "return 0; }"]
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "l.c"), os.path.join(d, "l")
        with open(src, "w") as f:
            f.write("\n".join(lines))
        subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", include, src, "-o", exe], check=True)
        return json.loads(subprocess.run([exe], check=True, capture_output=True, text=True).stdout)


def _mirror():
    return {c: [C.sizeof(t)] + [getattr(t, f[0]).offset for f in t._fields_] for c, t in STRUCTS}


def test_struct_layouts_match_mirror():
    got = _layouts(os.path.join(ROOT, "include"),
                   ["pih/plugin_sdk/plugin.h", "pih/contracts/device_cuda_v1.h"])
    assert got == _mirror()
    assert got["pih_cuda_allocation_v1"][0] == 48 and got["pih_host_api_v1"][0] == 48


@pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="reference headers not present on this machine")
def test_struct_layouts_match_reference_headers():
    headers = ["pih/plugin_sdk/abi.h", "pih/contracts/nvidia_cuda_v1.h", "pih/contracts/nvidia_cuda_memory_v1.h",
               "pih/contracts/nvidia_cuda_resources_v1.h", "pih/contracts/nvidia_cuda_async_v1.h",
               "pih/contracts/platform_linux_v1.h"]
    assert _layouts(REF_INCLUDE, headers) == _mirror()


def test_exports_only_the_entry_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", B.BACKEND_PLUGIN], capture_output=True, text=True,
                         check=True).stdout
    assert sorted(line.split()[-1] for line in out.splitlines() if " T " in line) == ["pih_plugin_entry_v1"]


def _run(body: str):
    script = "import ctypes as C, sys\nsys.path.insert(0, %r)\n" % ROOT
    script += "from pih_amd import backend as B\nfrom pih_amd.abi import *\n" + textwrap.dedent(body)
    r = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=120,
                       env=dict(os.environ, HIP_VISIBLE_DEVICES=""))
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_entry_validation_and_single_binding():
    out = _run("""
        import json
        h = B.PluginHost()
        res = {}
        res["null_host"] = h.enter(host=None).code
        bad = B.HostApi.from_buffer_copy(h.host); bad.activation_epoch = 0
        res["epoch0"] = h.enter(host=bad).code
        bad = B.HostApi.from_buffer_copy(h.host); bad.struct_size -= 8
        res["host_size"] = h.enter(host=bad).code
        res["null_plugin"] = h.enter(api=None).code
        p = B.PluginApi(); p.struct_size = C.sizeof(B.PluginApi) + 8; p.abi_version = 1
        res["plugin_size"] = h.enter(api=p).code
        h.load()
        res["id"] = [h.api.plugin_id.decode(), h.api.plugin_version.decode()]
        res["again"] = h.enter().code
        print(json.dumps(res))
    """)
    assert out == {"null_host": INVALID_ARGUMENT, "epoch0": INVALID_ARGUMENT, "host_size": INVALID_ARGUMENT,
                   "null_plugin": INVALID_ARGUMENT, "plugin_size": INVALID_ARGUMENT,
                   "id": ["pih.backend.amd-hip", "1.0.0"], "again": FAILED_PRECONDITION}


def test_lifecycle_order_capabilities_and_platform():
    out = _run("""
        import json
        h = B.PluginHost().load()
        seq = []
        for name in ["configure", "start", "ready", "drain", "stop", "register_plugin", "register_plugin",
                     "start", "ready", "configure", "configure", "ready", "start", "dispose", "start",
                     "drain", "ready", "ready", "dispose", "stop", "drain", "stop", "dispose", "dispose",
                     "register_plugin"]:
            seq.append(h.phase(name).code)
        foreign = h.phase("ready", context=C.c_void_p(0x1234)).code
        print(json.dumps({"seq": seq, "foreign": foreign, "platform_calls": h.platform_calls,
                          "resolves": h.resolves,
                          "registered": [r[:2] + r[3:] for r in h.registered]}))
    """)
    P, I = FAILED_PRECONDITION, INVALID_ARGUMENT
    assert out["seq"] == [P, P, P, P, P, OK, P,          # nothing before register; register once
                          P, P, OK, P, P, OK, P, P,      # configure, start; no dispose once started
                          P, OK, P, P, P, OK, OK, OK,    # ready; drain; stop; dispose
                          P, P]                          # a disposed plugin stays disposed
    assert out["foreign"] == I
    assert out["platform_calls"] == 1
    assert out["resolves"] == [["platform.linux.v1", "pih.platform.linux.v1", B.SCOPE_PROCESS, B.EXACTLY_ONE]]
    manifest = B.manifest_capabilities()
    got = {cap: (contract, B._NAMES["threading_model"][t], B._NAMES["scope"][s], B._NAMES["cardinality"][c])
           for cap, contract, t, s, c in out["registered"]}
    want = {cap: (m["contract_id"], m["threading_model"], m["scope"], m["cardinality"]) for cap, m in manifest.items()}
    assert got == want and len(got) == 4


def test_platform_failure_stops_start_and_allows_dispose():
    out = _run("""
        import json
        h = B.PluginHost(platform_status=UNAVAILABLE).load()
        seq = [h.phase(n).code for n in ("register_plugin", "configure", "start", "ready", "stop", "dispose")]
        print(json.dumps(seq))
    """)
    assert out == [OK, OK, 4, FAILED_PRECONDITION, FAILED_PRECONDITION, OK]


def test_device_calls_refused_before_ready_and_on_bad_arguments():
    out = _run("""
        import json
        h = B.PluginHost().load()
        h.phase("register_plugin")
        d = B.Device(h)
        r = {}
        r["prepare_early"] = d.prepare(0, 9, 5).code
        st, a = d.allocate(0, 4096); r["alloc_early"] = st.code
        r["retain_early"] = d.retain(0)[0].code
        h.phase("configure"); h.phase("start"); h.phase("ready")
        r["prepare_neg"] = d.prepare(-1, 9, 5).code
        r["prepare_major0"] = d.prepare(0, 0, 5).code
        st, a = d.allocate(0, 4096); r["alloc_unprepared"] = st.code
        st, a = d.allocate(0, 4096, alignment=48); r["alloc_align"] = st.code
        st, a = d.allocate(0, 4096, alignment=512); r["alloc_align512"] = st.code
        a = B.Allocation(C.sizeof(B.Allocation), 1); a.address = 64
        r["alloc_not_fresh"] = d.mem.allocate_device(d.mem.context, 0, 64, 256, C.byref(a)).code
        st, a = d.allocate(0, 4096, pinned=True); r["pinned_ordinal"] = st.code
        st, a = d.allocate(-1, 4096, pinned=True); r["pinned_unprepared"] = st.code
        r["retain_unprepared"] = d.retain(0)[0].code
        tok = B.UPTR(5)
        r["retain_nonzero_out"] = d.res.retain_primary_context(d.res.context, 0, 0, C.byref(tok)).code
        r["retain_bad_flags"] = d.retain(0, flags=0x10)[0].code
        r["stream_unknown_ctx"] = d.create_stream(0x1000)[0].code
        r["stream_null_ctx"] = d.create_stream(0)[0].code
        r["destroy_unknown"] = d.destroy_stream(0x2000).code
        r["copy_kind"] = d.copy_async(0x1000, 64, 64, 16, 9, 0x3000).code
        r["copy_unknown"] = d.copy_async(0x1000, 64, 64, 16, B.COPY_D2D, 0x3000).code
        r["memset_byte"] = d.memset_async(0x1000, 64, 256, 16, 0x3000).code
        r["memset_unknown"] = d.memset_async(0x1000, 64, 1, 16, 0x3000).code
        r["query_unknown"] = d.query(0x1000, 0x4000)[0].code
        r["sync_unknown"] = d.synchronize(0x1000, 0x3000).code
        r["last_error_unknown"] = d.clean_last_error(0x1000).code
        r["h2d_unprepared"] = d.copy_h2d(0, 64, C.c_char_p(b"x"), 1).code
        r["dealloc_null"] = d.mem.deallocate_device(d.mem.context, None).code
        r["foreign_ctx"] = d.rt.prepare_device(C.c_void_p(0x1234), 0, 9, 5).code
        h.shutdown()
        print(json.dumps(r))
    """)
    P, I = FAILED_PRECONDITION, INVALID_ARGUMENT
    assert out == {"prepare_early": P, "alloc_early": P, "retain_early": P, "prepare_neg": I,
                   "prepare_major0": I, "alloc_unprepared": P, "alloc_align": I, "alloc_align512": I,
                   "alloc_not_fresh": I, "pinned_ordinal": I, "pinned_unprepared": P, "retain_unprepared": P,
                   "retain_nonzero_out": I, "retain_bad_flags": I, "stream_unknown_ctx": P,
                   "stream_null_ctx": I, "destroy_unknown": P, "copy_kind": I, "copy_unknown": P,
                   "memset_byte": I, "memset_unknown": P, "query_unknown": P, "sync_unknown": P,
                   "last_error_unknown": P, "h2d_unprepared": P, "dealloc_null": I, "foreign_ctx": I}


def test_prepare_without_a_device_is_unavailable():
    out = _run("""
        import json
        h = B.PluginHost().load().activate()
        st = B.Device(h).prepare(0, 9, 5)
        h.shutdown()
        print(json.dumps([st.code, st.message.decode()]))
    """)
    assert out[0] in (4, FAILED_PRECONDITION)  # no visible device: unavailable (or identity failure)

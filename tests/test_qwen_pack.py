"""The gfx950 Qwen Kernel Pack and its code object, without a GPU.

Checks the pack's identity and exports, the bind_origin/root contract of
the reference's Qwen pack (plugins/kernels/qwen3/kernel_pack.cpp:10-36:
absolute path, the device image and manifest must exist under
<dir>/qwen3-<arch>/<arch>/, a second bind may not move the root, root()
before binding is a failed precondition), the manifest's field set and
digests, and the kernel symbols and kernarg layout recorded in the code
object's own metadata (qwen3_int4_gemm_plan.cpp:73-85: eight 64-bit
parameters at offsets 0..56).
"""
import json
import os
import shutil
import subprocess
import sys
import textwrap

import pytest

from pih_amd import abi, qwen

ROOT = os.path.join(abi.LIB_DIR, "qwen3-gfx950")
IMAGE = os.path.join(ROOT, "gfx950", "qwen_bf16_primitives.hsaco")
READELF = "/opt/rocm/llvm/bin/llvm-readelf"


def test_pack_identity_contract_and_root():
    p = abi.qwen_pack()
    assert (p.pack_id, p.pack_abi, p.architecture) == ("pih.kernels.qwen3.gfx950", "pih.qwen-kernels.v1", "gfx950")
    assert p.identity.pack_version == b"1.0.0"
    assert p.table.struct_size == abi.C.sizeof(abi.QWEN_API) == 24
    assert p.table.contract_version == 1 and p.table.target_sm == 950
    path = abi.C.c_char_p()
    st = p.table.root(abi.C.byref(path))
    assert st.code == abi.OK
    assert os.path.realpath(path.value.decode()) == os.path.realpath(ROOT)
    assert p.table.root(None).code == abi.INVALID_ARGUMENT


def test_pack_exports_exactly_two_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", abi.QWEN_PACK], capture_output=True, text=True, check=True)
    syms = sorted(line.split()[-1] for line in out.stdout.splitlines() if " T " in line)
    assert syms == ["pih_kernel_pack_api_v1_get", "pih_kernel_pack_identity_v1_get"]


def _fresh_process(body: str) -> str:
    """Run a script against a freshly loaded pack (its bound root is
    process-wide state)."""
    script = textwrap.dedent("""
        import ctypes as C, sys
        sys.path.insert(0, %r)
        from pih_amd import abi
        lib = C.CDLL(sys.argv[1])
        lib.pih_kernel_pack_api_v1_get.restype = C.POINTER(abi.PackApi)
        api = lib.pih_kernel_pack_api_v1_get().contents
        table = C.cast(api.contract_api, C.POINTER(abi.QWEN_API)).contents
        path = C.c_char_p()
    """ % os.path.dirname(os.path.dirname(os.path.abspath(__file__)))) + textwrap.dedent(body)
    return script


def _run(script: str, lib: str):
    r = subprocess.run([sys.executable, "-c", script, lib], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return r.stdout.split()


def test_root_before_bind_and_bind_rules(tmp_path):
    script = _fresh_process("""
        codes = [table.root(C.byref(path)).code]                       # before bind
        codes.append(api.bind_origin(b"relative/lib.so").code)         # not absolute
        codes.append(api.bind_origin(sys.argv[1].encode()).code)       # the pack itself
        codes.append(table.root(C.byref(path)).code)
        codes.append(api.bind_origin(sys.argv[1].encode()).code)       # same root again
        print(*codes, path.value.decode())
    """)
    out = _run(script, abi.QWEN_PACK)
    assert out[:5] == [str(abi.FAILED_PRECONDITION), str(abi.INVALID_ARGUMENT), str(abi.OK), str(abi.OK),
                       str(abi.OK)]
    assert os.path.realpath(out[5]) == os.path.realpath(ROOT)

    # a copy of the library without the code object beside it cannot bind
    lonely = tmp_path / "lonely" / os.path.basename(abi.QWEN_PACK)
    lonely.parent.mkdir()
    shutil.copy(abi.QWEN_PACK, lonely)
    out = _run(_fresh_process("print(api.bind_origin(sys.argv[1].encode()).code)"), str(lonely))
    assert out == [str(abi.INVALID_ARGUMENT)]

    # a complete second tree binds, but a process bound to one root may not move
    other = tmp_path / "other"
    shutil.copytree(ROOT, other / "qwen3-gfx950")
    shutil.copy(abi.QWEN_PACK, other / os.path.basename(abi.QWEN_PACK))
    script = _fresh_process("""
        a = api.bind_origin(sys.argv[1].encode()).code
        b = api.bind_origin(%r.encode()).code
        print(a, b)
    """ % abi.QWEN_PACK)
    out = _run(script, str(other / os.path.basename(abi.QWEN_PACK)))
    assert out == [str(abi.OK), str(abi.INVALID_ARGUMENT)]


MANIFEST_FIELDS = {"schema", "target", "producer_toolchain", "producer_flags_sha256", "code_object_sha256",
                   "code_object_bytes"}


def _signatures(digest: bytes):
    compat, p0 = qwen.w4a16_signature(abi.QWEN_INT4_COMPAT, digest)
    gfx, p1 = qwen.w4a16_signature(abi.QWEN_INT4_GFX950, digest)
    silu, p2, _ = qwen.silu_signature(digest)
    return [compat, gfx, silu], (p0, p1, p2)


def _verify(path, sigs):
    arr = (abi.KM_SIGNATURE * len(sigs))(*sigs)
    st = abi.kernel_module_lib().pih_hip_code_object_verify_v1(str(path).encode(), arr, len(sigs))
    return st.code, st.message.decode()


def test_driver_verifies_manifest_digest_and_kernarg_layout(tmp_path):
    """pih_hip_code_object_verify_v1 (no device): the shipped image and its
    manifest pass with the three signatures; a flipped byte, a truncated
    image, an extra or missing manifest field, another target, a signature
    made for another image, a symbol the image lacks, a parameter at the
    wrong offset or of the wrong size, a wrong packet size, duplicate symbols
    or logical ids, an empty symbol and a bad header are all refused
    (verified_kernel_module.cpp:8-70, cubin_artifact_manifest.cpp)."""
    with open(IMAGE + ".json") as f:
        m = json.load(f)
    assert set(m) == MANIFEST_FIELDS
    assert m["schema"] == "pih.code_object_artifact.v1" and m["target"] == "gfx950"
    assert m["code_object_bytes"] == os.path.getsize(IMAGE)
    digest = m["code_object_sha256"].encode()
    sigs, keep = _signatures(digest)
    assert _verify(IMAGE, sigs) == (abi.OK, "")

    bad = tmp_path / "qwen3-gfx950"
    shutil.copytree(ROOT, bad)
    img = bad / "gfx950" / "qwen_bf16_primitives.hsaco"
    man = bad / "gfx950" / "qwen_bf16_primitives.hsaco.json"
    data = bytearray(img.read_bytes())
    data[len(data) // 2] ^= 0x40
    img.write_bytes(bytes(data))
    assert _verify(img, sigs) == (abi.INVALID_ARGUMENT, "code_object_digest_differs_from_manifest")
    img.write_bytes(bytes(data[:-1]))
    assert _verify(img, sigs) == (abi.INVALID_ARGUMENT, "code_object_size_differs_from_manifest")
    shutil.copy(IMAGE, img)
    man.write_text(json.dumps(dict(m, extra=1)))
    assert _verify(img, sigs)[1] == "code_object_manifest_fields"
    man.write_text(json.dumps({k: v for k, v in m.items() if k != "producer_toolchain"}))
    assert _verify(img, sigs)[1] == "code_object_manifest_fields"
    man.write_text(json.dumps(dict(m, target="gfx942")))
    assert _verify(img, sigs)[1] == "code_object_manifest_target"
    man.write_text(json.dumps(m) + "{")
    assert _verify(img, sigs)[1] == "code_object_manifest_not_a_flat_json_object"
    man.write_text(json.dumps(m))
    assert _verify(img, sigs) == (abi.OK, "")

    other, _ = _signatures(b"0" * 64)
    assert _verify(IMAGE, other)[1] == "kernel_signature_names_another_image"
    s0 = sigs[0]
    missing = abi.KM_SIGNATURE.from_buffer_copy(s0)
    missing.symbol = b"pih_qwen_w4a16_gemm_absent_v1"
    missing.logical_id = b"qwen.absent.v1"
    assert _verify(IMAGE, [missing])[1] == "kernel_symbol_not_in_code_object"
    for field, value, msg in (("offset", 44, "kernel_signature_parameter_invalid"),
                              ("offset", 40, "kernel_parameter_layout_differs_from_signature"),
                              ("wire_type", 2, "kernel_parameter_layout_differs_from_signature")):
        params = (abi.KM_PARAMETER * 8)(*keep[0])
        setattr(params[6], field, value)
        moved = abi.KM_SIGNATURE.from_buffer_copy(s0)
        moved.parameters = params
        assert _verify(IMAGE, [moved])[1] == msg, (field, value)
    short = abi.KM_SIGNATURE.from_buffer_copy(s0)
    short.total_parameter_bytes = 72
    assert _verify(IMAGE, [short])[1] == "kernel_parameter_bytes_differ_from_signature"
    fewer = abi.KM_SIGNATURE.from_buffer_copy(s0)
    fewer.parameter_count = 7
    assert _verify(IMAGE, [fewer])[1] == "kernel_parameter_count_differs_from_signature"
    assert _verify(IMAGE, [s0, s0])[1] == "kernel_entrypoint_symbol_duplicated"
    twin = abi.KM_SIGNATURE.from_buffer_copy(sigs[1])
    twin.logical_id = s0.logical_id
    assert _verify(IMAGE, [s0, twin])[1] == "kernel_logical_id_duplicated"
    empty = abi.KM_SIGNATURE.from_buffer_copy(s0)
    empty.symbol = b""
    assert _verify(IMAGE, [empty])[1] == "kernel_symbol_empty_or_oversized"
    hdr = abi.KM_SIGNATURE.from_buffer_copy(s0)
    hdr.abi_version = 2
    assert _verify(IMAGE, [hdr])[1] == "kernel_signature_header_invalid"
    assert abi.kernel_module_lib().pih_hip_code_object_verify_v1(IMAGE.encode(), None, 0).code == abi.INVALID_ARGUMENT


def test_driver_exports_exactly_its_entries():
    out = subprocess.run(["nm", "-D", "--defined-only", abi.KERNEL_MODULE_LIB], capture_output=True, text=True,
                         check=True)
    syms = sorted(line.split()[-1] for line in out.stdout.splitlines() if " T " in line)
    assert syms == sorted(["pih_hip_code_object_verify_v1", "pih_hip_kernel_module_load_v1",
                           "pih_hip_kernel_module_find_v1", "pih_hip_kernel_submit_v1",
                           "pih_hip_kernel_module_unload_v1", "pih_qwen_int4_gemm_plan_create_v1",
                           "pih_qwen_int4_gemm_signature_v1"])
    # a NULL module / request never reaches the device
    L = abi.kernel_module_lib()
    assert L.pih_hip_kernel_module_unload_v1(None).code == abi.INVALID_ARGUMENT
    assert L.pih_hip_kernel_submit_v1(None, 0, None, 1, None).code == abi.INVALID_ARGUMENT


def test_int4_plan_reference_known_answers():
    """QwenInt4GemmPlan's known answers (tests/cpp/model/
    qwen3_int4_gemm_plan_test.cpp:9-37) for the compatibility variant: the
    five official (n, k) families at 7 tokens (packed, scale, input and
    output bytes), the logical id, the symbol, eight parameters in 64 bytes
    and the reference geometry ceil(m n / 256) x 256; 0 and 4097 tokens are
    refused.  The gfx950 variant: (n / 16, ceil(m / 16)) blocks of 64 x
    waves threads, waves splitting the 128-deep groups."""
    fams = [(2048, 1024, 1048576, 32768), (1024, 1024, 524288, 16384), (1024, 2048, 1048576, 32768),
            (3072, 1024, 1572864, 49152), (1024, 3072, 1572864, 49152)]
    for n, k, packed, scales in fams:
        p = qwen.w4a16_plan(7, n, k, abi.QWEN_INT4_COMPAT)
        assert (p.tokens, p.output_features, p.input_features) == (7, n, k)
        assert (p.packed_bytes, p.scale_bytes, p.input_bytes, p.output_bytes) == (packed, scales, 7 * k * 2, 7 * n * 2)
        assert p.logical_id == b"qwen.linear.w4a16.compatibility.v1"
        assert p.kernel_symbol == b"pih_qwen_w4a16_gemm_compat_v1"
        g = p.geometry
        assert (g.grid_x, g.grid_y, g.grid_z, g.block_x, g.block_y, g.block_z) == (-(-7 * n // 256), 1, 1, 256, 1, 1)
        q = qwen.w4a16_plan(7, n, k, abi.QWEN_INT4_GFX950)
        assert q.kernel_symbol == b"pih_qwen_w4a16_gemm_gfx950_v1" and q.packed_bytes == packed
        waves = min(16, k // 128)
        assert (q.geometry.grid_x, q.geometry.grid_y, q.geometry.block_x) == (n // 16, 1, 64 * waves)
        assert q.parameter_abi_sha256 != p.parameter_abi_sha256
    sig, params = qwen.w4a16_signature(abi.QWEN_INT4_COMPAT, b"a" * 64)
    assert (sig.parameter_count, sig.total_parameter_bytes) == (8, 64)
    assert [(params[j].offset, params[j].wire_type) for j in range(8)] == \
        [(8 * j, abi.WIRE_DEVICE_POINTER_U64 if j < 5 else abi.WIRE_U64) for j in range(8)]
    # prefill grids of >= 1024 blocks keep four waves per block
    assert qwen.w4a16_plan(4096, 3072, 1024, abi.QWEN_INT4_GFX950).geometry.block_x == 256
    for m, n, k, v in ((0, 2048, 1024, 1), (4097, 2048, 1024, 1), (1, 2048, 1000, 1), (1, 2064, 1024, 1),
                       (1, 2056, 1024, 2), (1, 2048, 1024, 3)):
        with pytest.raises(qwen.CodeObjectError):
            qwen.w4a16_plan(m, n, k, v)
    assert qwen.w4a16_plan(1, 2064, 1024, abi.QWEN_INT4_GFX950).geometry.grid_x == 129


@pytest.mark.skipif(not os.path.exists(READELF), reason="llvm-readelf not in this image")
def test_code_object_symbols_and_kernarg_layout():
    syms = subprocess.run([READELF, "-s", "--wide", IMAGE], capture_output=True, text=True, check=True).stdout
    for name in (qwen.W4A16_KERNEL, qwen.W4A16_GFX950_KERNEL, qwen.SILU_KERNEL):
        assert f" {name}\n" in syms or syms.rstrip().endswith(name) or f" {name} " in syms, name
        assert f"{name}.kd" in syms
    notes = subprocess.run([READELF, "--notes", "--wide", IMAGE], capture_output=True, text=True,
                           check=True).stdout
    import yaml

    doc = yaml.safe_load(notes[notes.index("---"):notes.rindex("...") if "..." in notes else None])
    kernels = {k[".name"]: k for k in doc["amdhsa.kernels"]}
    assert set(kernels) == {qwen.W4A16_KERNEL, qwen.W4A16_GFX950_KERNEL, qwen.SILU_KERNEL}
    explicit = [(a[".offset"], a[".size"], a[".value_kind"]) for a in kernels[qwen.W4A16_KERNEL][".args"]
                if not a[".value_kind"].startswith("hidden")]
    # input, packed_weight, scales, output, error_flag, m, n, k
    assert explicit == [(0, 8, "global_buffer"), (8, 8, "global_buffer"), (16, 8, "global_buffer"),
                        (24, 8, "global_buffer"), (32, 8, "global_buffer"), (40, 8, "by_value"),
                        (48, 8, "by_value"), (56, 8, "by_value")]
    explicit = [(a[".offset"], a[".size"]) for a in kernels[qwen.SILU_KERNEL][".args"]
                if not a[".value_kind"].startswith("hidden")]
    assert explicit == [(0, 8), (8, 8), (16, 8), (24, 8)]  # gate, up, output, elements
    for k in kernels.values():
        assert k[".private_segment_fixed_size"] == 0  # no scratch

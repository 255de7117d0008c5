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


def test_manifest_fields_and_digest(tmp_path):
    with open(IMAGE + ".json") as f:
        m = json.load(f)
    assert set(m) == qwen.MANIFEST_FIELDS
    assert m["schema"] == "pih.code_object_artifact.v1" and m["target"] == "gfx950"
    image = qwen.verified_image(ROOT)
    assert len(image) == m["code_object_bytes"] == os.path.getsize(IMAGE)

    # a flipped byte, a truncated image or an extra field are all rejected
    bad = tmp_path / "qwen3-gfx950"
    shutil.copytree(ROOT, bad)
    img = bad / "gfx950" / "qwen_bf16_primitives.hsaco"
    data = bytearray(img.read_bytes())
    data[len(data) // 2] ^= 0x40
    img.write_bytes(bytes(data))
    with pytest.raises(qwen.CodeObjectError, match="digest"):
        qwen.verified_image(str(bad))
    img.write_bytes(bytes(data[:-1]))
    with pytest.raises(qwen.CodeObjectError, match="size"):
        qwen.verified_image(str(bad))
    man = bad / "gfx950" / "qwen_bf16_primitives.hsaco.json"
    m2 = dict(m, extra=1)
    man.write_text(json.dumps(m2))
    with pytest.raises(qwen.CodeObjectError, match="exactly"):
        qwen.verified_image(str(bad))
    man.write_text(json.dumps(dict(m, target="gfx942")))
    with pytest.raises(qwen.CodeObjectError, match="target"):
        qwen.verified_image(str(bad))


@pytest.mark.skipif(not os.path.exists(READELF), reason="llvm-readelf not in this image")
def test_code_object_symbols_and_kernarg_layout():
    syms = subprocess.run([READELF, "-s", "--wide", IMAGE], capture_output=True, text=True, check=True).stdout
    for name in (qwen.W4A16_KERNEL, qwen.SILU_KERNEL):
        assert f" {name}\n" in syms or syms.rstrip().endswith(name) or f" {name} " in syms, name
        assert f"{name}.kd" in syms
    notes = subprocess.run([READELF, "--notes", "--wide", IMAGE], capture_output=True, text=True,
                           check=True).stdout
    import yaml

    doc = yaml.safe_load(notes[notes.index("---"):notes.rindex("...") if "..." in notes else None])
    kernels = {k[".name"]: k for k in doc["amdhsa.kernels"]}
    assert set(kernels) == {qwen.W4A16_KERNEL, qwen.SILU_KERNEL}
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

"""The Qwen model's side of the gfx950 code-object boundary.

The reference's Qwen plugin resolves the Qwen Kernel Pack, asks it for its
root(), checks the device image against the manifest beside it and loads it
(plugins/model-qwen3/qwen3_int4_kernel_bundle.cpp:33-74 with
src/backend/cuda/cubin_artifact_manifest.cpp), then launches kernels by name
with a packed kernarg buffer and its own launch geometry
(qwen3_int4_gemm_plan.cpp:55-85: ceil(m*n/256) blocks of 256 threads, eight
64-bit parameters at offsets 0..56).  ``QwenCodeObject`` does the same on
gfx950 through the HIP module API: the manifest check, ``hipModuleLoadData``,
``hipModuleGetFunction`` and ``hipModuleLaunchKernel`` with the 64-byte
packet in HIP_LAUNCH_PARAM_BUFFER_POINTER form.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import json
import os
import struct
from typing import Dict, Optional

from . import abi

CODE_OBJECT = os.path.join("gfx950", "qwen_bf16_primitives.hsaco")
MANIFEST_FIELDS = {"schema", "target", "producer_toolchain", "producer_flags_sha256", "code_object_sha256",
                   "code_object_bytes"}
MAX_MANIFEST_BYTES = 4096
MAX_CODE_OBJECT_BYTES = 64 << 20
W4A16_KERNEL = "pih_qwen_w4a16_gemm_compat_v1"
SILU_KERNEL = "pih_qwen_silu_mul_bf16_v1"
THREADS = 256

_LAUNCH_PARAM_BUFFER_POINTER = 1
_LAUNCH_PARAM_BUFFER_SIZE = 2
_LAUNCH_PARAM_END = 3


class CodeObjectError(RuntimeError):
    pass


def read_manifest(path: str) -> dict:
    """Parse and check the manifest's exact field set (the reference's
    manifest loader rejects missing, unknown and mistyped fields)."""
    if os.path.getsize(path) > MAX_MANIFEST_BYTES:
        raise CodeObjectError("code object manifest exceeds its byte budget")
    with open(path, "rb") as f:
        m = json.loads(f.read().decode("utf-8"))
    if not isinstance(m, dict) or set(m) != MANIFEST_FIELDS:
        raise CodeObjectError("code object manifest must contain exactly the v1 fields")
    if m["schema"] != "pih.code_object_artifact.v1":
        raise CodeObjectError("unsupported code object manifest schema")
    if m["target"] != "gfx950":
        raise CodeObjectError("code object target must be gfx950")
    for key in ("producer_toolchain", "producer_flags_sha256", "code_object_sha256"):
        if not isinstance(m[key], str) or not m[key] or len(m[key]) > 128:
            raise CodeObjectError(f"{key} must be a nonempty string")
    for key in ("producer_flags_sha256", "code_object_sha256"):
        if len(m[key]) != 64 or any(c not in "0123456789abcdef" for c in m[key]):
            raise CodeObjectError(f"{key} must be a lowercase sha256")
    if not isinstance(m["code_object_bytes"], int) or m["code_object_bytes"] < 64:
        raise CodeObjectError("code_object_bytes must include at least one ELF64 header")
    return m


def verified_image(root: str) -> bytes:
    """The code object under ``root``, checked against its manifest."""
    image_path = os.path.join(root, CODE_OBJECT)
    manifest = read_manifest(image_path + ".json")
    if manifest["code_object_bytes"] > MAX_CODE_OBJECT_BYTES:
        raise CodeObjectError("code object exceeds the configured byte budget")
    with open(image_path, "rb") as f:
        image = f.read(MAX_CODE_OBJECT_BYTES + 1)
    if len(image) != manifest["code_object_bytes"]:
        raise CodeObjectError("code object size differs from its manifest")
    if hashlib.sha256(image).hexdigest() != manifest["code_object_sha256"]:
        raise CodeObjectError("code object digest differs from its manifest")
    if image[:4] != b"\x7fELF" or image[4] != 2 or struct.unpack_from("<H", image, 18)[0] != 224:
        raise CodeObjectError("not an AMDGPU ELF64 code object")
    return image


def _hip() -> C.CDLL:
    lib = C.CDLL("libamdhip64.so")
    lib.hipModuleLoadData.argtypes = [C.POINTER(C.c_void_p), C.c_void_p]
    lib.hipModuleGetFunction.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_char_p]
    lib.hipModuleLaunchKernel.argtypes = [C.c_void_p] + [C.c_uint] * 7 + [C.c_void_p, C.c_void_p, C.c_void_p]
    lib.hipGetErrorString.restype = C.c_char_p
    return lib


class QwenCodeObject:
    """One loaded image; functions are resolved once, launches only enqueue."""

    def __init__(self, root: Optional[str] = None):
        if root is None:
            pack = abi.qwen_pack()
            path = C.c_char_p()
            st = pack.table.root(C.byref(path))
            if st.code != abi.OK or not path.value:
                raise CodeObjectError(f"qwen pack root() failed: {st}")
            if pack.table.target_sm != 950:
                raise CodeObjectError("qwen pack target is not gfx950")
            root = path.value.decode()
        self.root = root
        self._image = verified_image(root)  # kept alive for the module's lifetime
        self._hip = _hip()
        self._module = C.c_void_p()
        self._check(self._hip.hipModuleLoadData(C.byref(self._module), self._image), "hipModuleLoadData")
        self._functions: Dict[str, C.c_void_p] = {}
        for name in (W4A16_KERNEL, SILU_KERNEL):
            fn = C.c_void_p()
            self._check(self._hip.hipModuleGetFunction(C.byref(fn), self._module, name.encode()), name)
            self._functions[name] = fn

    def _check(self, rc: int, what: str) -> None:
        if rc != 0:
            raise CodeObjectError(f"{what}: {self._hip.hipGetErrorString(rc).decode()} ({rc})")

    def launch(self, name: str, packet: bytes, grid: int, block: int, stream: int) -> None:
        if not stream:
            raise CodeObjectError("launches need an explicit stream")
        buf = C.create_string_buffer(packet, len(packet))
        size = C.c_size_t(len(packet))
        extra = (C.c_void_p * 5)(_LAUNCH_PARAM_BUFFER_POINTER, C.cast(buf, C.c_void_p),
                                 _LAUNCH_PARAM_BUFFER_SIZE, C.cast(C.pointer(size), C.c_void_p), _LAUNCH_PARAM_END)
        self._check(self._hip.hipModuleLaunchKernel(self._functions[name], grid, 1, 1, block, 1, 1, 0,
                                                    C.c_void_p(stream), None, extra), name)

    def w4a16_gemm(self, x: int, packed: int, scales: int, out: int, error_flag: int, m: int, n: int, k: int,
                   stream: int, grid: Optional[int] = None, block: int = THREADS) -> None:
        """Launch with the model plan's geometry (override grid/block only to
        exercise the kernel's launch check)."""
        packet = struct.pack("<5Q3Q", x, packed, scales, out, error_flag, m, n, k)
        assert len(packet) == 64
        if grid is None:
            grid = (m * n + THREADS - 1) // THREADS
        self.launch(W4A16_KERNEL, packet, grid, block, stream)

    def silu_mul(self, gate: int, up: int, out: int, elements: int, stream: int, grid: Optional[int] = None) -> None:
        packet = struct.pack("<3QQ", gate, up, out, elements)
        if grid is None:
            grid = max(1, min((elements + THREADS - 1) // THREADS, 65535))
        self.launch(SILU_KERNEL, packet, grid, THREADS, stream)

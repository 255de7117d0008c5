"""The Qwen model's side of the gfx950 code-object boundary.

The reference's Qwen plugin resolves the Qwen Kernel Pack, asks it for its
root(), loads the device image through its kernel-module driver and
launches kernels by name with a typed 64-byte argument packet and its own
launch plan (plugins/model-qwen3/qwen3_int4_kernel_bundle.cpp:33-74,
qwen3_int4_gemm_plan.cpp:44-88, src/backend/cuda/verified_kernel_module.cpp,
verified_kernel_launcher.cpp).  ``QwenCodeObject`` makes the same calls into
the C++ driver ``libpih_hip_kernel_module.so``
(include/pih/backend/hip/kernel_module_v1.h): the manifest, digest and
per-kernel argument-layout checks, ``hipModuleLoadData`` / by-name
resolution, and identity-checked launches that refuse stream 0.  Launch
geometry comes from the plan entry
(include/pih/contracts/qwen_int4_plan_gfx950_v1.h): the reference's
geometry for the compatibility kernel, or the gfx950 kernel's own.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import json
import os
import struct
from typing import Optional

from . import abi

CODE_OBJECT = os.path.join("gfx950", "qwen_bf16_primitives.hsaco")
W4A16_KERNEL = "pih_qwen_w4a16_gemm_compat_v1"
W4A16_GFX950_KERNEL = "pih_qwen_w4a16_gemm_gfx950_v1"
SILU_KERNEL = "pih_qwen_silu_mul_bf16_v1"
THREADS = 256
# SiLU-mul packet: gate, up, output (device pointers at 0, 8, 16), elements (u64 at 24)
SILU_LOGICAL_ID = "qwen.elementwise.silu_mul.bf16.v1"
SILU_DESCRIPTOR = ("pih.typed_kernel_params.v1|qwen.elementwise.silu_mul.bf16.v1|gate:device_pointer_u64@0|"
                   "up:device_pointer_u64@8|output:device_pointer_u64@16|elements:u64@24|total:32|"
                   "activation:bf16|output:bf16")


class CodeObjectError(RuntimeError):
    pass


def _check(st, what: str) -> None:
    if st.code != abi.OK:
        raise CodeObjectError(f"{what}: {abi.STATUS_NAMES[st.code]} {st.message.decode(errors='replace')}")


def image_path(root: str) -> str:
    return os.path.join(root, CODE_OBJECT)


def manifest_digest(root: str) -> str:
    """The image digest the manifest names (the driver checks it against the
    image; the signatures are made for it)."""
    with open(image_path(root) + ".json", "rb") as f:
        return str(json.loads(f.read(4096).decode("utf-8")).get("code_object_sha256", ""))


def silu_signature(code_object_sha256: bytes):
    params = (abi.KM_PARAMETER * 4)(*[abi.KM_PARAMETER(abi.WIRE_DEVICE_POINTER_U64 if j < 3 else abi.WIRE_U64, 8 * j)
                                      for j in range(4)])
    digest = hashlib.sha256(SILU_DESCRIPTOR.encode()).hexdigest().encode()
    sig = abi.KM_SIGNATURE(C.sizeof(abi.KM_SIGNATURE), 1, SILU_KERNEL.encode(), SILU_LOGICAL_ID.encode(),
                           code_object_sha256, digest, params, 4, 32)
    return sig, params, digest


def w4a16_signature(variant: int, code_object_sha256: bytes):
    params = (abi.KM_PARAMETER * 8)()
    sig = abi.KM_SIGNATURE()
    _check(abi.kernel_module_lib().pih_qwen_int4_gemm_signature_v1(variant, code_object_sha256, params,
                                                                   C.byref(sig)), "qwen_int4_signature")
    return sig, params


def w4a16_plan(m: int, n: int, k: int, variant: int):
    plan = abi.QWEN_INT4_PLAN()
    plan.struct_size = C.sizeof(abi.QWEN_INT4_PLAN)
    _check(abi.kernel_module_lib().pih_qwen_int4_gemm_plan_create_v1(m, n, k, variant, C.byref(plan)),
           "qwen_int4_plan")
    return plan


class QwenCodeObject:
    """The loaded image with the compatibility and gfx950 W4A16 kernels and
    SiLU-mul resolved; launches only enqueue."""

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
        self._lib = abi.kernel_module_lib()
        digest = manifest_digest(root).encode()
        compat, p0 = w4a16_signature(abi.QWEN_INT4_COMPAT, digest)
        gfx, p1 = w4a16_signature(abi.QWEN_INT4_GFX950, digest)
        silu, p2, self._silu_digest = silu_signature(digest)
        self._keep = (p0, p1, p2)
        sigs = (abi.KM_SIGNATURE * 3)(compat, gfx, silu)
        self._module = C.c_void_p()
        _check(self._lib.pih_hip_kernel_module_load_v1(image_path(root).encode(), sigs, 3, C.byref(self._module)),
               "pih_hip_kernel_module_load_v1")
        self._index = {}
        for sig in (compat, gfx, silu):
            idx = C.c_uint32()
            _check(self._lib.pih_hip_kernel_module_find_v1(self._module, sig.logical_id, C.byref(idx)), "find")
            self._index[sig.logical_id.decode()] = (idx.value, sig.parameter_abi_sha256)

    def unload(self) -> None:
        if self._module:
            _check(self._lib.pih_hip_kernel_module_unload_v1(self._module), "unload")
            self._module = C.c_void_p()

    def submit(self, logical_id: str, packet: bytes, grid, block: int, stream: int, abi_digest: Optional[bytes] = None,
               packet_logical_id: Optional[str] = None):
        """One launch through the driver; returns its pih_status_v1 (the
        caller checks it).  ``abi_digest`` / ``packet_logical_id`` override
        the packet's identity (to exercise the driver's refusal)."""
        index, digest = self._index[logical_id]
        gx, gy = (grid, 1) if isinstance(grid, int) else grid
        geometry = abi.KM_GEOMETRY(C.sizeof(abi.KM_GEOMETRY), gx, gy, 1, block, 1, 1, 0)
        buf = C.create_string_buffer(packet, len(packet))
        args = abi.KM_ARGUMENTS(C.sizeof(abi.KM_ARGUMENTS), 1, (packet_logical_id or logical_id).encode(),
                                abi_digest if abi_digest is not None else digest, C.cast(buf, C.c_void_p),
                                len(packet))
        return self._lib.pih_hip_kernel_submit_v1(self._module, index, C.byref(geometry), stream, C.byref(args))

    def w4a16_gemm(self, x: int, packed: int, scales: int, out: int, error_flag: int, m: int, n: int, k: int,
                   stream: int, grid=None, block: Optional[int] = None, variant: int = abi.QWEN_INT4_COMPAT) -> None:
        """Launch with the plan's geometry for ``variant`` (override grid /
        block only to exercise the kernel's own launch check)."""
        packet = struct.pack("<5Q3Q", x, packed, scales, out, error_flag, m, n, k)
        assert len(packet) == 64
        if grid is None or block is None:
            plan = w4a16_plan(m, n, k, variant)
            g = plan.geometry
            grid = (g.grid_x, g.grid_y) if grid is None else grid
            block = g.block_x if block is None else block
        lid = "qwen.linear.w4a16.compatibility.v1" if variant == abi.QWEN_INT4_COMPAT else "qwen.linear.w4a16.gfx950.v1"
        _check(self.submit(lid, packet, grid, block, stream), W4A16_KERNEL if variant == abi.QWEN_INT4_COMPAT
               else W4A16_GFX950_KERNEL)

    def prepare_w4a16(self, x: int, packed: int, scales: int, out: int, error_flag: int, m: int, n: int, k: int,
                      stream: int, variant: int = abi.QWEN_INT4_COMPAT):
        """The launch with its plan and argument structs built once: the
        returned callable makes one driver call (a model's steady-state
        launch path; the bench times it)."""
        plan = w4a16_plan(m, n, k, variant)
        index, digest = self._index[plan.logical_id.decode()]
        geometry = abi.KM_GEOMETRY.from_buffer_copy(plan.geometry)
        buf = C.create_string_buffer(struct.pack("<5Q3Q", x, packed, scales, out, error_flag, m, n, k), 64)
        args = abi.KM_ARGUMENTS(C.sizeof(abi.KM_ARGUMENTS), 1, plan.logical_id, digest, C.cast(buf, C.c_void_p), 64)
        submit, module = self._lib.pih_hip_kernel_submit_v1, self._module
        keep = (buf, geometry, args, plan)

        def launch():
            st = submit(module, index, C.byref(geometry), stream, C.byref(args))
            if st.code != abi.OK:
                raise CodeObjectError(f"submit: {st.message.decode(errors='replace')} {len(keep)}")
        return launch

    def silu_mul(self, gate: int, up: int, out: int, elements: int, stream: int, grid: Optional[int] = None) -> None:
        packet = struct.pack("<3QQ", gate, up, out, elements)
        if grid is None:
            grid = max(1, min((elements + THREADS - 1) // THREADS, 65535))
        _check(self.submit(SILU_LOGICAL_ID, packet, grid, THREADS, stream), SILU_KERNEL)

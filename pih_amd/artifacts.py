"""ctypes front of libpih_amd_artifacts.so: the on-disk weight formats of the
linear path onto the device (declarations in
include/pih/contracts/amd_artifacts_v1.h).

* ``QwenInt4Artifact``: the canonical Qwen3-0.6B INT4 file ("XINGW4A1",
  xing-w4a16-sym-g128-v1), memory-mapped, verified the way the reference's
  loader verifies it (plugins/model-qwen3/artifact/qwen3_int4_artifact_io.cpp:35-52)
  and uploaded as one copy of its data region; ``linear(source)`` returns the
  device views the W4A16 symmetric kernels read.
* ``bind_expert_bundle`` / ``bundles_to_moe``: the DeepSeek V4 Flash routed
  expert bundle (deepseek_expert_bundle_layout.cpp:17-43) and its repack
  into the grouped MoE weights of ``launch_moe_layer``.
"""
from __future__ import annotations

import ctypes as C
import mmap
import os
from typing import Optional, Sequence, Tuple

import torch

from . import abi
from .device import stream_handle

LIB_PATH = os.path.join(abi.LIB_DIR, "libpih_amd_artifacts.so")
ABI_VERSION = 1
FILE_BYTES = 539_758_592
METADATA_BYTES = 1_048_576
DATA_BYTES = 538_710_016
RECORD_COUNT = 507
VERIFY_PAYLOADS = 1
PACKED_VALUES, FP16_SCALES, BF16_EMBEDDING, BF16_NORM, ALIAS = 1, 2, 3, 4, 5
BUNDLE_BYTES = 13_369_344
BUNDLE_ALIGNMENT = 256


class Info(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_version", C.c_uint32), ("record_count", C.c_uint32),
                ("payload_record_count", C.c_uint32), ("file_bytes", C.c_uint64), ("metadata_bytes", C.c_uint64),
                ("padded_data_bytes", C.c_uint64), ("logical_payload_bytes", C.c_uint64),
                ("encoded_metadata_bytes", C.c_uint32), ("reserved", C.c_uint32),
                ("source_artifact_root", C.c_uint8 * 32), ("source_binding_root", C.c_uint8 * 32),
                ("disposition_root", C.c_uint8 * 32)]


class Record(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_version", C.c_uint32), ("kind", C.c_uint32),
                ("reserved", C.c_uint32), ("file_offset", C.c_uint64), ("logical_bytes", C.c_uint64),
                ("extent_bytes", C.c_uint64), ("device_offset", C.c_uint64), ("rows", C.c_uint64),
                ("columns", C.c_uint64)]


class BundleView(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_version", C.c_uint32)] + [
        (n, C.c_size_t) for n in ("w1_packed", "w1_scales", "w2_packed", "w2_scales", "w3_packed", "w3_scales")] + [
        ("packed_bytes", C.c_uint64), ("scale_bytes", C.c_uint64)]


class BundlesToMoe(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_version", C.c_uint32), ("bundle_bases", C.POINTER(C.c_size_t)),
                ("w13_packed", C.c_size_t), ("w13_scales", C.c_size_t), ("w2_packed", C.c_size_t),
                ("w2_scales", C.c_size_t), ("stream", C.c_size_t), ("expert_count", C.c_uint32),
                ("reserved", C.c_uint32)]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise abi.PackError(f"{LIB_PATH} is not built (python -c 'import __graft_entry__ as g; g.build()')")
        L = C.CDLL(LIB_PATH)
        sigs = {
            "pih_amd_qwen_int4_artifact_verify_v1": [C.c_void_p, C.c_uint64, C.c_uint32, C.POINTER(Info)],
            "pih_amd_qwen_int4_artifact_record_v1": [C.c_char_p, C.POINTER(Record)],
            "pih_amd_qwen_int4_artifact_upload_v1": [C.c_void_p, C.c_uint64, C.c_size_t, C.c_uint64, C.c_size_t],
            "pih_amd_deepseek_expert_bundle_bind_v1": [C.c_size_t, C.POINTER(BundleView)],
            "pih_amd_deepseek_bundles_to_moe_v1": [C.POINTER(BundlesToMoe)],
        }
        for name, args in sigs.items():
            fn = getattr(L, name)
            fn.restype = abi.Status
            fn.argtypes = args
        _lib = L
    return _lib


def _new(struct):
    s = struct()
    s.struct_size = C.sizeof(struct)
    s.abi_version = ABI_VERSION
    return s


class ArtifactError(RuntimeError):
    def __init__(self, what: str, status: abi.Status):
        super().__init__(f"{what}: {abi.STATUS_NAMES[status.code]}: {status.message.decode(errors='replace')}")
        self.status = status


def _check(st: abi.Status, what: str) -> None:
    if st.code != abi.OK:
        raise ArtifactError(what, st)


def _host_ptr(buf) -> Tuple[int, object]:
    """The address of a writable bytes-like or mmap object's memory and the
    ctypes view that pins it (drop both before closing an mmap)."""
    arr = (C.c_uint8 * len(buf)).from_buffer(buf)
    return C.addressof(arr), arr


def verify_qwen_int4(buf, payloads: bool = True) -> Info:
    """Verifies a whole canonical file held in ``buf`` (writable mmap or
    bytearray)."""
    p, anchor = _host_ptr(buf)
    info = _new(Info)
    st = lib().pih_amd_qwen_int4_artifact_verify_v1(p, len(buf), VERIFY_PAYLOADS if payloads else 0, C.byref(info))
    del p, anchor
    _check(st, "qwen_int4_artifact_verify")
    return info


def qwen_int4_record(identity: str) -> Record:
    r = _new(Record)
    _check(lib().pih_amd_qwen_int4_artifact_record_v1(identity.encode(), C.byref(r)), f"record {identity}")
    return r


class QwenInt4Artifact:
    """A verified canonical artifact resident in device memory.

    ``linear(source)`` gives (packed u8 [N, K/2], scales fp16 [N, K/128]) for
    a projection such as ``model.layers.3.mlp.gate_proj.weight``; ``tensor``
    gives the bf16 embedding / norms (and the tied ``lm_head.weight``)."""

    def __init__(self, path: str, verify_payloads: bool = True, device: str = "cuda"):
        with open(path, "rb") as f:
            mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_COPY)
        try:
            self.info = verify_qwen_int4(mm, verify_payloads)
            self.data = torch.empty(DATA_BYTES, dtype=torch.uint8, device=device)
            p, anchor = _host_ptr(mm)
            st = lib().pih_amd_qwen_int4_artifact_upload_v1(p, len(mm), self.data.data_ptr(), DATA_BYTES,
                                                            stream_handle())
            del p, anchor
            _check(st, "qwen_int4_artifact_upload")
        finally:
            mm.close()

    def _view(self, identity: str):
        r = qwen_int4_record(identity)
        size = r.logical_bytes if r.kind != ALIAS else qwen_int4_record("model.embed_tokens.weight").logical_bytes
        return r, self.data[r.device_offset:r.device_offset + size]

    def linear(self, source: str) -> Tuple[torch.Tensor, torch.Tensor]:
        r, packed = self._view(source + ".packed_values")
        _, scales = self._view(source + ".scales")
        n, k = int(r.rows), int(r.columns)
        return packed.view(n, k // 2), scales.view(torch.float16).view(n, k // 128)

    def tensor(self, identity: str) -> torch.Tensor:
        r, raw = self._view(identity)
        if r.kind not in (BF16_EMBEDDING, BF16_NORM, ALIAS):
            raise ValueError(f"{identity} is not a bf16 tensor")
        return raw.view(torch.bfloat16).view(int(r.rows), int(r.columns))


def bind_expert_bundle(base: int) -> BundleView:
    v = _new(BundleView)
    _check(lib().pih_amd_deepseek_expert_bundle_bind_v1(base, C.byref(v)), "expert_bundle_bind")
    return v


def bundles_to_moe(bases: Sequence[int], w13: torch.Tensor, w13_scale: torch.Tensor, w2: torch.Tensor,
                   w2_scale: torch.Tensor) -> None:
    """Repacks device-resident expert bundles into the grouped MoE weights
    (w13 e2m1 [E, 4096, 2048] = W1 rows then W3 rows, w13_scale [E, 4096,
    128], w2 [E, 4096, 1024], w2_scale [E, 4096, 64]); enqueued on the
    current stream."""
    arr = (C.c_size_t * len(bases))(*bases)
    r = _new(BundlesToMoe)
    r.bundle_bases = arr
    r.w13_packed, r.w13_scales = w13.data_ptr(), w13_scale.data_ptr()
    r.w2_packed, r.w2_scales = w2.data_ptr(), w2_scale.data_ptr()
    r.stream = stream_handle()
    r.expert_count = len(bases)
    _check(lib().pih_amd_deepseek_bundles_to_moe_v1(C.byref(r)), "bundles_to_moe")


def split_bundle_host(bundle: bytes) -> dict:
    """Host-side segment slices of one bundle (the Bind offsets applied to a
    host buffer): name -> bytes."""
    v = bind_expert_bundle(BUNDLE_ALIGNMENT)  # offsets relative to an aligned base
    out = {}
    for name in ("w1_packed", "w1_scales", "w2_packed", "w2_scales", "w3_packed", "w3_scales"):
        off = getattr(v, name) - BUNDLE_ALIGNMENT
        n = v.packed_bytes if name.endswith("packed") else v.scale_bytes
        out[name] = bundle[off:off + n]
    return out

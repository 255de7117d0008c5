"""Host side of the backend-amd-hip plugin: a ctypes mirror of the plugin
ABI (include/pih/plugin_sdk/plugin.h) and of the four device contracts
(include/pih/contracts/device_cuda_v1.h), and a small host that loads the
plugin and drives its lifecycle the way the reference's activation runtime
does (src/microkernel/plugin_loader.cpp:74-128 for the entry and table
checks, activation_runtime.cpp:96-190 for register -> configure -> start ->
ready and drain -> stop -> dispose).

The native host (pih_amd/csrc/plugin_host.cpp) publishes
``platform.linux.v1`` itself (the reference's platform-linux plugin provides
it); the code its ``validate_runtime`` answers is settable so tests can make
start fail.
"""
from __future__ import annotations

import ctypes as C
import json
import os
from typing import Dict, List, Optional, Tuple

from .abi import LIB_DIR, OK, Status, U32, U64, I32, UPTR, valid_canonical_id

BACKEND_PLUGIN = os.path.join(LIB_DIR, "libpih_backend_amd_hip.so")
BACKEND_MANIFEST = os.path.join(LIB_DIR, "backend-amd-hip.manifest.json")

SINGLE_THREADED, SERIALIZED, CONCURRENT = 1, 2, 3
SCOPE_PROCESS, SCOPE_ACTIVATION, SCOPE_ENGINE, SCOPE_REQUEST = 1, 2, 3, 4
EXACTLY_ONE, ZERO_OR_ONE, ONE_OR_MORE, MANY = 1, 2, 3, 4
MEMORY_DEVICE, MEMORY_PINNED_HOST = 1, 2
COPY_H2D, COPY_D2H, COPY_D2D = 1, 2, 3
EVENT_COMPLETE, EVENT_PENDING = 1, 2
CONTEXT_SCHED_YIELD = 0x02
_NAMES = {"threading_model": {1: "single_threaded", 2: "serialized", 3: "concurrent"},
          "scope": {1: "process", 2: "activation", 3: "engine", 4: "request"},
          "cardinality": {1: "exactly_one", 2: "zero_or_one", 3: "one_or_more", 4: "many"}}


def _s(name, fields):
    return type(name, (C.Structure,), {"_fields_": fields})


Capability = _s("Capability", [("struct_size", U32), ("abi_version", U32), ("capability_id", C.c_char_p),
                               ("contract_id", C.c_char_p), ("api", C.c_void_p), ("threading_model", U32),
                               ("scope", U32), ("cardinality", U32)])
REGISTER_CB = C.CFUNCTYPE(Status, C.c_void_p, C.POINTER(Capability))
RESOLVE_CB = C.CFUNCTYPE(Status, C.c_void_p, C.c_char_p, C.c_char_p, U32, U32, C.POINTER(C.c_void_p))
LIFECYCLE_CB = C.CFUNCTYPE(Status, C.c_void_p)
LOG_CB = C.CFUNCTYPE(None, C.c_void_p, U32, C.c_char_p, C.c_char_p)
LIFECYCLE_PHASES = ("register_plugin", "configure", "start", "ready", "drain", "stop", "dispose")
Lifecycle = _s("Lifecycle", [("struct_size", U32), ("abi_version", U32)] +
               [(n, LIFECYCLE_CB) for n in LIFECYCLE_PHASES])
HostApi = _s("HostApi", [("struct_size", U32), ("abi_version", U32), ("context", C.c_void_p), ("log", LOG_CB),
                         ("register_capability", REGISTER_CB), ("resolve_capability", RESOLVE_CB),
                         ("activation_epoch", U64)])
PluginApi = _s("PluginApi", [("struct_size", U32), ("abi_version", U32), ("plugin_id", C.c_char_p),
                             ("plugin_version", C.c_char_p), ("context", C.c_void_p), ("lifecycle", Lifecycle)])
ENTRY = C.CFUNCTYPE(Status, C.POINTER(HostApi), C.POINTER(PluginApi))

Allocation = _s("Allocation", [("struct_size", U32), ("abi_version", U32), ("address", UPTR), ("bytes", U64),
                               ("alignment", U64), ("generation", U64), ("device_ordinal", I32),
                               ("memory_kind", U32)])
_V = C.c_void_p
RuntimeApi = _s("RuntimeApi", [("struct_size", U32), ("contract_version", U32), ("context", _V),
                               ("prepare_device", C.CFUNCTYPE(Status, _V, I32, U32, U32))])
_ALLOC = C.CFUNCTYPE(Status, _V, I32, U64, U64, C.POINTER(Allocation))
_DEALLOC = C.CFUNCTYPE(Status, _V, C.POINTER(Allocation))
MemoryApi = _s("MemoryApi", [("struct_size", U32), ("contract_version", U32), ("context", _V),
                             ("allocate_device", _ALLOC), ("deallocate_device", _DEALLOC),
                             ("allocate_pinned_host", _ALLOC), ("deallocate_pinned_host", _DEALLOC),
                             ("copy_h2d", C.CFUNCTYPE(Status, _V, I32, UPTR, _V, U64))])
_CREATE = C.CFUNCTYPE(Status, _V, UPTR, C.POINTER(UPTR))
_DESTROY = C.CFUNCTYPE(Status, _V, UPTR)
_CTX = C.CFUNCTYPE(Status, _V, I32, UPTR)
ResourcesApi = _s("ResourcesApi", [("struct_size", U32), ("contract_version", U32), ("context", _V),
                                   ("retain_primary_context", C.CFUNCTYPE(Status, _V, I32, U32, C.POINTER(UPTR))),
                                   ("bind_runtime", _CTX), ("create_nonblocking_stream", _CREATE),
                                   ("create_disable_timing_event", _CREATE), ("destroy_event", _DESTROY),
                                   ("destroy_stream", _DESTROY), ("release_primary_context", _CTX)])
AsyncApi = _s("AsyncApi", [("struct_size", U32), ("contract_version", U32), ("context", _V),
                           ("activate_context", C.CFUNCTYPE(Status, _V, UPTR)),
                           ("validate_pinned_host", C.CFUNCTYPE(Status, _V, UPTR, UPTR)),
                           ("copy_async", C.CFUNCTYPE(Status, _V, UPTR, UPTR, UPTR, U64, U32, UPTR)),
                           ("memset_async", C.CFUNCTYPE(Status, _V, UPTR, UPTR, U32, U64, UPTR)),
                           ("record_event", C.CFUNCTYPE(Status, _V, UPTR, UPTR, UPTR)),
                           ("query_event", C.CFUNCTYPE(Status, _V, UPTR, UPTR, C.POINTER(U32))),
                           ("synchronize_stream", C.CFUNCTYPE(Status, _V, UPTR, UPTR)),
                           ("require_clean_last_error", C.CFUNCTYPE(Status, _V, UPTR))])
PlatformApi = _s("PlatformApi", [("struct_size", U32), ("contract_version", U32), ("context", _V),
                                 ("validate_runtime", C.CFUNCTYPE(Status, _V))])

CONTRACT_TABLES = {"pih.device.cuda-runtime.v1": RuntimeApi, "pih.device.cuda-memory.v1": MemoryApi,
                   "pih.device.cuda-resources.v1": ResourcesApi, "pih.device.cuda-async.v1": AsyncApi}


class PluginError(RuntimeError):
    pass


HOST_LIB = os.path.join(LIB_DIR, "libpih_plugin_host.so")
PHASES = {n: i for i, n in enumerate(LIFECYCLE_PHASES)}
_host_lib = None


def _native_host() -> C.CDLL:
    global _host_lib
    if _host_lib is None:
        if not os.path.exists(HOST_LIB):
            raise PluginError(f"{HOST_LIB} not built (run __graft_entry__.build())")
        lib = C.CDLL(HOST_LIB)
        lib.pih_amd_host_create.restype = C.c_void_p
        lib.pih_amd_host_create.argtypes = [U64]
        lib.pih_amd_host_api.restype = C.POINTER(HostApi)
        lib.pih_amd_host_api.argtypes = [C.c_void_p]
        lib.pih_amd_host_plugin.restype = C.POINTER(PluginApi)
        lib.pih_amd_host_plugin.argtypes = [C.c_void_p]
        lib.pih_amd_host_load.restype = Status
        lib.pih_amd_host_load.argtypes = [C.c_void_p, C.c_char_p]
        lib.pih_amd_host_phase.restype = Status
        lib.pih_amd_host_phase.argtypes = [C.c_void_p, U32, C.c_void_p]
        lib.pih_amd_host_set_platform_status.argtypes = [C.c_void_p, U32]
        for f in ("platform_calls", "capability_count", "resolve_count"):
            getattr(lib, "pih_amd_host_" + f).restype = U32
            getattr(lib, "pih_amd_host_" + f).argtypes = [C.c_void_p]
        lib.pih_amd_host_capability.argtypes = [C.c_void_p, U32, C.POINTER(Capability)]
        lib.pih_amd_host_resolve.argtypes = [C.c_void_p, U32, C.c_char_p, U32]
        _host_lib = lib
    return _host_lib


class PluginHost:
    """One native plugin bound to one native host (libpih_plugin_host.so).

    The host table's callbacks (capability registry, platform.linux.v1) live
    in the native host because they return pih_status_v1 by value.  A plugin
    is never unloaded once its entry ran (plugin_loader.cpp:121-126).
    """

    def __init__(self, path: str = BACKEND_PLUGIN, epoch: int = 1, platform_status: int = OK):
        if not os.path.exists(path):
            raise PluginError(f"plugin_load_failed: {path} not built (run __graft_entry__.build())")
        self.path = os.path.abspath(path)
        self.native = _native_host()
        self.handle = self.native.pih_amd_host_create(epoch)
        if not self.handle:
            raise PluginError("plugin host allocation failed")
        self.native.pih_amd_host_set_platform_status(self.handle, platform_status)
        self.host = self.native.pih_amd_host_api(self.handle).contents
        self.api: Optional[PluginApi] = None

    def enter(self, host=..., api=...) -> Status:
        """Call the plugin's entry directly (for entry-validation checks);
        ``None`` passes a null pointer, ``...`` a fresh default."""
        lib = C.CDLL(self.path, mode=C.RTLD_LOCAL | os.RTLD_NOW)
        entry = ENTRY(("pih_plugin_entry_v1", lib))
        if host is ...:
            host = self.host
        if api is ...:
            api = PluginApi(C.sizeof(PluginApi), 1)
        return entry(C.byref(host) if host is not None else None, C.byref(api) if api is not None else None)

    def load(self) -> "PluginHost":
        st = self.native.pih_amd_host_load(self.handle, self.path.encode())
        if st.code != OK:
            raise PluginError(f"plugin_entry_failed:status={st.code}:{st.message.decode()}")
        self.api = self.native.pih_amd_host_plugin(self.handle).contents
        return self

    def phase(self, name: str, context=None) -> Status:
        return self.native.pih_amd_host_phase(self.handle, PHASES[name], context)

    def activate(self) -> "PluginHost":
        for name in ("register_plugin", "configure", "start", "ready"):
            st = self.phase(name)
            if st.code != OK:
                raise PluginError(f"plugin_{name}_failed:{st!r}")
        return self

    def shutdown(self) -> None:
        for name in ("drain", "stop", "dispose"):
            st = self.phase(name)
            if st.code != OK:
                raise PluginError(f"plugin_{name}_failed:{st!r}")

    @property
    def platform_calls(self) -> int:
        return self.native.pih_amd_host_platform_calls(self.handle)

    @property
    def registered(self) -> List[Tuple[str, str, int, int, int, int]]:
        out = []
        for i in range(self.native.pih_amd_host_capability_count(self.handle)):
            cap = Capability()
            self.native.pih_amd_host_capability(self.handle, i, C.byref(cap))
            out.append((cap.capability_id.decode(), cap.contract_id.decode(), cap.api, cap.threading_model,
                        cap.scope, cap.cardinality))
        return out

    @property
    def resolves(self) -> List[list]:
        out = []
        buf = C.create_string_buffer(1024)
        for i in range(self.native.pih_amd_host_resolve_count(self.handle)):
            self.native.pih_amd_host_resolve(self.handle, i, buf, 1024)
            cap, contract, scope, card = buf.value.decode().split()
            out.append([cap, contract, int(scope), int(card)])
        return out

    def table(self, contract_id: str):
        for cap, contract, api, *_ in self.registered:
            if contract == contract_id:
                t = C.cast(api, C.POINTER(CONTRACT_TABLES[contract_id])).contents
                if t.struct_size != C.sizeof(CONTRACT_TABLES[contract_id]) or t.contract_version != 1:
                    raise PluginError(f"{contract_id} table invalid")
                return t
        raise PluginError(f"{contract_id} not registered")


def manifest_capabilities(path: str = BACKEND_MANIFEST) -> Dict[str, dict]:
    with open(path) as f:
        m = json.load(f)
    return {p["capability_id"]: p for p in m["provides"]}


class Device:
    """Typed calls over the four contracts of an activated backend.

    Every method returns the plugin's Status (callers check ``.code``); the
    allocation helpers also return the filled record.
    """

    def __init__(self, host: PluginHost):
        self.host = host
        self.rt = host.table("pih.device.cuda-runtime.v1")
        self.mem = host.table("pih.device.cuda-memory.v1")
        self.res = host.table("pih.device.cuda-resources.v1")
        self.asy = host.table("pih.device.cuda-async.v1")

    def prepare(self, device: int, major: int, minor: int) -> Status:
        return self.rt.prepare_device(self.rt.context, device, major, minor)

    def allocate(self, device: int, nbytes: int, alignment: int = 256, pinned: bool = False):
        a = Allocation()
        a.struct_size = C.sizeof(Allocation)
        a.abi_version = 1
        fn = self.mem.allocate_pinned_host if pinned else self.mem.allocate_device
        st = fn(self.mem.context, device, nbytes, alignment, C.byref(a))
        return st, a

    def deallocate(self, a: Allocation, pinned: bool = False) -> Status:
        fn = self.mem.deallocate_pinned_host if pinned else self.mem.deallocate_device
        return fn(self.mem.context, C.byref(a))

    def copy_h2d(self, device: int, dst: int, src, nbytes: int) -> Status:
        return self.mem.copy_h2d(self.mem.context, device, dst, src, nbytes)

    def retain(self, device: int, flags: int = 0):
        tok = UPTR(0)
        st = self.res.retain_primary_context(self.res.context, device, flags, C.byref(tok))
        return st, tok.value

    def bind(self, device: int, token: int) -> Status:
        return self.res.bind_runtime(self.res.context, device, token)

    def create_stream(self, token: int):
        h = UPTR(0)
        return self.res.create_nonblocking_stream(self.res.context, token, C.byref(h)), h.value

    def create_event(self, token: int):
        h = UPTR(0)
        return self.res.create_disable_timing_event(self.res.context, token, C.byref(h)), h.value

    def destroy_event(self, h: int) -> Status:
        return self.res.destroy_event(self.res.context, h)

    def destroy_stream(self, h: int) -> Status:
        return self.res.destroy_stream(self.res.context, h)

    def release(self, device: int, token: int) -> Status:
        return self.res.release_primary_context(self.res.context, device, token)

    def activate(self, token: int) -> Status:
        return self.asy.activate_context(self.asy.context, token)

    def validate_pinned(self, token: int, ptr: int) -> Status:
        return self.asy.validate_pinned_host(self.asy.context, token, ptr)

    def copy_async(self, token: int, dst: int, src: int, nbytes: int, kind: int, stream: int) -> Status:
        return self.asy.copy_async(self.asy.context, token, dst, src, nbytes, kind, stream)

    def memset_async(self, token: int, dst: int, value: int, nbytes: int, stream: int) -> Status:
        return self.asy.memset_async(self.asy.context, token, dst, value, nbytes, stream)

    def record(self, token: int, event: int, stream: int) -> Status:
        return self.asy.record_event(self.asy.context, token, event, stream)

    def query(self, token: int, event: int):
        s = U32(0)
        return self.asy.query_event(self.asy.context, token, event, C.byref(s)), s.value

    def synchronize(self, token: int, stream: int) -> Status:
        return self.asy.synchronize_stream(self.asy.context, token, stream)

    def clean_last_error(self, token: int) -> Status:
        return self.asy.require_clean_last_error(self.asy.context, token)

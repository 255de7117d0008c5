// backend-amd-hip: the device backend plugin for gfx950, providing the four
// device capabilities the model plugins resolve (device.cuda-runtime.v1,
// device.cuda-memory.v1, device.cuda-resources.v1, device.cuda-async.v1;
// include/pih/contracts/device_cuda_v1.h) over HIP, in place of the
// reference's backend-nvidia-cuda plugin (plugins/backend-nvidia-cuda/
// entrypoint.cpp and manifest.json).  The capability ids, contract ids,
// table layouts, lifecycle order and status codes are the reference's; the
// mechanics are HIP's:
//   * a "retained context" is this provider's per-device token (HIP's device
//     model has no separate primary-context object); activating it makes
//     its device current with hipSetDevice;
//   * device memory comes from hipMalloc, pinned host memory from
//     hipHostMalloc (alignment a power of two <= 256); every allocation is
//     tracked with a generation number and copies and fills must stay inside
//     tracked ranges;
//   * streams are non-blocking hipStreams at the default priority, events
//     are created with timing disabled;
//   * memset_async is a fill kernel rather than hipMemsetAsync, so a caller
//     may capture it in a HIP graph.
// Lifecycle phases: 0 entry -> 1 registered -> 2 configured (platform.linux
// resolved) -> 3 started (platform runtime validated) -> 4 ready -> 5
// drained (no live resources) -> 6 stopped -> 7 disposed.  Device calls are
// accepted in phase 4, releases in phases 4 and 5.  Every entry point
// catches exceptions and answers with a status.
#include <hip/hip_runtime.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <unordered_map>

#include "host_common.hpp"
#include "pih/contracts/device_cuda_v1.h"
#include "pih/plugin_sdk/plugin.h"

namespace pih_amd {
namespace {

__global__ void fill_bytes_kernel(uint8_t* dst, uint32_t byte, uint64_t head, uint64_t body, uint64_t bytes) {
  const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t nthreads = (uint64_t)gridDim.x * blockDim.x;
  const uint32_t w = byte * 0x01010101u;
  const uint4 v = {w, w, w, w};
  for (uint64_t i = tid; i < head; i += nthreads) dst[i] = (uint8_t)byte;
  for (uint64_t i = tid; i < body / 16; i += nthreads) reinterpret_cast<uint4*>(dst + head)[i] = v;
  for (uint64_t i = head + body + tid; i < bytes; i += nthreads) dst[i] = (uint8_t)byte;
}

struct Allocation {
  uint64_t bytes, alignment, generation;
  int32_t device;
  uint32_t kind;
};

struct DeviceContext {
  int32_t device;
  uint32_t flags;
  uint32_t retains;
};

struct Provider {
  std::mutex mu;
  uint32_t phase = 0;
  const pih_host_api_v1* host = nullptr;
  const pih_platform_linux_api_v1* platform = nullptr;
  int32_t prepared_device = -1;
  uint32_t prepared_major = 0, prepared_minor = 0;
  uint64_t next_generation = 1;
  bool corrupted = false;
  std::map<uintptr_t, Allocation> allocations;  // base address -> record
  std::unordered_map<int32_t, std::unique_ptr<DeviceContext>> contexts;
  std::unordered_map<uintptr_t, uintptr_t> streams;  // stream -> context token
  std::unordered_map<uintptr_t, uintptr_t> events;   // event -> context token

  bool ready() const { return phase == 4 && !corrupted; }
  bool releasable() const { return phase == 4 || phase == 5; }
  bool idle() const { return allocations.empty() && contexts.empty() && streams.empty() && events.empty(); }

  DeviceContext* context_of(uintptr_t token) {
    for (auto& [dev, rec] : contexts)
      if (reinterpret_cast<uintptr_t>(rec.get()) == token) return rec.get();
    return nullptr;
  }
  // [address, address + bytes) inside one tracked allocation of this kind
  bool owns(uintptr_t address, uint64_t bytes, uint32_t kind, int32_t device) const {
    if (address == 0 || bytes == 0) return false;
    auto it = allocations.upper_bound(address);
    if (it == allocations.begin()) return false;
    --it;
    const Allocation& a = it->second;
    if (a.kind != kind || a.device != device) return false;
    const uint64_t off = address - it->first;
    return off <= a.bytes && bytes <= a.bytes - off;
  }
};

Provider g;

St Precond(const char* m) { return Precondition(m); }
St Exhausted(const char* m) { return St{PIH_STATUS_RESOURCE_EXHAUSTED_V1, m}; }

St FromHip(hipError_t e, const char* what) {
  if (e == hipSuccess) return Ok();
  if (e == hipErrorOutOfMemory) return Exhausted(what);
  if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) return Unavailable(what);
  return Internal(what);
}

template <typename F>
pih_status_v1 Contain(F body, const char* failure) noexcept {
  try {
    return ToAbi(body());
  } catch (const std::bad_alloc&) {
    return ToAbi(Exhausted("hip_provider_allocation_failed"));
  } catch (...) {
    return ToAbi(Internal(failure));
  }
}

// Makes `device` current for the scope and restores the previous device.
class DeviceScope {
 public:
  explicit DeviceScope(int32_t device) {
    if (hipGetDevice(&previous_) != hipSuccess) previous_ = -1;
    status_ = previous_ == device ? hipSuccess : hipSetDevice(device);
  }
  ~DeviceScope() {
    if (previous_ >= 0 && status_ == hipSuccess) (void)hipSetDevice(previous_);
  }
  hipError_t status() const { return status_; }

 private:
  int previous_ = -1;
  hipError_t status_ = hipSuccess;
};

bool FreshOutput(const pih_cuda_allocation_v1* a) {
  return a && a->struct_size == sizeof(*a) && a->abi_version == PIH_NVIDIA_CUDA_MEMORY_ABI_VERSION_V1 &&
         a->address == 0 && a->bytes == 0 && a->generation == 0;
}

// Requests name a power of two up to 256; hipMalloc and hipHostMalloc both
// return 256-byte aligned blocks, and the allocation record reports that.
constexpr uint64_t kGranted = 256;
bool AlignmentOk(uint64_t alignment) { return alignment && !(alignment & (alignment - 1)) && alignment <= kGranted; }

// ------------------------------------------------------- device.cuda-runtime
St PrepareDevice(int32_t device, uint32_t major, uint32_t minor) {
  if (device < 0 || major == 0 || minor > 9) return Invalid("hip_device_request_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  if (!g.ready()) return Precond("hip_provider_not_ready");
  if (g.prepared_device >= 0) {
    if (g.prepared_device != device || g.prepared_major != major || g.prepared_minor != minor)
      return Precond("hip_device_already_prepared");
    return Ok();
  }
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || device >= count) return Unavailable("hip_device_unavailable");
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return Precond("hip_device_identity_failed");
  if ((uint32_t)prop.major != major || (uint32_t)prop.minor != minor) return Precond("hip_device_arch_mismatch");
  g.prepared_device = device;
  g.prepared_major = major;
  g.prepared_minor = minor;
  return Ok();
}

// -------------------------------------------------------- device.cuda-memory
St Allocate(int32_t device, uint64_t bytes, uint64_t alignment, pih_cuda_allocation_v1* out, uint32_t kind) {
  const bool pinned = kind == PIH_CUDA_MEMORY_PINNED_HOST_V1;
  if ((pinned ? device != -1 : device < 0) || !FreshOutput(out)) return Invalid("hip_allocation_request_invalid");
  if (!AlignmentOk(alignment)) return Invalid("hip_allocation_alignment_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  if (!g.ready()) return Precond("hip_provider_not_ready");
  if (pinned ? g.prepared_device < 0 : g.prepared_device != device) return Precond("hip_device_not_prepared");
  void* p = nullptr;
  if (bytes) {
    DeviceScope scope(pinned ? g.prepared_device : device);
    if (scope.status() != hipSuccess) return FromHip(scope.status(), "hipSetDevice");
    const hipError_t e = pinned ? hipHostMalloc(&p, bytes, hipHostMallocDefault) : hipMalloc(&p, bytes);
    if (e != hipSuccess) return FromHip(e, pinned ? "hipHostMalloc" : "hipMalloc");
    if (reinterpret_cast<uintptr_t>(p) % kGranted) {
      (void)(pinned ? hipHostFree(p) : hipFree(p));
      return Internal("hip_allocation_misaligned");
    }
  }
  const uintptr_t addr = reinterpret_cast<uintptr_t>(p);
  const uint64_t gen = g.next_generation++;
  if (addr) {
    if (!g.allocations.emplace(addr, Allocation{bytes, kGranted, gen, device, kind}).second) {
      g.corrupted = true;  // an address handed out twice: stop trusting the table
      return Internal("hip_allocation_identity_duplicated");
    }
  }
  pih_cuda_allocation_v1 done{sizeof(done), PIH_NVIDIA_CUDA_MEMORY_ABI_VERSION_V1};
  done.address = addr;
  done.bytes = bytes;
  done.alignment = kGranted;
  done.generation = gen;
  done.device_ordinal = device;
  done.memory_kind = kind;
  *out = done;
  return Ok();
}

St Deallocate(const pih_cuda_allocation_v1* a, uint32_t kind) {
  const bool pinned = kind == PIH_CUDA_MEMORY_PINNED_HOST_V1;
  if (!a || a->struct_size != sizeof(*a) || a->abi_version != PIH_NVIDIA_CUDA_MEMORY_ABI_VERSION_V1 ||
      a->memory_kind != kind || (pinned ? a->device_ordinal != -1 : a->device_ordinal < 0))
    return Invalid("hip_allocation_handle_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  if (!g.releasable()) return Precond("hip_provider_not_releasable");
  if (a->address == 0) return Ok();
  auto it = g.allocations.find(a->address);
  if (it == g.allocations.end() || it->second.bytes != a->bytes || it->second.alignment != a->alignment ||
      it->second.generation != a->generation || it->second.device != a->device_ordinal ||
      it->second.kind != kind)
    return Precond("hip_allocation_owner_mismatch");
  void* p = reinterpret_cast<void*>(a->address);
  const hipError_t e = pinned ? hipHostFree(p) : hipFree(p);
  if (e != hipSuccess) return FromHip(e, pinned ? "hipHostFree" : "hipFree");
  g.allocations.erase(it);
  return Ok();
}

St CopyH2d(int32_t device, uintptr_t dst, const void* src, uint64_t bytes) {
  if (device < 0 || (bytes && (!dst || !src))) return Invalid("hip_copy_request_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  if (!g.ready()) return Precond("hip_provider_not_ready");
  if (g.prepared_device != device) return Precond("hip_device_not_prepared");
  if (bytes == 0) return Ok();
  if (!g.owns(dst, bytes, PIH_CUDA_MEMORY_DEVICE_V1, device)) return Precond("hip_copy_destination_not_owned");
  DeviceScope scope(device);
  if (scope.status() != hipSuccess) return FromHip(scope.status(), "hipSetDevice");
  return FromHip(hipMemcpy(reinterpret_cast<void*>(dst), src, bytes, hipMemcpyHostToDevice), "hipMemcpy");
}

// ----------------------------------------------------- device.cuda-resources
St RetainContext(int32_t device, uint32_t flags, uintptr_t* token) {
  if (device < 0 || !token || *token != 0 || (flags & ~PIH_CUDA_CONTEXT_SCHED_YIELD_V1))
    return Invalid("hip_context_request_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  if (!g.ready()) return Precond("hip_provider_not_ready");
  if (g.prepared_device != device) return Precond("hip_device_not_prepared");
  auto& rec = g.contexts[device];
  if (!rec) {
    rec.reset(new DeviceContext{device, flags, 0});
  } else if (rec->flags != flags || rec->retains == UINT32_MAX) {
    return Precond("hip_context_owner_conflict");
  }
  ++rec->retains;
  *token = reinterpret_cast<uintptr_t>(rec.get());
  return Ok();
}

St BindRuntime(int32_t device, uintptr_t token) {
  if (device < 0 || !token) return Invalid("hip_runtime_binding_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  if (!g.ready()) return Precond("hip_provider_not_ready");
  DeviceContext* c = g.context_of(token);
  if (!c || c->device != device) return Precond("hip_context_owner_mismatch");
  return FromHip(hipSetDevice(device), "hipSetDevice");
}

St CreateResource(uintptr_t token, uintptr_t* out, bool stream) {
  if (!token || !out || *out != 0) return Invalid(stream ? "hip_stream_request_invalid" : "hip_event_request_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  if (!g.ready()) return Precond("hip_provider_not_ready");
  DeviceContext* c = g.context_of(token);
  if (!c) return Precond("hip_context_owner_missing");
  const hipError_t set = hipSetDevice(c->device);
  if (set != hipSuccess) return FromHip(set, "hipSetDevice");
  uintptr_t handle = 0;
  if (stream) {
    hipStream_t s = nullptr;
    const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return FromHip(e, "hipStreamCreateWithFlags");
    handle = reinterpret_cast<uintptr_t>(s);
  } else {
    hipEvent_t ev = nullptr;
    const hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return FromHip(e, "hipEventCreateWithFlags");
    handle = reinterpret_cast<uintptr_t>(ev);
  }
  auto& table = stream ? g.streams : g.events;
  if (!handle || !table.emplace(handle, token).second) {
    g.corrupted = true;
    return Internal("hip_resource_identity_duplicated");
  }
  *out = handle;
  return Ok();
}

St DestroyResource(uintptr_t handle, bool stream) {
  if (!handle) return Invalid(stream ? "hip_stream_handle_invalid" : "hip_event_handle_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  if (!g.releasable()) return Precond("hip_provider_not_releasable");
  auto& table = stream ? g.streams : g.events;
  auto it = table.find(handle);
  if (it == table.end()) return Precond(stream ? "hip_stream_owner_mismatch" : "hip_event_owner_mismatch");
  DeviceContext* c = g.context_of(it->second);
  if (c) {
    const hipError_t set = hipSetDevice(c->device);
    if (set != hipSuccess) return FromHip(set, "hipSetDevice");
  }
  const hipError_t e = stream ? hipStreamDestroy(reinterpret_cast<hipStream_t>(handle))
                              : hipEventDestroy(reinterpret_cast<hipEvent_t>(handle));
  if (e != hipSuccess) return FromHip(e, stream ? "hipStreamDestroy" : "hipEventDestroy");
  table.erase(it);
  return Ok();
}

St ReleaseContext(int32_t device, uintptr_t token) {
  if (device < 0 || !token) return Invalid("hip_context_handle_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  if (!g.releasable()) return Precond("hip_provider_not_releasable");
  DeviceContext* c = g.context_of(token);
  if (!c || c->device != device) return Precond("hip_context_owner_mismatch");
  for (const auto& [h, owner] : g.streams)
    if (owner == token) return Precond("hip_context_has_live_streams");
  for (const auto& [h, owner] : g.events)
    if (owner == token) return Precond("hip_context_has_live_events");
  if (--c->retains == 0) g.contexts.erase(device);
  return Ok();
}

// --------------------------------------------------------- device.cuda-async
// The context must be owned and, for stream work, the stream created under it.
St StreamWork(uintptr_t token, uintptr_t stream, DeviceContext** out) {
  if (!g.ready()) return Precond("hip_provider_not_ready");
  DeviceContext* c = g.context_of(token);
  auto it = g.streams.find(stream);
  if (!c || it == g.streams.end() || it->second != token) return Precond("hip_stream_owner_mismatch");
  const hipError_t set = hipSetDevice(c->device);
  if (set != hipSuccess) return FromHip(set, "hipSetDevice");
  *out = c;
  return Ok();
}

bool IsPinnedHost(uintptr_t p) {
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, reinterpret_cast<const void*>(p)) != hipSuccess) {
    (void)hipGetLastError();  // an unknown host pointer is an answer, not a sticky error
    return false;
  }
  return attr.type == hipMemoryTypeHost;
}

St ActivateContext(uintptr_t token) {
  if (!token) return Invalid("hip_context_activate_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  if (!g.ready()) return Precond("hip_provider_not_ready");
  DeviceContext* c = g.context_of(token);
  if (!c) return Precond("hip_context_owner_mismatch");
  return FromHip(hipSetDevice(c->device), "hipSetDevice");
}

St ValidatePinnedHost(uintptr_t token, uintptr_t pointer) {
  if (!token || !pointer) return Invalid("hip_pinned_host_validation_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  if (!g.ready()) return Precond("hip_provider_not_ready");
  if (!g.context_of(token)) return Precond("hip_context_owner_mismatch");
  if (!g.owns(pointer, 1, PIH_CUDA_MEMORY_PINNED_HOST_V1, -1)) return Precond("hip_pinned_host_allocation_not_owned");
  return IsPinnedHost(pointer) ? Ok() : Precond("hip_pointer_is_not_pinned_host");
}

St CopyAsync(uintptr_t token, uintptr_t dst, uintptr_t src, uint64_t bytes, uint32_t kind, uintptr_t stream) {
  if (!token || !dst || !src || !bytes || !stream ||
      (kind != PIH_CUDA_COPY_H2D_V1 && kind != PIH_CUDA_COPY_D2H_V1 && kind != PIH_CUDA_COPY_D2D_V1))
    return Invalid("hip_async_copy_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  DeviceContext* c = nullptr;
  St s = StreamWork(token, stream, &c);
  if (!s.ok()) return s;
  const uint32_t dev = PIH_CUDA_MEMORY_DEVICE_V1, host = PIH_CUDA_MEMORY_PINNED_HOST_V1;
  const bool dst_ok = kind == PIH_CUDA_COPY_D2H_V1 ? g.owns(dst, bytes, host, -1) : g.owns(dst, bytes, dev, c->device);
  const bool src_ok = kind == PIH_CUDA_COPY_H2D_V1 ? g.owns(src, bytes, host, -1) : g.owns(src, bytes, dev, c->device);
  if (!dst_ok || !src_ok) return Precond("hip_async_copy_allocation_not_owned");
  if (kind != PIH_CUDA_COPY_D2D_V1 && !IsPinnedHost(kind == PIH_CUDA_COPY_H2D_V1 ? src : dst))
    return Precond("hip_async_copy_host_memory_not_pinned");
  const hipMemcpyKind mk = kind == PIH_CUDA_COPY_H2D_V1   ? hipMemcpyHostToDevice
                           : kind == PIH_CUDA_COPY_D2H_V1 ? hipMemcpyDeviceToHost
                                                          : hipMemcpyDeviceToDevice;
  return FromHip(hipMemcpyAsync(reinterpret_cast<void*>(dst), reinterpret_cast<const void*>(src), bytes, mk,
                                reinterpret_cast<hipStream_t>(stream)),
                 "hipMemcpyAsync");
}

St MemsetAsync(uintptr_t token, uintptr_t dst, uint32_t byte, uint64_t bytes, uintptr_t stream) {
  if (!token || !dst || byte > 255 || !bytes || !stream) return Invalid("hip_async_memset_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  DeviceContext* c = nullptr;
  St s = StreamWork(token, stream, &c);
  if (!s.ok()) return s;
  if (!g.owns(dst, bytes, PIH_CUDA_MEMORY_DEVICE_V1, c->device)) return Precond("hip_async_memset_allocation_not_owned");
  s = RequireCleanLastError();
  if (!s.ok()) return s;
  const uint64_t head = std::min<uint64_t>((16 - (dst & 15)) & 15, bytes);
  const uint64_t body = (bytes - head) / 16 * 16;
  const uint64_t units = std::max<uint64_t>(body / 16, head + (bytes - head - body));
  const uint32_t blocks = (uint32_t)std::min<uint64_t>(std::max<uint64_t>((units + 255) / 256, 1), 1024);
  hipLaunchKernelGGL(fill_bytes_kernel, dim3(blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<uint8_t*>(dst), byte, head, body, bytes);
  return AfterLaunch("hip_async_memset_launch_failed");
}

St RecordEvent(uintptr_t token, uintptr_t event, uintptr_t stream) {
  if (!token || !event || !stream) return Invalid("hip_event_record_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  DeviceContext* c = nullptr;
  St s = StreamWork(token, stream, &c);
  if (!s.ok()) return s;
  auto it = g.events.find(event);
  if (it == g.events.end() || it->second != token) return Precond("hip_event_owner_mismatch");
  return FromHip(hipEventRecord(reinterpret_cast<hipEvent_t>(event), reinterpret_cast<hipStream_t>(stream)),
                 "hipEventRecord");
}

St QueryEvent(uintptr_t token, uintptr_t event, uint32_t* status) {
  if (status) *status = 0;
  if (!token || !event || !status) return Invalid("hip_event_query_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  if (!g.ready()) return Precond("hip_provider_not_ready");
  DeviceContext* c = g.context_of(token);
  auto it = g.events.find(event);
  if (!c || it == g.events.end() || it->second != token) return Precond("hip_event_owner_mismatch");
  const hipError_t set = hipSetDevice(c->device);
  if (set != hipSuccess) return FromHip(set, "hipSetDevice");
  const hipError_t e = hipEventQuery(reinterpret_cast<hipEvent_t>(event));
  if (e == hipSuccess) {
    *status = PIH_CUDA_EVENT_COMPLETE_V1;
    return Ok();
  }
  if (e == hipErrorNotReady) {
    *status = PIH_CUDA_EVENT_PENDING_V1;
    return Ok();
  }
  return FromHip(e, "hipEventQuery");
}

St SynchronizeStream(uintptr_t token, uintptr_t stream) {
  if (!token || !stream) return Invalid("hip_stream_synchronize_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  DeviceContext* c = nullptr;
  St s = StreamWork(token, stream, &c);
  if (!s.ok()) return s;
  return FromHip(hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream)), "hipStreamSynchronize");
}

St CleanLastError(uintptr_t token) {
  if (!token) return Invalid("hip_last_error_probe_invalid");
  std::lock_guard<std::mutex> lock(g.mu);
  if (!g.ready()) return Precond("hip_provider_not_ready");
  DeviceContext* c = g.context_of(token);
  if (!c) return Precond("hip_context_owner_mismatch");
  int current = -1;
  if (hipGetDevice(&current) != hipSuccess || current != c->device) return Precond("hip_context_not_current");
  return FromHip(hipPeekAtLastError(), "hipPeekAtLastError");
}

// ------------------------------------------------------------ C-ABI tables
#define PIH_HIP_ENTRY(name, failure, params, call) \
  pih_status_v1 name params noexcept {             \
    if (ctx != &g) return ToAbi(Invalid("hip_provider_context_invalid")); \
    return Contain([&] { return call; }, failure); \
  }

PIH_HIP_ENTRY(CPrepareDevice, "hip_device_prepare_failed", (void* ctx, int32_t d, uint32_t ma, uint32_t mi),
              PrepareDevice(d, ma, mi))
PIH_HIP_ENTRY(CAllocateDevice, "hip_device_allocation_failed",
              (void* ctx, int32_t d, uint64_t b, uint64_t al, pih_cuda_allocation_v1* o),
              Allocate(d, b, al, o, PIH_CUDA_MEMORY_DEVICE_V1))
PIH_HIP_ENTRY(CDeallocateDevice, "hip_device_deallocation_failed", (void* ctx, const pih_cuda_allocation_v1* a),
              Deallocate(a, PIH_CUDA_MEMORY_DEVICE_V1))
PIH_HIP_ENTRY(CAllocatePinned, "hip_pinned_allocation_failed",
              (void* ctx, int32_t d, uint64_t b, uint64_t al, pih_cuda_allocation_v1* o),
              Allocate(d, b, al, o, PIH_CUDA_MEMORY_PINNED_HOST_V1))
PIH_HIP_ENTRY(CDeallocatePinned, "hip_pinned_deallocation_failed", (void* ctx, const pih_cuda_allocation_v1* a),
              Deallocate(a, PIH_CUDA_MEMORY_PINNED_HOST_V1))
PIH_HIP_ENTRY(CCopyH2d, "hip_h2d_copy_failed", (void* ctx, int32_t d, uintptr_t dst, const void* src, uint64_t b),
              CopyH2d(d, dst, src, b))
PIH_HIP_ENTRY(CRetainContext, "hip_context_retain_failed", (void* ctx, int32_t d, uint32_t f, uintptr_t* t),
              RetainContext(d, f, t))
PIH_HIP_ENTRY(CBindRuntime, "hip_runtime_binding_failed", (void* ctx, int32_t d, uintptr_t t), BindRuntime(d, t))
PIH_HIP_ENTRY(CCreateStream, "hip_stream_creation_failed", (void* ctx, uintptr_t t, uintptr_t* r),
              CreateResource(t, r, true))
PIH_HIP_ENTRY(CCreateEvent, "hip_event_creation_failed", (void* ctx, uintptr_t t, uintptr_t* r),
              CreateResource(t, r, false))
PIH_HIP_ENTRY(CDestroyEvent, "hip_event_destruction_failed", (void* ctx, uintptr_t r), DestroyResource(r, false))
PIH_HIP_ENTRY(CDestroyStream, "hip_stream_destruction_failed", (void* ctx, uintptr_t r), DestroyResource(r, true))
PIH_HIP_ENTRY(CReleaseContext, "hip_context_release_failed", (void* ctx, int32_t d, uintptr_t t),
              ReleaseContext(d, t))
PIH_HIP_ENTRY(CActivateContext, "hip_context_activation_failed", (void* ctx, uintptr_t t), ActivateContext(t))
PIH_HIP_ENTRY(CValidatePinned, "hip_pinned_host_validation_failed", (void* ctx, uintptr_t t, uintptr_t p),
              ValidatePinnedHost(t, p))
PIH_HIP_ENTRY(CCopyAsync, "hip_async_copy_failed",
              (void* ctx, uintptr_t t, uintptr_t d, uintptr_t s, uint64_t b, uint32_t k, uintptr_t st),
              CopyAsync(t, d, s, b, k, st))
PIH_HIP_ENTRY(CMemsetAsync, "hip_async_memset_failed",
              (void* ctx, uintptr_t t, uintptr_t d, uint32_t v, uint64_t b, uintptr_t st), MemsetAsync(t, d, v, b, st))
PIH_HIP_ENTRY(CRecordEvent, "hip_event_record_failed", (void* ctx, uintptr_t t, uintptr_t e, uintptr_t s),
              RecordEvent(t, e, s))
PIH_HIP_ENTRY(CQueryEvent, "hip_event_query_failed", (void* ctx, uintptr_t t, uintptr_t e, uint32_t* s),
              QueryEvent(t, e, s))
PIH_HIP_ENTRY(CSynchronizeStream, "hip_stream_synchronize_failed", (void* ctx, uintptr_t t, uintptr_t s),
              SynchronizeStream(t, s))
PIH_HIP_ENTRY(CCleanLastError, "hip_last_error_probe_failed", (void* ctx, uintptr_t t), CleanLastError(t))
#undef PIH_HIP_ENTRY

const pih_nvidia_cuda_api_v1 kRuntime = {sizeof(pih_nvidia_cuda_api_v1), PIH_NVIDIA_CUDA_ABI_VERSION_V1, &g,
                                         &CPrepareDevice};
const pih_nvidia_cuda_memory_api_v1 kMemory = {sizeof(pih_nvidia_cuda_memory_api_v1),
                                               PIH_NVIDIA_CUDA_MEMORY_ABI_VERSION_V1,
                                               &g,
                                               &CAllocateDevice,
                                               &CDeallocateDevice,
                                               &CAllocatePinned,
                                               &CDeallocatePinned,
                                               &CCopyH2d};
const pih_nvidia_cuda_resources_api_v1 kResources = {sizeof(pih_nvidia_cuda_resources_api_v1),
                                                     PIH_NVIDIA_CUDA_RESOURCES_ABI_VERSION_V1,
                                                     &g,
                                                     &CRetainContext,
                                                     &CBindRuntime,
                                                     &CCreateStream,
                                                     &CCreateEvent,
                                                     &CDestroyEvent,
                                                     &CDestroyStream,
                                                     &CReleaseContext};
const pih_nvidia_cuda_async_api_v1 kAsync = {sizeof(pih_nvidia_cuda_async_api_v1),
                                             PIH_NVIDIA_CUDA_ASYNC_ABI_VERSION_V1,
                                             &g,
                                             &CActivateContext,
                                             &CValidatePinned,
                                             &CCopyAsync,
                                             &CMemsetAsync,
                                             &CRecordEvent,
                                             &CQueryEvent,
                                             &CSynchronizeStream,
                                             &CCleanLastError};

// ---------------------------------------------------------------- lifecycle
St CheckedHostStatus(pih_status_v1 s, const char* invalid) {
  if (!pih_status_is_valid_v1(&s)) return Internal(invalid);
  return St{s.code, nullptr};
}

St Register() {
  if (g.phase != 0) return Precond("lifecycle_order_invalid");
  struct Cap {
    const char* id;
    const char* contract;
    const void* api;
  };
  const Cap caps[] = {{"device.cuda-runtime.v1", "pih.device.cuda-runtime.v1", &kRuntime},
                      {"device.cuda-memory.v1", "pih.device.cuda-memory.v1", &kMemory},
                      {"device.cuda-resources.v1", "pih.device.cuda-resources.v1", &kResources},
                      {"device.cuda-async.v1", "pih.device.cuda-async.v1", &kAsync}};
  for (const Cap& c : caps) {
    pih_capability_v1 cap{};
    cap.struct_size = sizeof(cap);
    cap.abi_version = PIH_CAPABILITY_ABI_VERSION_V1;
    cap.capability_id = c.id;
    cap.contract_id = c.contract;
    cap.api = c.api;
    cap.threading_model = PIH_CAPABILITY_THREADING_SERIALIZED_V1;
    cap.scope = PIH_CAPABILITY_SCOPE_PROCESS_V1;
    cap.cardinality = PIH_CAPABILITY_CARDINALITY_EXACTLY_ONE_V1;
    pih_status_v1 r = g.host->register_capability(g.host->context, &cap);
    if (!pih_status_is_valid_v1(&r)) return Internal("capability_registry_status_invalid");
    if (r.code != PIH_STATUS_OK_V1) return St{r.code, "capability_registration_rejected"};
  }
  g.phase = 1;
  return Ok();
}

St Configure() {
  if (g.phase != 1) return Precond("lifecycle_order_invalid");
  const void* api = nullptr;
  pih_status_v1 r = g.host->resolve_capability(g.host->context, "platform.linux.v1", "pih.platform.linux.v1",
                                               PIH_CAPABILITY_SCOPE_PROCESS_V1,
                                               PIH_CAPABILITY_CARDINALITY_EXACTLY_ONE_V1, &api);
  if (!pih_status_is_valid_v1(&r)) return Internal("capability_resolver_status_invalid");
  if (r.code != PIH_STATUS_OK_V1) return St{r.code, "platform_capability_unresolved"};
  const auto* platform = static_cast<const pih_platform_linux_api_v1*>(api);
  if (!platform || platform->struct_size != sizeof(*platform) ||
      platform->contract_version != PIH_PLATFORM_LINUX_ABI_VERSION_V1 || !platform->context ||
      !platform->validate_runtime)
    return Precond("linux_platform_capability_invalid");
  g.platform = platform;
  g.phase = 2;
  return Ok();
}

St Start() {
  if (g.phase != 2 || !g.platform) return Precond("hip_start_configuration_invalid");
  // the platform is only called after every plugin has been configured
  pih_status_v1 r = g.platform->validate_runtime(g.platform->context);
  if (!pih_status_is_valid_v1(&r)) return Internal("platform_provider_status_invalid");
  if (r.code != PIH_STATUS_OK_V1) return St{r.code, "platform_runtime_invalid"};
  g.phase = 3;
  return Ok();
}

St Ready() {
  if (g.phase != 3) return Precond("lifecycle_order_invalid");
  g.phase = 4;
  return Ok();
}

St Drain() {
  std::lock_guard<std::mutex> lock(g.mu);
  if (g.corrupted) return Precond("hip_resource_ownership_corrupted");
  if (!g.idle()) return Precond("hip_resources_still_live");
  if (g.phase != 4) return Precond("lifecycle_order_invalid");
  g.phase = 5;
  return Ok();
}

St Stop() {
  std::lock_guard<std::mutex> lock(g.mu);
  if (g.phase != 3 && g.phase != 5) return Precond("lifecycle_order_invalid");
  g.phase = 6;  // a started-but-never-ready provider may stop directly
  return Ok();
}

St Dispose() {
  std::lock_guard<std::mutex> lock(g.mu);
  if (g.phase != 1 && g.phase != 2 && g.phase != 6) return Precond("lifecycle_order_invalid");
  if (g.corrupted) return Precond("hip_resource_ownership_corrupted");
  if (!g.idle()) return Precond("hip_resources_still_live");
  g.prepared_device = -1;
  g.prepared_major = g.prepared_minor = 0;
  g.platform = nullptr;
  g.host = nullptr;
  g.phase = 7;
  return Ok();
}

#define PIH_HIP_LIFECYCLE(name, call, failure)                               \
  pih_status_v1 name(void* ctx) noexcept {                                  \
    if (ctx != &g) return ToAbi(Invalid("lifecycle_context_invalid"));      \
    return Contain([&] { return call(); }, failure);                        \
  }
PIH_HIP_LIFECYCLE(CRegister, Register, "hip_registration_failed")
PIH_HIP_LIFECYCLE(CConfigure, Configure, "hip_configuration_failed")
PIH_HIP_LIFECYCLE(CStart, Start, "hip_start_failed")
PIH_HIP_LIFECYCLE(CReady, Ready, "hip_ready_failed")
PIH_HIP_LIFECYCLE(CDrain, Drain, "hip_drain_failed")
PIH_HIP_LIFECYCLE(CStop, Stop, "hip_stop_failed")
PIH_HIP_LIFECYCLE(CDispose, Dispose, "hip_dispose_failed")
#undef PIH_HIP_LIFECYCLE

}  // namespace
}  // namespace pih_amd

extern "C" __attribute__((visibility("default"))) pih_status_v1 pih_plugin_entry_v1(
    const pih_host_api_v1* host, pih_plugin_api_v1* plugin) noexcept {
  using namespace pih_amd;
  if (!pih_host_api_is_valid_v1(host)) return ToAbi(Invalid("host_api_invalid"));
  if (!pih_plugin_api_accepts_v1(plugin)) return ToAbi(Invalid("plugin_api_invalid"));
  if (g.host != nullptr || g.phase != 0) return ToAbi(Precond("plugin_entry_already_bound"));
  g.host = host;
  plugin->plugin_id = "pih.backend.amd-hip";
  plugin->plugin_version = "1.0.0";
  plugin->context = &g;
  plugin->lifecycle.struct_size = sizeof(pih_plugin_lifecycle_v1);
  plugin->lifecycle.abi_version = PIH_PLUGIN_LIFECYCLE_ABI_VERSION_V1;
  plugin->lifecycle.register_plugin = &CRegister;
  plugin->lifecycle.configure = &CConfigure;
  plugin->lifecycle.start = &CStart;
  plugin->lifecycle.ready = &CReady;
  plugin->lifecycle.drain = &CDrain;
  plugin->lifecycle.stop = &CStop;
  plugin->lifecycle.dispose = &CDispose;
  return ToAbi(Ok());
}

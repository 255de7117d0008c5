// Host-side helpers of the gfx950 packs: the internal status value every
// launcher returns, its conversion to the C-ABI pih_status_v1, and the
// request-header checks the reference performs before any launch
// (plugins/kernels/deepseek-v4-sm89/kernel_pack.cpp:117-189,441-462).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <atomic>
#include <new>

#include "pih/plugin_sdk/status.h"

namespace pih_amd {

struct St {
  uint32_t code = PIH_STATUS_OK_V1;
  const char* message = nullptr;
  bool ok() const { return code == PIH_STATUS_OK_V1; }
};

inline St Ok() { return {}; }
inline St Invalid(const char* m) { return {PIH_STATUS_INVALID_ARGUMENT_V1, m}; }
inline St Internal(const char* m) { return {PIH_STATUS_INTERNAL_V1, m}; }
inline St Unavailable(const char* m) { return {PIH_STATUS_UNAVAILABLE_V1, m}; }
inline St Precondition(const char* m) { return {PIH_STATUS_FAILED_PRECONDITION_V1, m}; }

inline pih_status_v1 ToAbi(St s) {
  pih_status_v1 v;
  memset(&v, 0, sizeof(v));
  v.struct_size = sizeof(v);
  v.abi_version = PIH_STATUS_ABI_VERSION_V1;
  v.code = s.code;
  if (s.message) strncpy(v.message, s.message, sizeof(v.message) - 1);
  return v;
}

// A sticky HIP error left by earlier work is reported, not hidden
// (cudaPeekAtLastError in the reference launchers, e.g.
// deepseek_fp8_gemm.cu:85-87).
inline St RequireCleanLastError() {
  return hipPeekAtLastError() == hipSuccess ? Ok() : Internal("hip_sticky_error_before_launch");
}

inline St AfterLaunch(const char* what) {
  return hipGetLastError() == hipSuccess ? Ok() : St{PIH_STATUS_INTERNAL_V1, what};
}

inline hipStream_t AsStream(uintptr_t s) { return reinterpret_cast<hipStream_t>(s); }

template <typename T>
inline T* Ptr(uintptr_t p) {
  return reinterpret_cast<T*>(p);
}

// A one-time host step per device (raising a kernel's LDS limit): run()
// performs the step on the current device until it has succeeded there
// once.  Host threads that arrive together may both perform it (every such
// step is idempotent); the flags are atomics, so there is no data race.
constexpr int kHostMaxDevices = 64;
class PerDeviceOnce {
 public:
  template <typename F>
  St run(F&& step) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kHostMaxDevices) return step();
    if (done_[dev].load(std::memory_order_acquire)) return Ok();
    const St s = step();
    if (s.ok()) done_[dev].store(true, std::memory_order_release);
    return s;
  }

 private:
  std::atomic<bool> done_[kHostMaxDevices] = {};
};

// struct_size / abi_version gate shared by every entry point.
template <typename R>
inline bool HeaderOk(const R* r, uint32_t abi) {
  return r != nullptr && r->struct_size == sizeof(R) && r->abi_version == abi;
}

}  // namespace pih_amd

// C++ exceptions never cross the C ABI (reference kernel_pack.cpp:441-462).
#define PIH_AMD_CONTAINED(wrapper, body_fn, request_type)                    \
  static pih_status_v1 wrapper(const request_type* request) noexcept {      \
    try {                                                                   \
      return ::pih_amd::ToAbi(body_fn(request));                            \
    } catch (const std::bad_alloc&) {                                       \
      return ::pih_amd::ToAbi(                                              \
          {PIH_STATUS_RESOURCE_EXHAUSTED_V1, "kernel_pack_allocation_failed"}); \
    } catch (...) {                                                         \
      return ::pih_amd::ToAbi(                                              \
          {PIH_STATUS_INTERNAL_V1, "kernel_pack_callback_failed"});         \
    }                                                                       \
  }

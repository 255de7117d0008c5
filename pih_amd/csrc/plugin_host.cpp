// A minimal native plugin host for the backend plugin: the part of the
// reference's microkernel that loads a native plugin and activates it
// (src/microkernel/plugin_loader.cpp:74-128: entry, plugin/lifecycle table
// checks, the library stays mapped; activation_runtime.cpp:96-190: register
// -> configure -> start -> ready, then drain -> stop -> dispose).  It owns
// the host table the plugin is bound to, keeps every capability the plugin
// registers, and publishes platform.linux.v1 itself, whose validate_runtime
// answers a code the caller sets.  The C entry points below let a Python
// host (which cannot implement callbacks returning pih_status_v1 by value)
// drive it.
#include <dlfcn.h>
#include <string.h>

#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "pih/contracts/device_cuda_v1.h"
#include "pih/plugin_sdk/plugin.h"

namespace {

pih_status_v1 MakeStatus(uint32_t code, const char* message = "") {
  pih_status_v1 s;
  memset(&s, 0, sizeof(s));
  s.struct_size = sizeof(s);
  s.abi_version = PIH_STATUS_ABI_VERSION_V1;
  s.code = code;
  strncpy(s.message, message, sizeof(s.message) - 1);
  return s;
}

struct Registered {
  std::string capability, contract;
  const void* api;
  uint32_t threading, scope, cardinality;
};

struct Resolve {
  std::string capability, contract;
  uint32_t scope, cardinality;
};

bool CanonicalId(const char* s, size_t maximum) {
  if (!s) return false;
  const size_t n = strnlen(s, maximum + 1);
  if (n == 0 || n > maximum || s[0] == '.' || s[n - 1] == '.') return false;
  for (size_t i = 0; i < n; ++i) {
    const char c = s[i];
    if (!((c >= 'a' && c <= 'z') || (c >= '0' && c <= '9') || c == '.' || c == '-')) return false;
    if (c == '.' && i && s[i - 1] == '.') return false;
  }
  return true;
}

}  // namespace

struct pih_amd_plugin_host {
  std::mutex mu;
  pih_host_api_v1 host{};
  pih_plugin_api_v1 plugin{};
  pih_platform_linux_api_v1 platform{};
  void* library = nullptr;
  bool loaded = false;
  uint32_t platform_code = PIH_STATUS_OK_V1;
  uint32_t platform_calls = 0;
  std::vector<Registered> registered;
  std::vector<Resolve> resolves;
  std::vector<std::string> logs;
};

namespace {

void Log(void* context, uint32_t severity, const char* code, const char* message) {
  auto* h = static_cast<pih_amd_plugin_host*>(context);
  std::lock_guard<std::mutex> lock(h->mu);
  h->logs.push_back(std::to_string(severity) + ":" + (code ? code : "") + ":" + (message ? message : ""));
}

pih_status_v1 RegisterCapability(void* context, const pih_capability_v1* cap) {
  auto* h = static_cast<pih_amd_plugin_host*>(context);
  if (!cap || cap->struct_size != sizeof(*cap) || cap->abi_version != PIH_CAPABILITY_ABI_VERSION_V1 ||
      !CanonicalId(cap->capability_id, 256) || !CanonicalId(cap->contract_id, 256) || !cap->api)
    return MakeStatus(PIH_STATUS_INVALID_ARGUMENT_V1, "capability_invalid");
  std::lock_guard<std::mutex> lock(h->mu);
  for (const Registered& r : h->registered)
    if (r.capability == cap->capability_id) return MakeStatus(PIH_STATUS_FAILED_PRECONDITION_V1, "capability_duplicate");
  h->registered.push_back(
      {cap->capability_id, cap->contract_id, cap->api, cap->threading_model, cap->scope, cap->cardinality});
  return MakeStatus(PIH_STATUS_OK_V1);
}

pih_status_v1 ResolveCapability(void* context, const char* capability, const char* contract, uint32_t scope,
                                uint32_t cardinality, const void** api) {
  auto* h = static_cast<pih_amd_plugin_host*>(context);
  if (!capability || !contract || !api) return MakeStatus(PIH_STATUS_INVALID_ARGUMENT_V1, "resolve_invalid");
  *api = nullptr;
  std::lock_guard<std::mutex> lock(h->mu);
  h->resolves.push_back({capability, contract, scope, cardinality});
  if (strcmp(capability, "platform.linux.v1") == 0 && strcmp(contract, "pih.platform.linux.v1") == 0 &&
      scope == PIH_CAPABILITY_SCOPE_PROCESS_V1 && cardinality == PIH_CAPABILITY_CARDINALITY_EXACTLY_ONE_V1) {
    *api = &h->platform;
    return MakeStatus(PIH_STATUS_OK_V1);
  }
  for (const Registered& r : h->registered)
    if (r.capability == capability && r.contract == contract) {
      *api = r.api;
      return MakeStatus(PIH_STATUS_OK_V1);
    }
  return MakeStatus(PIH_STATUS_FAILED_PRECONDITION_V1, "capability_unresolved");
}

pih_status_v1 ValidateRuntime(void* context) {
  auto* h = static_cast<pih_amd_plugin_host*>(context);
  std::lock_guard<std::mutex> lock(h->mu);
  ++h->platform_calls;
  return MakeStatus(h->platform_code, h->platform_code == PIH_STATUS_OK_V1 ? "" : "platform_runtime_rejected");
}

}  // namespace

#define PIH_HOST_EXPORT extern "C" __attribute__((visibility("default")))

PIH_HOST_EXPORT pih_amd_plugin_host* pih_amd_host_create(uint64_t activation_epoch) {
  auto* h = new (std::nothrow) pih_amd_plugin_host();
  if (!h) return nullptr;
  h->host = {sizeof(pih_host_api_v1), PIH_PLUGIN_ABI_VERSION_V1, h, &Log, &RegisterCapability,
             &ResolveCapability, activation_epoch};
  h->platform = {sizeof(pih_platform_linux_api_v1), PIH_PLATFORM_LINUX_ABI_VERSION_V1, h, &ValidateRuntime};
  h->plugin.struct_size = sizeof(pih_plugin_api_v1);
  h->plugin.abi_version = PIH_PLUGIN_ABI_VERSION_V1;
  return h;  // hosts live until the process ends, like the plugins they bind
}

PIH_HOST_EXPORT const pih_host_api_v1* pih_amd_host_api(pih_amd_plugin_host* h) { return h ? &h->host : nullptr; }

PIH_HOST_EXPORT const pih_plugin_api_v1* pih_amd_host_plugin(pih_amd_plugin_host* h) {
  return h && h->loaded ? &h->plugin : nullptr;
}

// dlopen + entry + the reference loader's table checks.  A library whose
// entry ran stays mapped even when its tables are rejected.
PIH_HOST_EXPORT pih_status_v1 pih_amd_host_load(pih_amd_plugin_host* h, const char* path) {
  if (!h || !path || path[0] != '/') return MakeStatus(PIH_STATUS_INVALID_ARGUMENT_V1, "plugin_path_invalid");
  if (h->loaded) return MakeStatus(PIH_STATUS_FAILED_PRECONDITION_V1, "plugin_host_already_loaded");
  if (!pih_host_api_is_valid_v1(&h->host)) return MakeStatus(PIH_STATUS_INVALID_ARGUMENT_V1, "plugin_host_api_invalid");
  void* lib = dlopen(path, RTLD_NOW | RTLD_LOCAL);
  if (!lib) return MakeStatus(PIH_STATUS_UNAVAILABLE_V1, "plugin_load_failed");
  auto entry = reinterpret_cast<pih_plugin_entry_fn_v1>(dlsym(lib, "pih_plugin_entry_v1"));
  if (!entry) return MakeStatus(PIH_STATUS_INVALID_ARGUMENT_V1, "plugin_entry_missing");
  h->library = lib;
  pih_status_v1 st = entry(&h->host, &h->plugin);
  if (!pih_status_is_ok_v1(&st)) return pih_status_is_valid_v1(&st) ? st : MakeStatus(PIH_STATUS_INTERNAL_V1, "plugin_entry_status_invalid");
  const pih_plugin_api_v1& a = h->plugin;
  if (a.struct_size != sizeof(a) || a.abi_version != PIH_PLUGIN_ABI_VERSION_V1 || !CanonicalId(a.plugin_id, 256) ||
      !CanonicalId(a.plugin_version, 64) || !a.context)
    return MakeStatus(PIH_STATUS_INVALID_ARGUMENT_V1, "plugin_api_invalid");
  const pih_plugin_lifecycle_v1& l = a.lifecycle;
  if (l.struct_size != sizeof(l) || l.abi_version != PIH_PLUGIN_LIFECYCLE_ABI_VERSION_V1 || !l.register_plugin ||
      !l.configure || !l.start || !l.ready || !l.drain || !l.stop || !l.dispose)
    return MakeStatus(PIH_STATUS_INVALID_ARGUMENT_V1, "plugin_lifecycle_invalid");
  h->loaded = true;
  return MakeStatus(PIH_STATUS_OK_V1);
}

// phase: 0 register, 1 configure, 2 start, 3 ready, 4 drain, 5 stop, 6 dispose.
// `context` overrides the plugin's own context when non-null (to check
// that the plugin rejects a foreign one).
PIH_HOST_EXPORT pih_status_v1 pih_amd_host_phase(pih_amd_plugin_host* h, uint32_t phase, void* context) {
  if (!h || !h->loaded || phase > 6) return MakeStatus(PIH_STATUS_INVALID_ARGUMENT_V1, "host_phase_invalid");
  const pih_plugin_lifecycle_v1& l = h->plugin.lifecycle;
  const pih_lifecycle_callback_v1 fns[] = {l.register_plugin, l.configure, l.start, l.ready,
                                           l.drain,           l.stop,      l.dispose};
  pih_status_v1 st = fns[phase](context ? context : h->plugin.context);
  return pih_status_is_valid_v1(&st) ? st : MakeStatus(PIH_STATUS_INTERNAL_V1, "plugin_phase_status_invalid");
}

PIH_HOST_EXPORT void pih_amd_host_set_platform_status(pih_amd_plugin_host* h, uint32_t code) {
  if (!h) return;
  std::lock_guard<std::mutex> lock(h->mu);
  h->platform_code = code;
}

PIH_HOST_EXPORT uint32_t pih_amd_host_platform_calls(pih_amd_plugin_host* h) {
  if (!h) return 0;
  std::lock_guard<std::mutex> lock(h->mu);
  return h->platform_calls;
}

PIH_HOST_EXPORT uint32_t pih_amd_host_capability_count(pih_amd_plugin_host* h) {
  if (!h) return 0;
  std::lock_guard<std::mutex> lock(h->mu);
  return (uint32_t)h->registered.size();
}

// Fills the i-th registered capability; returns 0 when i is out of range.
PIH_HOST_EXPORT int pih_amd_host_capability(pih_amd_plugin_host* h, uint32_t i, pih_capability_v1* out) {
  if (!h || !out) return 0;
  std::lock_guard<std::mutex> lock(h->mu);
  if (i >= h->registered.size()) return 0;
  const Registered& r = h->registered[i];
  *out = {sizeof(pih_capability_v1), PIH_CAPABILITY_ABI_VERSION_V1, r.capability.c_str(), r.contract.c_str(),
          r.api, r.threading, r.scope, r.cardinality};
  return 1;
}

PIH_HOST_EXPORT uint32_t pih_amd_host_resolve_count(pih_amd_plugin_host* h) {
  if (!h) return 0;
  std::lock_guard<std::mutex> lock(h->mu);
  return (uint32_t)h->resolves.size();
}

// The i-th resolve request as "capability contract scope cardinality".
PIH_HOST_EXPORT int pih_amd_host_resolve(pih_amd_plugin_host* h, uint32_t i, char* out, uint32_t size) {
  if (!h || !out || !size) return 0;
  std::lock_guard<std::mutex> lock(h->mu);
  if (i >= h->resolves.size()) return 0;
  const Resolve& r = h->resolves[i];
  const std::string s =
      r.capability + " " + r.contract + " " + std::to_string(r.scope) + " " + std::to_string(r.cardinality);
  strncpy(out, s.c_str(), size - 1);
  out[size - 1] = 0;
  return 1;
}

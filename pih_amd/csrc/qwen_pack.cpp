// gfx950 Qwen Kernel Pack: the identity, the pih_qwen_kernels_api_v1 table
// and the two exported C symbols (include/pih/plugin_sdk/kernel_pack.h).
// The Qwen model loads its device code itself: after binding, root() hands
// it the directory holding gfx950/qwen_bf16_primitives.hsaco and the .json
// manifest beside it, the same shape as the reference's sm_89/sm_90 pack
// (plugins/kernels/qwen3/kernel_pack.cpp:10-36), whose cubin becomes a gfx950
// code object loaded with hipModuleLoadData.
//
// bind_origin(path) takes the absolute path of this library, canonicalises
// it and requires <dir>/qwen3-gfx950/gfx950/qwen_bf16_primitives.hsaco and
// .hsaco.json to be regular files; a second bind must name the same
// directory.  Neither call touches a device.
#include <filesystem>
#include <mutex>
#include <string>

#include "host_common.hpp"
#include "pih/contracts/qwen_kernels_v1.h"
#include "pih/plugin_sdk/kernel_pack.h"

namespace pih_amd {
namespace {

constexpr const char* kPackDirectory = "qwen3-gfx950";
constexpr const char* kArchDirectory = "gfx950";
constexpr const char* kCodeObject = "qwen_bf16_primitives.hsaco";
constexpr const char* kManifest = "qwen_bf16_primitives.hsaco.json";

const pih_kernel_pack_identity_v1 kIdentity = {sizeof(pih_kernel_pack_identity_v1), PIH_KERNEL_PACK_ABI_VERSION_V1,
                                               "pih.kernels.qwen3.gfx950", "1.0.0", "pih.qwen-kernels.v1",
                                               "gfx950"};

std::mutex g_mutex;
std::string g_root;  // set once by bind_origin; the pack is never unloaded

St Bind(const char* path) {
  if (!path || path[0] != '/') return Invalid("bind_origin_path_not_absolute");
  namespace fs = std::filesystem;
  std::error_code ec;
  const fs::path lib = fs::canonical(path, ec);
  if (ec) return Invalid("bind_origin_path_unresolvable");
  const fs::path dir = lib.parent_path() / kPackDirectory;
  const fs::path arch = dir / kArchDirectory;
  if (!fs::is_regular_file(arch / kCodeObject, ec) || !fs::is_regular_file(arch / kManifest, ec))
    return Invalid("bind_origin_code_object_missing");
  std::lock_guard<std::mutex> lock(g_mutex);
  if (g_root.empty()) {
    g_root = dir.string();  // never reassigned: root() hands out its c_str()
  } else if (g_root != dir.string()) {
    return Invalid("bind_origin_rebound_elsewhere");
  }
  return Ok();
}

pih_status_v1 BindOrigin(const char* path) noexcept {
  try {
    return ToAbi(Bind(path));
  } catch (...) {
    return ToAbi(Internal("bind_origin_failed"));
  }
}

pih_status_v1 Root(const char** path) noexcept {
  if (!path) return ToAbi(Invalid("root_path_null"));
  *path = nullptr;
  std::lock_guard<std::mutex> lock(g_mutex);
  if (g_root.empty()) return ToAbi(Precondition("root_before_bind_origin"));
  *path = g_root.c_str();
  return ToAbi(Ok());
}

const pih_qwen_kernels_api_v1 kContract = {sizeof(pih_qwen_kernels_api_v1), 1u, 950u, &Root};

const pih_kernel_pack_api_v1 kApi = {sizeof(pih_kernel_pack_api_v1), PIH_KERNEL_PACK_ABI_VERSION_V1, &kIdentity,
                                     &kContract, &BindOrigin};

}  // namespace
}  // namespace pih_amd

extern "C" PIH_PLUGIN_EXPORT const pih_kernel_pack_identity_v1* pih_kernel_pack_identity_v1_get(void) {
  return &pih_amd::kIdentity;
}

extern "C" PIH_PLUGIN_EXPORT const pih_kernel_pack_api_v1* pih_kernel_pack_api_v1_get(void) {
  return &pih_amd::kApi;
}

// Host loaders of the on-disk weight formats (libpih_amd_artifacts.so):
// the Qwen3 INT4 XINGW4A1 canonical artifact and the DeepSeek V4 Flash
// routed-expert bundle, onto gfx950 device memory.  The declarations and the
// reference interfaces each entry replaces are in
// include/pih/contracts/amd_artifacts_v1.h.
//
// The Qwen artifact is validated the way the reference's loader does it:
// the official record list is rebuilt here (28 layers x 7 projections as
// packed values + fp16 scales, 113 bf16 norms, the bf16 embedding and the
// tied lm_head alias, sorted by identity, extents 4096-aligned from 1 MiB),
// the metadata region must match it field by field, and the payload SHA-256
// digests are checked on up to 16 host threads.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "host_common.hpp"
#include "sha256.hpp"
#include "pih/contracts/amd_artifacts_v1.h"

namespace pih_amd {
namespace {

// ------------------------------------------------- official Qwen layout
constexpr uint64_t kMeta = PIH_AMD_QWEN_INT4_METADATA_BYTES_V1;
constexpr uint64_t kFileBytes = PIH_AMD_QWEN_INT4_FILE_BYTES_V1;
constexpr uint64_t kAlign = 4096;
constexpr const char kFormatId[] = "xing-w4a16-sym-g128-v1";
constexpr const char kLayoutId[] = "canonical-nk-low-nibble-k-v1";
constexpr uint32_t kHeaderBytes = 160, kChecksumOffset = 120;

struct Rec {
  std::string identity, source, alias;
  uint8_t kind;
  uint64_t logical, offset, extent, rows, cols;
};

struct Layout {
  std::vector<Rec> recs;
  uint64_t logical_total = 0, padded = 0;
  bool ok = false;
};

// qwen3_int4_linear_shape_ledger.cpp:14-31 (per-layer projections) and
// qwen3_int4_artifact_layout.cpp:41-104 (records, sort, offsets, totals)
const Layout& OfficialLayout() {
  static Layout L;
  static std::once_flag once;
  std::call_once(once, [] {
    struct Proj {
      const char* suffix;
      uint64_t rows, cols;
    };
    static const Proj kProj[7] = {{"self_attn.q_proj.weight", 2048, 1024}, {"self_attn.k_proj.weight", 1024, 1024},
                                  {"self_attn.v_proj.weight", 1024, 1024}, {"self_attn.o_proj.weight", 1024, 2048},
                                  {"mlp.gate_proj.weight", 3072, 1024},    {"mlp.up_proj.weight", 3072, 1024},
                                  {"mlp.down_proj.weight", 1024, 3072}};
    auto& r = L.recs;
    r.push_back({"model.embed_tokens.weight", "model.embed_tokens.weight", "", PIH_AMD_QWEN_INT4_BF16_EMBEDDING_V1,
                 151936ull * 1024 * 2, 0, 0, 151936, 1024});
    r.push_back({"lm_head.weight", "lm_head.weight", "model.embed_tokens.weight", PIH_AMD_QWEN_INT4_ALIAS_V1, 0, 0, 0,
                 151936, 1024});
    for (int layer = 0; layer < 28; ++layer) {
      const std::string pre = "model.layers." + std::to_string(layer) + ".";
      for (const Proj& p : kProj) {
        const std::string src = pre + p.suffix;
        r.push_back({src + ".packed_values", src, "", PIH_AMD_QWEN_INT4_PACKED_VALUES_V1, p.rows * p.cols / 2, 0, 0,
                     p.rows, p.cols});
        r.push_back({src + ".scales", src, "", PIH_AMD_QWEN_INT4_FP16_SCALES_V1, p.rows * (p.cols / 128) * 2, 0, 0,
                     p.rows, p.cols});
      }
      for (const auto& [name, width] : {std::pair<const char*, uint64_t>{"input_layernorm.weight", 1024},
                                        {"post_attention_layernorm.weight", 1024},
                                        {"self_attn.q_norm.weight", 128},
                                        {"self_attn.k_norm.weight", 128}})
        r.push_back({pre + name, pre + name, "", PIH_AMD_QWEN_INT4_BF16_NORM_V1, width * 2, 0, 0, 1, width});
    }
    r.push_back({"model.norm.weight", "model.norm.weight", "", PIH_AMD_QWEN_INT4_BF16_NORM_V1, 2048, 0, 0, 1, 1024});
    std::sort(r.begin(), r.end(), [](const Rec& a, const Rec& b) { return a.identity < b.identity; });
    uint64_t next = kMeta;
    size_t payloads = 0;
    for (size_t i = 0; i < r.size(); ++i) {
      if (i && r[i - 1].identity == r[i].identity) return;
      if (r[i].kind == PIH_AMD_QWEN_INT4_ALIAS_V1) continue;
      r[i].extent = (r[i].logical + kAlign - 1) / kAlign * kAlign;
      r[i].offset = next;
      next += r[i].extent;
      L.logical_total += r[i].logical;
      ++payloads;
    }
    L.padded = next - kMeta;
    L.ok = r.size() == PIH_AMD_QWEN_INT4_RECORD_COUNT_V1 && payloads == 506 && L.logical_total == 538378240ull &&
           L.padded == PIH_AMD_QWEN_INT4_DATA_BYTES_V1 && next == kFileBytes;
  });
  return L;
}

pih_status_v1 Fail(uint32_t code, const char* m) { return ToAbi(St{code, m}); }
pih_status_v1 Bad(const char* m) { return Fail(PIH_STATUS_INVALID_ARGUMENT_V1, m); }
pih_status_v1 Precond(const char* m) { return Fail(PIH_STATUS_FAILED_PRECONDITION_V1, m); }

uint64_t le(const uint8_t* p, int n) {
  uint64_t v = 0;
  for (int i = n - 1; i >= 0; --i) v = v << 8 | p[i];
  return v;
}
bool zero32(const uint8_t* p) {
  for (int i = 0; i < 32; ++i)
    if (p[i]) return false;
  return true;
}

struct Parsed {
  std::vector<std::array<uint8_t, 32>> digest;  // per layout record (alias: zero)
  uint32_t encoded = 0;
};

// QwenInt4ArtifactMetadata::ParseAndVerify (qwen3_int4_artifact_metadata.cpp:145-196)
pih_status_v1 ParseMetadata(const uint8_t* m, const Layout& L, Parsed& out) {
  if (memcmp(m, "XINGW4A1", 8) != 0) return Bad("Qwen INT4 metadata magic mismatch");
  const uint32_t version = (uint32_t)le(m + 8, 4), encoded = (uint32_t)le(m + 12, 4);
  const uint32_t count = (uint32_t)le(m + 16, 4), reserved = (uint32_t)le(m + 20, 4);
  if (version != 1 || reserved != 0 || encoded < kHeaderBytes || encoded > kMeta || count != L.recs.size())
    return Bad("Qwen INT4 metadata header mismatch");
  for (uint64_t i = encoded; i < kMeta; ++i)
    if (m[i]) return Bad("Qwen INT4 metadata tail is not zero");
  {
    Sha256 s;
    s.update(m, kChecksumOffset);
    const uint8_t zeros[32] = {};
    s.update(zeros, 32);
    s.update(m + kChecksumOffset + 32, encoded - kChecksumOffset - 32);
    if (s.finish() != *reinterpret_cast<const std::array<uint8_t, 32>*>(m + kChecksumOffset))
      return Precond("Qwen INT4 metadata checksum mismatch");
  }
  const uint32_t flen = (uint32_t)le(m + 152, 2), llen = (uint32_t)le(m + 154, 2);
  if (le(m + 156, 4) != 0) return Bad("Qwen INT4 metadata roots truncated");
  uint64_t pos = kHeaderBytes;
  auto str = [&](uint32_t n, std::string& s) -> bool {
    if (n > encoded - pos) return false;
    s.assign(reinterpret_cast<const char*>(m + pos), n);
    pos += n;
    return true;
  };
  std::string format, layout_id;
  if (!str(flen, format) || !str(llen, layout_id) || format != kFormatId || layout_id != kLayoutId)
    return Bad("Qwen INT4 metadata format mismatch");
  out.digest.assign(count, {});
  for (uint32_t i = 0; i < count; ++i) {
    if (encoded - pos < 64) return Bad("Qwen INT4 metadata record truncated");
    const uint8_t* r = m + pos;
    const uint8_t kind = r[0], zero = r[1];
    const uint32_t il = (uint32_t)le(r + 2, 2), sl = (uint32_t)le(r + 4, 2), al = (uint32_t)le(r + 6, 2);
    const uint64_t logical = le(r + 8, 8), offset = le(r + 16, 8), extent = le(r + 24, 8);
    memcpy(out.digest[i].data(), r + 32, 32);
    pos += 64;
    if (zero != 0) return Bad("Qwen INT4 metadata record truncated");
    std::string id, src, alias;
    if (!str(il, id) || !str(sl, src) || !str(al, alias)) return Bad("Qwen INT4 metadata record string truncated");
    const Rec& e = L.recs[i];
    const bool alias_rec = e.kind == PIH_AMD_QWEN_INT4_ALIAS_V1;
    if (id != e.identity || kind != e.kind || src != e.source || alias != e.alias || logical != e.logical ||
        offset != e.offset || extent != e.extent || alias_rec != zero32(r + 32))
      return Precond("Qwen INT4 metadata record mismatch");
  }
  if (pos != encoded) return Bad("Qwen INT4 metadata has trailing encoded bytes");
  for (int j = 0; j < 3; ++j)
    if (zero32(m + 24 + 32 * j)) return Precond("Qwen INT4 metadata root is empty");
  out.encoded = encoded;
  return ToAbi(Ok());
}

// verify_canonical_extent_file (src/core/canonical_extent_verifier.cpp:11-57)
// over the payload records, largest first on a small thread pool
pih_status_v1 VerifyPayloads(const uint8_t* file, const Layout& L, const Parsed& P) {
  std::vector<size_t> order;
  for (size_t i = 0; i < L.recs.size(); ++i)
    if (L.recs[i].kind != PIH_AMD_QWEN_INT4_ALIAS_V1) order.push_back(i);
  std::sort(order.begin(), order.end(), [&](size_t a, size_t b) { return L.recs[a].logical > L.recs[b].logical; });
  std::atomic<size_t> next{0};
  std::atomic<int> bad{0};  // 1 digest mismatch, 2 padding
  auto work = [&] {
    for (size_t j; !bad.load(std::memory_order_relaxed) && (j = next.fetch_add(1)) < order.size();) {
      const Rec& r = L.recs[order[j]];
      if (Sha256::of(file + r.offset, r.logical) != P.digest[order[j]]) {
        bad.store(1);
        return;
      }
      for (uint64_t b = r.offset + r.logical; b < r.offset + r.extent; ++b)
        if (file[b]) {
          bad.store(2);
          return;
        }
    }
  };
  const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  std::vector<std::thread> pool;
  try {
    for (unsigned t = 1; t < hw; ++t) pool.emplace_back(work);
  } catch (...) {
    // fewer threads than asked for: the records are shared out by the
    // atomic counter, so the ones started (and this one) cover them all
  }
  work();
  for (auto& t : pool) t.join();
  if (bad.load() == 1) return Precond("canonical payload checksum mismatch");
  if (bad.load() == 2) return Precond("canonical extent padding is not zero");
  return ToAbi(Ok());
}

constexpr uint64_t kBundlePacked = 4194304, kBundleScales = 262144;
constexpr uint64_t kBundle = PIH_AMD_EXPERT_BUNDLE_BYTES_V1;
static_assert(3 * (kBundlePacked + kBundleScales) == kBundle, "bundle segments");

}  // namespace
}  // namespace pih_amd

using namespace pih_amd;

extern "C" {

__attribute__((visibility("default"))) pih_status_v1 pih_amd_qwen_int4_artifact_verify_v1(
    const uint8_t* file, uint64_t file_bytes, uint32_t flags, pih_amd_qwen_int4_artifact_info_v1* info) {
  try {
    if (!file || !info || info->struct_size != sizeof(*info) || info->abi_version != PIH_AMD_ARTIFACTS_ABI_VERSION_V1 ||
        (flags & ~PIH_AMD_VERIFY_PAYLOADS_V1))
      return Bad("qwen_int4_verify_request_invalid");
    if (file_bytes != kFileBytes) return Precond("Qwen INT4 artifact file length mismatch");
    const Layout& L = OfficialLayout();
    if (!L.ok) return Fail(PIH_STATUS_INTERNAL_V1, "Qwen INT4 canonical artifact totals drifted");
    Parsed P;
    pih_status_v1 st = ParseMetadata(file, L, P);
    if (st.code != PIH_STATUS_OK_V1) return st;
    if (flags & PIH_AMD_VERIFY_PAYLOADS_V1) {
      st = VerifyPayloads(file, L, P);
      if (st.code != PIH_STATUS_OK_V1) return st;
    }
    info->record_count = (uint32_t)L.recs.size();
    info->payload_record_count = 506;
    info->file_bytes = kFileBytes;
    info->metadata_bytes = kMeta;
    info->padded_data_bytes = L.padded;
    info->logical_payload_bytes = L.logical_total;
    info->encoded_metadata_bytes = P.encoded;
    memcpy(info->source_artifact_root, file + 24, 32);
    memcpy(info->source_binding_root, file + 56, 32);
    memcpy(info->disposition_root, file + 88, 32);
    return ToAbi(Ok());
  } catch (...) {
    return Fail(PIH_STATUS_INTERNAL_V1, "qwen_int4_verify_failed");
  }
}

__attribute__((visibility("default"))) pih_status_v1 pih_amd_qwen_int4_artifact_record_v1(
    const char* identity, pih_amd_artifact_record_v1* out) {
  try {
    if (!identity || !out || out->struct_size != sizeof(*out) || out->abi_version != PIH_AMD_ARTIFACTS_ABI_VERSION_V1)
      return Bad("qwen_int4_record_request_invalid");
    const Layout& L = OfficialLayout();
    if (!L.ok) return Fail(PIH_STATUS_INTERNAL_V1, "Qwen INT4 canonical artifact totals drifted");
    const std::string id(identity);
    auto it = std::lower_bound(L.recs.begin(), L.recs.end(), id,
                               [](const Rec& r, const std::string& k) { return r.identity < k; });
    if (it == L.recs.end() || it->identity != id) return Bad("qwen_int4_record_unknown");
    const Rec* data = &*it;
    if (it->kind == PIH_AMD_QWEN_INT4_ALIAS_V1) {
      auto owner = std::lower_bound(L.recs.begin(), L.recs.end(), it->alias,
                                    [](const Rec& r, const std::string& k) { return r.identity < k; });
      data = &*owner;
    }
    out->kind = it->kind;
    out->file_offset = it->offset;
    out->logical_bytes = it->logical;
    out->extent_bytes = it->extent;
    out->device_offset = data->offset - kMeta;
    out->rows = it->rows;
    out->columns = it->cols;
    return ToAbi(Ok());
  } catch (...) {
    return Fail(PIH_STATUS_INTERNAL_V1, "qwen_int4_record_failed");
  }
}

__attribute__((visibility("default"))) pih_status_v1 pih_amd_qwen_int4_artifact_upload_v1(
    const uint8_t* file, uint64_t file_bytes, uintptr_t device_dst, uint64_t dst_bytes, uintptr_t stream) {
  if (!file || !device_dst || !stream) return Bad("qwen_int4_upload_request_invalid");
  if (file_bytes != kFileBytes || memcmp(file, "XINGW4A1", 8) != 0)
    return Precond("Qwen INT4 artifact file length mismatch");
  if (dst_bytes < PIH_AMD_QWEN_INT4_DATA_BYTES_V1) return Bad("qwen_int4_upload_destination_too_small");
  hipStream_t s = AsStream(stream);
  if (hipMemcpyAsync(reinterpret_cast<void*>(device_dst), file + kMeta, PIH_AMD_QWEN_INT4_DATA_BYTES_V1,
                     hipMemcpyHostToDevice, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return Fail(PIH_STATUS_INTERNAL_V1, "qwen_int4_upload_copy_failed");
  return ToAbi(Ok());
}

__attribute__((visibility("default"))) pih_status_v1 pih_amd_deepseek_expert_bundle_bind_v1(
    uintptr_t base, pih_amd_expert_bundle_view_v1* out) {
  if (!out || out->struct_size != sizeof(*out) || out->abi_version != PIH_AMD_ARTIFACTS_ABI_VERSION_V1)
    return Bad("expert_bundle_request_invalid");
  if (base == 0 || base % PIH_AMD_EXPERT_BUNDLE_ALIGNMENT_V1 != 0 || base > UINTPTR_MAX - kBundle)
    return Bad("DeepSeek canonical expert bundle base is invalid");
  out->w1_packed = base;
  out->w1_scales = base + kBundlePacked;
  out->w2_packed = out->w1_scales + kBundleScales;
  out->w2_scales = out->w2_packed + kBundlePacked;
  out->w3_packed = out->w2_scales + kBundleScales;
  out->w3_scales = out->w3_packed + kBundlePacked;
  out->packed_bytes = kBundlePacked;
  out->scale_bytes = kBundleScales;
  return ToAbi(Ok());
}

__attribute__((visibility("default"))) pih_status_v1 pih_amd_deepseek_bundles_to_moe_v1(
    const pih_amd_bundles_to_moe_v1* r) {
  if (!r || r->struct_size != sizeof(*r) || r->abi_version != PIH_AMD_ARTIFACTS_ABI_VERSION_V1)
    return Bad("bundles_to_moe_request_invalid");
  if (!r->bundle_bases || !r->w13_packed || !r->w13_scales || !r->w2_packed || !r->w2_scales || !r->stream ||
      r->expert_count == 0)
    return Bad("bundles_to_moe_request_invalid");
  hipStream_t s = AsStream(r->stream);
  auto copy = [&](uintptr_t dst, uintptr_t src, uint64_t n) {
    return hipMemcpyAsync(reinterpret_cast<void*>(dst), reinterpret_cast<const void*>(src), n,
                          hipMemcpyDeviceToDevice, s) == hipSuccess;
  };
  for (uint32_t e = 0; e < r->expert_count; ++e) {
    pih_amd_expert_bundle_view_v1 v{};
    v.struct_size = sizeof(v);
    v.abi_version = PIH_AMD_ARTIFACTS_ABI_VERSION_V1;
    const pih_status_v1 st = pih_amd_deepseek_expert_bundle_bind_v1(r->bundle_bases[e], &v);
    if (st.code != PIH_STATUS_OK_V1) return st;
    const uint64_t e13p = (uint64_t)e * 2 * kBundlePacked, e13s = (uint64_t)e * 2 * kBundleScales;
    if (!copy(r->w13_packed + e13p, v.w1_packed, kBundlePacked) ||
        !copy(r->w13_packed + e13p + kBundlePacked, v.w3_packed, kBundlePacked) ||
        !copy(r->w13_scales + e13s, v.w1_scales, kBundleScales) ||
        !copy(r->w13_scales + e13s + kBundleScales, v.w3_scales, kBundleScales) ||
        !copy(r->w2_packed + (uint64_t)e * kBundlePacked, v.w2_packed, kBundlePacked) ||
        !copy(r->w2_scales + (uint64_t)e * kBundleScales, v.w2_scales, kBundleScales))
      return Fail(PIH_STATUS_INTERNAL_V1, "bundles_to_moe_copy_failed");
  }
  return ToAbi(Ok());
}

}  // extern "C"

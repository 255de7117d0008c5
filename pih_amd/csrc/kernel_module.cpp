// gfx950 kernel-module driver and the Qwen W4A16 launch plan
// (libpih_hip_kernel_module.so); declarations and the reference interfaces
// each entry replaces are in include/pih/backend/hip/kernel_module_v1.h and
// include/pih/contracts/qwen_int4_plan_gfx950_v1.h.
//
// Verification reads three things, none of which needs a device:
//   * the manifest beside the code object: a JSON object with exactly the
//     fields schema, target, producer_toolchain, producer_flags_sha256,
//     code_object_sha256 and code_object_bytes (string or unsigned integer
//     values, no nesting), checked like the reference's cubin manifest;
//   * the image: size and SHA-256 against the manifest, an AMDGPU ELF64;
//   * the image's AMDGPU metadata note (NT_AMDGPU_METADATA, a MessagePack
//     map): for each kernel its name, kernarg segment size and argument
//     list, of which the arguments whose value kind is not "hidden_*" are
//     the explicit ones a packet carries.  This is the layout the
//     reference obtains from cuFuncGetParamCount / cuFuncGetParamInfo.
// The device side is hipModuleLoadData / hipModuleGetFunction /
// hipModuleLaunchKernel with the packet as HIP_LAUNCH_PARAM_BUFFER_POINTER.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <cstdio>
#include <map>
#include <memory>
#include <new>
#include <set>
#include <string>
#include <vector>

#include "host_common.hpp"
#include "pih/backend/hip/kernel_module_v1.h"
#include "pih/plugin_sdk/kernel_pack.h"
#include "pih/contracts/qwen_int4_plan_gfx950_v1.h"
#include "sha256.hpp"

namespace pih_amd {

// one resolved entrypoint of a loaded module
struct Function {
  std::string symbol, logical_id, parameter_abi;
  uint32_t packet_bytes = 0;
  hipFunction_t handle = nullptr;
};

namespace {

constexpr uint64_t kMaxManifestBytes = 4096, kMaxImageBytes = 64ull << 20;
constexpr uint32_t kMaxParameters = 256, kMaxParameterBytes = 32764;

// ------------------------------------------------------------ files
bool ReadFile(const char* path, uint64_t limit, std::vector<uint8_t>& out) {
  FILE* f = fopen(path, "rb");
  if (!f) return false;
  out.clear();
  uint8_t buf[65536];
  size_t got;
  bool ok = true;
  while ((got = fread(buf, 1, sizeof(buf), f)) > 0) {
    if (out.size() + got > limit) {
      ok = false;
      break;
    }
    out.insert(out.end(), buf, buf + got);
  }
  if (ferror(f)) ok = false;
  fclose(f);
  return ok;
}

// ------------------------------------------------------- manifest JSON
// A flat JSON object of string / unsigned integer values.
struct Flat {
  std::map<std::string, std::string> str;
  std::map<std::string, uint64_t> num;
  std::set<std::string> keys;
};

class JsonReader {
 public:
  JsonReader(const std::vector<uint8_t>& t) : p_(t.data()), e_(t.data() + t.size()) {}
  bool object(Flat& out) {
    ws();
    if (!take('{')) return false;
    ws();
    if (take('}')) return end();
    for (;;) {
      std::string key;
      ws();
      if (!string(key) || out.keys.count(key)) return false;  // duplicate keys are rejected
      out.keys.insert(key);
      ws();
      if (!take(':')) return false;
      ws();
      if (p_ < e_ && *p_ == '"') {
        std::string v;
        if (!string(v)) return false;
        out.str[key] = v;
      } else {
        uint64_t v = 0;
        if (!number(v)) return false;
        out.num[key] = v;
      }
      ws();
      if (take('}')) return end();
      if (!take(',')) return false;
    }
  }

 private:
  void ws() {
    while (p_ < e_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
  }
  bool take(char c) {
    if (p_ < e_ && *p_ == (uint8_t)c) {
      ++p_;
      return true;
    }
    return false;
  }
  bool end() {
    ws();
    return p_ == e_;
  }
  // printable ASCII strings with the escapes \" \\ \/ only
  bool string(std::string& s) {
    if (!take('"')) return false;
    while (p_ < e_ && *p_ != '"') {
      uint8_t c = *p_++;
      if (c < 0x20 || c > 0x7e) return false;
      if (c == '\\') {
        if (p_ >= e_) return false;
        c = *p_++;
        if (c != '"' && c != '\\' && c != '/') return false;
      }
      s.push_back((char)c);
    }
    return take('"');
  }
  bool number(uint64_t& v) {
    const uint8_t* start = p_;
    v = 0;
    while (p_ < e_ && *p_ >= '0' && *p_ <= '9') {
      if (v > (UINT64_MAX - 9) / 10) return false;
      v = v * 10 + (*p_++ - '0');
    }
    if (p_ == start || (p_ - start > 1 && *start == '0')) return false;
    return true;
  }
  const uint8_t* p_;
  const uint8_t* e_;
};

bool IsHex64(const std::string& s) {
  return s.size() == 64 && std::all_of(s.begin(), s.end(), [](char c) { return (c >= '0' && c <= '9') || (c >= 'a' && c <= 'f'); });
}

// --------------------------------------------------------- MessagePack
// A bounded reader of the subset the AMDGPU metadata uses (maps, arrays,
// strings, integers, booleans, nil, binary, floats); values are kept as a
// small tree.
struct MsgValue {
  enum Kind { kNil, kBool, kInt, kStr, kArr, kMap, kOther } kind = kNil;
  int64_t i = 0;
  std::string s;
  std::vector<MsgValue> items;                        // array
  std::vector<std::pair<MsgValue, MsgValue>> pairs;  // map
  const MsgValue* get(const char* key) const {
    for (const auto& kv : pairs)
      if (kv.first.kind == kStr && kv.first.s == key) return &kv.second;
    return nullptr;
  }
};

class MsgReader {
 public:
  MsgReader(const uint8_t* p, size_t n) : p_(p), e_(p + n) {}
  bool read(MsgValue& v, int depth = 0) {
    if (depth > 16 || p_ >= e_) return false;
    const uint8_t c = *p_++;
    if (c <= 0x7f) return integer(v, c);
    if (c >= 0xe0) return integer(v, (int8_t)c);
    if ((c & 0xf0) == 0x80) return map(v, c & 0x0f, depth);
    if ((c & 0xf0) == 0x90) return array(v, c & 0x0f, depth);
    if ((c & 0xe0) == 0xa0) return str(v, c & 0x1f);
    uint64_t n = 0;
    switch (c) {
      case 0xc0: v.kind = MsgValue::kNil; return true;
      case 0xc2: case 0xc3: v.kind = MsgValue::kBool; v.i = c == 0xc3; return true;
      case 0xcc: return uint(1, n) && integer(v, (int64_t)n);
      case 0xcd: return uint(2, n) && integer(v, (int64_t)n);
      case 0xce: return uint(4, n) && integer(v, (int64_t)n);
      case 0xcf: return uint(8, n) && n <= (uint64_t)INT64_MAX && integer(v, (int64_t)n);
      case 0xd0: return uint(1, n) && integer(v, (int8_t)n);
      case 0xd1: return uint(2, n) && integer(v, (int16_t)n);
      case 0xd2: return uint(4, n) && integer(v, (int32_t)n);
      case 0xd3: return uint(8, n) && integer(v, (int64_t)n);
      case 0xca: return skip(4, v);
      case 0xcb: return skip(8, v);
      case 0xd9: return uint(1, n) && str(v, n);
      case 0xda: return uint(2, n) && str(v, n);
      case 0xdb: return uint(4, n) && str(v, n);
      case 0xc4: return uint(1, n) && skip(n, v);
      case 0xc5: return uint(2, n) && skip(n, v);
      case 0xc6: return uint(4, n) && skip(n, v);
      case 0xdc: return uint(2, n) && array(v, n, depth);
      case 0xdd: return uint(4, n) && array(v, n, depth);
      case 0xde: return uint(2, n) && map(v, n, depth);
      case 0xdf: return uint(4, n) && map(v, n, depth);
      default: return false;
    }
  }

 private:
  bool uint(int bytes, uint64_t& n) {
    if ((size_t)(e_ - p_) < (size_t)bytes) return false;
    n = 0;
    for (int b = 0; b < bytes; ++b) n = n << 8 | *p_++;
    return true;
  }
  bool integer(MsgValue& v, int64_t x) {
    v.kind = MsgValue::kInt;
    v.i = x;
    return true;
  }
  bool str(MsgValue& v, uint64_t n) {
    if ((uint64_t)(e_ - p_) < n) return false;
    v.kind = MsgValue::kStr;
    v.s.assign(reinterpret_cast<const char*>(p_), n);
    p_ += n;
    return true;
  }
  bool skip(uint64_t n, MsgValue& v) {
    if ((uint64_t)(e_ - p_) < n) return false;
    p_ += n;
    v.kind = MsgValue::kOther;
    return true;
  }
  bool array(MsgValue& v, uint64_t n, int depth) {
    if (n > (uint64_t)(e_ - p_)) return false;  // every element takes at least one byte
    v.kind = MsgValue::kArr;
    v.items.resize(n);
    for (auto& it : v.items)
      if (!read(it, depth + 1)) return false;
    return true;
  }
  bool map(MsgValue& v, uint64_t n, int depth) {
    if (2 * n > (uint64_t)(e_ - p_)) return false;
    v.kind = MsgValue::kMap;
    v.pairs.resize(n);
    for (auto& kv : v.pairs)
      if (!read(kv.first, depth + 1) || !read(kv.second, depth + 1)) return false;
    return true;
  }
  const uint8_t* p_;
  const uint8_t* e_;
};

// ------------------------------------------------------------- ELF note
struct KernelArgs {
  uint32_t kernarg_bytes = 0;
  std::vector<std::pair<uint32_t, uint32_t>> explicit_args;  // (offset, size)
};

template <typename T>
bool ReadAt(const std::vector<uint8_t>& b, uint64_t off, T& v) {
  if (off > b.size() || b.size() - off < sizeof(T)) return false;
  memcpy(&v, b.data() + off, sizeof(T));
  return true;
}

St ParseKernels(const std::vector<uint8_t>& img, std::map<std::string, KernelArgs>& out) {
  // ELF64 little-endian AMDGPU (e_machine 224)
  if (img.size() < 64 || memcmp(img.data(), "\x7f" "ELF", 4) != 0 || img[4] != 2 || img[5] != 1)
    return Invalid("code_object_not_elf64");
  uint16_t machine = 0, shentsize = 0, shnum = 0;
  uint64_t shoff = 0;
  if (!ReadAt(img, 18, machine) || !ReadAt(img, 40, shoff) || !ReadAt(img, 58, shentsize) ||
      !ReadAt(img, 60, shnum))
    return Invalid("code_object_elf_header_truncated");
  if (machine != 224) return Invalid("code_object_not_amdgpu");
  if (shentsize != 64) return Invalid("code_object_elf_section_size");
  bool found = false;
  for (uint32_t i = 0; i < shnum; ++i) {
    const uint64_t sh = shoff + (uint64_t)i * 64;
    uint32_t type = 0;
    uint64_t off = 0, size = 0;
    if (!ReadAt(img, sh + 4, type) || !ReadAt(img, sh + 24, off) || !ReadAt(img, sh + 32, size))
      return Invalid("code_object_elf_sections_truncated");
    if (type != 7) continue;  // SHT_NOTE
    if (off > img.size() || img.size() - off < size) return Invalid("code_object_note_out_of_range");
    for (uint64_t q = off; q + 12 <= off + size;) {
      uint32_t namesz = 0, descsz = 0, ntype = 0;
      ReadAt(img, q, namesz);
      ReadAt(img, q + 4, descsz);
      ReadAt(img, q + 8, ntype);
      const uint64_t name_at = q + 12, desc_at = name_at + ((namesz + 3ull) & ~3ull);
      const uint64_t next = desc_at + ((descsz + 3ull) & ~3ull);
      if (next > off + size) return Invalid("code_object_note_truncated");
      if (ntype == 32 && namesz == 7 && memcmp(img.data() + name_at, "AMDGPU", 7) == 0) {
        MsgValue root;
        MsgReader r(img.data() + desc_at, descsz);
        if (!r.read(root) || root.kind != MsgValue::kMap) return Invalid("code_object_metadata_unreadable");
        const MsgValue* kernels = root.get("amdhsa.kernels");
        if (!kernels || kernels->kind != MsgValue::kArr) return Invalid("code_object_metadata_no_kernels");
        for (const MsgValue& k : kernels->items) {
          const MsgValue* name = k.get(".name");
          const MsgValue* seg = k.get(".kernarg_segment_size");
          const MsgValue* args = k.get(".args");
          if (!name || name->kind != MsgValue::kStr || !seg || seg->kind != MsgValue::kInt || seg->i < 0)
            return Invalid("code_object_metadata_kernel_malformed");
          KernelArgs ka;
          ka.kernarg_bytes = (uint32_t)seg->i;
          if (args) {
            if (args->kind != MsgValue::kArr) return Invalid("code_object_metadata_args_malformed");
            for (const MsgValue& a : args->items) {
              const MsgValue* o = a.get(".offset");
              const MsgValue* s = a.get(".size");
              const MsgValue* vk = a.get(".value_kind");
              if (!o || !s || !vk || o->kind != MsgValue::kInt || s->kind != MsgValue::kInt ||
                  vk->kind != MsgValue::kStr || o->i < 0 || s->i < 0)
                return Invalid("code_object_metadata_args_malformed");
              if (vk->s.rfind("hidden_", 0) == 0) continue;
              ka.explicit_args.emplace_back((uint32_t)o->i, (uint32_t)s->i);
            }
          }
          if (out.count(name->s)) return Invalid("code_object_metadata_duplicate_kernel");
          out[name->s] = std::move(ka);
        }
        found = true;
      }
      q = next;
    }
  }
  return found ? Ok() : Invalid("code_object_metadata_note_missing");
}

// ---------------------------------------------------------- verification
uint32_t WireSize(uint32_t t) {
  switch (t) {
    case PIH_HIP_WIRE_U8_V1: return 1;
    case PIH_HIP_WIRE_U16_V1: case PIH_HIP_WIRE_F16_BITS_V1: case PIH_HIP_WIRE_BF16_BITS_V1: return 2;
    case PIH_HIP_WIRE_U32_V1: case PIH_HIP_WIRE_I32_V1: case PIH_HIP_WIRE_F32_V1: return 4;
    case PIH_HIP_WIRE_U64_V1: case PIH_HIP_WIRE_I64_V1: case PIH_HIP_WIRE_F64_V1:
    case PIH_HIP_WIRE_DEVICE_POINTER_U64_V1: return 8;
    default: return 0;
  }
}

bool CString(const char* s, size_t max, std::string& out) {
  if (!s) return false;
  const size_t n = strnlen(s, max + 1);
  if (n == 0 || n > max) return false;
  out.assign(s, n);
  return true;
}

St Verify(const char* path, const pih_hip_kernel_signature_v1* sigs, uint32_t count, std::vector<uint8_t>& image,
          std::vector<Function>& fns) {
  if (!path || !sigs || count == 0 || count > PIH_HIP_KERNEL_MODULE_MAX_ENTRYPOINTS_V1)
    return Invalid("kernel_module_request_invalid");
  const std::string image_path(path), manifest_path = image_path + ".json";
  std::vector<uint8_t> manifest;
  if (!ReadFile(manifest_path.c_str(), kMaxManifestBytes, manifest)) return Invalid("code_object_manifest_unreadable");
  Flat m;
  if (!JsonReader(manifest).object(m)) return Invalid("code_object_manifest_not_a_flat_json_object");
  static const char* kStr[] = {"schema", "target", "producer_toolchain", "producer_flags_sha256", "code_object_sha256"};
  if (m.keys.size() != 6 || m.num.size() != 1 || !m.num.count("code_object_bytes"))
    return Invalid("code_object_manifest_fields");
  for (const char* k : kStr)
    if (!m.str.count(k) || m.str[k].empty() || m.str[k].size() > 128) return Invalid("code_object_manifest_fields");
  if (m.str["schema"] != "pih.code_object_artifact.v1") return Invalid("code_object_manifest_schema");
  if (m.str["target"] != "gfx950") return Invalid("code_object_manifest_target");
  if (!IsHex64(m.str["producer_flags_sha256"]) || !IsHex64(m.str["code_object_sha256"]))
    return Invalid("code_object_manifest_digest_format");
  const uint64_t bytes = m.num["code_object_bytes"];
  if (bytes < 64 || bytes > kMaxImageBytes) return Invalid("code_object_manifest_size");
  if (!ReadFile(path, kMaxImageBytes, image)) return Invalid("code_object_unreadable");
  if (image.size() != bytes) return Invalid("code_object_size_differs_from_manifest");
  const std::string digest = Sha256Hex(Sha256::of(image.data(), image.size()));
  if (digest != m.str["code_object_sha256"]) return Invalid("code_object_digest_differs_from_manifest");
  std::map<std::string, KernelArgs> kernels;
  St s = ParseKernels(image, kernels);
  if (!s.ok()) return s;
  std::set<std::string> symbols, ids;
  fns.clear();
  for (uint32_t i = 0; i < count; ++i) {
    const pih_hip_kernel_signature_v1& g = sigs[i];
    if (g.struct_size != sizeof(g) || g.abi_version != PIH_HIP_KERNEL_MODULE_ABI_VERSION_V1)
      return Invalid("kernel_signature_header_invalid");
    Function f;
    std::string co;
    if (!CString(g.symbol, PIH_HIP_KERNEL_SYMBOL_MAX_BYTES_V1, f.symbol)) return Invalid("kernel_symbol_empty_or_oversized");
    if (!CString(g.logical_id, 128, f.logical_id)) return Invalid("kernel_logical_id_invalid");
    if (!CString(g.parameter_abi_sha256, 64, f.parameter_abi) || !IsHex64(f.parameter_abi))
      return Invalid("kernel_parameter_abi_digest_invalid");
    if (!CString(g.code_object_sha256, 64, co) || co != digest) return Invalid("kernel_signature_names_another_image");
    if (!symbols.insert(f.symbol).second) return Invalid("kernel_entrypoint_symbol_duplicated");
    if (!ids.insert(f.logical_id).second) return Invalid("kernel_logical_id_duplicated");
    if (g.parameter_count > kMaxParameters || (g.parameter_count && !g.parameters) ||
        g.total_parameter_bytes > kMaxParameterBytes)
      return Invalid("kernel_signature_parameters_invalid");
    const auto it = kernels.find(f.symbol);
    if (it == kernels.end()) return Invalid("kernel_symbol_not_in_code_object");
    const KernelArgs& ka = it->second;
    if (ka.explicit_args.size() != g.parameter_count) return Invalid("kernel_parameter_count_differs_from_signature");
    uint32_t end = 0;
    for (uint32_t j = 0; j < g.parameter_count; ++j) {
      const uint32_t size = WireSize(g.parameters[j].wire_type);
      if (!size || g.parameters[j].offset % size) return Invalid("kernel_signature_parameter_invalid");
      if (ka.explicit_args[j].first != g.parameters[j].offset || ka.explicit_args[j].second != size)
        return Invalid("kernel_parameter_layout_differs_from_signature");
      end = std::max(end, g.parameters[j].offset + size);
    }
    if (end != g.total_parameter_bytes || g.total_parameter_bytes > ka.kernarg_bytes)
      return Invalid("kernel_parameter_bytes_differ_from_signature");
    f.packet_bytes = g.total_parameter_bytes;
    fns.push_back(std::move(f));
  }
  return Ok();
}

}  // namespace
}  // namespace pih_amd

struct pih_hip_kernel_module_v1 {
  int device = -1;
  hipModule_t module = nullptr;
  std::vector<uint8_t> image;  // the loaded bytes, kept for the module's lifetime
  std::vector<pih_amd::Function> functions;
};

namespace pih_amd {
namespace {

St CurrentGfx950(int& dev) {
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return Precondition("kernel_module_no_current_device");
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return Internal("kernel_module_device_query_failed");
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0 || (prop.gcnArchName[6] != '\0' && prop.gcnArchName[6] != ':'))
    return Precondition("kernel_module_device_is_not_gfx950");
  return Ok();
}

St Load(const char* path, const pih_hip_kernel_signature_v1* sigs, uint32_t count, pih_hip_kernel_module_v1** out) {
  if (!out) return Invalid("kernel_module_out_null");
  *out = nullptr;
  std::unique_ptr<pih_hip_kernel_module_v1> m(new pih_hip_kernel_module_v1());
  St s = Verify(path, sigs, count, m->image, m->functions);
  if (!s.ok()) return s;
  if (!(s = CurrentGfx950(m->device)).ok()) return s;
  if (!(s = RequireCleanLastError()).ok()) return s;
  if (hipModuleLoadData(&m->module, m->image.data()) != hipSuccess || !m->module) {
    (void)hipGetLastError();
    return Internal("hipModuleLoadData_failed");
  }
  for (Function& f : m->functions) {
    if (hipModuleGetFunction(&f.handle, m->module, f.symbol.c_str()) != hipSuccess || !f.handle) {
      (void)hipGetLastError();
      (void)hipModuleUnload(m->module);  // rollback: nothing stays loaded
      return Internal("hipModuleGetFunction_failed");
    }
  }
  *out = m.release();
  return Ok();
}

St Submit(const pih_hip_kernel_module_v1* m, uint32_t index, const pih_hip_launch_geometry_v1* g, uintptr_t stream,
          const pih_hip_kernel_arguments_v1* a) {
  if (!m || !g || !a) return Invalid("kernel_launch_request_null");
  if (g->struct_size != sizeof(*g) || a->struct_size != sizeof(*a) ||
      a->abi_version != PIH_HIP_KERNEL_MODULE_ABI_VERSION_V1)
    return Invalid("kernel_launch_request_header_invalid");
  if (index >= m->functions.size() || !m->functions[index].handle) return Invalid("kernel_function_index_invalid");
  if (!g->grid_x || !g->grid_y || !g->grid_z || !g->block_x || !g->block_y || !g->block_z)
    return Invalid("kernel_launch_dimensions_must_be_nonzero");
  if (g->grid_x > 0x7fffffffu || g->grid_y > 65535u || g->grid_z > 65535u || g->block_x > 1024u ||
      g->block_y > 1024u || g->block_z > 64u || (uint64_t)g->block_x * g->block_y * g->block_z > 1024u)
    return Invalid("kernel_launch_dimensions_exceed_bounds");
  if (g->dynamic_shared_bytes > 160u * 1024u) return Invalid("kernel_launch_shared_memory_exceeds_lds");
  if (stream == 0) return Invalid("verified_kernel_launch_forbids_default_stream");
  const Function& f = m->functions[index];
  std::string id, abi;
  if (!CString(a->logical_id, 128, id) || !CString(a->parameter_abi_sha256, 64, abi) || id != f.logical_id ||
      abi != f.parameter_abi)
    return Invalid("kernel_function_and_argument_packet_identities_differ");
  if (!a->packet || a->packet_bytes != f.packet_bytes) return Invalid("kernel_argument_packet_size_differs");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != m->device) return Precondition("current_device_differs_from_module_owner");
  St s = RequireCleanLastError();
  if (!s.ok()) return s;
  // the argument buffer is consumed when the launch is enqueued; a copy
  // (on the stack for packets up to 1 KiB) keeps the caller's bytes as they
  // were checked
  alignas(16) uint8_t small[1024];
  std::vector<uint8_t> large;
  uint8_t* packet = small;
  if (a->packet_bytes > sizeof(small)) {
    large.resize(a->packet_bytes);
    packet = large.data();
  }
  memcpy(packet, a->packet, a->packet_bytes);
  size_t size = a->packet_bytes;
  void* extra[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, packet, HIP_LAUNCH_PARAM_BUFFER_SIZE, &size,
                   HIP_LAUNCH_PARAM_END};
  const hipError_t e = hipModuleLaunchKernel(f.handle, g->grid_x, g->grid_y, g->grid_z, g->block_x, g->block_y,
                                             g->block_z, g->dynamic_shared_bytes, AsStream(stream), nullptr, extra);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return Internal("hipModuleLaunchKernel_failed");
  }
  return RequireCleanLastError();
}

// ----------------------------------------------------- Qwen W4A16 plan
// The compatibility descriptor is the reference's
// (plugins/model-qwen3/qwen3_int4_gemm_plan.cpp:13-20): its digest is the
// packet identity an unchanged model computes.
constexpr const char kCompatDescriptor[] =
    "pih.typed_kernel_params.v1|qwen.linear.w4a16.compatibility.v1|"
    "input:device_pointer_u64@0|packed_weight:device_pointer_u64@8|"
    "scales:device_pointer_u64@16|output:device_pointer_u64@24|error_flag:"
    "device_pointer_u64@32|m:u64@40|n:u64@48|k:u64@56|total:64|"
    "activation:bf16|weight:xing-w4a16-sym-g128-v1|scales:fp16|"
    "accumulator:fp32|output:bf16|layout:canonical-nk-low-nibble-k-v1|"
    "reduction:strict-increasing-k-v1";
constexpr const char kGfx950Descriptor[] =
    "pih.typed_kernel_params.v1|qwen.linear.w4a16.gfx950.v1|"
    "input:device_pointer_u64@0|packed_weight:device_pointer_u64@8|"
    "scales:device_pointer_u64@16|output:device_pointer_u64@24|error_flag:"
    "device_pointer_u64@32|m:u64@40|n:u64@48|k:u64@56|total:64|"
    "activation:bf16|weight:xing-w4a16-sym-g128-v1|scales:fp16|"
    "accumulator:fp32|output:bf16|layout:canonical-nk-low-nibble-k-v1|"
    "reduction:wave-split-k-groups-v1|geometry:n16-by-m16-blocks-v1";

struct Variant {
  const char* symbol;
  const char* logical_id;
  const char* descriptor;
};
const Variant kVariants[2] = {
    {"pih_qwen_w4a16_gemm_compat_v1", "qwen.linear.w4a16.compatibility.v1", kCompatDescriptor},
    {"pih_qwen_w4a16_gemm_gfx950_v1", "qwen.linear.w4a16.gfx950.v1", kGfx950Descriptor}};

const char* DescriptorDigest(uint32_t variant) {
  static const std::string digests[2] = {
      Sha256Hex(Sha256::of(reinterpret_cast<const uint8_t*>(kCompatDescriptor), sizeof(kCompatDescriptor) - 1)),
      Sha256Hex(Sha256::of(reinterpret_cast<const uint8_t*>(kGfx950Descriptor), sizeof(kGfx950Descriptor) - 1))};
  return digests[variant - 1].c_str();
}

St Plan(uint64_t m, uint64_t n, uint64_t k, uint32_t variant, pih_qwen_int4_gemm_plan_v1* p) {
  if (!p || p->struct_size != sizeof(*p)) return Invalid("qwen_int4_plan_header_invalid");
  if (variant != PIH_QWEN_INT4_VARIANT_COMPATIBILITY_V1 && variant != PIH_QWEN_INT4_VARIANT_GFX950_V1)
    return Invalid("qwen_int4_plan_variant_invalid");
  const bool compat = variant == PIH_QWEN_INT4_VARIANT_COMPATIBILITY_V1;
  if (m == 0 || m > PIH_QWEN_INT4_MAX_TOKENS_V1 || n == 0 || k == 0 || k % 128 || n % (compat ? 256 : 16) ||
      n > (1ull << 31) || k > (1ull << 31))
    return Invalid("qwen_int4_plan_predicate_mismatch");
  const uint32_t size = p->struct_size;
  memset(p, 0, sizeof(*p));
  p->struct_size = size;
  p->abi_version = PIH_HIP_KERNEL_MODULE_ABI_VERSION_V1;
  p->variant = variant;
  const Variant& v = kVariants[variant - 1];
  p->kernel_symbol = v.symbol;
  p->logical_id = v.logical_id;
  p->parameter_abi_sha256 = DescriptorDigest(variant);
  p->tokens = m;
  p->output_features = n;
  p->input_features = k;
  p->input_bytes = m * k * 2;
  p->packed_bytes = n * k / 2;
  p->scale_bytes = n * (k / 128) * 2;
  p->output_bytes = m * n * 2;
  pih_hip_launch_geometry_v1& g = p->geometry;
  g.struct_size = sizeof(g);
  g.grid_y = g.grid_z = g.block_y = g.block_z = 1;
  if (compat) {
    // the reference's geometry (qwen3_int4_gemm_plan.cpp:58-61)
    const uint64_t blocks = (m * n + 255) / 256;
    if (blocks > 0x7fffffffull) return Invalid("qwen_int4_plan_grid_overflow");
    g.grid_x = (uint32_t)blocks;
    g.block_x = 256;
  } else {
    // 16 W rows x 16 tokens per block; its waves split the 128-deep groups:
    // a decode grid (tens to hundreds of blocks) gives every wave one or
    // two groups, a prefill grid of >= 1024 blocks four waves per block
    const uint64_t groups = k / 128, row_blocks = n / 16, tok_blocks = (m + 15) / 16;
    const uint64_t blocks = row_blocks * tok_blocks;
    uint64_t waves = blocks >= 1024 ? 4 : std::min<uint64_t>(16, groups);
    waves = std::max<uint64_t>(1, std::min(waves, groups));
    g.grid_x = (uint32_t)row_blocks;
    g.grid_y = (uint32_t)tok_blocks;
    g.block_x = (uint32_t)(64 * waves);
  }
  return Ok();
}

St Signature(uint32_t variant, const char* code_object_sha256, pih_hip_kernel_parameter_v1* params,
             pih_hip_kernel_signature_v1* sig) {
  if (!params || !sig || !code_object_sha256) return Invalid("qwen_int4_signature_request_null");
  if (variant != PIH_QWEN_INT4_VARIANT_COMPATIBILITY_V1 && variant != PIH_QWEN_INT4_VARIANT_GFX950_V1)
    return Invalid("qwen_int4_plan_variant_invalid");
  // input, packed_weight, scales, output, error_flag (device pointers), m, n, k (u64)
  for (uint32_t j = 0; j < 8; ++j) {
    params[j].wire_type = j < 5 ? PIH_HIP_WIRE_DEVICE_POINTER_U64_V1 : PIH_HIP_WIRE_U64_V1;
    params[j].offset = 8 * j;
  }
  const Variant& v = kVariants[variant - 1];
  sig->struct_size = sizeof(*sig);
  sig->abi_version = PIH_HIP_KERNEL_MODULE_ABI_VERSION_V1;
  sig->symbol = v.symbol;
  sig->logical_id = v.logical_id;
  sig->code_object_sha256 = code_object_sha256;
  sig->parameter_abi_sha256 = DescriptorDigest(variant);
  sig->parameters = params;
  sig->parameter_count = 8;
  sig->total_parameter_bytes = 64;
  return Ok();
}

template <typename F>
pih_status_v1 Contained(F&& f) noexcept {
  try {
    return ToAbi(f());
  } catch (const std::bad_alloc&) {
    return ToAbi({PIH_STATUS_RESOURCE_EXHAUSTED_V1, "kernel_module_allocation_failed"});
  } catch (...) {
    return ToAbi(Internal("kernel_module_failed"));
  }
}

}  // namespace
}  // namespace pih_amd

extern "C" {

PIH_PLUGIN_EXPORT pih_status_v1 pih_hip_code_object_verify_v1(const char* code_object_path,
                                                              const pih_hip_kernel_signature_v1* signatures,
                                                              uint32_t signature_count) {
  return pih_amd::Contained([&] {
    std::vector<uint8_t> image;
    std::vector<pih_amd::Function> fns;
    return pih_amd::Verify(code_object_path, signatures, signature_count, image, fns);
  });
}

PIH_PLUGIN_EXPORT pih_status_v1 pih_hip_kernel_module_load_v1(const char* code_object_path,
                                                              const pih_hip_kernel_signature_v1* signatures,
                                                              uint32_t signature_count,
                                                              pih_hip_kernel_module_v1** module) {
  return pih_amd::Contained([&] { return pih_amd::Load(code_object_path, signatures, signature_count, module); });
}

PIH_PLUGIN_EXPORT pih_status_v1 pih_hip_kernel_module_find_v1(const pih_hip_kernel_module_v1* module,
                                                              const char* logical_id, uint32_t* function_index) {
  return pih_amd::Contained([&]() -> pih_amd::St {
    if (!module || !logical_id || !function_index) return pih_amd::Invalid("kernel_module_find_request_null");
    for (uint32_t i = 0; i < module->functions.size(); ++i)
      if (module->functions[i].logical_id == logical_id) {
        *function_index = i;
        return pih_amd::Ok();
      }
    return pih_amd::Invalid("kernel_logical_id_not_in_module");
  });
}

PIH_PLUGIN_EXPORT pih_status_v1 pih_hip_kernel_submit_v1(const pih_hip_kernel_module_v1* module,
                                                         uint32_t function_index,
                                                         const pih_hip_launch_geometry_v1* geometry, uintptr_t stream,
                                                         const pih_hip_kernel_arguments_v1* arguments) {
  return pih_amd::Contained([&] { return pih_amd::Submit(module, function_index, geometry, stream, arguments); });
}

PIH_PLUGIN_EXPORT pih_status_v1 pih_hip_kernel_module_unload_v1(pih_hip_kernel_module_v1* module) {
  return pih_amd::Contained([&]() -> pih_amd::St {
    if (!module) return pih_amd::Invalid("cannot_unload_a_null_module");
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev != module->device)
      return pih_amd::Precondition("current_device_differs_from_module_owner");
    const hipError_t e = module->module ? hipModuleUnload(module->module) : hipSuccess;
    delete module;
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return pih_amd::Internal("hipModuleUnload_failed");
    }
    return pih_amd::Ok();
  });
}

PIH_PLUGIN_EXPORT pih_status_v1 pih_qwen_int4_gemm_plan_create_v1(uint64_t tokens, uint64_t output_features,
                                                                  uint64_t input_features, uint32_t variant,
                                                                  pih_qwen_int4_gemm_plan_v1* plan) {
  return pih_amd::Contained([&] { return pih_amd::Plan(tokens, output_features, input_features, variant, plan); });
}

PIH_PLUGIN_EXPORT pih_status_v1 pih_qwen_int4_gemm_signature_v1(uint32_t variant, const char* code_object_sha256,
                                                                pih_hip_kernel_parameter_v1* parameters,
                                                                pih_hip_kernel_signature_v1* signature) {
  return pih_amd::Contained([&] { return pih_amd::Signature(variant, code_object_sha256, parameters, signature); });
}

}  // extern "C"

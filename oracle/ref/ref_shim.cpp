// ref_shim.cpp — extern "C" access to the reference's own CPU oracles.
// TEST INFRASTRUCTURE ONLY: linked with the reference's oracle sources,
// compiled where they lie under the reference checkout (see Makefile in this
// directory), into oracle/_ref/libpih_ref.so.  Used to validate the C
// restatement in oracle/pih_oracle.c; never loaded by product code.
//
// Return convention: 0 OK, 1 the reference returned a non-OK status.
#include <array>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <span>
#include <vector>

#include "pih/core/bfloat16.h"
#include "pih/core/float16.h"
#include "pih/model/deepseek_expert_accumulator_oracle.h"
#include "pih/model/deepseek_expert_subwave_plan.h"
#include "pih/model/deepseek_expert_swiglu_oracle.h"
#include "pih/model/deepseek_fp4_gemm_oracle.h"
#include "pih/model/deepseek_fp8_activation_codec.h"
#include "pih/model/deepseek_fp8_gemm_oracle.h"
#include "pih/model/deepseek_learned_router.h"
#include "pih/model/deepseek_mxfp4_codec.h"
#include "pih/model/deepseek_routed_expert_oracle.h"
#include "pih/model/qwen3_cpu_oracle.h"
#include "pih/model/qwen3_int4_artifact_layout.h"
#include "pih/model/qwen3_int4_artifact_metadata.h"
#include "qwen3_int4_reference_quantizer.h"
#include "weight_dequantize.h"
#include "weight_expert_convert.h"

using namespace pih;

namespace {
std::span<const std::byte> bytes(const std::uint8_t* p, std::size_t n) {
  return {reinterpret_cast<const std::byte*>(p), n};
}
DeepSeekFp8Activation activation(const std::uint8_t* codes,
                                 const std::uint8_t* scales,
                                 std::uint32_t tokens, std::uint32_t k) {
  DeepSeekFp8Activation a;
  a.token_count = tokens;
  a.logical_k = k;
  a.e4m3_bits.assign(codes, codes + static_cast<std::size_t>(tokens) * k);
  a.scale_bits.assign(scales, scales + static_cast<std::size_t>(tokens) * (k / 128U));
  return a;
}
}  // namespace

extern "C" {

uint16_t pr_bf16_from_f32(float v) { return BFloat16::FromFloat(v).bits; }
uint16_t pr_f16_from_f32(float v) { return Float16::FromFloat(v).bits; }
float pr_f16_to_f32(uint16_t b) { return Float16{b}.to_float(); }

int pr_e4m3_decode(uint8_t bits, float* out) {
  auto r = DeepSeekFp8ActivationCodec::DecodeE4m3Fn(bits);
  if (!r.ok()) return 1;
  *out = *r;
  return 0;
}

int pr_e4m3_encode(float v, uint8_t* out) {
  auto r = DeepSeekFp8ActivationCodec::EncodeE4m3Fn(v);
  if (!r.ok()) return 1;
  *out = *r;
  return 0;
}

int pr_fp8_quant(const float* in, uint32_t tokens, uint32_t k, uint8_t* codes,
                 uint8_t* scales) {
  auto r = DeepSeekFp8ActivationCodec::Quantize(
      std::span<const float>(in, static_cast<std::size_t>(tokens) * k), tokens, k);
  if (!r.ok()) return 1;
  std::memcpy(codes, r->e4m3_bits.data(), r->e4m3_bits.size());
  std::memcpy(scales, r->scale_bits.data(), r->scale_bits.size());
  return 0;
}

int pr_fp8_gemm(const uint8_t* a, const uint8_t* sa, const uint8_t* w,
                const uint8_t* sw, uint32_t m, uint32_t n, uint32_t k, float* out) {
  auto act = activation(a, sa, m, k);
  auto r = DeepSeekFp8GemmOracle::Multiply(
      act, bytes(w, static_cast<std::size_t>(n) * k),
      bytes(sw, static_cast<std::size_t>(n / 128U) * (k / 128U)), n);
  if (!r.ok()) return 1;
  std::memcpy(out, r->data(), r->size() * sizeof(float));
  return 0;
}

int pr_fp4_gemm(const uint8_t* a, const uint8_t* sa, const uint8_t* packed,
                const uint8_t* sw, uint32_t m, uint32_t n, uint32_t k, float* out) {
  auto act = activation(a, sa, m, k);
  auto r = DeepSeekFp4GemmOracle::Multiply(
      act, bytes(packed, static_cast<std::size_t>(n) * (k / 2U)),
      bytes(sw, static_cast<std::size_t>(n) * (k / 32U)), n);
  if (!r.ok()) return 1;
  std::memcpy(out, r->data(), r->size() * sizeof(float));
  return 0;
}

int pr_mxfp4_decode_row(const uint8_t* packed, const uint8_t* scales,
                        uint32_t k, float* out) {
  auto r = DeepSeekMxfp4Codec::DecodeRow(bytes(packed, (k + 1U) / 2U),
                                         bytes(scales, (k + 31U) / 32U), k);
  if (!r.ok()) return 1;
  std::memcpy(out, r->data(), r->size() * sizeof(float));
  return 0;
}

int pr_swiglu(const float* g, const float* u, uint32_t tokens, uint32_t inter,
              float limit, float* out) {
  const std::size_t n = static_cast<std::size_t>(tokens) * inter;
  auto r = DeepSeekExpertSwiGluOracle::Apply(std::span<const float>(g, n),
                                             std::span<const float>(u, n),
                                             tokens, inter, limit);
  if (!r.ok()) return 1;
  std::memcpy(out, r->data(), n * sizeof(float));
  return 0;
}

int pr_silu_mul(const uint16_t* g, const uint16_t* u, std::size_t n, uint16_t* out) {
  std::vector<BFloat16> gb(n), ub(n), ob(n);
  for (std::size_t i = 0; i < n; ++i) { gb[i].bits = g[i]; ub[i].bits = u[i]; }
  if (!qwen_silu_mul_oracle(gb, ub, ob).ok()) return 1;
  for (std::size_t i = 0; i < n; ++i) out[i] = ob[i].bits;
  return 0;
}

// Six routes per token, 256 experts (the reference's fixed geometry).
// Outputs: offsets[257]; sorted routes as parallel arrays.
int pr_subwave_plan(const uint16_t* expert, const uint32_t* token,
                    const uint8_t* ordinal, const float* weight,
                    uint32_t token_count, uint32_t* offsets,
                    uint16_t* s_expert, uint32_t* s_token, uint8_t* s_ordinal,
                    float* s_weight) {
  const std::size_t n = static_cast<std::size_t>(token_count) * 6U;
  std::vector<DeepSeekExpertRoute> routes(n);
  for (std::size_t i = 0; i < n; ++i)
    routes[i] = {expert[i], token[i], ordinal[i], weight[i]};
  auto plan = DeepSeekExpertSubwavePlan::Create(token_count, routes);
  if (!plan.ok()) return 1;
  for (std::size_t e = 0; e <= 256; ++e) offsets[e] = plan->expert_offsets()[e];
  for (std::size_t i = 0; i < n; ++i) {
    const auto& r = plan->routes()[i];
    s_expert[i] = r.expert_id;
    s_token[i] = r.token_index;
    s_ordinal[i] = r.route_ordinal;
    s_weight[i] = r.weight;
  }
  return 0;
}

// Ordered accumulation over experts (hidden fixed at 4096 by the reference).
// Rows are grouped by expert with offsets[experts+1]; out_f32 is [rows, 4096].
int pr_accumulate(const uint32_t* offsets, uint32_t experts,
                  const uint32_t* row_token, const float* expert_out,
                  uint32_t token_count, const float* shared, float* result) {
  auto acc = DeepSeekExpertAccumulatorOracle::Create(token_count);
  if (!acc.ok()) return 1;
  for (uint32_t e = 0; e < experts; ++e) {
    const auto begin = offsets[e], end = offsets[e + 1];
    if (begin == end) continue;
    std::vector<DeepSeekExpertRoute> routes;
    for (uint32_t r = begin; r < end; ++r)
      routes.push_back({static_cast<std::uint16_t>(e), row_token[r], 0, 1.0F});
    auto st = acc->add_expert(
        static_cast<std::uint16_t>(e), routes,
        std::span<const float>(expert_out + static_cast<std::size_t>(begin) * 4096U,
                               static_cast<std::size_t>(end - begin) * 4096U));
    if (!st.ok()) return 1;
  }
  auto fin = acc->finalize(std::span<const float>(
      shared, static_cast<std::size_t>(token_count) * 4096U));
  if (!fin.ok()) return 1;
  std::memcpy(result, fin->data(), fin->size() * sizeof(float));
  return 0;
}

int pr_routed_expert(const uint16_t* input, const float* route_weights,
                     uint32_t tokens, uint32_t hidden, uint32_t inter,
                     const uint8_t* w1p, const uint8_t* w1s, const uint8_t* w2p,
                     const uint8_t* w2s, const uint8_t* w3p, const uint8_t* w3s,
                     uint16_t* out) {
  std::vector<BFloat16> x(static_cast<std::size_t>(tokens) * hidden);
  for (std::size_t i = 0; i < x.size(); ++i) x[i].bits = input[i];
  const std::size_t up_bytes = static_cast<std::size_t>(inter) * hidden / 2U;
  const std::size_t up_scales = static_cast<std::size_t>(inter) * hidden / 32U;
  DeepSeekFp4MatrixView w1{bytes(w1p, up_bytes), bytes(w1s, up_scales)};
  DeepSeekFp4MatrixView w3{bytes(w3p, up_bytes), bytes(w3s, up_scales)};
  DeepSeekFp4MatrixView w2{bytes(w2p, up_bytes), bytes(w2s, up_scales)};
  auto r = DeepSeekRoutedExpertOracle::Forward(
      x, std::span<const float>(route_weights, tokens), tokens, hidden, inter,
      w1, w2, w3);
  if (!r.ok()) return 1;
  for (std::size_t i = 0; i < r->size(); ++i) out[i] = (*r)[i].bits;
  return 0;
}

// Reference INT4 quantizer (xing-w4a16-sym-g128-v1): bf16 [rows, cols] ->
// packed u8 [rows, cols/2] + fp16 scale bits [rows, cols/128].
int pr_int4_quantize(const uint16_t* src, uint64_t rows, uint64_t cols,
                     uint8_t* packed, uint16_t* scales) {
  std::vector<BFloat16> s(rows * cols);
  for (std::size_t i = 0; i < s.size(); ++i) s[i].bits = src[i];
  auto q = QwenInt4QuantizedTensor::Quantize(s, rows, cols);
  if (!q.ok()) return 1;
  std::memcpy(packed, q->packed_values().data(), q->packed_values().size());
  std::memcpy(scales, q->scale_bits().data(), q->scale_bits().size() * 2U);
  return 0;
}

// The V4 learned router (256 experts, top-6, x1.5): raw scores [tokens, 256]
// and bias [256] -> expert ids and weights [tokens, 6] by (token, ordinal).
int pr_learned_router(const float* raw, uint32_t token_count, const float* bias,
                      uint32_t* ids, float* weights) {
  std::vector<float> scores(raw, raw + static_cast<std::size_t>(token_count) * 256U);
  std::array<float, 256> b{};
  for (std::size_t e = 0; e < 256; ++e) b[e] = bias[e];
  auto plan = DeepSeekLearnedRouter::Route(token_count, scores, b);
  if (!plan.ok()) return 1;
  for (const auto& r : plan->routes()) {
    const std::size_t at = static_cast<std::size_t>(r.token_index) * 6U + r.route_ordinal;
    ids[at] = r.expert_id;
    weights[at] = r.weight;
  }
  return 0;
}

// Qwen INT4 XINGW4A1 metadata region (1 MiB) serialised by the reference for
// the official layout, the given roots (3 x 32 bytes) and payload digests
// (32 bytes per payload record, in the layout's record order, aliases
// skipped).  Writes the region to out (1 MiB) and the encoded length.
int pr_qwen_int4_metadata(const uint8_t* roots, const uint8_t* digests, uint8_t* out, uint32_t* encoded) {
  auto layout = QwenInt4ArtifactLayout::CreateOfficialPureW4();
  if (!layout.ok()) return 1;
  QwenInt4ArtifactRoots r;
  std::memcpy(r.source_artifact.bytes.data(), roots, 32);
  std::memcpy(r.source_binding.bytes.data(), roots + 32, 32);
  std::memcpy(r.disposition.bytes.data(), roots + 64, 32);
  std::vector<QwenInt4PayloadDigest> list;
  std::size_t i = 0;
  for (const auto& rec : layout->records()) {
    if (rec.kind == QwenInt4ArtifactRecordKind::kAlias) continue;
    QwenInt4PayloadDigest d;
    d.identity = rec.identity;
    std::memcpy(d.sha256.bytes.data(), digests + 32 * i++, 32);
    list.push_back(std::move(d));
  }
  auto meta = QwenInt4ArtifactMetadata::Create(*layout, r, std::move(list));
  if (!meta.ok()) return 1;
  auto region = meta->serialize_fixed_region();
  if (!region.ok()) return 1;
  std::memcpy(out, region->data(), region->size());
  *encoded = static_cast<uint32_t>(meta->encoded_bytes());
  return 0;
}

// ParseAndVerify of a 1 MiB metadata region against the official layout.
int pr_qwen_int4_parse(const uint8_t* region) {
  auto layout = QwenInt4ArtifactLayout::CreateOfficialPureW4();
  if (!layout.ok()) return 2;
  auto meta = QwenInt4ArtifactMetadata::ParseAndVerify(bytes(region, QwenInt4ArtifactLayout::kMetadataBytes), *layout);
  return meta.ok() ? 0 : 1;
}

// V4.1 expert FP4 -> FP8 32x32 block conversion (weight_expert_convert.cpp).
int pr_v41_fp4_block_to_fp8(const uint8_t* packed, const uint8_t* scales, uint8_t* weight, uint8_t* scale) {
  auto block = deepseek_v41::ConvertExpertFp4Block(bytes(packed, 512), bytes(scales, 32));
  if (!block.ok()) return 1;
  std::memcpy(weight, block->weight.data(), 1024);
  *scale = std::to_integer<uint8_t>(block->scale);
  return 0;
}

// V4.1 wo_a block dequantisation E4M3FN x scale -> bf16 (weight_dequantize.cpp).
int pr_v41_dequant_block(const uint8_t* source, float scale, uint32_t block, uint16_t* out) {
  std::vector<std::byte> dst(static_cast<std::size_t>(block) * block * 2U);
  auto st = deepseek_v41::DequantizeWoABlock(bytes(source, static_cast<std::size_t>(block) * block), scale, block,
                                             dst);
  if (!st.ok()) return 1;
  std::memcpy(out, dst.data(), dst.size());
  return 0;
}

}  // extern "C"

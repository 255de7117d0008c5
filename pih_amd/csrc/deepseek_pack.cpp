// gfx950 DeepSeek V4 Kernel Pack: identity, the 29-entry
// pih_deepseek_kernels_api_v1 table and the two exported C symbols.
//
// Drop-in for plugins/kernels/deepseek-v4-sm89/kernel_pack.cpp:42-585.  The
// table keeps the reference's order and request structs.  Linear/MoE entries
// run the gfx950 kernels of this library; the attention, compressor,
// indexer, hyper-connection, embedding and sampling entries stay in the
// table so its size and order match, and answer UNAVAILABLE; the LM head
// runs the BF16 GEMM/GEMV.
//
// Shapes fixed by the reference ABI (no size field in the request): route
// gather, expert accumulate and finalize use hidden 4096; expert and shared
// SwiGLU use intermediate 2048 with clamp limit 10
// (include/pih/backend/cuda/deepseek_route_gather.h:10,
// deepseek_expert_swiglu.h:10-11, deepseek_expert_accumulate.cu:11).
#include <hip/hip_runtime.h>
#include <string.h>

#include "host_common.hpp"
#include "kernels.hpp"
#include "pih/contracts/deepseek_kernels_v1.h"

namespace pih_amd {
namespace {

constexpr uint32_t kAbi = PIH_DEEPSEEK_KERNELS_ABI_VERSION_V1;
constexpr uint32_t kHidden = 4096;
constexpr uint32_t kIntermediate = 2048;
constexpr uint32_t kVocab = 129280;
constexpr float kSwiGluLimit = 10.0f;

const pih_kernel_pack_identity_v1 kIdentity = {
    sizeof(pih_kernel_pack_identity_v1), PIH_KERNEL_PACK_ABI_VERSION_V1,
    "pih.kernels.deepseek-v4.gfx950", "1.0.0", "pih.deepseek-gfx950-kernel-pack.v1", "gfx950"};

#define PIH_AMD_REQUIRE_HEADER(req, msg) \
  if (!HeaderOk(req, kAbi)) return Invalid(msg)

St Fp8ActivationQuant(const pih_deepseek_fp8_activation_quant_launch_v1* r) {
  PIH_AMD_REQUIRE_HEADER(r, "fp8_quant_request_invalid");
  Fp8QuantArgs a;
  a.input = Ptr<const uint16_t>(r->input_bf16);
  a.codes = Ptr<uint8_t>(r->output_e4m3);
  a.scales = Ptr<void>(r->scale_bits);
  a.error_flag = Ptr<uint32_t>(r->error_flag);
  a.stream = AsStream(r->stream);
  a.row_count = r->token_count;
  a.k = r->logical_k;
  a.fmt = kScaleUe8m0;
  return LaunchFp8Quant(a);
}

St Fp8Gemm(const pih_deepseek_fp8_gemm_launch_v1* r) {
  if (!HeaderOk(r, kAbi) || (r->output_type != 1 && r->output_type != 2))
    return Invalid("fp8_gemm_request_invalid");
  // reference bounds (deepseek_fp8_gemm.cpp:5-20)
  if (r->m == 0 || r->m > 4096 || r->n > 129280 || r->k > 32768) return Invalid("fp8_gemm_shape_invalid");
  BlockGemmArgs a;
  a.a = Ptr<const uint8_t>(r->activation_e4m3);
  a.a_scale = Ptr<const void>(r->activation_scale_bits);
  a.w = Ptr<const uint8_t>(r->weight_e4m3);
  a.w_scale = Ptr<const void>(r->weight_scale_bits);
  a.out = Ptr<void>(r->output);
  a.error_flag = Ptr<uint32_t>(r->error_flag);
  a.stream = AsStream(r->stream);
  a.m = r->m;
  a.n = r->n;
  a.k = r->k;
  a.a_rows_total = r->m;
  a.scale_fmt = kScaleUe8m0;
  a.out_kind = r->output_type == 2 ? kOutF32 : kOutBf16;
  a.check_codes = true;
  return LaunchFp8BlockGemm(a);
}

St GroupedFp8Gemm(const pih_deepseek_grouped_fp8_gemm_launch_v1* r) {
  PIH_AMD_REQUIRE_HEADER(r, "grouped_fp8_request_invalid");
  // The reference fixes G=8, N_g=1024, K_g=4096 (attention wo_a,
  // deepseek_attention_dense_primitives.cpp:58-71); any N_g, K_g that are
  // multiples of 128 are accepted here.
  if (r->token_count == 0 || r->group_count == 0 || r->output_per_group == 0 ||
      r->output_per_group % 128 || r->input_per_group == 0 || r->input_per_group % 128 ||
      (uint64_t)r->token_count * r->group_count > 0x7fffffffull)
    return Invalid("grouped_fp8_shape_invalid");
  if (!r->activation_e4m3 || !r->activation_scale_bits) return Invalid("grouped_fp8_null_argument");
  const uint32_t rows = r->token_count * r->group_count;
  Fp8QuantArgs q;
  q.input = Ptr<const uint16_t>(r->input_bf16);
  q.codes = Ptr<uint8_t>(r->activation_e4m3);
  q.scales = Ptr<void>(r->activation_scale_bits);
  q.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  q.stream = AsStream(r->stream);
  q.row_count = rows;
  q.k = r->input_per_group;
  q.fmt = kScaleUe8m0;
  St s = LaunchFp8Quant(q);
  if (!s.ok()) return s;
  BlockGemmArgs a;
  a.a = Ptr<const uint8_t>(r->activation_e4m3);
  a.a_scale = Ptr<const void>(r->activation_scale_bits);
  a.w = Ptr<const uint8_t>(r->weight_e4m3);
  a.w_scale = Ptr<const void>(r->weight_scale_bits);
  a.out = Ptr<void>(r->output_bf16);
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.m = r->token_count;
  a.n = r->output_per_group;
  a.k = r->input_per_group;
  a.problems = r->group_count;
  a.a_rows_total = rows;
  a.a_row_stride = r->group_count;
  a.a_prob_row = 1;
  a.out_row_stride = (uint64_t)r->group_count * r->output_per_group;
  a.out_prob_col = r->output_per_group;
  a.scale_fmt = kScaleUe8m0;
  a.out_kind = kOutBf16;
  // the reference grouped kernel reports scale 0xFF as 1024 and a
  // non-finite sum as 2048, and stores the non-finite bf16 value all the
  // same (deepseek_attention_dense_primitives.cu:205-250)
  a.err_scale_bit = 1024u;
  a.err_nonfinite_bit = 2048u;
  a.write_nonfinite = true;
  return LaunchFp8BlockGemm(a);
}

St RouteGather(const pih_deepseek_route_gather_launch_v1* r) {
  PIH_AMD_REQUIRE_HEADER(r, "route_gather_request_invalid");
  GatherArgs a;
  a.source = Ptr<const uint16_t>(r->source_hidden_bf16);
  a.token_index = Ptr<const uint32_t>(r->token_indices_u32);
  a.dest = Ptr<uint16_t>(r->route_hidden_bf16);
  a.error_flag = Ptr<uint32_t>(r->error_flag);
  a.stream = AsStream(r->stream);
  a.routes = r->route_count;
  a.tokens = r->packed_token_count;
  a.hidden = kHidden;
  return LaunchRouteGather(a);
}

St Fp4Gemm(const pih_deepseek_fp4_gemm_launch_v1* r) {
  PIH_AMD_REQUIRE_HEADER(r, "fp4_gemm_request_invalid");
  if (r->m == 0 || r->m > 4096 || r->n == 0 || r->k == 0) return Invalid("fp4_gemm_shape_invalid");
  Fp4GemmArgs a;
  a.a = Ptr<const void>(r->activation_e4m3);
  a.a_scale = Ptr<const uint8_t>(r->activation_scale_bits);
  a.w = Ptr<const uint8_t>(r->packed_weight);
  a.w_scale = Ptr<const uint8_t>(r->weight_scale_bits);
  a.out = Ptr<void>(r->output_bf16);
  a.error_flag = Ptr<uint32_t>(r->error_flag);
  a.stream = AsStream(r->stream);
  a.m = r->m;
  a.n = r->n;
  a.k = r->k;
  a.a_rows_total = r->m;
  a.act = kActE4m3;
  a.out_kind = kOutBf16;
  return LaunchFp4Gemm(a);
}

St ExpertSwiGlu(const pih_deepseek_expert_swiglu_launch_v1* r) {
  PIH_AMD_REQUIRE_HEADER(r, "expert_swiglu_request_invalid");
  if (!r->route_weights_f32) return Invalid("expert_swiglu_null_argument");
  SwiGluArgs a;
  a.gate = Ptr<const uint16_t>(r->gate_bf16);
  a.up = Ptr<const uint16_t>(r->up_bf16);
  a.weights = Ptr<const float>(r->route_weights_f32);
  a.out = Ptr<uint16_t>(r->output_bf16);
  a.error_flag = Ptr<uint32_t>(r->error_flag);
  a.stream = AsStream(r->stream);
  a.rows = r->token_count;
  a.cols = kIntermediate;
  a.limit = kSwiGluLimit;
  return LaunchSwiGlu(a);
}

St SharedSwiGlu(const pih_deepseek_shared_swiglu_launch_v1* r) {
  PIH_AMD_REQUIRE_HEADER(r, "shared_swiglu_request_invalid");
  SwiGluArgs a;
  a.gate = Ptr<const uint16_t>(r->gate_bf16);
  a.up = Ptr<const uint16_t>(r->up_bf16);
  a.out = Ptr<uint16_t>(r->output_bf16);
  a.error_flag = Ptr<uint32_t>(r->error_flag);
  a.stream = AsStream(r->stream);
  a.rows = r->token_count;
  a.cols = kIntermediate;
  a.limit = kSwiGluLimit;
  return LaunchSwiGlu(a);
}

St ExpertAccumulate(const pih_deepseek_expert_accumulate_launch_v1* r) {
  PIH_AMD_REQUIRE_HEADER(r, "expert_accumulate_invalid");
  AccumulateArgs a;
  a.expert_out = Ptr<const uint16_t>(r->expert_output_bf16);
  a.token_index = Ptr<const uint32_t>(r->token_indices);
  a.acc = Ptr<float>(r->accumulator_f32);
  a.error_flag = Ptr<uint32_t>(r->error_flag);
  a.stream = AsStream(r->stream);
  a.routes = r->route_count;
  a.tokens = r->token_count;
  a.hidden = kHidden;
  return LaunchOrderedAccumulate(a);
}

St ExpertFinalize(const pih_deepseek_expert_finalize_launch_v1* r) {
  PIH_AMD_REQUIRE_HEADER(r, "expert_finalize_invalid");
  if (!r->shared_output_bf16) return Invalid("expert_finalize_null_argument");
  FinalizeArgs a;
  a.acc = Ptr<const float>(r->accumulator_f32);
  a.shared = Ptr<const uint16_t>(r->shared_output_bf16);
  a.out = Ptr<uint16_t>(r->output_bf16);
  a.error_flag = Ptr<uint32_t>(r->error_flag);
  a.stream = AsStream(r->stream);
  a.count = (uint64_t)r->token_count * kHidden;
  return LaunchFinalize(a);
}

St RouterGemm(const pih_deepseek_router_gemm_launch_v1* r) {
  PIH_AMD_REQUIRE_HEADER(r, "router_gemm_request_invalid");
  Bf16GemmArgs a;
  a.a = Ptr<const uint16_t>(r->input_bf16);
  a.w = Ptr<const uint16_t>(r->weight_bf16);
  a.out = Ptr<void>(r->scores_f32);
  a.stream = AsStream(r->stream);
  a.m = r->token_count;
  a.n = r->expert_count;
  a.k = r->hidden_size;
  a.out_kind = kOutF32;
  // the request carries no workspace: decode shapes run without k-split
  return LaunchBf16Gemm(a);
}

// LM head: logits f32 [rows, 129280] = x bf16 [rows, 4096] . W bf16
// [129280, 4096]^T (reference deepseek_endpoint.cu:94-115, launcher
// :484-497, validator deepseek_endpoint.cpp:57-66).  Error bits as the
// reference: 128 for a non-finite logit (the logit is still written), 64
// for a non-finite x or W element.  Decode row counts run the
// weight-streaming GEMV, larger ones the MFMA GEMM; the fp32 sums run in
// the kernels' order, not the reference's 256-thread tree.
St LmHead(const pih_deepseek_lm_head_launch_v1* r) {
  if (!HeaderOk(r, kAbi)) return Invalid("lm_head_request_invalid");
  if (!r->input_bf16 || !r->weight_bf16 || !r->logits_f32 || !r->error_flag_u32 || !r->stream ||
      r->output_rows == 0 || r->output_rows > 4096 || r->vocab_size != kVocab || r->hidden_size != kHidden ||
      r->logits_f32 == r->input_bf16 || r->logits_f32 == r->weight_bf16)
    return Invalid("lm_head_launch_invalid");
  Bf16GemmArgs g;
  g.a = Ptr<const uint16_t>(r->input_bf16);
  g.w = Ptr<const uint16_t>(r->weight_bf16);
  g.out = Ptr<void>(r->logits_f32);
  g.stream = AsStream(r->stream);
  g.m = r->output_rows;
  g.n = r->vocab_size;
  g.k = r->hidden_size;
  g.out_kind = kOutF32;
  g.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  g.nonfinite_bit = 128u;
  St s = LaunchBf16Gemm(g);
  if (!s.ok()) return s;
  NonfiniteScanArgs c;
  c.x = g.a;
  c.w = g.w;
  c.x_elems = (uint64_t)r->output_rows * r->hidden_size;
  c.w_elems = (uint64_t)r->vocab_size * r->hidden_size;
  c.error_flag = g.error_flag;
  c.stream = g.stream;
  c.trigger_bit = 128u;
  c.set_bit = 64u;
  return LaunchNonfiniteScan(c);
}

// Entries outside the linear/MoE path: present, validated, unavailable.
#define PIH_AMD_UNAVAILABLE_ENTRY(fn, type, name)                     \
  St fn(const type* r) {                                              \
    if (!HeaderOk(r, kAbi)) return Invalid(name "_request_invalid");  \
    return Unavailable(name "_not_in_gfx950_linear_pack");           \
  }
PIH_AMD_UNAVAILABLE_ENTRY(RopeTable, pih_deepseek_rope_table_launch_v1, "rope_table")
PIH_AMD_UNAVAILABLE_ENTRY(RmsNorm, pih_deepseek_rms_norm_launch_v1, "rms_norm")
PIH_AMD_UNAVAILABLE_ENTRY(HeadRms, pih_deepseek_head_rms_launch_v1, "head_rms")
PIH_AMD_UNAVAILABLE_ENTRY(Rotary, pih_deepseek_rotary_launch_v1, "rotary")
PIH_AMD_UNAVAILABLE_ENTRY(KvFp8Simulate, pih_deepseek_kv_fp8_simulate_launch_v1, "kv_fp8")
PIH_AMD_UNAVAILABLE_ENTRY(Embedding, pih_deepseek_embedding_launch_v1, "embedding")
PIH_AMD_UNAVAILABLE_ENTRY(HcHead, pih_deepseek_hc_head_launch_v1, "hc_head")
PIH_AMD_UNAVAILABLE_ENTRY(Argmax, pih_deepseek_argmax_launch_v1, "argmax")
PIH_AMD_UNAVAILABLE_ENTRY(StochasticSample, pih_deepseek_stochastic_sample_launch_v1, "sample")
PIH_AMD_UNAVAILABLE_ENTRY(CompressorPooling, pih_deepseek_compressor_pooling_launch_v1, "compressor_pooling")
PIH_AMD_UNAVAILABLE_ENTRY(CompressorProjection, pih_deepseek_compressor_projection_launch_v1, "compressor_projection")
PIH_AMD_UNAVAILABLE_ENTRY(CompressorStore, pih_deepseek_compressor_store_launch_v1, "compressor_store")
PIH_AMD_UNAVAILABLE_ENTRY(IndexerProjection, pih_deepseek_indexer_projection_launch_v1, "indexer_projection")
PIH_AMD_UNAVAILABLE_ENTRY(IndexScore, pih_deepseek_index_score_launch_v1, "index_score")
PIH_AMD_UNAVAILABLE_ENTRY(SparseAttention, pih_deepseek_sparse_attention_launch_v1, "sparse_attention")
PIH_AMD_UNAVAILABLE_ENTRY(MhcPre, pih_deepseek_mhc_pre_launch_v1, "mhc_pre")
PIH_AMD_UNAVAILABLE_ENTRY(MhcPost, pih_deepseek_mhc_post_launch_v1, "mhc_post")
PIH_AMD_UNAVAILABLE_ENTRY(MhcTargetTap, pih_deepseek_mhc_target_tap_launch_v1, "mhc_target_tap")
#undef PIH_AMD_UNAVAILABLE_ENTRY

PIH_AMD_CONTAINED(CRopeTable, RopeTable, pih_deepseek_rope_table_launch_v1)
PIH_AMD_CONTAINED(CRmsNorm, RmsNorm, pih_deepseek_rms_norm_launch_v1)
PIH_AMD_CONTAINED(CFp8ActivationQuant, Fp8ActivationQuant, pih_deepseek_fp8_activation_quant_launch_v1)
PIH_AMD_CONTAINED(CFp8Gemm, Fp8Gemm, pih_deepseek_fp8_gemm_launch_v1)
PIH_AMD_CONTAINED(CHeadRms, HeadRms, pih_deepseek_head_rms_launch_v1)
PIH_AMD_CONTAINED(CRotary, Rotary, pih_deepseek_rotary_launch_v1)
PIH_AMD_CONTAINED(CKvFp8Simulate, KvFp8Simulate, pih_deepseek_kv_fp8_simulate_launch_v1)
PIH_AMD_CONTAINED(CGroupedFp8Gemm, GroupedFp8Gemm, pih_deepseek_grouped_fp8_gemm_launch_v1)
PIH_AMD_CONTAINED(CRouteGather, RouteGather, pih_deepseek_route_gather_launch_v1)
PIH_AMD_CONTAINED(CFp4Gemm, Fp4Gemm, pih_deepseek_fp4_gemm_launch_v1)
PIH_AMD_CONTAINED(CExpertSwiGlu, ExpertSwiGlu, pih_deepseek_expert_swiglu_launch_v1)
PIH_AMD_CONTAINED(CExpertAccumulate, ExpertAccumulate, pih_deepseek_expert_accumulate_launch_v1)
PIH_AMD_CONTAINED(CEmbedding, Embedding, pih_deepseek_embedding_launch_v1)
PIH_AMD_CONTAINED(CHcHead, HcHead, pih_deepseek_hc_head_launch_v1)
PIH_AMD_CONTAINED(CLmHead, LmHead, pih_deepseek_lm_head_launch_v1)
PIH_AMD_CONTAINED(CArgmax, Argmax, pih_deepseek_argmax_launch_v1)
PIH_AMD_CONTAINED(CStochasticSample, StochasticSample, pih_deepseek_stochastic_sample_launch_v1)
PIH_AMD_CONTAINED(CCompressorPooling, CompressorPooling, pih_deepseek_compressor_pooling_launch_v1)
PIH_AMD_CONTAINED(CCompressorProjection, CompressorProjection, pih_deepseek_compressor_projection_launch_v1)
PIH_AMD_CONTAINED(CCompressorStore, CompressorStore, pih_deepseek_compressor_store_launch_v1)
PIH_AMD_CONTAINED(CIndexerProjection, IndexerProjection, pih_deepseek_indexer_projection_launch_v1)
PIH_AMD_CONTAINED(CIndexScore, IndexScore, pih_deepseek_index_score_launch_v1)
PIH_AMD_CONTAINED(CSparseAttention, SparseAttention, pih_deepseek_sparse_attention_launch_v1)
PIH_AMD_CONTAINED(CRouterGemm, RouterGemm, pih_deepseek_router_gemm_launch_v1)
PIH_AMD_CONTAINED(CMhcPre, MhcPre, pih_deepseek_mhc_pre_launch_v1)
PIH_AMD_CONTAINED(CMhcPost, MhcPost, pih_deepseek_mhc_post_launch_v1)
PIH_AMD_CONTAINED(CMhcTargetTap, MhcTargetTap, pih_deepseek_mhc_target_tap_launch_v1)
PIH_AMD_CONTAINED(CSharedSwiGlu, SharedSwiGlu, pih_deepseek_shared_swiglu_launch_v1)
PIH_AMD_CONTAINED(CExpertFinalize, ExpertFinalize, pih_deepseek_expert_finalize_launch_v1)

const pih_deepseek_kernels_api_v1 kContract = {
    sizeof(pih_deepseek_kernels_api_v1), kAbi, &kIdentity,
    &CRopeTable, &CRmsNorm, &CFp8ActivationQuant, &CFp8Gemm, &CHeadRms, &CRotary,
    &CKvFp8Simulate, &CGroupedFp8Gemm, &CRouteGather, &CFp4Gemm, &CExpertSwiGlu,
    &CExpertAccumulate, &CEmbedding, &CHcHead, &CLmHead, &CArgmax, &CStochasticSample,
    &CCompressorPooling, &CCompressorProjection, &CCompressorStore, &CIndexerProjection,
    &CIndexScore, &CSparseAttention, &CRouterGemm, &CMhcPre, &CMhcPost, &CMhcTargetTap,
    &CSharedSwiGlu, &CExpertFinalize};

// Device images are embedded in this library; binding only checks the path
// (reference kernel_pack.cpp:564-569) and touches no device.
pih_status_v1 BindOrigin(const char* path) noexcept {
  return ToAbi(path && path[0] == '/' ? Ok() : Invalid("bind_origin_path_not_absolute"));
}

const pih_kernel_pack_api_v1 kApi = {sizeof(pih_kernel_pack_api_v1), PIH_KERNEL_PACK_ABI_VERSION_V1,
                                     &kIdentity, &kContract, &BindOrigin};

}  // namespace
}  // namespace pih_amd

extern "C" PIH_PLUGIN_EXPORT const pih_kernel_pack_identity_v1* pih_kernel_pack_identity_v1_get(void) {
  return &pih_amd::kIdentity;
}

extern "C" PIH_PLUGIN_EXPORT const pih_kernel_pack_api_v1* pih_kernel_pack_api_v1_get(void) {
  return &pih_amd::kApi;
}

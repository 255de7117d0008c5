// gfx950 AMD linear-layer Kernel Pack: identity, the
// pih_amd_linear_kernels_api_v1 table and the two exported C symbols
// (the Kernel Pack ABI of include/pih/plugin_sdk/kernel_pack.h, as loaded by
// the reference's KernelPackLoader, src/microkernel/kernel_pack_loader.cpp:
// 90-133).  Each entry checks the request header, maps the request onto an
// internal launcher and returns its status; nothing here allocates or
// touches a device outside the enqueue.
#include <hip/hip_runtime.h>
#include <string.h>

#include "host_common.hpp"
#include "kernels.hpp"
#include "pih/contracts/amd_linear_kernels_v1.h"

namespace pih_amd {
namespace {

constexpr uint32_t kAbi = PIH_AMD_LINEAR_KERNELS_ABI_VERSION_V1;

const pih_kernel_pack_identity_v1 kIdentity = {
    sizeof(pih_kernel_pack_identity_v1), PIH_KERNEL_PACK_ABI_VERSION_V1,
    "pih.kernels.amd-linear.gfx950", "1.0.0", "pih.amd-linear-kernels.v1", "gfx950"};

bool ScaleFmtOk(uint32_t f) { return f == PIH_AMD_SCALE_F32_V1 || f == PIH_AMD_SCALE_UE8M0_V1; }
bool OutOk(uint32_t o) {
  return o == PIH_AMD_OUTPUT_BF16_V1 || o == PIH_AMD_OUTPUT_F32_V1 || o == PIH_AMD_OUTPUT_SWIGLU_BF16_V1;
}

St QueryWorkspace(const pih_amd_workspace_query_v1* r) {
  if (!HeaderOk(r, kAbi) || !r->bytes_u64) return Invalid("workspace_query_invalid");
  uint64_t bytes;
  switch (r->kind) {
    case PIH_AMD_WORKSPACE_ROUTE_PLAN_V1:
      if (r->m == 0 || r->n == 0 || r->k == 0) return Invalid("workspace_query_shape_invalid");
      bytes = RoutePlanWorkspaceBytes(r->m, r->n, r->k);
      break;
    case PIH_AMD_WORKSPACE_BF16_GEMM_V1:
      bytes = Bf16GemmWorkspaceBytes(r->m, r->n, r->k);
      break;
    case PIH_AMD_WORKSPACE_W4A16_V1:
      bytes = W4a16WorkspaceBytes(r->m, r->n, r->k);
      break;
    default:
      return Invalid("workspace_query_kind_invalid");
  }
  *Ptr<uint64_t>(r->bytes_u64) = bytes;
  return Ok();
}

St RoutePlan(const pih_amd_route_plan_launch_v1* r) {
  if (!HeaderOk(r, kAbi)) return Invalid("route_plan_request_invalid");
  RoutePlanArgs a;
  a.topk_ids = Ptr<const uint32_t>(r->topk_ids_u32);
  a.topk_weights = Ptr<const float>(r->topk_weights_f32);
  a.expert_offsets = Ptr<uint32_t>(r->expert_offsets_u32);
  a.row_token = Ptr<uint32_t>(r->row_token_u32);
  a.row_weight = Ptr<float>(r->row_weight_f32);
  a.token_rows = Ptr<uint32_t>(r->token_rows_u32);
  a.workspace = Ptr<void>(r->workspace);
  a.workspace_bytes = r->workspace_bytes;
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.tokens = r->token_count;
  a.topk = r->top_k;
  a.experts = r->expert_count;
  return LaunchRoutePlan(a);
}

St RoutePlanNoAlloc(const pih_amd_route_plan_launch_v1* r) {
  if (!HeaderOk(r, kAbi)) return Invalid("route_plan_request_invalid");
  static_assert(PIH_AMD_ROUTE_PLAN_NOALLOC_MAX_SCRATCH_V1 == kRoutePlanNoAllocScratchBytes,
                "contract limit and scratch array size differ");
  RoutePlanArgs a;
  a.topk_ids = Ptr<const uint32_t>(r->topk_ids_u32);
  a.topk_weights = Ptr<const float>(r->topk_weights_f32);
  a.expert_offsets = Ptr<uint32_t>(r->expert_offsets_u32);
  a.row_token = Ptr<uint32_t>(r->row_token_u32);
  a.row_weight = Ptr<float>(r->row_weight_f32);
  a.token_rows = Ptr<uint32_t>(r->token_rows_u32);
  a.workspace = Ptr<void>(r->workspace);
  a.workspace_bytes = r->workspace_bytes;
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.tokens = r->token_count;
  a.topk = r->top_k;
  a.experts = r->expert_count;
  return LaunchRoutePlanNoAlloc(a);
}

St RouterTopk(const pih_amd_router_topk_launch_v1* r) {
  if (!HeaderOk(r, kAbi)) return Invalid("router_topk_request_invalid");
  RouterTopkArgs a;
  a.scores = Ptr<const float>(r->scores_f32);
  a.bias = Ptr<const float>(r->bias_f32);
  a.ids = Ptr<uint32_t>(r->topk_ids_u32);
  a.weights = Ptr<float>(r->topk_weights_f32);
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.tokens = r->token_count;
  a.experts = r->expert_count;
  a.topk = r->top_k;
  a.mode = r->mode;
  a.scale = r->route_scale;
  return LaunchRouterTopk(a);
}

// The reference's region checks (plugins/model-deepseek-v41/linear_fp8.cpp:
// 6-13): non-zero, aligned, exactly the layout's size, no address overflow.
bool RegionOk(uintptr_t address, uint64_t bytes, uint64_t want, unsigned align) {
  return address && address % align == 0 && bytes == want && want <= UINTPTR_MAX - address;
}
bool RegionsOverlap(uintptr_t a, uint64_t na, uintptr_t b, uint64_t nb) { return a < b + nb && b < a + na; }

St V41Linear(const pih_amd_v41_linear_launch_v1* r) {
  if (!HeaderOk(r, kAbi)) return Invalid("v41_linear_request_invalid");
  const bool fp4 = r->weight_format == PIH_AMD_V41_WEIGHT_MXFP4_V1;
  if (!fp4 && r->weight_format != PIH_AMD_V41_WEIGHT_FP8_BLOCK32_V1) return Invalid("v41_linear_weight_format_invalid");
  // linear_fp8.cpp:15-17 / linear_fp4.cpp:14-16
  if (!r->stream || !r->rows || r->rows > 4096 || !r->in_features || r->in_features > 32768 || !r->out_features ||
      r->out_features > 32768 || r->in_features % 32 || r->out_features % 32)
    return Invalid("V4.1 linear requires bounded block-32 dimensions");
  const uint64_t m = r->rows, k = r->in_features, n = r->out_features;
  const uint64_t wbytes = fp4 ? n * k / 2 : n * k, wsbytes = fp4 ? n * (k / 32) : (n / 32) * (k / 32);
  if (!RegionOk(r->input_bf16, r->input_bytes, m * k * 2, 2) || !RegionOk(r->weight, r->weight_bytes, wbytes, 1) ||
      !RegionOk(r->weight_scales, r->weight_scale_bytes, wsbytes, 1) ||
      !RegionOk(r->quantized_e4m3, r->quantized_bytes, m * k, 1) ||
      !RegionOk(r->activation_scales, r->activation_scale_bytes, m * (k / 32), 1) ||
      !RegionOk(r->output_bf16, r->output_bytes, m * n * 2, 2) ||
      !RegionOk(r->error_flag_u32, r->error_flag_bytes, 4, 4))
    return Invalid("V4.1 linear buffer layout invalid");
  const uintptr_t reads[3][2] = {{r->input_bf16, r->input_bytes}, {r->weight, r->weight_bytes},
                                 {r->weight_scales, r->weight_scale_bytes}};
  const uintptr_t writes[4][2] = {{r->quantized_e4m3, r->quantized_bytes},
                                  {r->activation_scales, r->activation_scale_bytes},
                                  {r->output_bf16, r->output_bytes},
                                  {r->error_flag_u32, r->error_flag_bytes}};
  for (int i = 0; i < 4; ++i) {
    for (int j = 0; j < 3; ++j)
      if (RegionsOverlap(writes[i][0], writes[i][1], reads[j][0], reads[j][1]))
        return Invalid("V4.1 linear overwrites an input");
    for (int j = 0; j < i; ++j)
      if (RegionsOverlap(writes[i][0], writes[i][1], writes[j][0], writes[j][1]))
        return Invalid("V4.1 linear writable alias");
  }
  // the MX MFMA tiles take 128-deep steps over 128-row W tiles
  if (k % 128 || n % 128) return Invalid("v41_linear_requires_128_multiples");
  V41Quant32Args q;
  q.input = Ptr<const uint16_t>(r->input_bf16);
  q.codes = Ptr<uint8_t>(r->quantized_e4m3);
  q.scales = Ptr<uint8_t>(r->activation_scales);
  q.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  q.stream = AsStream(r->stream);
  q.rows = r->rows;
  q.k = r->in_features;
  St s = LaunchV41Quant32(q);
  if (!s.ok()) return s;
  Mx32GemmArgs g;
  g.a = q.codes;
  g.a_scale = q.scales;
  g.w = Ptr<const uint8_t>(r->weight);
  g.w_scale = Ptr<const uint8_t>(r->weight_scales);
  g.out = Ptr<uint16_t>(r->output_bf16);
  g.error_flag = q.error_flag;
  g.stream = q.stream;
  g.m = r->rows;
  g.n = r->out_features;
  g.k = r->in_features;
  g.fp4_weight = fp4;
  return LaunchMx32Gemm(g);
}

St V41Fp4ToFp8(const pih_amd_v41_fp4_to_fp8_launch_v1* r) {
  if (!HeaderOk(r, kAbi)) return Invalid("v41_fp4_to_fp8_request_invalid");
  V41Fp4ToFp8Args a;
  a.packed = Ptr<const uint8_t>(r->packed);
  a.scales = Ptr<const uint8_t>(r->scales);
  a.weight = Ptr<uint8_t>(r->weight_e4m3);
  a.weight_scales = Ptr<uint8_t>(r->weight_scales);
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.rows = r->rows;
  a.cols = r->columns;
  return LaunchV41Fp4ToFp8(a);
}

St V41BlockDequant(const pih_amd_v41_block_dequant_launch_v1* r) {
  if (!HeaderOk(r, kAbi)) return Invalid("v41_block_dequant_request_invalid");
  if (r->scale_storage != PIH_AMD_V41_SCALE_E8M0_V1 && r->scale_storage != PIH_AMD_V41_SCALE_F32_V1)
    return Invalid("v41_dequant_scale_storage_invalid");
  V41BlockDequantArgs a;
  a.source = Ptr<const uint8_t>(r->source_e4m3);
  a.scales = Ptr<const void>(r->scales);
  a.output = Ptr<uint16_t>(r->output_bf16);
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.rows = r->rows;
  a.cols = r->columns;
  a.block = r->block;
  a.scale_f32 = r->scale_storage == PIH_AMD_V41_SCALE_F32_V1 ? 1u : 0u;
  return LaunchV41BlockDequant(a);
}

St Fp8Quant(const pih_amd_fp8_quant_launch_v1* r) {
  if (!HeaderOk(r, kAbi) || !ScaleFmtOk(r->scale_format)) return Invalid("fp8_quant_request_invalid");
  Fp8QuantArgs a;
  a.input = Ptr<const uint16_t>(r->input_bf16);
  a.rows = Ptr<const uint32_t>(r->row_index_u32);
  a.codes = Ptr<uint8_t>(r->output_e4m3);
  a.scales = Ptr<void>(r->scale);
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.row_count = r->row_count;
  a.k = r->logical_k;
  a.input_rows = r->input_rows;
  a.fmt = (ScaleFmt)r->scale_format;
  return LaunchFp8Quant(a);
}

St Fp8Gemm(const pih_amd_fp8_gemm_launch_v1* r) {
  if (!HeaderOk(r, kAbi) || !ScaleFmtOk(r->scale_format) ||
      (r->output_type != PIH_AMD_OUTPUT_BF16_V1 && r->output_type != PIH_AMD_OUTPUT_F32_V1))
    return Invalid("fp8_gemm_request_invalid");
  BlockGemmArgs a;
  a.a = Ptr<const uint8_t>(r->activation_e4m3);
  a.a_scale = Ptr<const void>(r->activation_scale);
  a.w = Ptr<const uint8_t>(r->weight_e4m3);
  a.w_scale = Ptr<const void>(r->weight_scale);
  a.out = Ptr<void>(r->output);
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.m = r->m;
  a.n = r->n;
  a.k = r->k;
  a.a_rows_total = r->m;
  a.scale_fmt = (ScaleFmt)r->scale_format;
  a.out_kind = (OutKind)r->output_type;
  a.check_codes = true;
  return LaunchFp8BlockGemm(a);
}

St MoeFp8Gemm(const pih_amd_moe_fp8_gemm_launch_v1* r) {
  if (!HeaderOk(r, kAbi) || !ScaleFmtOk(r->scale_format) ||
      !(OutOk(r->output_type) || r->output_type == PIH_AMD_OUTPUT_SWIGLU_E4M3_V1))
    return Invalid("moe_fp8_gemm_request_invalid");
  if (r->expert_count == 0 || r->row_capacity == 0 || r->activation_rows == 0)
    return Invalid("moe_fp8_gemm_shape_invalid");
  BlockGemmArgs a;
  a.a = Ptr<const uint8_t>(r->activation_e4m3);
  a.a_scale = Ptr<const void>(r->activation_scale);
  a.a_gather = Ptr<const uint32_t>(r->row_token_u32);
  a.w = Ptr<const uint8_t>(r->weight_e4m3);
  a.w_scale = Ptr<const void>(r->weight_scale);
  a.offsets = Ptr<const uint32_t>(r->expert_offsets_u32);
  a.row_weight = Ptr<const float>(r->row_weight_f32);
  a.out = Ptr<void>(r->output);
  a.out_scale = Ptr<void>(r->output_scale);
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.m = r->row_capacity;
  a.n = r->n;
  a.k = r->k;
  a.problems = r->expert_count;
  a.a_rows_total = r->activation_rows;
  a.moe = true;
  a.scale_fmt = (ScaleFmt)r->scale_format;
  a.out_kind = (OutKind)r->output_type;
  a.swiglu_limit = r->swiglu_limit;
  return LaunchFp8BlockGemm(a);
}

St MoeMxfp4Gemm(const pih_amd_moe_mxfp4_gemm_launch_v1* r) {
  if (!HeaderOk(r, kAbi) || !OutOk(r->output_type) ||
      (r->activation_type != PIH_AMD_ACTIVATION_E4M3_V1 &&
       r->activation_type != PIH_AMD_ACTIVATION_BF16_V1))
    return Invalid("moe_mxfp4_gemm_request_invalid");
  if (r->expert_count == 0 || r->row_capacity == 0 || r->activation_rows == 0)
    return Invalid("moe_mxfp4_gemm_shape_invalid");
  Fp4GemmArgs a;
  a.a = Ptr<const void>(r->activation);
  a.a_scale = Ptr<const uint8_t>(r->activation_scale_ue8m0);
  a.a_gather = Ptr<const uint32_t>(r->row_token_u32);
  a.w = Ptr<const uint8_t>(r->packed_weight);
  a.w_scale = Ptr<const uint8_t>(r->weight_scale_ue8m0);
  a.offsets = Ptr<const uint32_t>(r->expert_offsets_u32);
  a.row_weight = Ptr<const float>(r->row_weight_f32);
  a.out = Ptr<void>(r->output);
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.m = r->row_capacity;
  a.n = r->n;
  a.k = r->k;
  a.problems = r->expert_count;
  a.a_rows_total = r->activation_rows;
  a.moe = true;
  a.act = (ActKind)r->activation_type;
  a.out_kind = (OutKind)r->output_type;
  a.swiglu_limit = r->swiglu_limit;
  return LaunchFp4Gemm(a);
}

St MoeCombine(const pih_amd_moe_combine_launch_v1* r) {
  if (!HeaderOk(r, kAbi)) return Invalid("moe_combine_request_invalid");
  CombineArgs a;
  a.expert_out = Ptr<const uint16_t>(r->expert_output_bf16);
  a.token_rows = Ptr<const uint32_t>(r->token_rows_u32);
  a.shared = Ptr<const uint16_t>(r->shared_bf16);
  a.out = Ptr<uint16_t>(r->output_bf16);
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.tokens = r->token_count;
  a.topk = r->top_k;
  a.hidden = r->hidden_size;
  a.rows = r->row_count;
  return LaunchMoeCombine(a);
}

St Bf16Gemm(const pih_amd_bf16_gemm_launch_v1* r) {
  if (!HeaderOk(r, kAbi) ||
      (r->output_type != PIH_AMD_OUTPUT_BF16_V1 && r->output_type != PIH_AMD_OUTPUT_F32_V1))
    return Invalid("bf16_gemm_request_invalid");
  Bf16GemmArgs a;
  a.a = Ptr<const uint16_t>(r->a_bf16);
  a.w = Ptr<const uint16_t>(r->w_bf16);
  a.out = Ptr<void>(r->output);
  a.workspace = Ptr<void>(r->workspace);
  a.workspace_bytes = r->workspace_bytes;
  a.stream = AsStream(r->stream);
  a.m = r->m;
  a.n = r->n;
  a.k = r->k;
  a.out_kind = (OutKind)r->output_type;
  return LaunchBf16Gemm(a);
}

St W4a16(const pih_amd_w4a16_launch_v1* r) {
  if (!HeaderOk(r, kAbi) ||
      (r->format != PIH_AMD_W4A16_SYMMETRIC_V1 && r->format != PIH_AMD_W4A16_ASYMMETRIC_V1))
    return Invalid("w4a16_request_invalid");
  W4a16Args a;
  a.x = Ptr<const uint16_t>(r->input_bf16);
  a.qweight = Ptr<const void>(r->qweight);
  a.scales = Ptr<const uint16_t>(r->scales);
  a.zeros = Ptr<const uint32_t>(r->zeros);
  a.out = Ptr<uint16_t>(r->output_bf16);
  a.workspace = Ptr<void>(r->workspace);
  a.workspace_bytes = r->workspace_bytes;
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.m = r->m;
  a.n = r->n;
  a.k = r->k;
  a.symmetric = r->format == PIH_AMD_W4A16_SYMMETRIC_V1;
  return LaunchW4a16(a);
}

St W4a16Grouped(const pih_amd_w4a16_grouped_launch_v1* r) {
  if (!HeaderOk(r, kAbi) ||
      (r->format != PIH_AMD_W4A16_SYMMETRIC_V1 && r->format != PIH_AMD_W4A16_ASYMMETRIC_V1))
    return Invalid("w4a16_grouped_request_invalid");
  if (!r->problems || r->problem_count == 0 || r->problem_count > PIH_AMD_W4A16_GROUP_MAX_V1)
    return Invalid("w4a16_grouped_problem_count_invalid");
  const auto* probs = Ptr<const pih_amd_w4a16_problem_v1>(r->problems);
  W4a16Args a[PIH_AMD_W4A16_GROUP_MAX_V1];
  for (uint32_t i = 0; i < r->problem_count; ++i) {
    a[i].x = Ptr<const uint16_t>(probs[i].input_bf16);
    a[i].qweight = Ptr<const void>(probs[i].qweight);
    a[i].scales = Ptr<const uint16_t>(probs[i].scales);
    a[i].zeros = Ptr<const uint32_t>(probs[i].zeros);
    a[i].out = Ptr<uint16_t>(probs[i].output_bf16);
    a[i].error_flag = Ptr<uint32_t>(r->error_flag_u32);
    a[i].stream = AsStream(r->stream);
    a[i].m = r->m;
    a[i].n = probs[i].n;
    a[i].k = r->k;
    a[i].symmetric = r->format == PIH_AMD_W4A16_SYMMETRIC_V1;
  }
  return LaunchW4a16Grouped(a, r->problem_count);
}

MoeLayerArgs LayerArgs(const pih_amd_moe_layer_launch_v1* r) {
  MoeLayerArgs a;
  a.x = Ptr<const uint16_t>(r->input_bf16);
  a.topk_ids = Ptr<const uint32_t>(r->topk_ids_u32);
  a.topk_weights = Ptr<const float>(r->topk_weights_f32);
  a.w13 = Ptr<const void>(r->w13);
  a.w13_scale = Ptr<const void>(r->w13_scale);
  a.w2 = Ptr<const void>(r->w2);
  a.w2_scale = Ptr<const void>(r->w2_scale);
  a.shared = Ptr<const uint16_t>(r->shared_bf16);
  a.out = Ptr<uint16_t>(r->output_bf16);
  a.workspace = Ptr<void>(r->workspace);
  a.workspace_bytes = r->workspace_bytes;
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.tokens = r->token_count;
  a.topk = r->top_k;
  a.experts = r->expert_count;
  a.hidden = r->hidden_size;
  a.inter = r->intermediate_size;
  a.weight_format = (WeightFmt)r->weight_format;
  a.scale_fmt = (ScaleFmt)r->scale_format;
  a.act = (ActKind)r->activation_type;
  a.swiglu_limit = r->swiglu_limit;
  return a;
}

St QueryMoeLayer(const pih_amd_moe_layer_launch_v1* r) {
  if (!HeaderOk(r, kAbi) || !r->required_bytes_u64) return Invalid("moe_layer_query_invalid");
  const uint64_t bytes = MoeLayerWorkspaceBytes(LayerArgs(r));
  if (bytes == 0) return Invalid("moe_layer_shape_invalid");
  *Ptr<uint64_t>(r->required_bytes_u64) = bytes;
  return Ok();
}

St MoeLayer(const pih_amd_moe_layer_launch_v1* r) {
  if (!HeaderOk(r, kAbi)) return Invalid("moe_layer_request_invalid");
  return LaunchMoeLayer(LayerArgs(r));
}

St SiluMul(const pih_amd_silu_mul_launch_v1* r) {
  if (!HeaderOk(r, kAbi)) return Invalid("silu_mul_request_invalid");
  SiluMulArgs a;
  a.gate = Ptr<const uint16_t>(r->gate_bf16);
  a.up = Ptr<const uint16_t>(r->up_bf16);
  a.out = Ptr<uint16_t>(r->output_bf16);
  a.stream = AsStream(r->stream);
  a.count = r->count;
  return LaunchSiluMul(a);
}

St SwiGlu(const pih_amd_swiglu_launch_v1* r) {
  if (!HeaderOk(r, kAbi)) return Invalid("swiglu_request_invalid");
  SwiGluArgs a;
  a.gate = Ptr<const uint16_t>(r->gate_bf16);
  a.up = Ptr<const uint16_t>(r->up_bf16);
  a.weights = Ptr<const float>(r->route_weights_f32);
  a.out = Ptr<uint16_t>(r->output_bf16);
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.rows = r->rows;
  a.cols = r->cols;
  a.limit = r->limit;
  return LaunchSwiGlu(a);
}

St Mxfp4Decode(const pih_amd_mxfp4_decode_launch_v1* r) {
  if (!HeaderOk(r, kAbi)) return Invalid("mxfp4_decode_request_invalid");
  Mxfp4DecodeArgs a;
  a.packed = Ptr<const uint8_t>(r->packed);
  a.scales = Ptr<const uint8_t>(r->scales_ue8m0);
  a.out = Ptr<uint16_t>(r->output_bf16);
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.rows = r->rows;
  a.k = r->k;
  return LaunchMxfp4Decode(a);
}

St W4a16Dequant(const pih_amd_w4a16_dequant_launch_v1* r) {
  if (!HeaderOk(r, kAbi) ||
      (r->format != PIH_AMD_W4A16_SYMMETRIC_V1 && r->format != PIH_AMD_W4A16_ASYMMETRIC_V1))
    return Invalid("w4a16_dequant_request_invalid");
  W4a16Args a;
  a.qweight = Ptr<const void>(r->qweight);
  a.scales = Ptr<const uint16_t>(r->scales);
  a.zeros = Ptr<const uint32_t>(r->zeros);
  a.error_flag = Ptr<uint32_t>(r->error_flag_u32);
  a.stream = AsStream(r->stream);
  a.n = r->n;
  a.k = r->k;
  a.symmetric = r->format == PIH_AMD_W4A16_SYMMETRIC_V1;
  return LaunchW4a16Dequant(a, Ptr<float>(r->output_f32));
}

PIH_AMD_CONTAINED(CQueryWorkspace, QueryWorkspace, pih_amd_workspace_query_v1)
PIH_AMD_CONTAINED(CRoutePlan, RoutePlan, pih_amd_route_plan_launch_v1)
PIH_AMD_CONTAINED(CFp8Quant, Fp8Quant, pih_amd_fp8_quant_launch_v1)
PIH_AMD_CONTAINED(CFp8Gemm, Fp8Gemm, pih_amd_fp8_gemm_launch_v1)
PIH_AMD_CONTAINED(CMoeFp8Gemm, MoeFp8Gemm, pih_amd_moe_fp8_gemm_launch_v1)
PIH_AMD_CONTAINED(CMoeMxfp4Gemm, MoeMxfp4Gemm, pih_amd_moe_mxfp4_gemm_launch_v1)
PIH_AMD_CONTAINED(CMoeCombine, MoeCombine, pih_amd_moe_combine_launch_v1)
PIH_AMD_CONTAINED(CBf16Gemm, Bf16Gemm, pih_amd_bf16_gemm_launch_v1)
PIH_AMD_CONTAINED(CW4a16, W4a16, pih_amd_w4a16_launch_v1)
PIH_AMD_CONTAINED(CSiluMul, SiluMul, pih_amd_silu_mul_launch_v1)
PIH_AMD_CONTAINED(CSwiGlu, SwiGlu, pih_amd_swiglu_launch_v1)
PIH_AMD_CONTAINED(CMxfp4Decode, Mxfp4Decode, pih_amd_mxfp4_decode_launch_v1)
PIH_AMD_CONTAINED(CW4a16Dequant, W4a16Dequant, pih_amd_w4a16_dequant_launch_v1)
PIH_AMD_CONTAINED(CW4a16Grouped, W4a16Grouped, pih_amd_w4a16_grouped_launch_v1)
PIH_AMD_CONTAINED(CQueryMoeLayer, QueryMoeLayer, pih_amd_moe_layer_launch_v1)
PIH_AMD_CONTAINED(CMoeLayer, MoeLayer, pih_amd_moe_layer_launch_v1)
PIH_AMD_CONTAINED(CRoutePlanNoAlloc, RoutePlanNoAlloc, pih_amd_route_plan_launch_v1)
PIH_AMD_CONTAINED(CRouterTopk, RouterTopk, pih_amd_router_topk_launch_v1)
PIH_AMD_CONTAINED(CV41Linear, V41Linear, pih_amd_v41_linear_launch_v1)
PIH_AMD_CONTAINED(CV41Fp4ToFp8, V41Fp4ToFp8, pih_amd_v41_fp4_to_fp8_launch_v1)
PIH_AMD_CONTAINED(CV41BlockDequant, V41BlockDequant, pih_amd_v41_block_dequant_launch_v1)

const pih_amd_linear_kernels_api_v1 kContract = {
    sizeof(pih_amd_linear_kernels_api_v1), kAbi, &kIdentity, &CQueryWorkspace, &CRoutePlan,
    &CFp8Quant, &CFp8Gemm, &CMoeFp8Gemm, &CMoeMxfp4Gemm, &CMoeCombine, &CBf16Gemm, &CW4a16,
    &CSiluMul, &CSwiGlu, &CMxfp4Decode, &CW4a16Dequant, &CW4a16Grouped, &CQueryMoeLayer, &CMoeLayer,
    &CRoutePlanNoAlloc, &CRouterTopk, &CV41Linear, &CV41Fp4ToFp8, &CV41BlockDequant};

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

// One MoE expert layer per call: the C++ host sequence that replaces the
// reference's per-expert submission loop (plugins/model-deepseek-v4-flash/
// cuda/deepseek_expert_cuda_backend.cpp:23-103, which gathers, quantises,
// runs W1/W3, SwiGLU, re-quantises, runs W2 and accumulates expert by expert
// with a host event poll between experts) and its host route plan
// (deepseek_expert_subwave_plan.cpp:32-101).  Here every stage is one launch
// over all experts, enqueued back to back on the caller's stream with no
// host synchronisation:
//   route plan + activation quant -> grouped gate/up GEMM (+ SwiGLU x route
//   weight) -> intermediate quant -> grouped down GEMM -> ordered combine.
// The activation quant does not depend on the routing, so its blocks ride in
// the route plan's first launch (the route-mask blocks first); it is not a
// prologue of the gate/up GEMM because every token row feeds top_k experts
// times n / 256 tiles there and would be quantised that many times over.
// FP8 weights fold the intermediate quant into the gate/up epilogue (one
// launch and the bf16 intermediate's write and read fewer); it quantises the
// bf16-rounded SwiGLU values with the quant entry's arithmetic, so the
// layer's output still equals launching the stages one by one.
//
// Weights: FP8 e4m3 with 128x128 block scales (fp32 or UE8M0), or MXFP4
// (e2m1 + UE8M0 per 32 k) with e4m3 (UE8M0 per 128) or bf16 activations.
// Scratch (caller-provided, sized by MoeLayerWorkspaceBytes) holds the route
// plan, the quantised activations, the intermediate and the expert outputs.
#include "kernels.hpp"

namespace pih_amd {
namespace {

constexpr uint64_t kAlign = 256;

uint64_t Up(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct Carve {
  uint64_t route_ws = 0, offsets = 0, row_token = 0, row_weight = 0, token_rows = 0;
  uint64_t xq = 0, xs = 0, mid = 0, mq = 0, ms = 0, y = 0, total = 0;
  bool quant_x = false, quant_mid = false;
};

// Offsets of every scratch buffer; `total` is the size the caller provides.
Carve Layout(const MoeLayerArgs& a) {
  Carve c;
  const uint64_t T = a.tokens, R = (uint64_t)a.tokens * a.topk, H = a.hidden, I = a.inter;
  const bool fp8 = a.weight_format == kWeightFp8;
  c.quant_x = c.quant_mid = fp8 || a.act == kActE4m3;
  const uint64_t ssz = fp8 && a.scale_fmt == kScaleF32 ? 4 : 1;  // MXFP4 activations: UE8M0
  uint64_t o = 0;
  auto take = [&](uint64_t& at, uint64_t bytes) {
    at = o;
    o += Up(bytes);
  };
  take(c.route_ws, RoutePlanWorkspaceBytes(a.tokens, a.topk, a.experts));
  take(c.offsets, (uint64_t)(a.experts + 1) * 4);
  take(c.row_token, R * 4);
  take(c.row_weight, R * 4);
  take(c.token_rows, R * 4);
  if (c.quant_x) {
    take(c.xq, T * H);
    take(c.xs, T * (H / 128) * ssz);
  }
  // FP8 weights: the gate/up epilogue writes the e4m3 intermediate
  // directly, so only MXFP4 needs the bf16 one
  if (!fp8) take(c.mid, R * I * 2);
  if (c.quant_mid) {
    take(c.mq, R * I);
    take(c.ms, R * (I / 128) * ssz);
  }
  take(c.y, R * H * 2);
  c.total = o;
  return c;
}

St Check(const MoeLayerArgs& a) {
  if (a.tokens == 0 || a.topk == 0 || a.topk > 32 || a.experts == 0 || a.experts > 1024)
    return Invalid("moe_layer_routing_shape_invalid");
  if (a.hidden == 0 || a.hidden % 128 || a.inter == 0 || a.inter % 128)
    return Invalid("moe_layer_dims_invalid");
  if ((uint64_t)a.tokens * a.topk > 0xffffffffull) return Invalid("moe_layer_too_many_routes");
  if (a.weight_format != kWeightFp8 && a.weight_format != kWeightMxfp4) return Invalid("moe_layer_format_invalid");
  if (a.weight_format == kWeightFp8 && a.scale_fmt != kScaleF32 && a.scale_fmt != kScaleUe8m0)
    return Invalid("moe_layer_scale_format_invalid");
  if (a.weight_format == kWeightMxfp4 && a.act != kActE4m3 && a.act != kActBf16)
    return Invalid("moe_layer_activation_invalid");
  return Ok();
}

}  // namespace

uint64_t MoeLayerWorkspaceBytes(const MoeLayerArgs& a) { return Check(a).ok() ? Layout(a).total : 0; }

St LaunchMoeLayer(const MoeLayerArgs& a) {
  St s = Check(a);
  if (!s.ok()) return s;
  if (!a.x || !a.topk_ids || !a.topk_weights || !a.w13 || !a.w13_scale || !a.w2 || !a.w2_scale || !a.out ||
      !a.workspace || !a.error_flag || !a.stream)
    return Invalid("moe_layer_null_argument");
  const Carve c = Layout(a);
  if (a.workspace_bytes < c.total) return Invalid("moe_layer_workspace_too_small");
  uint8_t* ws = static_cast<uint8_t*>(a.workspace);
  auto at = [&](uint64_t off) { return ws + off; };
  const uint32_t R = a.tokens * a.topk;
  uint32_t* offsets = reinterpret_cast<uint32_t*>(at(c.offsets));
  uint32_t* row_token = reinterpret_cast<uint32_t*>(at(c.row_token));
  float* row_weight = reinterpret_cast<float*>(at(c.row_weight));
  uint32_t* token_rows = reinterpret_cast<uint32_t*>(at(c.token_rows));
  const bool fp8 = a.weight_format == kWeightFp8;
  uint16_t* mid = fp8 ? nullptr : reinterpret_cast<uint16_t*>(at(c.mid));
  uint16_t* y = reinterpret_cast<uint16_t*>(at(c.y));
  const ScaleFmt act_fmt = fp8 ? a.scale_fmt : kScaleUe8m0;

  RoutePlanArgs rp;
  rp.topk_ids = a.topk_ids;
  rp.topk_weights = a.topk_weights;
  rp.expert_offsets = offsets;
  rp.row_token = row_token;
  rp.row_weight = row_weight;
  rp.token_rows = token_rows;
  rp.workspace = at(c.route_ws);
  rp.workspace_bytes = c.offsets - c.route_ws;
  rp.error_flag = a.error_flag;
  rp.stream = a.stream;
  rp.tokens = a.tokens;
  rp.topk = a.topk;
  rp.experts = a.experts;

  auto quant_args = [&](const uint16_t* in, uint32_t rows, uint32_t k, uint64_t codes, uint64_t scales) {
    Fp8QuantArgs q;
    q.input = in;
    q.codes = at(codes);
    q.scales = at(scales);
    q.error_flag = a.error_flag;
    q.stream = a.stream;
    q.row_count = rows;
    q.k = k;
    q.input_rows = rows;
    q.fmt = act_fmt;
    return q;
  };
  // the token activations are quantized by the route plan's first launch
  if (c.quant_x) s = LaunchRoutePlanWithQuant(rp, quant_args(a.x, a.tokens, a.hidden, c.xq, c.xs));
  else s = LaunchRoutePlan(rp);
  if (!s.ok()) return s;

  // gate/up: logical row r reads token row_token[r]; SwiGLU x route weight
  auto gemm = [&](bool gate_up) -> St {
    const void* act = gate_up ? (c.quant_x ? (const void*)at(c.xq) : (const void*)a.x)
                              : (c.quant_mid ? (const void*)at(c.mq) : (const void*)mid);
    const void* act_scale = gate_up ? (c.quant_x ? at(c.xs) : nullptr) : (c.quant_mid ? at(c.ms) : nullptr);
    const uint32_t n = gate_up ? 2 * a.inter : a.hidden, k = gate_up ? a.hidden : a.inter;
    if (fp8) {
      BlockGemmArgs g;
      g.a = static_cast<const uint8_t*>(act);
      g.a_scale = act_scale;
      g.a_gather = gate_up ? row_token : nullptr;
      g.w = static_cast<const uint8_t*>(gate_up ? a.w13 : a.w2);
      g.w_scale = gate_up ? a.w13_scale : a.w2_scale;
      // FP8 experts: the gate/up epilogue writes the e4m3 intermediate and
      // its group scales itself (kOutSwiGluFp8, the values LaunchFp8Quant
      // would produce from the bf16 SwiGLU output)
      g.out = gate_up ? (void*)at(c.mq) : (void*)y;
      g.out_scale = gate_up ? (void*)at(c.ms) : nullptr;
      g.row_weight = gate_up ? row_weight : nullptr;
      g.offsets = offsets;
      g.error_flag = a.error_flag;
      g.stream = a.stream;
      g.m = R;
      g.n = n;
      g.k = k;
      g.problems = a.experts;
      g.a_rows_total = gate_up ? a.tokens : R;
      g.moe = true;
      g.scale_fmt = a.scale_fmt;
      g.out_kind = gate_up ? kOutSwiGluFp8 : kOutBf16;
      g.swiglu_limit = a.swiglu_limit;
      return LaunchFp8BlockGemm(g);
    }
    Fp4GemmArgs g;
    g.a = act;
    g.a_scale = static_cast<const uint8_t*>(act_scale);
    g.a_gather = gate_up ? row_token : nullptr;
    g.w = static_cast<const uint8_t*>(gate_up ? a.w13 : a.w2);
    g.w_scale = static_cast<const uint8_t*>(gate_up ? a.w13_scale : a.w2_scale);
    g.out = gate_up ? (void*)mid : (void*)y;
    g.row_weight = gate_up ? row_weight : nullptr;
    g.offsets = offsets;
    g.error_flag = a.error_flag;
    g.stream = a.stream;
    g.m = R;
    g.n = n;
    g.k = k;
    g.problems = a.experts;
    g.a_rows_total = gate_up ? a.tokens : R;
    g.moe = true;
    g.act = a.act;
    g.out_kind = gate_up ? kOutSwiGlu : kOutBf16;
    g.swiglu_limit = a.swiglu_limit;
    g.max_expert_rows = a.tokens;  // the route plan's rows: at most one per token and expert
    return LaunchFp4Gemm(g);
  };
  if (!(s = gemm(true)).ok()) return s;
  if (!fp8 && c.quant_mid && !(s = LaunchFp8Quant(quant_args(mid, R, a.inter, c.mq, c.ms))).ok()) return s;
  if (!(s = gemm(false)).ok()) return s;

  CombineArgs cb;
  cb.expert_out = y;
  cb.token_rows = token_rows;
  cb.shared = a.shared;
  cb.out = a.out;
  cb.error_flag = a.error_flag;
  cb.stream = a.stream;
  cb.tokens = a.tokens;
  cb.topk = a.topk;
  cb.hidden = a.hidden;
  cb.rows = R;
  return LaunchMoeCombine(cb);
}

}  // namespace pih_amd

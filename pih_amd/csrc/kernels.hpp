// Internal launcher interface of the gfx950 packs.  Every launcher validates
// its arguments on the host, enqueues on the caller's stream and returns St;
// none allocates memory or synchronises the host.  The pack tables
// (deepseek_pack.cpp, linear_pack.cpp) translate the C-ABI request structs
// into these calls.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "host_common.hpp"

namespace pih_amd {

enum ScaleFmt : uint32_t { kScaleF32 = 1, kScaleUe8m0 = 2 };
// kOutSwiGluFp8 (MoE FP8 GEMM only): the SwiGLU output rounded to bf16 and
// quantised to e4m3 with one scale per (row, 128 columns) in the GEMM's
// scale format, exactly as LaunchFp8Quant would quantise the bf16 output
enum OutKind : uint32_t { kOutBf16 = 1, kOutF32 = 2, kOutSwiGlu = 3, kOutSwiGluFp8 = 4 };
enum ActKind : uint32_t { kActE4m3 = 1, kActBf16 = 2 };

// ------------------------------------------------------------- FP8 quant
// Per (row, 128 columns): amax -> scale -> e4m3 codes.  kScaleUe8m0 follows
// the reference codec (deepseek_fp8_activation_codec.cpp:53-107): scale byte
// e+127 with e the least integer such that max(amax,1e-4) <= 448*2^e.
// kScaleF32 writes s = max(amax,1e-4)/448.  rows == nullptr reads input row
// r for output row r; otherwise input row rows[r] (bounded by input_rows).
struct Fp8QuantArgs {
  const uint16_t* input = nullptr;
  const uint32_t* rows = nullptr;
  uint8_t* codes = nullptr;
  void* scales = nullptr;
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t row_count = 0, k = 0, input_rows = 0;
  ScaleFmt fmt = kScaleUe8m0;
};
St LaunchFp8Quant(const Fp8QuantArgs& a);

// ------------------------------------------------- block-scaled FP8 GEMM
// out = A . W^T over one or more problems, with one scale per (A row, 128 k)
// and one per (128 W rows, 128 k), fp32 or UE8M0.  Problems are either
// strided (dense GEMM, grouped projections) or MoE segments given by
// device-resident expert offsets.
struct BlockGemmArgs {
  const uint8_t* a = nullptr;      // e4m3 [a_rows_total, k]
  const void* a_scale = nullptr;   // [a_rows_total, k/128]
  const uint32_t* a_gather = nullptr;  // MoE: logical row -> A row
  const uint8_t* w = nullptr;      // e4m3 [problems][n][k]
  const void* w_scale = nullptr;   // [problems][n/128][k/128]
  void* out = nullptr;
  void* out_scale = nullptr;           // kOutSwiGluFp8: [m, n/256] scales (codes in out)
  const float* row_weight = nullptr;   // SwiGLU epilogue, per logical row
  const uint32_t* offsets = nullptr;   // MoE: [problems+1] on device
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t m = 0;        // strided: rows per problem; MoE: total rows bound
  uint32_t n = 0, k = 0; // per-problem weight rows and depth
  uint32_t problems = 1;
  uint32_t a_rows_total = 0;
  // strided addressing: A row = i*a_row_stride + p*a_prob_row,
  // out element = out[i*out_row_stride + p*out_prob_col + col]
  uint32_t a_row_stride = 1, a_prob_row = 0;
  uint64_t out_row_stride = 0;
  uint32_t out_prob_col = 0;
  bool moe = false;
  bool check_codes = false;
  ScaleFmt scale_fmt = kScaleUe8m0;
  OutKind out_kind = kOutBf16;
  float swiglu_limit = 0.0f;  // <= 0: plain SiLU-mul
  // error bits for: invalid code / A row, UE8M0 0xFF, non-finite result
  uint32_t err_code_bit = 1u, err_scale_bit = 2u, err_nonfinite_bit = 4u;
  // a non-finite result is flagged and, when set, also stored (the
  // reference's grouped FP8 kernel stores it; its dense FP8 and FP4 kernels
  // skip the element)
  bool write_nonfinite = false;
};
St LaunchFp8BlockGemm(const BlockGemmArgs& a);
// MoE problems without the code scan (called by LaunchFp8BlockGemm after its
// checks): the 128x256-tile grouped kernel of gemm_fp8_moe.hip
St LaunchFp8MoeGemm(const BlockGemmArgs& a);

// ----------------------------------------------------- MXFP4 weight GEMM
// out = A . W^T with W e2m1 packed two per byte (low nibble = even k) and a
// UE8M0 scale per (W row, 32 k).  A is e4m3 with a UE8M0 scale per
// (row, 128 k) (reference deepseek_fp4_gemm_oracle.cpp:11-91) or bf16.
struct Fp4GemmArgs {
  const void* a = nullptr;
  const uint8_t* a_scale = nullptr;   // e4m3 activations only
  const uint32_t* a_gather = nullptr;
  const uint8_t* w = nullptr;         // [problems][n][k/2]
  const uint8_t* w_scale = nullptr;   // [problems][n][k/32]
  void* out = nullptr;
  const float* row_weight = nullptr;
  const uint32_t* offsets = nullptr;
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t m = 0, n = 0, k = 0, problems = 1, a_rows_total = 0;
  bool moe = false;
  ActKind act = kActE4m3;
  OutKind out_kind = kOutBf16;
  float swiglu_limit = 0.0f;
  // MoE: a bound on every expert's row count that the caller guarantees (0:
  // none).  The layer passes its token count (the route plan gives an
  // expert at most one row per token); at or below the light-expert limit
  // no expert can need the tiled kernels, so they are not launched.
  uint32_t max_expert_rows = 0;
};
St LaunchFp4Gemm(const Fp4GemmArgs& a);

// Small-M dense GEMM with FP8 or MXFP4 weights and e4m3 activations
// (gemm_small_m.hip): 16 weight rows and up to 64 activation rows per
// block, the block's waves splitting K.  It takes m <= 64, and m up to
// kSmallMRows while the 128 x 128 tiled kernel would have fewer than 128
// tiles (too few blocks to stream the weights).  `taken` is false when it
// does not take the shape (the caller then uses the tiled kernel); the
// callers' checks come first.
constexpr uint32_t kSmallMChunkRows = 64, kSmallMRows = 256;
inline bool SmallMTakes(uint32_t m, uint32_t n, uint32_t problems) {
  if (m <= kSmallMChunkRows) return m > 0;
  return m <= kSmallMRows && (uint64_t)((m + 127) / 128) * ((n + 127) / 128) * problems < 128;
}
St LaunchFp8SmallM(const BlockGemmArgs& a, bool& taken);
St LaunchFp4SmallM(const Fp4GemmArgs& a, bool& taken);
// MoE problems: experts with at most Fp4MoeLightRows(a) rows (64; 0 when
// the shape does not fit the streaming kernel) go to the weight-streaming
// kernel of moe_stream.hip, the others to the tiled kernel; LaunchFp4Gemm
// enqueues both on a.stream.
constexpr uint32_t kMoeLightRows = 64;
uint32_t Fp4MoeLightRows(const Fp4GemmArgs& a);
St LaunchFp4MoeStream(const Fp4GemmArgs& a);
// The other experts of an e4m3 MoE problem run on the 128 x 256 tiles of
// gemm_fp8_moe.hip with an FP4 W operand when the shape fits
// (Fp4MoeBigTileTakes), on the 128 x 128 tiles of gemm_mfma.hip otherwise.
bool Fp4MoeBigTileTakes(const Fp4GemmArgs& a);
St LaunchFp4MoeBigTile(const Fp4GemmArgs& a, uint32_t light_rows);
// One dense FP4 problem with e4m3 activations on the 128 x 256 tiles (every
// block exits at once when *skip_if holds skip_bit)
bool Fp4DenseBigTileTakes(const Fp4GemmArgs& a);
St LaunchFp4DenseBigTile(const Fp4GemmArgs& a, const uint32_t* skip_if, uint32_t skip_bit);

// ------------------------------------------------------------- BF16 GEMM
// C[m,n] = A[m,k] . W[n,k]^T, fp32 accumulate, bf16 or fp32 out.
struct Bf16GemmArgs {
  const uint16_t* a = nullptr;
  const uint16_t* w = nullptr;
  void* out = nullptr;
  void* workspace = nullptr;
  uint64_t workspace_bytes = 0;
  hipStream_t stream = nullptr;
  uint32_t m = 0, n = 0, k = 0;
  OutKind out_kind = kOutBf16;
  // optional: a non-finite output is stored and ORs nonfinite_bit into
  // *error_flag (the DeepSeek LM head's bit 128)
  uint32_t* error_flag = nullptr;
  uint32_t nonfinite_bit = 0;
};
St LaunchBf16Gemm(const Bf16GemmArgs& a);

// Dense GEMM on the MoE kernel's 128 x 256 tiles (gemm_fp8_moe.hip), one or
// more strided problems: out [m, n] = A [m, k] . W [n, k]^T, either
// e4m3 with 128x128 block scales (fp32 or UE8M0, no NaN-code handling) or
// bf16.  n % 128 == 0, k % 128 (e4m3) or % 64 (bf16) == 0.
struct BigTileArgs {
  const void* a = nullptr;
  const void* a_scale = nullptr;
  const void* w = nullptr;
  const void* w_scale = nullptr;
  void* out = nullptr;
  uint32_t* error_flag = nullptr;  // optional for bf16
  hipStream_t stream = nullptr;
  uint32_t m = 0, n = 0, k = 0;
  // strided problems (W [problems][n][k]): A row i of problem q is
  // i * a_row_stride + q * a_prob_row (< a_rows_total, 0 = m * problems);
  // its output row starts at i * out_row_stride (0 = n) + q * out_prob_col
  uint32_t problems = 1, a_rows_total = 0, a_row_stride = 1, a_prob_row = 0;
  uint64_t out_row_stride = 0, out_prob_col = 0;
  bool bf16 = false;
  ScaleFmt scale_fmt = kScaleF32;
  OutKind out_kind = kOutBf16;
  uint32_t err_code_bit = 1u, err_scale_bit = 2u, err_nonfinite_bit = 4u;
  bool write_nonfinite = false;
  // when set, every block exits at once if (*skip_if & skip_bit) != 0
  const uint32_t* skip_if = nullptr;
  uint32_t skip_bit = 0;
  // > 1: one problem with K split into this many equal parts; `out` then
  // holds k_splits fp32 slabs [m][out_row_stride] of partial sums, summed
  // by LaunchSplitKReduce (out_kind kOutF32)
  uint32_t k_splits = 1;
  // FP8, one problem of contiguous rows, A and W on 16-byte boundaries:
  // the reference's NaN-code semantics (a code decodes as 0 and raises
  // err_code_bit).  A persistent launch handles them in its tiles
  // (*codes_in_tiles set); otherwise a scan raises the bit before the tiles,
  // which then exit at once if it is set, and the caller enqueues the
  // checking kernel, which computes the result when the bit is set.
  // skip_if is not used.
  bool code_check = false;
};
St LaunchBigTileGemm(const BigTileArgs& a, bool* codes_in_tiles = nullptr);
// K splits for a dense big-tile GEMM of k_steps 128-byte K steps (1: none):
// below a round of tiles on the 256 CUs
uint32_t DenseKSplits(uint32_t m, uint32_t n, uint32_t k_steps);
// out[m, n] = sum over the splits in order of ws[q][m][n] (bf16 or fp32)
St LaunchSplitKReduce(const float* ws, uint32_t splits, uint32_t m, uint32_t n, void* out, OutKind out_kind,
                      uint32_t* err, uint32_t bit, hipStream_t stream);

// ORs `bit` into *error_flag when A or W holds an e4m3 NaN code (0x7F or
// 0xFF byte) -- the test the big-tile FP8 path runs before it trusts the
// MFMA to see no NaN codes (elementwise.hip).
struct NanCodeScanArgs {
  const void* a = nullptr;
  uint64_t a_bytes = 0;
  const void* w = nullptr;
  uint64_t w_bytes = 0;
  uint32_t* error_flag = nullptr;
  uint32_t bit = 0;
  hipStream_t stream = nullptr;
};
St LaunchNanCodeScan(const NanCodeScanArgs& a);
// the big-tile path pays from 64 tiles on (measured at M = 2048: N = 1024,
// 64 tiles on 64 CUs, 40.7 us against 64 us for the 128 x 128 kernel's 128
// tiles)
inline bool BigTileWorthIt(uint32_t m, uint32_t n) {
  return m >= 256 && (uint64_t)((m + 127) / 128) * ((n + 255) / 256) >= 64;
}
// BF16 GEMMs above 64 rows take the big tiles (K split into the queried
// workspace when their tiles are few) from 512-deep K and 256 columns on:
// against the 128 x 128 kernel, Qwen3-8B projections at M 65-384 ran
// 1.3-3.8x faster (4096 -> 4096 M 192 64 -> 25 us, 12288 -> 4096 M 192
// 181 -> 47 us, 4096 -> 1024 M 1024 58 -> 28 us) and nowhere slower.
inline bool Bf16BigTiles(uint32_t m, uint32_t n, uint32_t k) {
  return BigTileWorthIt(m, n) || (m > 64 && k >= 512 && n >= 256);
}
uint64_t Bf16GemmWorkspaceBytes(uint32_t m, uint32_t n, uint32_t k);
// decode shapes (m <= 64): the weight-streaming GEMV with split-K
St LaunchBf16Gemv(const Bf16GemmArgs& a);
uint64_t Bf16GemvWorkspaceBytes(uint32_t m, uint32_t n, uint32_t k);

// ------------------------------------------------------------- W4A16 GEMV
struct W4a16Args {
  const uint16_t* x = nullptr;       // bf16 [m, k]
  const void* qweight = nullptr;     // asym: u32 [n, k/8]; sym: u8 [n, k/2]
  const uint16_t* scales = nullptr;  // asym: bf16 [n, k/128]; sym: fp16
  const uint32_t* zeros = nullptr;   // asym: u32 [n, ceil(k/1024)]
  uint16_t* out = nullptr;           // bf16 [m, n]
  void* workspace = nullptr;
  uint64_t workspace_bytes = 0;
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t m = 0, n = 0, k = 0;
  bool symmetric = false;
};
St LaunchW4a16(const W4a16Args& a);
// up to 8 problems with one m, k and format in one launch (x, qweight,
// scales, zeros, out and n per problem; the rest from probs[0])
St LaunchW4a16Grouped(const W4a16Args* probs, uint32_t count);
uint64_t W4a16WorkspaceBytes(uint32_t m, uint32_t n, uint32_t k);
// exact dequant (q - z) * s (or q * s) to fp32 [n, k]
St LaunchW4a16Dequant(const W4a16Args& a, float* out);

// ---------------------------------------------------------- router top-k
// Raw router scores [tokens, experts] -> ids u32 / weights f32 [tokens,
// topk] in rank order (router.hip).  Error bits: 1 non-finite score,
// 2 non-finite bias, 4 top-k weight sum invalid.
enum RouterMode : uint32_t { kRouterSoftmax = 1, kRouterSqrtSoftplus = 2 };
struct RouterTopkArgs {
  const float* scores = nullptr;  // [tokens, experts]
  const float* bias = nullptr;    // [experts], sqrt-softplus selection only (nullptr: 0)
  uint32_t* ids = nullptr;        // [tokens, topk]
  float* weights = nullptr;       // [tokens, topk]
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t tokens = 0, experts = 0, topk = 0;
  uint32_t mode = kRouterSoftmax;
  float scale = 1.0f;
};
St LaunchRouterTopk(const RouterTopkArgs& a);

// --------------------------------------------------------------- MoE glue
struct RoutePlanArgs {
  const uint32_t* topk_ids = nullptr;     // [tokens, topk]
  const float* topk_weights = nullptr;    // [tokens, topk]
  uint32_t* expert_offsets = nullptr;     // [experts + 1]
  uint32_t* row_token = nullptr;          // [tokens * topk]
  float* row_weight = nullptr;            // [tokens * topk]
  uint32_t* token_rows = nullptr;         // [tokens * topk]
  void* workspace = nullptr;
  uint64_t workspace_bytes = 0;
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t tokens = 0, topk = 0, experts = 0;
};
St LaunchRoutePlan(const RoutePlanArgs& a);
// The route plan whose first launch also quantizes the token activations
// (quant: input [tokens, k] bf16, no row gather, same stream and error flag)
// -- the MoE layer's activation quant without a launch of its own.
St LaunchRoutePlanWithQuant(const RoutePlanArgs& a, const Fp8QuantArgs& quant);
uint64_t RoutePlanWorkspaceBytes(uint32_t tokens, uint32_t topk, uint32_t experts);
// LaunchRoutePlan with the pack's own per-device scratch array instead of a
// caller workspace (a.workspace and a.workspace_bytes must be 0); plans
// needing more than kRoutePlanNoAllocScratchBytes are rejected.  Calls that
// overlap on one device share the array and race.
constexpr uint64_t kRoutePlanNoAllocScratchBytes = 1ull << 20;
St LaunchRoutePlanNoAlloc(const RoutePlanArgs& a);

struct GatherArgs {
  const uint16_t* source = nullptr;   // bf16 [tokens, hidden]
  const uint32_t* token_index = nullptr;  // [routes]
  uint16_t* dest = nullptr;           // bf16 [routes, hidden]
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t routes = 0, tokens = 0, hidden = 0;
};
St LaunchRouteGather(const GatherArgs& a);

// Ordered accumulate: acc[token[r], :] += out[r, :] for r in order.
struct AccumulateArgs {
  const uint16_t* expert_out = nullptr;  // bf16 [routes, hidden]
  const uint32_t* token_index = nullptr;
  float* acc = nullptr;                  // [tokens, hidden]
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t routes = 0, tokens = 0, hidden = 0;
};
St LaunchOrderedAccumulate(const AccumulateArgs& a);

// Combine: out[t,:] = bf16(sum over t's rows in ascending row order + shared)
struct CombineArgs {
  const uint16_t* expert_out = nullptr;  // bf16 [rows, hidden]
  const uint32_t* token_rows = nullptr;  // [tokens, topk]
  const uint16_t* shared = nullptr;      // bf16 [tokens, hidden] or null
  uint16_t* out = nullptr;               // bf16 [tokens, hidden]
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t tokens = 0, topk = 0, hidden = 0, rows = 0;
};
St LaunchMoeCombine(const CombineArgs& a);

// One MoE expert layer (route plan -> quant -> gate/up -> quant -> down ->
// combine) on the caller's stream; moe_layer.cpp.
enum WeightFmt : uint32_t { kWeightFp8 = 1, kWeightMxfp4 = 2 };
struct MoeLayerArgs {
  const uint16_t* x = nullptr;          // bf16 [tokens, hidden]
  const uint32_t* topk_ids = nullptr;   // [tokens, topk]
  const float* topk_weights = nullptr;  // [tokens, topk]
  const void* w13 = nullptr;            // fp8 [E][2I][H] or e2m1 [E][2I][H/2]
  const void* w13_scale = nullptr;      // fp8 [E][2I/128][H/128]; mxfp4 UE8M0 [E][2I][H/32]
  const void* w2 = nullptr;             // fp8 [E][H][I] or e2m1 [E][H][I/2]
  const void* w2_scale = nullptr;
  const uint16_t* shared = nullptr;     // bf16 [tokens, hidden] or null
  uint16_t* out = nullptr;              // bf16 [tokens, hidden]
  void* workspace = nullptr;
  uint64_t workspace_bytes = 0;
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t tokens = 0, topk = 0, experts = 0, hidden = 0, inter = 0;
  WeightFmt weight_format = kWeightFp8;
  ScaleFmt scale_fmt = kScaleF32;  // FP8 weights and their activations
  ActKind act = kActE4m3;          // MXFP4 weights: e4m3 (UE8M0) or bf16 activations
  float swiglu_limit = 0.0f;
};
uint64_t MoeLayerWorkspaceBytes(const MoeLayerArgs& a);  // 0 for an invalid shape
St LaunchMoeLayer(const MoeLayerArgs& a);

struct FinalizeArgs {
  const float* acc = nullptr;
  const uint16_t* shared = nullptr;
  uint16_t* out = nullptr;
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint64_t count = 0;
};
St LaunchFinalize(const FinalizeArgs& a);

// ------------------------------------------------------------ elementwise
// out = bf16(silu(min(g,L)) * clamp(u,-L,L) * w[row]) with L <= 0 meaning no
// clamp and weights == nullptr meaning 1.
struct SwiGluArgs {
  const uint16_t* gate = nullptr;
  const uint16_t* up = nullptr;
  const float* weights = nullptr;
  uint16_t* out = nullptr;
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t rows = 0, cols = 0;
  float limit = 0.0f;
};
St LaunchSwiGlu(const SwiGluArgs& a);

struct SiluMulArgs {
  const uint16_t* gate = nullptr;
  const uint16_t* up = nullptr;
  uint16_t* out = nullptr;
  hipStream_t stream = nullptr;
  uint64_t count = 0;
};
St LaunchSiluMul(const SiluMulArgs& a);

struct Mxfp4DecodeArgs {
  const uint8_t* packed = nullptr;
  const uint8_t* scales = nullptr;
  uint16_t* out = nullptr;
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t rows = 0, k = 0;
};
St LaunchMxfp4Decode(const Mxfp4DecodeArgs& a);

// Sets set_bit in *error_flag when a bf16 element of x or w is non-finite,
// scanning only when trigger_bit is already set (elementwise.hip).
struct NonfiniteScanArgs {
  const uint16_t* x = nullptr;
  const uint16_t* w = nullptr;
  uint64_t x_elems = 0, w_elems = 0;  // multiples of 8, 16-byte aligned pointers
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t trigger_bit = 0, set_bit = 0;
};
St LaunchNonfiniteScan(const NonfiniteScanArgs& a);

// ------------------------------------------- DeepSeek V4.1 32-block formats
// (v41_formats.hip, gemm_mfma.hip; plugins/model-deepseek-v41)
struct V41Quant32Args {
  const uint16_t* input = nullptr;  // bf16 [rows, k]
  uint8_t* codes = nullptr;         // e4m3 [rows, k]
  uint8_t* scales = nullptr;        // UE8M0 [rows, k/32]
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t rows = 0, k = 0;
};
St LaunchV41Quant32(const V41Quant32Args& a);
// out bf16 [m, n] = A . W^T with A e4m3 + UE8M0 per (row, 32 k) and W e4m3
// + UE8M0 per (32 rows, 32 k) or W e2m1 + UE8M0 per (row, 32 k), on the
// MX MFMA (each lane group's scale covers its 32-deep k block).  Error bit
// 1: a NaN code or a 255 scale; 2: a non-finite output (stored).
struct Mx32GemmArgs {
  const uint8_t* a = nullptr;
  const uint8_t* a_scale = nullptr;
  const uint8_t* w = nullptr;
  const uint8_t* w_scale = nullptr;
  uint16_t* out = nullptr;
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t m = 0, n = 0, k = 0;
  bool fp4_weight = false;
};
St LaunchMx32Gemm(const Mx32GemmArgs& a);
struct V41Fp4ToFp8Args {
  const uint8_t* packed = nullptr;  // e2m1 [rows, cols/2]
  const uint8_t* scales = nullptr;  // UE8M0 [rows, cols/32]
  uint8_t* weight = nullptr;        // e4m3 [rows, cols]
  uint8_t* weight_scales = nullptr; // UE8M0 [rows/32, cols/32]
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t rows = 0, cols = 0;
};
St LaunchV41Fp4ToFp8(const V41Fp4ToFp8Args& a);
struct V41BlockDequantArgs {
  const uint8_t* source = nullptr;  // e4m3 [rows, cols]
  const void* scales = nullptr;     // [rows/block, cols/block] UE8M0 or fp32
  uint16_t* output = nullptr;       // bf16 [rows, cols]
  uint32_t* error_flag = nullptr;
  hipStream_t stream = nullptr;
  uint32_t rows = 0, cols = 0, block = 0;
  uint32_t scale_f32 = 0;
};
St LaunchV41BlockDequant(const V41BlockDequantArgs& a);

}  // namespace pih_amd

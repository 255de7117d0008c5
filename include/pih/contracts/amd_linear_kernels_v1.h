/* AMD linear-layer Kernel Pack contract (contract id
 * "pih.amd-linear-kernels.v1"), function-table ABI version 1.
 *
 * The entries here have no one-to-one counterpart in the reference's
 * pih_deepseek_kernels_api_v1 table; each names the reference code whose
 * work it takes over:
 *   launch_route_plan      host DeepSeekExpertSubwavePlan::materialize
 *                          (plugins/model-deepseek-v4-flash/
 *                          deepseek_expert_subwave_plan.cpp:32-101), moved
 *                          onto the device (histogram, prefix scan, stable
 *                          permutation) so no D2H copy or host sort sits
 *                          between router and experts;
 *   launch_fp8_quant       fp8_activation_quant (deepseek_kernels_v1.h
 *                          entry 3) with fp32 or UE8M0 scales, any K%128,
 *                          optional row gather;
 *   launch_fp8_gemm        fp8_gemm (entry 4) with fp32 or UE8M0 scales;
 *   launch_moe_fp8_gemm    the per-expert loop of DeepSeekExpertCudaBackend
 *                          (plugins/model-deepseek-v4-flash/cuda/
 *                          deepseek_expert_cuda_backend.cpp:23-103) as ONE
 *                          grouped launch over every expert's contiguous row
 *                          segment, FP8 weights with 128x128 block scales,
 *                          optional fused gate/up SwiGLU*route-weight
 *                          epilogue;
 *   launch_moe_mxfp4_gemm  the same over MXFP4 (e2m1 + UE8M0/32) weights
 *                          (fp4_gemm, entry 10, generalised);
 *   launch_moe_combine     ordered_expert_accumulate + expert_finalize
 *                          (entries 12 and 29) for all experts at once, in
 *                          the same fp32 add order;
 *   launch_bf16_gemm       GemmPlan::execute (src/backend/cuda/
 *                          gemm_plan.cpp:169-198): C = A.W^T, bf16 in, fp32
 *                          accumulate, bf16 or fp32 out;
 *   launch_w4a16_gemm      pih_qwen_w4a16_gemm_compat_v1 (kernels/cuda/
 *                          qwen_bf16_primitives.cu:98-149) in the
 *                          reference's symmetric format and the asymmetric
 *                          u32-packed format;
 *   launch_silu_mul, launch_swiglu, launch_mxfp4_decode
 *                          pih_qwen_silu_mul_bf16_v1, expert/shared SwiGLU
 *                          (entries 11 and 28), deepseek_mxfp4_decode;
 *   launch_w4a16_dequant   the INT4 unpack of the W4A16 GEMV on its own
 *                          (the reference's quantizer format,
 *                          plugins/offline-qwen/
 *                          qwen3_int4_reference_quantizer.cpp:30-108);
 *   query_moe_layer_workspace, launch_moe_layer
 *                          DeepSeekExpertCudaBackend::submit's whole
 *                          per-expert loop (cuda/deepseek_expert_cuda_
 *                          backend.cpp:23-103) as one host call that
 *                          enqueues the six grouped stages above;
 *   launch_w4a16_grouped   several launch_w4a16_gemm problems with one m
 *                          and K in one launch (the Qwen decode step's
 *                          q/k/v and gate/up projections each read the
 *                          same input; the reference issues one launch per
 *                          projection, qwen3_int4_gemm_plan.cpp:55-85);
 *   launch_route_plan_noalloc
 *                          launch_route_plan with the pack's own scratch
 *                          (no reference counterpart; for callers that
 *                          cannot allocate);
 *   launch_router_topk     the host DeepSeekLearnedRouter::Route
 *                          (plugins/model-deepseek-v4-flash/
 *                          deepseek_learned_router.cpp:21-94) on the device,
 *                          plus BASELINE's softmax top-k, so router scores
 *                          never travel to the host;
 *   launch_v41_linear      the DeepSeek V4.1 FP8 and mixed FP8/FP4 linears
 *                          (plugins/model-deepseek-v41/linear_fp8.cu:
 *                          82-105, validators linear_fp8.cpp:14-32,
 *                          linear_fp4.cpp:13-29): per-32 activation quant,
 *                          then the 32-block-scaled GEMM on MX MFMAs;
 *   launch_v41_fp4_to_fp8  the V4.1 expert FP4 -> FP8 32x32 conversion
 *                          (weight_expert_convert.cpp:33-100) on the device;
 *   launch_v41_block_dequant
 *                          the V4.1 wo_a e4m3 x block-scale -> bf16
 *                          dequantisation (weight_dequantize.cpp:17-50,
 *                          DequantizeWoATensor) on the device.
 *
 * Conventions are those of the reference's pack tables: one request pointer
 * in, pih_status_v1 by value out; a NULL request, wrong struct_size or wrong
 * abi_version gives PIH_STATUS_INVALID_ARGUMENT_V1; tensors are caller-owned
 * device addresses; stream is a caller-owned hipStream_t and 0 is rejected;
 * error_flag is a caller-owned device u32 the kernels OR error bits into;
 * scratch memory is caller-provided (sizes from query_workspace); entries
 * only enqueue work and never allocate or synchronise the host. */
#ifndef PIH_CONTRACTS_AMD_LINEAR_KERNELS_V1_H_
#define PIH_CONTRACTS_AMD_LINEAR_KERNELS_V1_H_

#include <stdint.h>

#include "pih/plugin_sdk/kernel_pack.h"
#include "pih/plugin_sdk/status.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PIH_AMD_LINEAR_KERNELS_ABI_VERSION_V1 1U

#define PIH_AMD_SCALE_F32_V1 1U   /* fp32 scale values */
#define PIH_AMD_SCALE_UE8M0_V1 2U /* one byte b, value 2^(b-127) */

#define PIH_AMD_OUTPUT_BF16_V1 1U
#define PIH_AMD_OUTPUT_F32_V1 2U
/* Fused gate/up epilogue: the weight holds [2I, K] (gate rows 0..I-1, then
 * up rows I..2I-1); the output is bf16 [rows, I] with
 * mid = bf16(silu(min(g,L)) * clamp(u,-L,L) * route_weight[row]) where
 * g, u are the bf16-rounded GEMM results and L = swiglu_limit (<= 0: no
 * clamp). */
#define PIH_AMD_OUTPUT_SWIGLU_BF16_V1 3U
#define PIH_AMD_OUTPUT_SWIGLU_E4M3_V1 4U /* launch_moe_fp8_gemm only */

#define PIH_AMD_ACTIVATION_E4M3_V1 1U
#define PIH_AMD_ACTIVATION_BF16_V1 2U

#define PIH_AMD_W4A16_SYMMETRIC_V1 1U  /* xing-w4a16-sym-g128-v1 */
#define PIH_AMD_W4A16_ASYMMETRIC_V1 2U /* u32 x8, bf16 scale, int4 zero */

#define PIH_AMD_WORKSPACE_ROUTE_PLAN_V1 1U
#define PIH_AMD_WORKSPACE_BF16_GEMM_V1 2U
#define PIH_AMD_WORKSPACE_W4A16_V1 3U

/* Scratch size query (host only; touches no device). */
typedef struct pih_amd_workspace_query_v1 {
  uint32_t struct_size, abi_version;
  uint32_t kind;          /* PIH_AMD_WORKSPACE_* */
  uint32_t m, n, k;       /* route plan: tokens, top_k, experts */
  uintptr_t bytes_u64;    /* host address the size is written to */
} pih_amd_workspace_query_v1;

/* Device route plan. topk_ids u32 [T, top_k], topk_weights f32 [T, top_k]
 * -> expert_offsets u32 [E+1] (exclusive prefix of per-expert counts),
 * row_token u32 [T*top_k] and row_weight f32 [T*top_k] in (expert, token)
 * order, token_rows u32 [T, top_k] (the row of route (t, j); 0xFFFFFFFF for
 * a rejected route).  Error bits: 1 expert id >= E, 2 expert repeated in a
 * token, 4 weight non-finite or negative.  top_k <= 32, E <= 1024. */
typedef struct pih_amd_route_plan_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t topk_ids_u32, topk_weights_f32;
  uintptr_t expert_offsets_u32, row_token_u32, row_weight_f32, token_rows_u32;
  uintptr_t workspace;
  uint64_t workspace_bytes;
  uintptr_t error_flag_u32, stream;
  uint32_t token_count, top_k, expert_count;
} pih_amd_route_plan_launch_v1;

/* bf16 [input_rows, K] -> e4m3 [row_count, K] + scale [row_count, K/128].
 * row_index_u32 == 0: output row r reads input row r (input_rows ignored);
 * otherwise input row row_index[r]. */
typedef struct pih_amd_fp8_quant_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t input_bf16, row_index_u32, output_e4m3, scale;
  uintptr_t error_flag_u32, stream;
  uint32_t row_count, logical_k, input_rows, scale_format;
} pih_amd_fp8_quant_launch_v1;

/* Dense block-scaled FP8 GEMM: out[m,n] = sum_kb (A.W over the block) *
 * sa[m,kb] * sw[n/128,kb].  Error bits: 1 e4m3 NaN code, 2 UE8M0 0xFF,
 * 4 non-finite result (element not written). */
typedef struct pih_amd_fp8_gemm_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t activation_e4m3, activation_scale, weight_e4m3, weight_scale;
  uintptr_t output, error_flag_u32, stream;
  uint32_t m, n, k, scale_format, output_type;
} pih_amd_fp8_gemm_launch_v1;

/* Grouped FP8 GEMM over MoE expert segments.  Logical row r (0 <= r <
 * expert_offsets[E]) belongs to the expert e with offsets[e] <= r <
 * offsets[e+1] and reads activation row row_token[r] (row_token == 0:
 * row r) of activation [activation_rows, K]; weight e4m3 [E, N, K] and
 * weight_scale [E, N/128, K/128]; output row r.  row_capacity bounds
 * offsets[E] (the output has row_capacity rows).  row_weight_f32 is read by
 * the SwiGLU epilogue only (0 = weight 1). */
typedef struct pih_amd_moe_fp8_gemm_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t activation_e4m3, activation_scale, row_token_u32;
  uintptr_t weight_e4m3, weight_scale, expert_offsets_u32, row_weight_f32;
  uintptr_t output, error_flag_u32, stream;
  uint32_t row_capacity, expert_count, n, k, activation_rows;
  uint32_t scale_format, output_type;
  float swiglu_limit;
  /* output_type PIH_AMD_OUTPUT_SWIGLU_E4M3_V1 only: the SwiGLU output is
   * rounded to bf16 and quantised to e4m3 as launch_fp8_quant would quantise
   * it; output receives the codes [row_capacity, n/2], output_scale the
   * scales [row_capacity, n/256] in scale_format.  Otherwise 0. */
  uintptr_t output_scale;
} pih_amd_moe_fp8_gemm_launch_v1;

/* Grouped MXFP4-weight GEMM over MoE expert segments: weight e2m1 packed
 * two per byte, low nibble = even k, [E, N, K/2], UE8M0 scale [E, N, K/32].
 * Activations e4m3 with UE8M0 scale [rows, K/128], or bf16. */
typedef struct pih_amd_moe_mxfp4_gemm_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t activation, activation_scale_ue8m0, row_token_u32;
  uintptr_t packed_weight, weight_scale_ue8m0, expert_offsets_u32, row_weight_f32;
  uintptr_t output, error_flag_u32, stream;
  uint32_t row_capacity, expert_count, n, k, activation_rows;
  uint32_t activation_type, output_type;
  float swiglu_limit;
} pih_amd_moe_mxfp4_gemm_launch_v1;

/* out[t, :] = bf16(sum over t's rows in ascending row order of
 * expert_output[row, :] + shared[t, :]) (shared_bf16 == 0: no shared). */
typedef struct pih_amd_moe_combine_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t expert_output_bf16, token_rows_u32, shared_bf16, output_bf16;
  uintptr_t error_flag_u32, stream;
  uint32_t token_count, top_k, hidden_size, row_count;
} pih_amd_moe_combine_launch_v1;

/* C[m,n] = A[m,k] . W[n,k]^T (row-major, bf16 in, fp32 accumulate). */
typedef struct pih_amd_bf16_gemm_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t a_bf16, w_bf16, output, workspace;
  uint64_t workspace_bytes;
  uintptr_t stream;
  uint32_t m, n, k, output_type;
} pih_amd_bf16_gemm_launch_v1;

/* W4A16: y[m,n] = bf16(sum_k x[m,k] * w[n,k]).
 * SYMMETRIC: qweight u8 [N, K/2] (low nibble = even k, signed int4 in
 *   [-7, 7], nibble 8 reserved), scales fp16 [N, K/128], w = q * s.
 * ASYMMETRIC: qweight u32 [N, K/8] (nibble j of a word = k%8 == j), scales
 *   bf16 [N, K/128], zeros u32 [N, ceil(K/1024)] (nibble j = group%8 == j),
 *   w = (q - z) * s.
 * The error flag takes the first failure's code (compare-and-swap from 0),
 * with the reference's QwenCudaInvariant numbers
 * (include/pih/model/qwen3_cuda_invariant.h:20-23): 12 reserved nibble,
 * 13 scale not finite and positive, 14 non-finite output. */
typedef struct pih_amd_w4a16_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t input_bf16, qweight, scales, zeros, output_bf16, workspace;
  uint64_t workspace_bytes;
  uintptr_t error_flag_u32, stream;
  uint32_t m, n, k, format;
} pih_amd_w4a16_launch_v1;

/* Several independent W4A16 GEMVs in one launch (for example q, k and v,
 * or gate and up, of one decode step): problem i computes
 * output_i[m, n_i] = input_i[m, k] . w_i^T exactly as
 * pih_amd_w4a16_launch_v1 would, with one m, k and format for the whole
 * group.  `problems` is a HOST pointer to problem_count (1..8) entries,
 * read during the call (so a captured launch keeps its own copy). */
#define PIH_AMD_W4A16_GROUP_MAX_V1 8U
typedef struct pih_amd_w4a16_problem_v1 {
  uintptr_t input_bf16, qweight, scales, zeros, output_bf16;
  uint32_t n, reserved;
} pih_amd_w4a16_problem_v1;

typedef struct pih_amd_w4a16_grouped_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t problems; /* const pih_amd_w4a16_problem_v1* (host) */
  uintptr_t error_flag_u32, stream;
  uint32_t problem_count, m, k, format;
} pih_amd_w4a16_grouped_launch_v1;

/* One MoE expert layer per call, enqueued on `stream` with no host wait:
 * route plan -> activation quant -> grouped gate/up GEMM with the SwiGLU x
 * route-weight epilogue -> intermediate quant -> grouped down GEMM ->
 * ordered combine (+ shared).  The output equals launching those entries
 * one by one in that order; fewer launches run (the activation quant rides
 * in the route plan's first launch, and with FP8 weights the intermediate
 * quant in the gate/up epilogue).
 * FP8 weights: w13 e4m3 [E][2I][H] (gate rows, then up rows), w13_scale
 *   [E][2I/128][H/128], w2 e4m3 [E][H][I], w2_scale [E][H/128][I/128];
 *   scale_format applies to weights and activations.
 * MXFP4 weights: w13 e2m1 [E][2I][H/2], UE8M0 [E][2I][H/32]; w2 e2m1
 *   [E][H][I/2], UE8M0 [E][H][I/32]; activation_type e4m3 (UE8M0 per 128)
 *   or bf16 (no quant stages).
 * Scratch: query_moe_layer_workspace writes the byte count to
 * *required_bytes_u64 (a host address); launch_moe_layer needs at least
 * that much in `workspace`.  Error bits are those of the stage entries. */
#define PIH_AMD_WEIGHT_FP8_V1 1U
#define PIH_AMD_WEIGHT_MXFP4_V1 2U
typedef struct pih_amd_moe_layer_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t input_bf16, topk_ids_u32, topk_weights_f32;
  uintptr_t w13, w13_scale, w2, w2_scale;
  uintptr_t shared_bf16, output_bf16;
  uintptr_t workspace;
  uint64_t workspace_bytes;
  uintptr_t required_bytes_u64;
  uintptr_t error_flag_u32, stream;
  uint32_t token_count, top_k, expert_count, hidden_size, intermediate_size;
  uint32_t weight_format, scale_format, activation_type;
  float swiglu_limit;
} pih_amd_moe_layer_launch_v1;

/* Exact INT4 dequant, the unpack the W4A16 GEMV applies: output fp32
 * [N, K] with w = (q - z) * s (ASYMMETRIC) or q * s (SYMMETRIC); same
 * layouts and error codes as pih_amd_w4a16_launch_v1. */
typedef struct pih_amd_w4a16_dequant_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t qweight, scales, zeros, output_f32, error_flag_u32, stream;
  uint32_t n, k, format;
} pih_amd_w4a16_dequant_launch_v1;

typedef struct pih_amd_silu_mul_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t gate_bf16, up_bf16, output_bf16, stream;
  uint64_t count;
} pih_amd_silu_mul_launch_v1;

typedef struct pih_amd_swiglu_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t gate_bf16, up_bf16, route_weights_f32, output_bf16;
  uintptr_t error_flag_u32, stream;
  uint32_t rows, cols;
  float limit;
} pih_amd_swiglu_launch_v1;

typedef struct pih_amd_mxfp4_decode_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t packed, scales_ue8m0, output_bf16, error_flag_u32, stream;
  uint32_t rows, k;
} pih_amd_mxfp4_decode_launch_v1;

/* Router top-k on the device (the step between the router GEMM and the
 * route plan): raw scores f32 [T, E] -> topk_ids u32 [T, top_k] and
 * topk_weights f32 [T, top_k] in rank order, ranked by (selection
 * descending, expert id ascending).
 * SQRT_SOFTPLUS: the V4 learned router (plugins/model-deepseek-v4-flash/
 *   deepseek_learned_router.cpp:21-81; E = 256, top-6, scale 1.5 there):
 *   base = sqrt(softplus(raw)), selection = base + bias[e] (bias_f32 [E],
 *   0 = none), weight = base / sum of the top-k bases * route_scale.
 * SOFTMAX: softmax over the E scores, top-k, renormalised to sum
 *   route_scale (BASELINE's DeepSeek-V3-style router; selection by score,
 *   which orders like the probability).
 * E <= 1024, top_k <= min(32, E), route_scale finite and > 0.  Error bits:
 * 1 non-finite score, 2 non-finite bias, 4 top-k weight sum non-finite or
 * <= 0 (the reference rejects all three). */
#define PIH_AMD_ROUTER_SOFTMAX_V1 1U
#define PIH_AMD_ROUTER_SQRT_SOFTPLUS_V1 2U
typedef struct pih_amd_router_topk_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t scores_f32, bias_f32, topk_ids_u32, topk_weights_f32;
  uintptr_t error_flag_u32, stream;
  uint32_t token_count, expert_count, top_k, mode;
  float route_scale;
} pih_amd_router_topk_launch_v1;

/* DeepSeek V4.1 linear: out bf16 [rows, N] = quant32(input bf16 [rows, K])
 * . W^T.  weight_format 1: W e4m3 [N, K] + UE8M0 [N/32, K/32] (one per 32x32
 * block); 2: W e2m1 [N, K/2] (even k in the low nibble) + UE8M0 [N, K/32].
 * quantized_e4m3 [rows, K] and activation_scales UE8M0 [rows, K/32] are
 * caller scratch the entry writes (the per-32 quant of the reference's
 * Quantize kernel).  Every region carries its byte count, which must equal
 * the layout's (the reference's Valid: non-zero, aligned, exact size), and
 * no written region may overlap another region.  1 <= rows <= 4096,
 * K and N in [1, 32768] and multiples of 32 (the reference's bounds); this
 * pack also needs K and N multiples of 128 (every V4.1 projection is) and
 * answers INVALID_ARGUMENT otherwise.  Error bits: 1 a non-finite input, a
 * NaN code or a 255 scale; 2 a non-finite result (stored, as the reference
 * stores it). */
#define PIH_AMD_V41_WEIGHT_FP8_BLOCK32_V1 1U
#define PIH_AMD_V41_WEIGHT_MXFP4_V1 2U
typedef struct pih_amd_v41_linear_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t input_bf16;
  uint64_t input_bytes;
  uintptr_t weight;
  uint64_t weight_bytes;
  uintptr_t weight_scales;
  uint64_t weight_scale_bytes;
  uintptr_t quantized_e4m3;
  uint64_t quantized_bytes;
  uintptr_t activation_scales;
  uint64_t activation_scale_bytes;
  uintptr_t output_bf16;
  uint64_t output_bytes;
  uintptr_t error_flag_u32;
  uint64_t error_flag_bytes;
  uintptr_t stream;
  uint32_t rows, in_features, out_features, weight_format;
} pih_amd_v41_linear_launch_v1;

/* V4.1 expert FP4 -> FP8 32x32: packed e2m1 [rows, cols/2] + UE8M0 [rows,
 * cols/32] -> e4m3 [rows, cols] + UE8M0 [rows/32, cols/32]; rows and cols
 * multiples of 32.  Error bits: 1 a NaN (255) row scale, 2 a block whose
 * largest row scale is below 6 (shared scale under the E8M0 range); such
 * blocks are left unwritten and the whole output must be discarded, as the
 * reference rejects the tensor. */
typedef struct pih_amd_v41_fp4_to_fp8_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t packed, scales, weight_e4m3, weight_scales, error_flag_u32, stream;
  uint32_t rows, columns;
} pih_amd_v41_fp4_to_fp8_launch_v1;

/* V4.1 block dequantisation: e4m3 [rows, columns] x one scale per square
 * block (block 32 or 128; scale_storage 1: UE8M0 bytes, 0 meaning 2^-127;
 * 2: fp32) -> bf16, fp32 product rounded to nearest even.  Error bits: 1 a
 * NaN code, 2 a 255 / non-finite / non-positive scale, 4 a non-finite
 * product or bf16; those elements are left unwritten. */
#define PIH_AMD_V41_SCALE_E8M0_V1 1U
#define PIH_AMD_V41_SCALE_F32_V1 2U
typedef struct pih_amd_v41_block_dequant_launch_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t source_e4m3, scales, output_bf16, error_flag_u32, stream;
  uint32_t rows, columns, block, scale_storage;
} pih_amd_v41_block_dequant_launch_v1;

typedef struct pih_amd_linear_kernels_api_v1 {
  uint32_t struct_size;
  uint32_t contract_version;
  const pih_kernel_pack_identity_v1* identity;
  pih_status_v1 (*query_workspace)(const pih_amd_workspace_query_v1*);
  pih_status_v1 (*launch_route_plan)(const pih_amd_route_plan_launch_v1*);
  pih_status_v1 (*launch_fp8_quant)(const pih_amd_fp8_quant_launch_v1*);
  pih_status_v1 (*launch_fp8_gemm)(const pih_amd_fp8_gemm_launch_v1*);
  pih_status_v1 (*launch_moe_fp8_gemm)(const pih_amd_moe_fp8_gemm_launch_v1*);
  pih_status_v1 (*launch_moe_mxfp4_gemm)(const pih_amd_moe_mxfp4_gemm_launch_v1*);
  pih_status_v1 (*launch_moe_combine)(const pih_amd_moe_combine_launch_v1*);
  pih_status_v1 (*launch_bf16_gemm)(const pih_amd_bf16_gemm_launch_v1*);
  pih_status_v1 (*launch_w4a16_gemm)(const pih_amd_w4a16_launch_v1*);
  pih_status_v1 (*launch_silu_mul)(const pih_amd_silu_mul_launch_v1*);
  pih_status_v1 (*launch_swiglu)(const pih_amd_swiglu_launch_v1*);
  pih_status_v1 (*launch_mxfp4_decode)(const pih_amd_mxfp4_decode_launch_v1*);
  pih_status_v1 (*launch_w4a16_dequant)(const pih_amd_w4a16_dequant_launch_v1*);
  pih_status_v1 (*launch_w4a16_grouped)(const pih_amd_w4a16_grouped_launch_v1*);
  pih_status_v1 (*query_moe_layer_workspace)(const pih_amd_moe_layer_launch_v1*);
  pih_status_v1 (*launch_moe_layer)(const pih_amd_moe_layer_launch_v1*);
  /* launch_route_plan_noalloc: no counterpart in the reference.  For callers
   * that cannot allocate device memory (code under HIP graph capture, tight
   * serving loops): launch_route_plan with its scratch (per-chunk expert
   * masks and bases) in a device array the pack owns, one per GPU, instead
   * of a caller workspace.  `workspace` and `workspace_bytes` must be 0.
   * Limit: the scratch launch_route_plan would need,
   * query_workspace(ROUTE_PLAN, tokens, top_k, experts), must not exceed
   * PIH_AMD_ROUTE_PLAN_NOALLOC_MAX_SCRATCH_V1 bytes (for example T <= 16384
   * tokens at E = 256, or T <= 4096 at E = 1024); larger plans are
   * INVALID_ARGUMENT.  Every call on one GPU uses that GPU's one array, so
   * calls that overlap on one GPU (other streams, other threads) race; the
   * kernels rewrite all of it on every call, so no state carries over.
   * Outputs equal launch_route_plan's bit for bit. */
  pih_status_v1 (*launch_route_plan_noalloc)(const pih_amd_route_plan_launch_v1*);
  /* Router top-k (pih_amd_router_topk_launch_v1 above); replaces the host
   * DeepSeekLearnedRouter::Route (deepseek_learned_router.cpp:84-94) and the
   * scores D2H before it. */
  pih_status_v1 (*launch_router_topk)(const pih_amd_router_topk_launch_v1*);
  /* DeepSeek V4.1 32-block formats (the three structs above). */
  pih_status_v1 (*launch_v41_linear)(const pih_amd_v41_linear_launch_v1*);
  pih_status_v1 (*launch_v41_fp4_to_fp8)(const pih_amd_v41_fp4_to_fp8_launch_v1*);
  pih_status_v1 (*launch_v41_block_dequant)(const pih_amd_v41_block_dequant_launch_v1*);
} pih_amd_linear_kernels_api_v1;

#define PIH_AMD_ROUTE_PLAN_NOALLOC_MAX_SCRATCH_V1 (1ULL << 20)

#ifdef __cplusplus
}
#endif

#endif /* PIH_CONTRACTS_AMD_LINEAR_KERNELS_V1_H_ */

/* pih_oracle — CPU restatement of the reference's arithmetic for the
 * linear-layer hot path.  TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker or as the timed CPU baseline.
 * No product code path links, loads or calls it; the HIP packs fail loudly
 * instead of falling back to it.
 *
 * Every function follows the loop nesting of the reference function it cites
 * (fp32 accumulate, strict increasing k, rounding only where the reference
 * rounds).  Built with -O2 -ffp-contract=off and without -ffast-math, like the
 * reference's CPU oracles.  OpenMP parallelises over output rows only, so the
 * per-element arithmetic (and therefore every bit of the result) is the same
 * for any thread count.
 *
 * Return convention: 0 = OK, otherwise a small positive code naming the
 * rejection (the reference returns Status::InvalidArgument at the same
 * points).
 *
 * Pinning (what checks each function, see tests/test_oracle_*.py):
 *   codecs (bf16, fp16, e4m3, e2m1/ue8m0)  reference KATs + exhaustive
 *                                          closed-form sweeps + oracle/_ref
 *   fp8 quant (ue8m0)                      reference KATs + oracle/_ref
 *   fp8 quant (fp32 scale)                 closed form (scale*448 == amax,
 *                                          codes round-trip) - BASELINE-only
 *   fp8 gemm (ue8m0)                       reference KAT 384 + oracle/_ref
 *   fp8 gemm (fp32 scale)                  reduces to the ue8m0 gemm when all
 *                                          scales are powers of two; brute
 *                                          force in float64 on tiny inputs
 *   fp4 gemm                               reference KATs 128/256, nibble
 *                                          order -1, oracle/_ref
 *   w4a16 sym                              reference fixture (closed-form
 *                                          expected bf16 for 5 shapes)
 *   w4a16 asym                             reduces to the sym form when z=8
 *                                          and scales equal; float64 brute
 *   bf16 gemm                              float64 brute force (exact for
 *                                          small integer-valued inputs)
 *   silu_mul / swiglu                      reference KATs + oracle/_ref
 *   route plan / accumulate                reference KATs + oracle/_ref
 *   routed expert chain                    reference KAT (all 0.75) +
 *                                          oracle/_ref
 */
#ifndef PIH_ORACLE_H_
#define PIH_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- threads */
void po_set_threads(int threads);
int po_get_threads(void);

/* ----------------------------------------------------------------- codecs */
/* include/pih/core/bfloat16.h:13-27 */
uint16_t po_bf16_from_f32(float value);
float po_bf16_to_f32(uint16_t bits);
/* src/core/float16.cpp:8-68 */
uint16_t po_f16_from_f32(float value);
float po_f16_to_f32(uint16_t bits);
/* plugins/model-deepseek-v4-flash/deepseek_fp8_activation_codec.cpp:11-25;
 * returns 1 for the NaN code (S.1111.111), 0 otherwise. */
int po_e4m3_decode(uint8_t bits, float* value);
/* deepseek_fp8_activation_codec.cpp:27-51: nearest finite e4m3fn code, ties
 * to the even code; |value| must be finite and <= 448 (returns 1 otherwise). */
int po_e4m3_encode(float value, uint8_t* bits);
/* plugins/model-deepseek-v4-flash/deepseek_mxfp4_codec.cpp:9-19 */
int po_mxfp4_decode_scalar(uint8_t e2m1_bits, uint8_t ue8m0_bits, double* value);
/* deepseek_mxfp4_codec.cpp:21-46; packed holds (k+1)/2 bytes, low nibble =
 * even k; one scale byte per 32 values. */
int po_mxfp4_decode_row(const uint8_t* packed, const uint8_t* scale_bits,
                        uint32_t logical_k, float* out);

/* ------------------------------------------------------- activation quant */
/* deepseek_fp8_activation_codec.cpp:53-107: per (token, 128 columns) amax with
 * floor 1e-4, e = ceil(log2(amax/448)), scale byte e+127,
 * code = e4m3(clamp(x / 2^e, +-448)). */
int po_fp8_quant_ue8m0(const float* input, uint32_t tokens, uint32_t logical_k,
                       uint8_t* codes, uint8_t* scale_bits);
/* Same grouping with an fp32 scale s = max(amax, 1e-4) / 448 and
 * code = e4m3(clamp(x / s, +-448)) (the BASELINE fp8 MoE activation format;
 * no reference counterpart). */
int po_fp8_quant_f32(const float* input, uint32_t tokens, uint32_t logical_k,
                     uint8_t* codes, float* scales);

/* ------------------------------------------------------------------ GEMMs */
/* src/model/deepseek_fp8_gemm_oracle.cpp:10-80.  out[m,n] (fp32) =
 * sum_kb (sum_{i<128} a*w) * 2^(sa-127) * 2^(sw-127). */
int po_fp8_gemm_ue8m0(const uint8_t* a, const uint8_t* a_scale_bits,
                      const uint8_t* w, const uint8_t* w_scale_bits,
                      uint32_t m, uint32_t n, uint32_t k, float* out);
/* Same nesting with fp32 scales: a_scale [m, k/128], w_scale [n/128, k/128]. */
int po_fp8_gemm_f32(const uint8_t* a, const float* a_scale, const uint8_t* w,
                    const float* w_scale, uint32_t m, uint32_t n, uint32_t k,
                    float* out);
/* src/model/deepseek_fp4_gemm_oracle.cpp:11-91. a_scale_bits [m, k/128],
 * packed [n, k/2] (low nibble = even k), w_scale_bits [n, k/32]. */
int po_fp4_gemm(const uint8_t* a, const uint8_t* a_scale_bits,
                const uint8_t* packed, const uint8_t* w_scale_bits, uint32_t m,
                uint32_t n, uint32_t k, float* out);
/* MXFP4 weights against bf16 activations: out[m,n] = sum_k x*w with w the
 * exact fp32 value of e2m1 * 2^(e-127), strict increasing k (BASELINE cfg5
 * bf16-activation variant; decode semantics from deepseek_mxfp4_codec.cpp). */
int po_mxfp4_bf16_gemm(const uint16_t* x, const uint8_t* packed,
                       const uint8_t* w_scale_bits, uint32_t m, uint32_t n,
                       uint32_t k, float* out);
/* kernels/cuda/qwen_bf16_primitives.cu:98-149 (reference W4A16 format):
 * packed u8 [n, k/2] signed int4 (nibble 8 reserved), fp16 scale per
 * (n, k/128), acc += x * (q * s), bf16 out.  Returns 12 for a reserved
 * nibble, 13 for a bad scale, 14 for a non-finite output. */
int po_w4a16_sym(const uint16_t* x, const uint8_t* packed,
                 const uint16_t* scales_f16, uint32_t m, uint32_t n, uint32_t k,
                 uint16_t* out);
/* BASELINE W4A16 format: qweight u32 [n, k/8] (nibble j of word = k%8 == j),
 * bf16 scale [n, k/128], zero points u32 [n, ceil(k/1024)] (nibble j of word
 * = group%8 == j); w = (q - z) * s exactly in fp32; acc += x * w, bf16 out. */
int po_w4a16_asym(const uint16_t* x, const uint32_t* qweight,
                  const uint16_t* scales_bf16, const uint32_t* zeros,
                  uint32_t m, uint32_t n, uint32_t k, uint16_t* out);
int po_w4a16_asym_dequant(const uint32_t* qweight, const uint16_t* scales_bf16,
                          const uint32_t* zeros, uint32_t n, uint32_t k,
                          float* w);
/* BF16 linear as cuBLASLt computes it for GemmPlan
 * (src/backend/cuda/gemm_plan.cpp:83-198): C[m,n] = A[m,k] . W[n,k]^T with a
 * strict-k fp32 dot.  fp32 result; callers round to bf16 with RNE. */
/* DeepSeek LM head in the reference's reduction order; returns error bits 64/128. */
uint32_t po_lm_head(const uint16_t* x, const uint16_t* w, uint32_t rows, uint32_t vocab,
                    uint32_t hidden, float* logits);
/* DeepSeek V4.1 32-block formats (weight_expert_convert.cpp, weight_dequantize.cpp, linear_fp8.cu). */
int po_v41_fp4_block_to_fp8(const uint8_t* packed, const uint8_t* scales, uint8_t* weight, uint8_t* scale);
int po_v41_fp4_to_fp8(const uint8_t* packed, const uint8_t* scales, uint32_t rows, uint32_t cols, uint8_t* weight,
                      uint8_t* out_scales);
int po_v41_dequant_block(const uint8_t* src, float scale, uint32_t block, uint16_t* out);
uint32_t po_v41_quant32(const uint16_t* x, uint32_t rows, uint32_t k, uint8_t* codes, uint8_t* scales);
uint32_t po_v41_linear(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, uint32_t rows,
                       uint32_t n, uint32_t k, int fp4, uint16_t* out);
void po_bf16_gemm(const uint16_t* a, const uint16_t* w, uint32_t m, uint32_t n,
                  uint32_t k, float* out);

/* ------------------------------------------------------------ elementwise */
/* plugins/model-qwen3/qwen3_cpu_oracle.cpp:114-126 */
void po_silu_mul(const uint16_t* gate, const uint16_t* up, size_t count,
                 uint16_t* out);
/* src/model/deepseek_expert_swiglu_oracle.cpp:11-42 (fp32 out, no rounding);
 * limit <= 0 disables the clamp (BASELINE's plain SiLU-mul). */
int po_swiglu(const float* gate, const float* up, size_t count, float limit,
              float* out);

/* ------------------------------------------------------------ router top-k */
/* Router selection over raw scores [tokens, experts] (one token's scores
 * contiguous), top_k <= 32, ranked by (selection descending, expert id
 * ascending); ids/weights [tokens, top_k] in rank order.
 * mode 2 (V4 learned router, plugins/model-deepseek-v4-flash/
 *   deepseek_learned_router.cpp:10-81, generalised from E=256, k=6):
 *   base = sqrt(softplus(raw)) with the stable softplus, selection = base +
 *   bias[e] (bias NULL: 0), weight = base / sum(base over the top-k, rank
 *   order) * scale (the reference's 1.5).
 * mode 1 (BASELINE softmax top-k, no reference counterpart): selection =
 *   raw (softmax is strictly increasing); p = exp(raw - max) / sum over all
 *   experts (expert order), weight = p / sum(p over the top-k, rank order)
 *   * scale.
 * Codes: 1 geometry/mode, 2 non-finite score, 3 non-finite bias, 4 top-k
 * weight sum non-finite or <= 0 (mode 2). */
int po_router_topk(const float* scores, const float* bias, uint32_t tokens,
                   uint32_t experts, uint32_t topk, uint32_t mode, float scale,
                   uint32_t* ids, float* weights);

/* -------------------------------------------------------- MoE route plan */
/* plugins/model-deepseek-v4-flash/deepseek_expert_subwave_plan.cpp:32-101,
 * generalised to any top-k and expert count: validates, sorts routes by
 * (expert, token, ordinal) and writes expert_offsets[experts+1],
 * row_token[R], row_weight[R] and token_rows[T*topk] (the sorted row of the
 * route (t, ordinal)). Route (t, j) is topk_ids[t*topk+j] / topk_weights[..].
 * Codes: 1 geometry, 2 expert id out of range, 3 duplicate expert in a
 * token, 4 bad weight. */
int po_route_plan(const uint32_t* topk_ids, const float* topk_weights,
                  uint32_t tokens, uint32_t topk, uint32_t experts,
                  uint32_t* expert_offsets, uint32_t* row_token,
                  float* row_weight, uint32_t* token_rows);

/* src/model/deepseek_expert_accumulator_oracle.cpp:20-85 generalised to any
 * hidden size: for sorted rows r (experts ascending, tokens ascending within
 * an expert) acc[row_token[r], :] += out[r, :] (fp32), then
 * final = bf16(acc + shared) with shared == NULL meaning zero. */
int po_ordered_accumulate(const uint16_t* expert_out_bf16,
                          const uint32_t* row_token, uint32_t rows,
                          uint32_t tokens, uint32_t hidden, float* acc);
int po_finalize(const float* acc, const uint16_t* shared_bf16, size_t count,
                uint16_t* out);

/* src/model/deepseek_routed_expert_oracle.cpp:50-95 (reference format):
 * quant -> fp4 gemm W1 -> bf16 -> quant -> fp4 gemm W3 -> bf16 -> SwiGLU
 * (limit 10) -> * w -> bf16 -> quant -> fp4 gemm W2 -> bf16. */
int po_routed_expert_fp4(const uint16_t* input_bf16, const float* route_weights,
                         uint32_t tokens, uint32_t hidden,
                         uint32_t intermediate, const uint8_t* w1_packed,
                         const uint8_t* w1_scales, const uint8_t* w2_packed,
                         const uint8_t* w2_scales, const uint8_t* w3_packed,
                         const uint8_t* w3_scales, uint16_t* out_bf16);

/* BASELINE cfg4 expert chain with the same rounding points, FP8 weights with
 * fp32 128x128 block scales and a fused gate/up weight [2I, H] (gate rows
 * first): quant_f32(x) -> fp8 gemm -> bf16 gate/up -> SwiGLU(limit, <=0 off)
 * -> * w -> bf16 -> quant_f32 -> fp8 gemm W2 -> bf16. */
int po_expert_fp8(const uint16_t* input_bf16, const float* route_weights,
                  uint32_t tokens, uint32_t hidden, uint32_t intermediate,
                  const uint8_t* w13, const float* w13_scale, const uint8_t* w2,
                  const float* w2_scale, float limit, uint16_t* out_bf16);

#ifdef __cplusplus
}
#endif

#endif /* PIH_ORACLE_H_ */

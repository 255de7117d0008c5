/* Launch plan of the Qwen W4A16 linear for the gfx950 code object: the
 * model-side plan the Qwen plugin computes before launching
 * pih_qwen_w4a16_gemm_* by name through the kernel-module driver
 * (include/pih/backend/hip/kernel_module_v1.h).  It replaces
 * QwenInt4GemmPlan::Create / signature (plugins/model-qwen3/
 * qwen3_int4_gemm_plan.cpp:44-88, include/pih/model/qwen3_int4_gemm_plan.h):
 *   PIH_QWEN_INT4_VARIANT_COMPATIBILITY_V1: the reference's kernel and
 *     geometry (pih_qwen_w4a16_gemm_compat_v1, ceil(m n / 256) blocks of
 *     256 threads), the launch an unchanged model makes;
 *   PIH_QWEN_INT4_VARIANT_GFX950_V1: pih_qwen_w4a16_gemm_gfx950_v1 with a
 *     grid of (n / 16, ceil(m / 16)) blocks whose waves split K.
 * Both take the same 64-byte packet (input, packed_weight, scales, output,
 * error_flag as device pointers at 0..32; m, n, k as u64 at 40, 48, 56).
 * Library: libpih_hip_kernel_module.so. */
#ifndef PIH_CONTRACTS_QWEN_INT4_PLAN_GFX950_V1_H_
#define PIH_CONTRACTS_QWEN_INT4_PLAN_GFX950_V1_H_

#include <stdint.h>

#include "pih/backend/hip/kernel_module_v1.h"
#include "pih/plugin_sdk/status.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PIH_QWEN_INT4_VARIANT_COMPATIBILITY_V1 1u
#define PIH_QWEN_INT4_VARIANT_GFX950_V1 2u
#define PIH_QWEN_INT4_MAX_TOKENS_V1 4096u

typedef struct pih_qwen_int4_gemm_plan_v1 {
  uint32_t struct_size;
  uint32_t abi_version; /* PIH_HIP_KERNEL_MODULE_ABI_VERSION_V1 */
  uint32_t variant;
  uint32_t reserved;
  const char* kernel_symbol;         /* static strings */
  const char* logical_id;
  const char* parameter_abi_sha256;  /* SHA-256 of the parameter descriptor */
  pih_hip_launch_geometry_v1 geometry;
  uint64_t tokens, output_features, input_features;
  uint64_t input_bytes, packed_bytes, scale_bytes, output_bytes;
} pih_qwen_int4_gemm_plan_v1;

/* The plan for m tokens of an (n, k) linear (k % 128 == 0; the
 * compatibility variant needs n % 256 == 0, the gfx950 one n % 16 == 0;
 * 1 <= m <= 4096). */
pih_status_v1 pih_qwen_int4_gemm_plan_create_v1(uint64_t tokens, uint64_t output_features,
                                                uint64_t input_features, uint32_t variant,
                                                pih_qwen_int4_gemm_plan_v1* plan);

/* The eight-parameter signature of the plan's kernel (parameters and
 * descriptor digest), for pih_hip_kernel_module_load_v1; `parameters`
 * must hold 8 entries and lives as long as the signature is used. */
pih_status_v1 pih_qwen_int4_gemm_signature_v1(uint32_t variant, const char* code_object_sha256,
                                              pih_hip_kernel_parameter_v1* parameters,
                                              pih_hip_kernel_signature_v1* signature);

#ifdef __cplusplus
}
#endif

#endif /* PIH_CONTRACTS_QWEN_INT4_PLAN_GFX950_V1_H_ */

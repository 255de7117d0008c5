/* Qwen Kernel Pack contract (contract id "pih.qwen-kernels.v1").
 *
 * Layout-compatible restatement of the reference's
 * include/pih/contracts/qwen_kernels_v1.h:7-14. The model plugin
 * (plugins/model-qwen3/entrypoint.cpp:415-427) resolves the pack, calls
 * root() and loads the device image found under it. For the gfx950 pack the
 * directory holds qwen3-gfx950/gfx950/qwen_bf16_primitives.hsaco plus its
 * .json manifest; target_sm carries 950 (the gfx950 major/minor/stepping
 * digits) in place of an sm_XY number. */
#ifndef PIH_CONTRACTS_QWEN_KERNELS_V1_H_
#define PIH_CONTRACTS_QWEN_KERNELS_V1_H_

#include <stdint.h>

#include "pih/plugin_sdk/status.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct pih_qwen_kernels_api_v1 {
  uint32_t struct_size;
  uint32_t contract_version; /* 1 */
  uint32_t target_sm;        /* 950 on this pack */
  /* Pack-owned, absolute path of the code-object directory. Valid for as long
   * as the pack stays loaded (packs are never unloaded). */
  pih_status_v1 (*root)(const char** path);
} pih_qwen_kernels_api_v1;

#ifdef __cplusplus
}
#endif

#endif /* PIH_CONTRACTS_QWEN_KERNELS_V1_H_ */

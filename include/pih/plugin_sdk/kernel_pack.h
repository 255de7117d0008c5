/* Kernel Pack C-ABI: the two symbols every pack exports.
 *
 * Layout-compatible restatement of the reference's
 * include/pih/plugin_sdk/kernel_pack.h:1-44. The host (the reference's
 * KernelPackLoader, src/microkernel/kernel_pack_loader.cpp:90-133) dlopens a
 * pack, resolves exactly these two symbols, checks struct_size/abi_version and
 * canonical ids, then calls bind_origin() with the absolute library path.
 * bind_origin must copy whatever it keeps and must not touch a device. */
#ifndef PIH_PLUGIN_SDK_KERNEL_PACK_H_
#define PIH_PLUGIN_SDK_KERNEL_PACK_H_

#include <stdint.h>

#include "pih/plugin_sdk/status.h"

#define PIH_KERNEL_PACK_ABI_VERSION_V1 1u
#define PIH_KERNEL_PACK_IDENTITY_SYMBOL_V1 "pih_kernel_pack_identity_v1_get"
#define PIH_KERNEL_PACK_API_SYMBOL_V1 "pih_kernel_pack_api_v1_get"

#if defined(__GNUC__)
#define PIH_PLUGIN_EXPORT __attribute__((visibility("default")))
#else
#define PIH_PLUGIN_EXPORT
#endif

typedef struct pih_kernel_pack_identity_v1 {
  uint32_t struct_size;
  uint32_t abi_version;
  const char* pack_id;      /* canonical [a-z0-9.-] */
  const char* pack_version; /* "1.0.0" */
  const char* pack_abi;     /* contract id the model resolves */
  const char* architecture; /* "gfx950" for every pack in this repository */
} pih_kernel_pack_identity_v1;

typedef const pih_kernel_pack_identity_v1* (*pih_kernel_pack_identity_fn_v1)(
    void);

typedef struct pih_kernel_pack_api_v1 {
  uint32_t struct_size;
  uint32_t abi_version;
  const pih_kernel_pack_identity_v1* identity; /* same pointer as identity_get */
  const void* contract_api;                    /* contract-specific table */
  pih_status_v1 (*bind_origin)(const char* absolute_library_path);
} pih_kernel_pack_api_v1;

typedef const pih_kernel_pack_api_v1* (*pih_kernel_pack_api_fn_v1)(void);

#ifdef __cplusplus
extern "C" {
#endif

const pih_kernel_pack_identity_v1* pih_kernel_pack_identity_v1_get(void);
const pih_kernel_pack_api_v1* pih_kernel_pack_api_v1_get(void);

#ifdef __cplusplus
}
#endif

#endif /* PIH_PLUGIN_SDK_KERNEL_PACK_H_ */

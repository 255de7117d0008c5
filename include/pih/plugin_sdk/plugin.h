/* Native plugin ABI (plugin ABI "pih.native-plugin.v1").
 *
 * Layout-compatible restatement of the reference's plugin SDK headers
 * include/pih/plugin_sdk/abi.h:20-58 (host and plugin tables, entry point),
 * capability.h (capability record, registry callbacks) and lifecycle.h
 * (seven lifecycle callbacks).  A plugin exports
 *   pih_status_v1 pih_plugin_entry_v1(const pih_host_api_v1*, pih_plugin_api_v1*)
 * which fills in its id, version, context and lifecycle table; the host then
 * drives register -> configure -> start -> ready -> drain -> stop -> dispose,
 * and the plugin publishes capabilities (capability id + contract id + API
 * table) through host->register_capability during register and resolves the
 * ones it needs through host->resolve_capability during configure. */
#ifndef PIH_PLUGIN_SDK_PLUGIN_H_
#define PIH_PLUGIN_SDK_PLUGIN_H_

#include <stdint.h>

#include "pih/plugin_sdk/status.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PIH_PLUGIN_ABI_VERSION_V1 1U
#define PIH_PLUGIN_LIFECYCLE_ABI_VERSION_V1 1U
#define PIH_CAPABILITY_ABI_VERSION_V1 1U

enum {
  PIH_CAPABILITY_THREADING_SINGLE_THREADED_V1 = 1,
  PIH_CAPABILITY_THREADING_SERIALIZED_V1 = 2,
  PIH_CAPABILITY_THREADING_CONCURRENT_V1 = 3
};
enum {
  PIH_CAPABILITY_SCOPE_PROCESS_V1 = 1,
  PIH_CAPABILITY_SCOPE_ACTIVATION_V1 = 2,
  PIH_CAPABILITY_SCOPE_ENGINE_V1 = 3,
  PIH_CAPABILITY_SCOPE_REQUEST_V1 = 4
};
enum {
  PIH_CAPABILITY_CARDINALITY_EXACTLY_ONE_V1 = 1,
  PIH_CAPABILITY_CARDINALITY_ZERO_OR_ONE_V1 = 2,
  PIH_CAPABILITY_CARDINALITY_ONE_OR_MORE_V1 = 3,
  PIH_CAPABILITY_CARDINALITY_MANY_V1 = 4
};

typedef struct pih_capability_v1 {
  uint32_t struct_size;
  uint32_t abi_version;
  const char* capability_id;
  const char* contract_id;
  const void* api;
  uint32_t threading_model;
  uint32_t scope;
  uint32_t cardinality;
} pih_capability_v1;

typedef pih_status_v1 (*pih_register_capability_callback_v1)(void* context, const pih_capability_v1* capability);
typedef pih_status_v1 (*pih_resolve_capability_callback_v1)(void* context, const char* capability_id,
                                                            const char* contract_id, uint32_t required_scope,
                                                            uint32_t required_cardinality, const void** api);

typedef pih_status_v1 (*pih_lifecycle_callback_v1)(void* context);

typedef struct pih_plugin_lifecycle_v1 {
  uint32_t struct_size;
  uint32_t abi_version;
  pih_lifecycle_callback_v1 register_plugin;
  pih_lifecycle_callback_v1 configure;
  pih_lifecycle_callback_v1 start;
  pih_lifecycle_callback_v1 ready;
  pih_lifecycle_callback_v1 drain;
  pih_lifecycle_callback_v1 stop;
  pih_lifecycle_callback_v1 dispose;
} pih_plugin_lifecycle_v1;

typedef void (*pih_log_callback_v1)(void* context, uint32_t severity, const char* code, const char* message);

typedef struct pih_host_api_v1 {
  uint32_t struct_size;
  uint32_t abi_version;
  void* context;
  pih_log_callback_v1 log;
  pih_register_capability_callback_v1 register_capability;
  pih_resolve_capability_callback_v1 resolve_capability;
  uint64_t activation_epoch;
} pih_host_api_v1;

typedef struct pih_plugin_api_v1 {
  uint32_t struct_size;
  uint32_t abi_version;
  const char* plugin_id;
  const char* plugin_version;
  void* context;
  pih_plugin_lifecycle_v1 lifecycle;
} pih_plugin_api_v1;

typedef pih_status_v1 (*pih_plugin_entry_fn_v1)(const pih_host_api_v1* host, pih_plugin_api_v1* plugin);

/* A usable host table: every callback present, non-zero context and epoch. */
static inline int pih_host_api_is_valid_v1(const pih_host_api_v1* host) {
  return host != 0 && host->struct_size == sizeof(pih_host_api_v1) &&
         host->abi_version == PIH_PLUGIN_ABI_VERSION_V1 && host->context != 0 && host->log != 0 &&
         host->register_capability != 0 && host->resolve_capability != 0 && host->activation_epoch != 0;
}

static inline int pih_plugin_api_accepts_v1(const pih_plugin_api_v1* plugin) {
  return plugin != 0 && plugin->struct_size == sizeof(pih_plugin_api_v1) &&
         plugin->abi_version == PIH_PLUGIN_ABI_VERSION_V1;
}

#ifdef __cplusplus
}
#endif

#endif /* PIH_PLUGIN_SDK_PLUGIN_H_ */

/* Device backend contracts provided by the backend plugin, under the
 * capability ids the reference's Locks select:
 *   device.cuda-runtime.v1   / pih.device.cuda-runtime.v1    pih_nvidia_cuda_api_v1
 *   device.cuda-memory.v1    / pih.device.cuda-memory.v1     pih_nvidia_cuda_memory_api_v1
 *   device.cuda-resources.v1 / pih.device.cuda-resources.v1  pih_nvidia_cuda_resources_api_v1
 *   device.cuda-async.v1     / pih.device.cuda-async.v1      pih_nvidia_cuda_async_api_v1
 * and the platform contract the provider resolves (platform.linux.v1).
 *
 * Layout-compatible restatement of the reference's
 * include/pih/contracts/nvidia_cuda_v1.h:9-18, nvidia_cuda_memory_v1.h:13-47,
 * nvidia_cuda_resources_v1.h:11-37, nvidia_cuda_async_v1.h:11-54 and
 * platform_linux_v1.h.  The struct names keep their reference spelling so
 * that model plugins bind unchanged; on gfx950 the "retained context" is the
 * HIP provider's device-context token, streams are hipStream_t and events
 * hipEvent_t, all carried as uintptr_t. */
#ifndef PIH_CONTRACTS_DEVICE_CUDA_V1_H_
#define PIH_CONTRACTS_DEVICE_CUDA_V1_H_

#include <stdint.h>

#include "pih/plugin_sdk/status.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- device.cuda-runtime.v1 */
#define PIH_NVIDIA_CUDA_ABI_VERSION_V1 1U
typedef pih_status_v1 (*pih_nvidia_cuda_prepare_device_v1)(void* context, int32_t device_ordinal,
                                                            uint32_t expected_sm_major, uint32_t expected_sm_minor);
typedef struct pih_nvidia_cuda_api_v1 {
  uint32_t struct_size;
  uint32_t contract_version;
  void* context;
  pih_nvidia_cuda_prepare_device_v1 prepare_device;
} pih_nvidia_cuda_api_v1;

/* ---- device.cuda-memory.v1 */
#define PIH_NVIDIA_CUDA_MEMORY_ABI_VERSION_V1 1U
enum pih_cuda_memory_kind_v1 { PIH_CUDA_MEMORY_DEVICE_V1 = 1, PIH_CUDA_MEMORY_PINNED_HOST_V1 = 2 };
typedef struct pih_cuda_allocation_v1 {
  uint32_t struct_size;
  uint32_t abi_version;
  uintptr_t address;
  uint64_t bytes;
  uint64_t alignment;
  uint64_t generation;
  int32_t device_ordinal;
  uint32_t memory_kind;
} pih_cuda_allocation_v1;
typedef pih_status_v1 (*pih_cuda_allocate_v1)(void* context, int32_t device_ordinal, uint64_t bytes,
                                               uint64_t alignment, pih_cuda_allocation_v1* allocation);
typedef pih_status_v1 (*pih_cuda_deallocate_v1)(void* context, const pih_cuda_allocation_v1* allocation);
typedef pih_status_v1 (*pih_cuda_copy_h2d_v1)(void* context, int32_t device_ordinal, uintptr_t destination,
                                               const void* source, uint64_t bytes);
typedef struct pih_nvidia_cuda_memory_api_v1 {
  uint32_t struct_size;
  uint32_t contract_version;
  void* context;
  pih_cuda_allocate_v1 allocate_device;
  pih_cuda_deallocate_v1 deallocate_device;
  pih_cuda_allocate_v1 allocate_pinned_host;
  pih_cuda_deallocate_v1 deallocate_pinned_host;
  pih_cuda_copy_h2d_v1 copy_h2d;
} pih_nvidia_cuda_memory_api_v1;

/* ---- device.cuda-resources.v1 */
#define PIH_NVIDIA_CUDA_RESOURCES_ABI_VERSION_V1 1U
#define PIH_CUDA_CONTEXT_SCHED_YIELD_V1 0x02U
typedef pih_status_v1 (*pih_cuda_retain_primary_context_v1)(void* context, int32_t device_ordinal,
                                                             uint32_t context_flags, uintptr_t* retained_context);
typedef pih_status_v1 (*pih_cuda_bind_runtime_v1)(void* context, int32_t device_ordinal,
                                                   uintptr_t retained_context);
typedef pih_status_v1 (*pih_cuda_create_context_resource_v1)(void* context, uintptr_t retained_context,
                                                              uintptr_t* resource);
typedef pih_status_v1 (*pih_cuda_destroy_resource_v1)(void* context, uintptr_t resource);
typedef pih_status_v1 (*pih_cuda_release_primary_context_v1)(void* context, int32_t device_ordinal,
                                                              uintptr_t retained_context);
typedef struct pih_nvidia_cuda_resources_api_v1 {
  uint32_t struct_size;
  uint32_t contract_version;
  void* context;
  pih_cuda_retain_primary_context_v1 retain_primary_context;
  pih_cuda_bind_runtime_v1 bind_runtime;
  pih_cuda_create_context_resource_v1 create_nonblocking_stream;
  pih_cuda_create_context_resource_v1 create_disable_timing_event;
  pih_cuda_destroy_resource_v1 destroy_event;
  pih_cuda_destroy_resource_v1 destroy_stream;
  pih_cuda_release_primary_context_v1 release_primary_context;
} pih_nvidia_cuda_resources_api_v1;

/* ---- device.cuda-async.v1 */
#define PIH_NVIDIA_CUDA_ASYNC_ABI_VERSION_V1 1U
#define PIH_CUDA_COPY_H2D_V1 1U
#define PIH_CUDA_COPY_D2H_V1 2U
#define PIH_CUDA_COPY_D2D_V1 3U
#define PIH_CUDA_EVENT_COMPLETE_V1 1U
#define PIH_CUDA_EVENT_PENDING_V1 2U
typedef pih_status_v1 (*pih_cuda_activate_context_v1)(void* context, uintptr_t retained_context);
typedef pih_status_v1 (*pih_cuda_require_clean_last_error_v1)(void* context, uintptr_t retained_context);
typedef pih_status_v1 (*pih_cuda_validate_pinned_host_v1)(void* context, uintptr_t retained_context,
                                                           uintptr_t pointer);
typedef pih_status_v1 (*pih_cuda_copy_async_v1)(void* context, uintptr_t retained_context, uintptr_t destination,
                                                 uintptr_t source, uint64_t bytes, uint32_t copy_kind,
                                                 uintptr_t stream);
typedef pih_status_v1 (*pih_cuda_memset_async_v1)(void* context, uintptr_t retained_context, uintptr_t destination,
                                                   uint32_t byte_value, uint64_t bytes, uintptr_t stream);
typedef pih_status_v1 (*pih_cuda_record_event_v1)(void* context, uintptr_t retained_context, uintptr_t event,
                                                   uintptr_t stream);
typedef pih_status_v1 (*pih_cuda_query_event_v1)(void* context, uintptr_t retained_context, uintptr_t event,
                                                  uint32_t* event_status);
typedef pih_status_v1 (*pih_cuda_synchronize_stream_v1)(void* context, uintptr_t retained_context,
                                                         uintptr_t stream);
typedef struct pih_nvidia_cuda_async_api_v1 {
  uint32_t struct_size;
  uint32_t contract_version;
  void* context;
  pih_cuda_activate_context_v1 activate_context;
  pih_cuda_validate_pinned_host_v1 validate_pinned_host;
  pih_cuda_copy_async_v1 copy_async;
  pih_cuda_memset_async_v1 memset_async;
  pih_cuda_record_event_v1 record_event;
  pih_cuda_query_event_v1 query_event;
  pih_cuda_synchronize_stream_v1 synchronize_stream;
  pih_cuda_require_clean_last_error_v1 require_clean_last_error;
} pih_nvidia_cuda_async_api_v1;

/* ---- platform.linux.v1 (resolved during configure, called at start) */
#define PIH_PLATFORM_LINUX_ABI_VERSION_V1 1U
typedef pih_status_v1 (*pih_platform_linux_validate_runtime_v1)(void* context);
typedef struct pih_platform_linux_api_v1 {
  uint32_t struct_size;
  uint32_t contract_version;
  void* context;
  pih_platform_linux_validate_runtime_v1 validate_runtime;
} pih_platform_linux_api_v1;

#ifdef __cplusplus
}
#endif

#endif /* PIH_CONTRACTS_DEVICE_CUDA_V1_H_ */

/* gfx950 kernel-module driver: the C ABI a model plugin links to load a
 * verified code object by kernel name and launch it with a packed kernel
 * argument buffer.  It replaces, for HIP on MI355X:
 *   - KernelModuleDriver / NvidiaKernelModuleDriver
 *     (include/pih/backend/cuda/verified_kernel_module.h:24-37,
 *     src/backend/cuda/nvidia_kernel_module_driver.cpp:69-158): module load
 *     and unload, function by name, the parameter layout of a function;
 *   - VerifiedKernelModule::Load (verified_kernel_module.h:38-82,
 *     src/backend/cuda/verified_kernel_module.cpp:47-100): entrypoint
 *     checks, image digest against each signature, every function's
 *     parameter layout against its signature, rollback on failure;
 *   - submit_verified_kernel and KernelLaunchGeometry::Create
 *     (src/backend/cuda/verified_kernel_launcher.cpp:10-57): geometry
 *     bounds, stream 0 refused, the packet's identity against the
 *     function's, clean error state before and after the launch;
 *   - the cubin artifact manifest check (src/backend/cuda/
 *     cubin_artifact_manifest.cpp) for the code object's .json manifest
 *     (schema pih.code_object_artifact.v1).
 * CUDA's cuFuncGetParamInfo has no HIP counterpart: the parameter layout
 * of a function is read from the code object's own AMDGPU metadata note
 * (the explicit kernel arguments, their offsets and sizes).
 *
 * Library: libpih_hip_kernel_module.so (exports exactly the functions
 * below).  Status codes are those of pih_status_v1; no call throws. */
#ifndef PIH_BACKEND_HIP_KERNEL_MODULE_V1_H_
#define PIH_BACKEND_HIP_KERNEL_MODULE_V1_H_

#include <stdint.h>

#include "pih/plugin_sdk/status.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PIH_HIP_KERNEL_MODULE_ABI_VERSION_V1 1u
#define PIH_HIP_KERNEL_MODULE_MAX_ENTRYPOINTS_V1 1024u
#define PIH_HIP_KERNEL_SYMBOL_MAX_BYTES_V1 256u

/* Wire types of kernel parameters, in the order of the reference's
 * KernelWireType (include/pih/backend/cuda/kernel_signature_manifest.h:15-27). */
enum pih_hip_kernel_wire_type_v1 {
  PIH_HIP_WIRE_U8_V1 = 0,
  PIH_HIP_WIRE_U16_V1 = 1,
  PIH_HIP_WIRE_U32_V1 = 2,
  PIH_HIP_WIRE_U64_V1 = 3,
  PIH_HIP_WIRE_I32_V1 = 4,
  PIH_HIP_WIRE_I64_V1 = 5,
  PIH_HIP_WIRE_F32_V1 = 6,
  PIH_HIP_WIRE_F64_V1 = 7,
  PIH_HIP_WIRE_F16_BITS_V1 = 8,
  PIH_HIP_WIRE_BF16_BITS_V1 = 9,
  PIH_HIP_WIRE_DEVICE_POINTER_U64_V1 = 10
};

typedef struct pih_hip_kernel_parameter_v1 {
  uint32_t wire_type; /* pih_hip_kernel_wire_type_v1 */
  uint32_t offset;    /* byte offset in the kernel argument buffer */
} pih_hip_kernel_parameter_v1;

/* One entrypoint's expected signature (the reference's
 * KernelEntrypointRequest + KernelSignatureManifest). */
typedef struct pih_hip_kernel_signature_v1 {
  uint32_t struct_size;
  uint32_t abi_version;
  const char* symbol;               /* kernel name in the code object */
  const char* logical_id;           /* e.g. "qwen.linear.w4a16.compatibility.v1" */
  const char* code_object_sha256;   /* lowercase hex digest of the image it was made for */
  const char* parameter_abi_sha256; /* lowercase hex digest of the parameter descriptor */
  const pih_hip_kernel_parameter_v1* parameters;
  uint32_t parameter_count;
  uint32_t total_parameter_bytes; /* explicit argument bytes (packet size) */
} pih_hip_kernel_signature_v1;

typedef struct pih_hip_launch_geometry_v1 {
  uint32_t struct_size;
  uint32_t grid_x, grid_y, grid_z;
  uint32_t block_x, block_y, block_z;
  uint32_t dynamic_shared_bytes;
} pih_hip_launch_geometry_v1;

/* A ready kernel argument packet (the reference's KernelArgumentPacket
 * after ready_kernel_params): the explicit arguments at their offsets. */
typedef struct pih_hip_kernel_arguments_v1 {
  uint32_t struct_size;
  uint32_t abi_version;
  const char* logical_id;
  const char* parameter_abi_sha256;
  const void* packet;
  uint32_t packet_bytes;
} pih_hip_kernel_arguments_v1;

typedef struct pih_hip_kernel_module_v1 pih_hip_kernel_module_v1; /* opaque */

/* Checks the code object at `code_object_path` and its manifest
 * `<code_object_path>.json` (exact v1 field set, target gfx950, byte count,
 * SHA-256, AMDGPU ELF64) and every signature against the image: unique
 * symbols and logical ids, the image digest the signature names, and the
 * kernel's explicit arguments in the image's metadata equal to the
 * signature's parameters (count, offsets, sizes) and total bytes.  Touches
 * no device: usable on a host without a GPU. */
pih_status_v1 pih_hip_code_object_verify_v1(const char* code_object_path,
                                            const pih_hip_kernel_signature_v1* signatures,
                                            uint32_t signature_count);

/* pih_hip_code_object_verify_v1, then the current device must be gfx950;
 * hipModuleLoadData of the verified bytes and hipModuleGetFunction per
 * signature.  On any failure nothing stays loaded.  The module belongs to
 * the device current at this call. */
pih_status_v1 pih_hip_kernel_module_load_v1(const char* code_object_path,
                                            const pih_hip_kernel_signature_v1* signatures,
                                            uint32_t signature_count, pih_hip_kernel_module_v1** module);

/* Index of the function whose logical id is `logical_id`. */
pih_status_v1 pih_hip_kernel_module_find_v1(const pih_hip_kernel_module_v1* module, const char* logical_id,
                                            uint32_t* function_index);

/* Enqueues one launch: geometry dimensions non-zero and within the
 * hardware's bounds (grid x < 2^31, y and z <= 65535, block <= 1024
 * threads), stream != 0, the packet's logical id and parameter ABI digest
 * equal to the function's, packet_bytes equal to its total parameter
 * bytes, the current device equal to the module's, no sticky HIP error
 * before; then hipModuleLaunchKernel with the packet as the argument
 * buffer and the error state checked after.  Enqueue only. */
pih_status_v1 pih_hip_kernel_submit_v1(const pih_hip_kernel_module_v1* module, uint32_t function_index,
                                       const pih_hip_launch_geometry_v1* geometry, uintptr_t stream,
                                       const pih_hip_kernel_arguments_v1* arguments);

/* Unloads the module on its device and frees the handle (NULL is an
 * invalid argument). */
pih_status_v1 pih_hip_kernel_module_unload_v1(pih_hip_kernel_module_v1* module);

#ifdef __cplusplus
}
#endif

#endif /* PIH_BACKEND_HIP_KERNEL_MODULE_V1_H_ */

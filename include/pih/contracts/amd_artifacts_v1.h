/* On-disk weight formats of the linear path -> gfx950 device memory.
 *
 * Host C-ABI of libpih_amd_artifacts.so (plain pointers and sizes, no
 * device-framework types).  Every call returns pih_status_v1; none throws.
 *
 *   Qwen3 INT4 artifact "XINGW4A1" (xing-w4a16-sym-g128-v1,
 *   canonical-nk-low-nibble-k-v1): the 539,758,592-byte canonical file of
 *   Qwen3-0.6B -- a 1 MiB metadata region, then 506 payload extents in
 *   identity order, 4096-aligned and zero-padded.  Replaces the reference's
 *   QwenInt4ArtifactLayout::CreateOfficialPureW4
 *   (plugins/model-qwen3/artifact/qwen3_int4_artifact_layout.cpp:41-104),
 *   QwenInt4ArtifactMetadata::ParseAndVerify
 *   (qwen3_int4_artifact_metadata.cpp:145-196) and verify_qwen_int4_artifact
 *   (qwen3_int4_artifact_io.cpp:35-52, src/core/canonical_extent_verifier.cpp:11-57).
 *   Packed values are [N][K/2] bytes (low nibble = even k, signed int4 with
 *   0x8 reserved) and scales fp16 [N][K/128]: the layout the W4A16
 *   symmetric kernels read, so the upload is one copy of the data region and
 *   a record's device address is base + file_offset - metadata bytes.
 *
 *   DeepSeek V4 Flash expert bundle: 13,369,344 bytes per routed expert, six
 *   segments W1 packed, W1 scales, W2 packed, W2 scales, W3 packed, W3 scales
 *   (H 4096, I 2048; MXFP4 [rows][cols/2] + UE8M0 [rows][cols/32]).
 *   Replaces DeepSeekExpertBundleLayout::Bind
 *   (plugins/model-deepseek-v4-flash/deepseek_expert_bundle_layout.cpp:17-43),
 *   and repacks bundles into the grouped MoE weights of the linear pack's
 *   launch_moe_layer (gate rows W1 then up rows W3 per expert; W2). */
#ifndef PIH_CONTRACTS_AMD_ARTIFACTS_V1_H_
#define PIH_CONTRACTS_AMD_ARTIFACTS_V1_H_

#include <stdint.h>

#include "pih/plugin_sdk/status.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PIH_AMD_ARTIFACTS_ABI_VERSION_V1 1U

#define PIH_AMD_QWEN_INT4_FILE_BYTES_V1 539758592ULL
#define PIH_AMD_QWEN_INT4_METADATA_BYTES_V1 1048576ULL
#define PIH_AMD_QWEN_INT4_DATA_BYTES_V1 538710016ULL
#define PIH_AMD_QWEN_INT4_RECORD_COUNT_V1 507U

/* record kinds (QwenInt4ArtifactRecordKind) */
#define PIH_AMD_QWEN_INT4_PACKED_VALUES_V1 1U
#define PIH_AMD_QWEN_INT4_FP16_SCALES_V1 2U
#define PIH_AMD_QWEN_INT4_BF16_EMBEDDING_V1 3U
#define PIH_AMD_QWEN_INT4_BF16_NORM_V1 4U
#define PIH_AMD_QWEN_INT4_ALIAS_V1 5U

/* verify flags */
#define PIH_AMD_VERIFY_PAYLOADS_V1 1U /* payload SHA-256 digests and zero padding */

typedef struct pih_amd_qwen_int4_artifact_info_v1 {
  uint32_t struct_size, abi_version;
  uint32_t record_count, payload_record_count;
  uint64_t file_bytes, metadata_bytes, padded_data_bytes, logical_payload_bytes;
  uint32_t encoded_metadata_bytes, reserved;
  uint8_t source_artifact_root[32], source_binding_root[32], disposition_root[32];
} pih_amd_qwen_int4_artifact_info_v1;

typedef struct pih_amd_artifact_record_v1 {
  uint32_t struct_size, abi_version;
  uint32_t kind, reserved;
  uint64_t file_offset, logical_bytes, extent_bytes;
  uint64_t device_offset; /* file_offset - metadata bytes (alias: its owner's) */
  uint64_t rows, columns; /* source tensor [rows, columns]; norms: [1, width] */
} pih_amd_artifact_record_v1;

/* Checks a whole canonical file in host memory (e.g. mmap): size, metadata
 * region (magic, version, record count, zero tail, SHA-256 checksum, format
 * and layout identifiers, every record equal to the official layout,
 * non-empty roots) and, with PIH_AMD_VERIFY_PAYLOADS_V1, every payload's
 * SHA-256 and zero padding.  Fills *info on success. */
pih_status_v1 pih_amd_qwen_int4_artifact_verify_v1(const uint8_t* file, uint64_t file_bytes, uint32_t flags,
                                                   pih_amd_qwen_int4_artifact_info_v1* info);

/* Official-layout record of `identity` (e.g.
 * "model.layers.0.mlp.gate_proj.weight.packed_values"); no file needed. */
pih_status_v1 pih_amd_qwen_int4_artifact_record_v1(const char* identity, pih_amd_artifact_record_v1* out);

/* Copies the data region of a verified file (bytes [metadata, end)) to
 * device memory at device_dst (dst_bytes >= PIH_AMD_QWEN_INT4_DATA_BYTES_V1)
 * on `stream`; returns when the copy has completed. */
pih_status_v1 pih_amd_qwen_int4_artifact_upload_v1(const uint8_t* file, uint64_t file_bytes, uintptr_t device_dst,
                                                   uint64_t dst_bytes, uintptr_t stream);

#define PIH_AMD_EXPERT_BUNDLE_BYTES_V1 13369344ULL
#define PIH_AMD_EXPERT_BUNDLE_ALIGNMENT_V1 256ULL

typedef struct pih_amd_expert_bundle_view_v1 {
  uint32_t struct_size, abi_version;
  uintptr_t w1_packed, w1_scales, w2_packed, w2_scales, w3_packed, w3_scales;
  uint64_t packed_bytes, scale_bytes;
} pih_amd_expert_bundle_view_v1;

/* DeepSeekExpertBundleLayout::Bind: base non-zero, 256-byte aligned, and
 * base + 13,369,344 representable. */
pih_status_v1 pih_amd_deepseek_expert_bundle_bind_v1(uintptr_t base, pih_amd_expert_bundle_view_v1* out);

typedef struct pih_amd_bundles_to_moe_v1 {
  uint32_t struct_size, abi_version;
  const uintptr_t* bundle_bases; /* host array [expert_count] of device bundle addresses */
  uintptr_t w13_packed;          /* e2m1 [E][4096][2048]: W1 rows then W3 rows */
  uintptr_t w13_scales;          /* UE8M0 [E][4096][128] */
  uintptr_t w2_packed;           /* e2m1 [E][4096][1024] */
  uintptr_t w2_scales;           /* UE8M0 [E][4096][64] */
  uintptr_t stream;
  uint32_t expert_count, reserved;
} pih_amd_bundles_to_moe_v1;

/* Enqueues device copies of each bundle into expert slot e of the grouped
 * MoE weights (gate/up fused as launch_moe_layer reads them). */
pih_status_v1 pih_amd_deepseek_bundles_to_moe_v1(const pih_amd_bundles_to_moe_v1* request);

#ifdef __cplusplus
}
#endif

#endif /* PIH_CONTRACTS_AMD_ARTIFACTS_V1_H_ */

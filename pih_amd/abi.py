"""ctypes mirror of the C ABI the gfx950 packs export.

Struct layouts restate ``include/pih/plugin_sdk/*.h`` and
``include/pih/contracts/*.h`` field for field (``tests/test_abi_layout.py``
compiles the headers and checks every size and offset against this file).
``load_pack`` performs the same checks as the reference's
``KernelPackLoader`` (src/microkernel/kernel_pack_loader.cpp:90-123): both
symbols resolve, identity/api struct sizes and ABI versions match, ids are
canonical ``[a-z0-9.-]``, ``api.identity`` is the identity pointer, the
contract table is present and ``bind_origin`` accepts the absolute path.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os
from typing import Dict, Optional

U32, U64, UPTR, F32, F64, I32 = C.c_uint32, C.c_uint64, C.c_size_t, C.c_float, C.c_double, C.c_int32

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
DEEPSEEK_PACK = os.path.join(LIB_DIR, "libpih_kernels_deepseek_v4_gfx950.so")
LINEAR_PACK = os.path.join(LIB_DIR, "libpih_kernels_amd_linear_gfx950.so")
QWEN_PACK = os.path.join(LIB_DIR, "libpih_kernels_qwen3_gfx950.so")

# pih_status_code_v1
OK, INVALID_ARGUMENT, FAILED_PRECONDITION, INTERNAL, UNAVAILABLE, RESOURCE_EXHAUSTED, DEADLINE_EXCEEDED = range(7)
STATUS_NAMES = ["OK", "INVALID_ARGUMENT", "FAILED_PRECONDITION", "INTERNAL", "UNAVAILABLE",
                "RESOURCE_EXHAUSTED", "DEADLINE_EXCEEDED"]


class Status(C.Structure):
    _fields_ = [("struct_size", U32), ("abi_version", U32), ("code", U32), ("message", C.c_char * 256)]

    def __repr__(self):
        name = STATUS_NAMES[self.code] if self.code < len(STATUS_NAMES) else str(self.code)
        return f"Status({name}, {self.message.decode(errors='replace')!r})"


class Identity(C.Structure):
    _fields_ = [("struct_size", U32), ("abi_version", U32), ("pack_id", C.c_char_p),
                ("pack_version", C.c_char_p), ("pack_abi", C.c_char_p), ("architecture", C.c_char_p)]


BIND_ORIGIN = C.CFUNCTYPE(Status, C.c_char_p)


class PackApi(C.Structure):
    _fields_ = [("struct_size", U32), ("abi_version", U32), ("identity", C.POINTER(Identity)),
                ("contract_api", C.c_void_p), ("bind_origin", BIND_ORIGIN)]


def _struct(name: str, fields):
    return type(name, (C.Structure,), {"_fields_": fields})


def _hdr(*rest):
    return [("struct_size", U32), ("abi_version", U32)] + list(rest)


def _u(*names):
    return [(n, UPTR) for n in names]


def _i(*names):
    return [(n, U32) for n in names]


# ---------------------------------------------------------------- DeepSeek
DS = {}
DS["rope_table"] = _struct("RopeTable", _hdr(*_u("output_f32", "error_flag_u32", "stream"),
                                             *_i("position_count", "rope_dimension"),
                                             ("theta", F64), ("scaling_factor", F64),
                                             *_i("original_maximum_positions", "beta_fast", "beta_slow", "yarn")))
DS["rms_norm"] = _struct("RmsNorm", _hdr(*_u("input_bf16", "weight_bf16", "output_bf16", "error_flag", "stream"),
                                         *_i("rows", "hidden_size"), ("epsilon", F32)))
DS["fp8_activation_quant"] = _struct("Fp8ActivationQuant", _hdr(
    *_u("input_bf16", "output_e4m3", "scale_bits", "error_flag", "stream"), *_i("token_count", "logical_k")))
DS["fp8_gemm"] = _struct("Fp8Gemm", _hdr(
    *_u("activation_e4m3", "activation_scale_bits", "weight_e4m3", "weight_scale_bits", "output",
        "error_flag", "stream"), *_i("m", "n", "k", "output_type")))
DS["head_rms"] = _struct("HeadRms", _hdr(*_u("input_bf16", "output_bf16", "error_flag_u32", "stream"),
                                         *_i("token_count", "head_count", "head_dimension"), ("epsilon", F32)))
DS["rotary"] = _struct("Rotary", _hdr(*_u("input_bf16", "frequencies_f32", "error_flag_u32", "stream"),
                                      *_i("token_count", "head_count", "head_dimension", "rope_dimension", "inverse"),
                                      ("positions_u32", UPTR), ("table_position_count", U32)))
DS["kv_fp8_simulate"] = _struct("KvFp8Simulate", _hdr(*_u("kv_bf16", "error_flag_u32", "stream"),
                                                      *_i("token_count", "vector_dimension",
                                                          "quantized_dimension", "group_size")))
DS["grouped_fp8_gemm"] = _struct("GroupedFp8Gemm", _hdr(
    *_u("input_bf16", "activation_e4m3", "activation_scale_bits", "weight_e4m3", "weight_scale_bits",
        "output_bf16", "error_flag_u32", "stream"),
    *_i("token_count", "group_count", "output_per_group", "input_per_group")))
DS["route_gather"] = _struct("RouteGather", _hdr(
    *_u("source_hidden_bf16", "token_indices_u32", "route_hidden_bf16", "error_flag", "stream"),
    *_i("route_count", "packed_token_count")))
DS["fp4_gemm"] = _struct("Fp4Gemm", _hdr(
    *_u("activation_e4m3", "activation_scale_bits", "packed_weight", "weight_scale_bits", "output_bf16",
        "error_flag", "stream"), *_i("m", "n", "k")))
DS["expert_swiglu"] = _struct("ExpertSwiGlu", _hdr(
    *_u("gate_bf16", "up_bf16", "route_weights_f32", "output_bf16", "error_flag", "stream"), *_i("token_count")))
DS["expert_accumulate"] = _struct("ExpertAccumulate", _hdr(
    *_u("expert_output_bf16", "token_indices", "accumulator_f32", "error_flag", "stream"),
    *_i("route_count", "token_count")))
DS["embedding"] = _struct("Embedding", _hdr(*_u("token_ids_u32", "weight_bf16", "output_hc_bf16",
                                                "error_flag_u32", "stream"),
                                            *_i("token_count", "vocab_size", "hidden_size", "hc_multiplicity")))
DS["hc_head"] = _struct("HcHead", _hdr(*_u("input_hc_bf16", "fn_f32", "scale_f32", "base_f32", "output_bf16",
                                           "error_flag_u32", "stream"),
                                       *_i("token_count", "hidden_size", "hc_multiplicity"),
                                       ("rms_epsilon", F32), ("hc_epsilon", F32)))
DS["lm_head"] = _struct("LmHead", _hdr(*_u("input_bf16", "weight_bf16", "logits_f32", "error_flag_u32", "stream"),
                                       *_i("output_rows", "vocab_size", "hidden_size")))
Suppressed = _struct("Suppressed", [("token_ids", U32 * 17), ("token_count", U32)])
DS["argmax"] = _struct("Argmax", _hdr(*_u("logits_f32", "token_id_u32", "error_flag_u32", "stream"),
                                      ("vocab_size", U32),
                                      *_u("selected_logprob_f32", "top_logprobs_ids_u32", "top_logprobs_f32"),
                                      ("top_logprobs_count", U32), ("suppressed_tokens", Suppressed)))
DS["stochastic_sample"] = _struct("StochasticSample", _hdr(
    *_u("logits_f32", "token_id_u32", "selected_logprob_f32", "rng_word_u32", "workspace_values_f32",
        "workspace_ids_u32", "error_flag_u32", "stream"),
    *_i("vocab_size", "workspace_capacity"), ("temperature", F32), ("top_p", F32), ("top_k", U32),
    ("seed", U64), ("sample_ordinal", U64), *_u("top_logprobs_ids_u32", "top_logprobs_f32"),
    ("top_logprobs_count", U32), ("suppressed_tokens", Suppressed)))
DS["compressor_pooling"] = _struct("CompressorPooling", _hdr(
    *_u("kv_projection_f32", "gate_projection_f32", "ape_row_f32", "kv_state_f32", "score_state_f32",
        "output_f32", "error_flag_u32", "stream"), *_i("batch_count", "ratio", "head_dim", "absolute_position")))
DS["compressor_projection"] = _struct("CompressorProjection", _hdr(
    *_u("input_bf16", "kv_weight_bf16", "gate_weight_bf16", "kv_projection_f32", "gate_projection_f32",
        "error_flag_u32", "stream"), *_i("token_count", "ratio", "head_dim", "hidden_size")))
DS["compressor_store"] = _struct("CompressorStore", _hdr(
    *_u("compressed_f32", "rms_weight_bf16", "cos_sin_cache_f32", "destination_bf16", "error_flag_u32", "stream"),
    *_i("head_dim", "rope_head_dim", "rope_position"), ("rms_epsilon", F32)))
DS["indexer_projection"] = _struct("IndexerProjection", _hdr(
    *_u("qr_bf16", "hidden_bf16", "wq_b_e4m3", "wq_b_scale_bits", "qr_e4m3", "qr_scale_bits",
        "weights_proj_bf16", "frequencies_f32", "positions_u32", "query_bf16", "head_weight_f32",
        "error_flag_u32", "stream"), *_i("token_count", "table_position_count")))
DS["index_score"] = _struct("IndexScore", _hdr(
    *_u("query_bf16", "index_kv_bf16", "head_weight_f32", "score_f32", "error_flag_u32", "stream"),
    *_i("query_count", "head_count", "slot_count"), ("page_slots_u32", UPTR),
    *_i("slot_base", "logical_page_count", "physical_page_count")))
DS["sparse_attention"] = _struct("SparseAttention", _hdr(
    *_u("query_bf16", "latent_kv_bf16", "attention_sink_f32", "indices_i32", "output_bf16", "error_flag_u32",
        "stream"), *_i("query_count", "head_count", "kv_count", "index_count"),
    *_u("compressed_kv_bf16", "page_slots_u32"), ("recent_physical_offset", I32),
    ("compressed_physical_offset", I32), *_i("compressed_slot_count", "logical_page_count",
                                             "physical_page_count")))
DS["router_gemm"] = _struct("RouterGemm", _hdr(*_u("input_bf16", "weight_bf16", "scores_f32", "error_flag_u32",
                                                   "stream"), *_i("token_count", "expert_count", "hidden_size")))
DS["mhc_pre"] = _struct("MhcPre", _hdr(
    *_u("residual_bf16", "fn_f32", "scale_f32", "base_f32", "norm_weight_bf16", "post_mix_f32",
        "residual_mix_f32", "layer_input_bf16", "error_flag_u32", "stream"), *_i("token_count", "hidden_size"),
    ("rms_epsilon", F32), ("pre_epsilon", F32), ("sinkhorn_epsilon", F32), ("post_multiplier", F32),
    ("sinkhorn_iterations", U32)))
DS["mhc_post"] = _struct("MhcPost", _hdr(*_u("layer_output_bf16", "residual_bf16", "post_mix_f32",
                                             "residual_mix_f32", "output_bf16", "error_flag_u32", "stream"),
                                         *_i("token_count", "hidden_size")))
DS["mhc_target_tap"] = _struct("MhcTargetTap", _hdr(
    *_u("residual_hc_bf16", "target_hidden_bf16", "error_flag_u32", "stream"),
    *_i("token_count", "hidden_size", "source_stream_count", "target_stage_count", "target_stage_index")))
DS["shared_swiglu"] = _struct("SharedSwiGlu", _hdr(*_u("gate_bf16", "up_bf16", "output_bf16", "error_flag", "stream"),
                                                   *_i("token_count")))
DS["expert_finalize"] = _struct("ExpertFinalize", _hdr(
    *_u("accumulator_f32", "shared_output_bf16", "output_bf16", "error_flag", "stream"), *_i("token_count")))

DS_ORDER = ["rope_table", "rms_norm", "fp8_activation_quant", "fp8_gemm", "head_rms", "rotary",
            "kv_fp8_simulate", "grouped_fp8_gemm", "route_gather", "fp4_gemm", "expert_swiglu",
            "expert_accumulate", "embedding", "hc_head", "lm_head", "argmax", "stochastic_sample",
            "compressor_pooling", "compressor_projection", "compressor_store", "indexer_projection",
            "index_score", "sparse_attention", "router_gemm", "mhc_pre", "mhc_post", "mhc_target_tap",
            "shared_swiglu", "expert_finalize"]
DS_API = _struct("DeepSeekKernelsApi", [("struct_size", U32), ("contract_version", U32),
                                        ("identity", C.POINTER(Identity))] +
                 [("launch_" + n, C.CFUNCTYPE(Status, C.POINTER(DS[n]))) for n in DS_ORDER])

# ------------------------------------------------------------ AMD linear
LN = {}
LN["workspace_query"] = _struct("WorkspaceQuery", _hdr(*_i("kind", "m", "n", "k"), ("bytes_u64", UPTR)))
LN["route_plan"] = _struct("RoutePlan", _hdr(
    *_u("topk_ids_u32", "topk_weights_f32", "expert_offsets_u32", "row_token_u32", "row_weight_f32",
        "token_rows_u32", "workspace"), ("workspace_bytes", U64), *_u("error_flag_u32", "stream"),
    *_i("token_count", "top_k", "expert_count")))
LN["fp8_quant"] = _struct("Fp8Quant", _hdr(*_u("input_bf16", "row_index_u32", "output_e4m3", "scale",
                                               "error_flag_u32", "stream"),
                                           *_i("row_count", "logical_k", "input_rows", "scale_format")))
LN["fp8_gemm"] = _struct("AmdFp8Gemm", _hdr(*_u("activation_e4m3", "activation_scale", "weight_e4m3",
                                                "weight_scale", "output", "error_flag_u32", "stream"),
                                            *_i("m", "n", "k", "scale_format", "output_type")))
LN["moe_fp8_gemm"] = _struct("MoeFp8Gemm", _hdr(
    *_u("activation_e4m3", "activation_scale", "row_token_u32", "weight_e4m3", "weight_scale",
        "expert_offsets_u32", "row_weight_f32", "output", "error_flag_u32", "stream"),
    *_i("row_capacity", "expert_count", "n", "k", "activation_rows", "scale_format", "output_type"),
    ("swiglu_limit", F32), *_u("output_scale")))
LN["moe_mxfp4_gemm"] = _struct("MoeMxfp4Gemm", _hdr(
    *_u("activation", "activation_scale_ue8m0", "row_token_u32", "packed_weight", "weight_scale_ue8m0",
        "expert_offsets_u32", "row_weight_f32", "output", "error_flag_u32", "stream"),
    *_i("row_capacity", "expert_count", "n", "k", "activation_rows", "activation_type", "output_type"),
    ("swiglu_limit", F32)))
LN["moe_combine"] = _struct("MoeCombine", _hdr(*_u("expert_output_bf16", "token_rows_u32", "shared_bf16",
                                                   "output_bf16", "error_flag_u32", "stream"),
                                               *_i("token_count", "top_k", "hidden_size", "row_count")))
LN["bf16_gemm"] = _struct("Bf16Gemm", _hdr(*_u("a_bf16", "w_bf16", "output", "workspace"),
                                           ("workspace_bytes", U64), ("stream", UPTR),
                                           *_i("m", "n", "k", "output_type")))
LN["w4a16"] = _struct("W4a16", _hdr(*_u("input_bf16", "qweight", "scales", "zeros", "output_bf16", "workspace"),
                                    ("workspace_bytes", U64), *_u("error_flag_u32", "stream"),
                                    *_i("m", "n", "k", "format")))
LN["router_topk"] = _struct("RouterTopk", _hdr(*_u("scores_f32", "bias_f32", "topk_ids_u32", "topk_weights_f32",
                                                    "error_flag_u32", "stream"),
                                                *_i("token_count", "expert_count", "top_k", "mode"),
                                                ("route_scale", C.c_float)))
_V41_BYTES = {"input_bf16": "input_bytes", "weight": "weight_bytes", "weight_scales": "weight_scale_bytes",
              "quantized_e4m3": "quantized_bytes", "activation_scales": "activation_scale_bytes",
              "output_bf16": "output_bytes", "error_flag_u32": "error_flag_bytes"}
LN["v41_linear"] = _struct("V41Linear", _hdr(
    *[f for name in ("input_bf16", "weight", "weight_scales", "quantized_e4m3", "activation_scales", "output_bf16",
                     "error_flag_u32") for f in ((name, UPTR), (_V41_BYTES[name], U64))],
    ("stream", UPTR), *_i("rows", "in_features", "out_features", "weight_format")))
LN["v41_fp4_to_fp8"] = _struct("V41Fp4ToFp8", _hdr(*_u("packed", "scales", "weight_e4m3", "weight_scales",
                                                        "error_flag_u32", "stream"), *_i("rows", "columns")))
LN["v41_block_dequant"] = _struct("V41BlockDequant", _hdr(*_u("source_e4m3", "scales", "output_bf16",
                                                              "error_flag_u32", "stream"),
                                                          *_i("rows", "columns", "block", "scale_storage")))
V41_WEIGHT_FP8_BLOCK32, V41_WEIGHT_MXFP4 = 1, 2
V41_SCALE_E8M0, V41_SCALE_F32 = 1, 2
LN["silu_mul"] = _struct("SiluMul", _hdr(*_u("gate_bf16", "up_bf16", "output_bf16", "stream"), ("count", U64)))
LN["swiglu"] = _struct("SwiGlu", _hdr(*_u("gate_bf16", "up_bf16", "route_weights_f32", "output_bf16",
                                          "error_flag_u32", "stream"), *_i("rows", "cols"), ("limit", F32)))
LN["mxfp4_decode"] = _struct("Mxfp4Decode", _hdr(*_u("packed", "scales_ue8m0", "output_bf16", "error_flag_u32",
                                                     "stream"), *_i("rows", "k")))
LN["w4a16_dequant"] = _struct("W4a16Dequant", _hdr(*_u("qweight", "scales", "zeros", "output_f32", "error_flag_u32",
                                                      "stream"), *_i("n", "k", "format")))
LN["w4a16_grouped"] = _struct("W4a16Grouped", _hdr(*_u("problems", "error_flag_u32", "stream"),
                                                    *_i("problem_count", "m", "k", "format")))
LN["moe_layer"] = _struct("MoeLayer", _hdr(*_u("input_bf16", "topk_ids_u32", "topk_weights_f32", "w13", "w13_scale",
                                             "w2", "w2_scale", "shared_bf16", "output_bf16", "workspace"),
                                          ("workspace_bytes", U64), *_u("required_bytes_u64", "error_flag_u32",
                                                                        "stream"),
                                          *_i("token_count", "top_k", "expert_count", "hidden_size",
                                              "intermediate_size", "weight_format", "scale_format",
                                              "activation_type"), ("swiglu_limit", F32)))
WEIGHT_FP8, WEIGHT_MXFP4 = 1, 2
# pih_amd_w4a16_problem_v1: one entry of the grouped launch's host array
W4A16_PROBLEM = _struct("W4a16Problem", _u("input_bf16", "qweight", "scales", "zeros", "output_bf16") +
                        _i("n", "reserved"))
W4A16_GROUP_MAX = 8
LN_ORDER = [("query_workspace", "workspace_query"), ("launch_route_plan", "route_plan"),
            ("launch_fp8_quant", "fp8_quant"), ("launch_fp8_gemm", "fp8_gemm"),
            ("launch_moe_fp8_gemm", "moe_fp8_gemm"), ("launch_moe_mxfp4_gemm", "moe_mxfp4_gemm"),
            ("launch_moe_combine", "moe_combine"), ("launch_bf16_gemm", "bf16_gemm"),
            ("launch_w4a16_gemm", "w4a16"), ("launch_silu_mul", "silu_mul"), ("launch_swiglu", "swiglu"),
            ("launch_mxfp4_decode", "mxfp4_decode"), ("launch_w4a16_dequant", "w4a16_dequant"),
            ("launch_w4a16_grouped", "w4a16_grouped"), ("query_moe_layer_workspace", "moe_layer"),
            ("launch_moe_layer", "moe_layer"), ("launch_route_plan_noalloc", "route_plan"),
            ("launch_router_topk", "router_topk"), ("launch_v41_linear", "v41_linear"),
            ("launch_v41_fp4_to_fp8", "v41_fp4_to_fp8"), ("launch_v41_block_dequant", "v41_block_dequant")]
LN_API = _struct("AmdLinearKernelsApi", [("struct_size", U32), ("contract_version", U32),
                                         ("identity", C.POINTER(Identity))] +
                 [(f, C.CFUNCTYPE(Status, C.POINTER(LN[s]))) for f, s in LN_ORDER])

# pih_qwen_kernels_api_v1 (include/pih/contracts/qwen_kernels_v1.h)
QWEN_API = _struct("QwenKernelsApi", [("struct_size", U32), ("contract_version", U32), ("target_sm", U32),
                                      ("root", C.CFUNCTYPE(Status, C.POINTER(C.c_char_p)))])

# kernel-module driver and Qwen W4A16 plan (include/pih/backend/hip/
# kernel_module_v1.h, include/pih/contracts/qwen_int4_plan_gfx950_v1.h),
# libpih_hip_kernel_module.so
KERNEL_MODULE_LIB = os.path.join(LIB_DIR, "libpih_hip_kernel_module.so")
WIRE_U64, WIRE_DEVICE_POINTER_U64 = 3, 10
KM_PARAMETER = _struct("HipKernelParameter", [("wire_type", U32), ("offset", U32)])
KM_SIGNATURE = _struct("HipKernelSignature", [("struct_size", U32), ("abi_version", U32), ("symbol", C.c_char_p),
                                              ("logical_id", C.c_char_p), ("code_object_sha256", C.c_char_p),
                                              ("parameter_abi_sha256", C.c_char_p),
                                              ("parameters", C.POINTER(KM_PARAMETER)), ("parameter_count", U32),
                                              ("total_parameter_bytes", U32)])
KM_GEOMETRY = _struct("HipLaunchGeometry", [("struct_size", U32), ("grid_x", U32), ("grid_y", U32), ("grid_z", U32),
                                            ("block_x", U32), ("block_y", U32), ("block_z", U32),
                                            ("dynamic_shared_bytes", U32)])
KM_ARGUMENTS = _struct("HipKernelArguments", [("struct_size", U32), ("abi_version", U32), ("logical_id", C.c_char_p),
                                              ("parameter_abi_sha256", C.c_char_p), ("packet", C.c_void_p),
                                              ("packet_bytes", U32)])
QWEN_INT4_COMPAT, QWEN_INT4_GFX950 = 1, 2
QWEN_INT4_PLAN = _struct("QwenInt4GemmPlan", [("struct_size", U32), ("abi_version", U32), ("variant", U32),
                                              ("reserved", U32), ("kernel_symbol", C.c_char_p),
                                              ("logical_id", C.c_char_p), ("parameter_abi_sha256", C.c_char_p),
                                              ("geometry", KM_GEOMETRY), ("tokens", U64), ("output_features", U64),
                                              ("input_features", U64), ("input_bytes", U64), ("packed_bytes", U64),
                                              ("scale_bytes", U64), ("output_bytes", U64)])

_kernel_module = None


def kernel_module_lib() -> C.CDLL:
    """libpih_hip_kernel_module.so with its seven entries typed."""
    global _kernel_module
    if _kernel_module is None:
        if not os.path.exists(KERNEL_MODULE_LIB):
            raise PackError(f"kernel-module driver not built: {KERNEL_MODULE_LIB}")
        L = C.CDLL(KERNEL_MODULE_LIB)
        P = C.c_void_p
        sigs = {
            "pih_hip_code_object_verify_v1": [C.c_char_p, C.POINTER(KM_SIGNATURE), U32],
            "pih_hip_kernel_module_load_v1": [C.c_char_p, C.POINTER(KM_SIGNATURE), U32, C.POINTER(P)],
            "pih_hip_kernel_module_find_v1": [P, C.c_char_p, C.POINTER(U32)],
            "pih_hip_kernel_submit_v1": [P, U32, C.POINTER(KM_GEOMETRY), UPTR, C.POINTER(KM_ARGUMENTS)],
            "pih_hip_kernel_module_unload_v1": [P],
            "pih_qwen_int4_gemm_plan_create_v1": [U64, U64, U64, U32, C.POINTER(QWEN_INT4_PLAN)],
            "pih_qwen_int4_gemm_signature_v1": [U32, C.c_char_p, C.POINTER(KM_PARAMETER), C.POINTER(KM_SIGNATURE)],
        }
        for name, args in sigs.items():
            fn = getattr(L, name)
            fn.restype = Status
            fn.argtypes = args
        _kernel_module = L
    return _kernel_module


SCALE_F32, SCALE_UE8M0 = 1, 2
OUTPUT_BF16, OUTPUT_F32, OUTPUT_SWIGLU_BF16, OUTPUT_SWIGLU_E4M3 = 1, 2, 3, 4
ACTIVATION_E4M3, ACTIVATION_BF16 = 1, 2
W4A16_SYMMETRIC, W4A16_ASYMMETRIC = 1, 2
WORKSPACE_ROUTE_PLAN, WORKSPACE_BF16_GEMM, WORKSPACE_W4A16 = 1, 2, 3
ROUTER_SOFTMAX, ROUTER_SQRT_SOFTPLUS = 1, 2


class PackError(RuntimeError):
    pass


def valid_canonical_id(value: Optional[bytes], maximum: int) -> bool:
    """kernel_pack_loader.cpp:49-65: [a-z0-9.-], no leading/trailing/double dot."""
    if not value or len(value) > maximum:
        return False
    s = value.decode("ascii", errors="replace")
    if s[0] == "." or s[-1] == ".":
        return False
    prev = ""
    for ch in s:
        if not (("a" <= ch <= "z") or ("0" <= ch <= "9") or ch in ".-") or (ch == "." and prev == "."):
            return False
        prev = ch
    return True


class KernelPack:
    def __init__(self, path, handle, identity, api, table):
        self.path = path
        self.handle = handle
        self.identity = identity
        self.api = api
        self.table = table

    @property
    def pack_id(self) -> str:
        return self.identity.pack_id.decode()

    @property
    def pack_abi(self) -> str:
        return self.identity.pack_abi.decode()

    @property
    def architecture(self) -> str:
        return self.identity.architecture.decode()

    def call(self, entry: str, request) -> Status:
        fn = getattr(self.table, entry)
        if not fn:
            raise PackError(f"{entry} is null")
        return fn(C.byref(request))


_loaded: Dict[str, KernelPack] = {}


def load_pack(path: str, contract: str, expected_sha256: Optional[str] = None) -> KernelPack:
    """Load a Kernel Pack with the reference loader's checks; packs are never
    unloaded (kernel_pack_loader.cpp:117-119)."""
    path = os.path.abspath(path)
    if path in _loaded:
        pack = _loaded[path]
        if pack.pack_abi != contract:
            raise PackError(f"contract mismatch: pack exports {pack.pack_abi!r}, caller wants {contract!r}")
        return pack
    if not os.path.exists(path):
        raise PackError(f"kernel_pack_load_failed: {path} not built (run __graft_entry__.build())")
    if expected_sha256 is not None:
        with open(path, "rb") as f:
            if hashlib.sha256(f.read()).hexdigest() != expected_sha256.lower():
                raise PackError("kernel_pack_load_failed: sha256 mismatch")
    handle = C.CDLL(path, mode=C.RTLD_LOCAL | os.RTLD_NOW)
    try:
        get_identity = handle.pih_kernel_pack_identity_v1_get
    except AttributeError as e:
        raise PackError("kernel_pack_identity_missing") from e
    try:
        get_api = handle.pih_kernel_pack_api_v1_get
    except AttributeError as e:
        raise PackError("kernel_pack_api_missing") from e
    get_identity.restype = C.POINTER(Identity)
    get_api.restype = C.POINTER(PackApi)
    ident_p = get_identity()
    if not ident_p:
        raise PackError("kernel_pack_identity_invalid")
    ident = ident_p.contents
    if (ident.struct_size != C.sizeof(Identity) or ident.abi_version != 1 or
            not valid_canonical_id(ident.pack_id, 256) or not valid_canonical_id(ident.pack_version, 64) or
            not valid_canonical_id(ident.pack_abi, 256) or not valid_canonical_id(ident.architecture, 64)):
        raise PackError("kernel_pack_identity_invalid")
    api_p = get_api()
    if not api_p:
        raise PackError("kernel_pack_api_invalid")
    api = api_p.contents
    if (api.struct_size != C.sizeof(PackApi) or api.abi_version != 1 or
            C.cast(api.identity, C.c_void_p).value != C.cast(ident_p, C.c_void_p).value or
            not api.contract_api or not api.bind_origin):
        raise PackError("kernel_pack_api_invalid")
    bound = api.bind_origin(path.encode())
    if bound.struct_size != C.sizeof(Status) or bound.abi_version != 1 or bound.code != OK:
        raise PackError("kernel_pack_origin_binding_failed")
    table_type = {"pih.deepseek-gfx950-kernel-pack.v1": DS_API, "pih.amd-linear-kernels.v1": LN_API,
                  "pih.qwen-kernels.v1": QWEN_API}.get(contract)
    if table_type is None or ident.pack_abi.decode() != contract:
        raise PackError(f"contract mismatch: pack exports {ident.pack_abi!r}, caller wants {contract!r}")
    table = C.cast(api.contract_api, C.POINTER(table_type)).contents
    if table.struct_size != C.sizeof(table_type) or table.contract_version != 1:
        raise PackError("contract_table_invalid")
    pack = KernelPack(path, handle, ident, api, table)
    _loaded[path] = pack
    return pack


def deepseek_pack() -> KernelPack:
    return load_pack(DEEPSEEK_PACK, "pih.deepseek-gfx950-kernel-pack.v1")


def linear_pack() -> KernelPack:
    return load_pack(LINEAR_PACK, "pih.amd-linear-kernels.v1")


def qwen_pack() -> KernelPack:
    return load_pack(QWEN_PACK, "pih.qwen-kernels.v1")


def request(struct_type, **fields):
    """Build a request with its header filled in."""
    r = struct_type()
    r.struct_size = C.sizeof(struct_type)
    r.abi_version = 1
    for k, v in fields.items():
        setattr(r, k, v)
    return r

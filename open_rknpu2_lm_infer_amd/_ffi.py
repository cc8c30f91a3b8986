"""ctypes declarations of the hip_matmul C ABI (include/*.h).

This module plays the role bindgen plays for the reference's Rust layer
(build.rs:132-158): it mirrors every struct and entry point of the headers.
Loading fails loudly when the built library is missing: there is no fallback.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import (POINTER, Structure, c_char_p, c_double, c_float, c_int, c_int8, c_int32,
                    c_uint32, c_uint64, c_void_p)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libhip_matmul.so")

RK_NPU_OK = 0
RK_NPU_ERR_PARAM = -1
RK_NPU_ERR_NOMEM = -2
RK_NPU_ERR_DEVICE = -3
RK_NPU_ERR_CACHE_MISS = -4
RK_NPU_ERR_BUSY = -5
RK_NPU_ERR_UNSUPPORTED = -6
RK_NPU_ERR_FORMAT = -7
RK_NPU_IOMMU_DOMAIN_COUNT = 16
RK_NPU_MATMUL_F32I8F32_DYNAMIC = 1
RK_NPU_MATMUL_A_LAYOUT_NORMAL = 0
RK_NPU_MATMUL_C_LAYOUT_NATIVE = 0
RK_NPU_W4A8_SERIAL = 0
RK_NPU_W4A8_PIPELINED = 1
RK_NPU_W4A8_REDUCE_DEVICE = 0
RK_NPU_W4A8_REDUCE_CPU = 1
RK_NPU_MOE_QUANT_BLOB_VERSION = 1
RK_NPU_HIP_F32 = 0
RK_NPU_HIP_F16 = 1
RK_NPU_HIP_PLAIN = 0
RK_NPU_HIP_SWIGLU = 1
RK_NPU_HIP_PACK_QUANTIZED = 0
RK_NPU_HIP_INT_QUANTIZED = 1
RK_NPU_HIP_STATIC_SCRATCH_BYTES = 16 << 20
RK_NPU_HIP_STATIC_MAX_ROWS = 256
RK_NPU_ATTENTION_F16_CAUSAL = 0
RK_NPU_ATTENTION_F16_NO_MASK = 1
RK_NPU_ATTENTION_F16_STABLE_SOFTMAX = 1


class rk_npu_domain_memory_stats(Structure):
    _fields_ = [("live_bytes", c_uint64), ("peak_bytes", c_uint64), ("creates", c_uint64),
                ("destroys", c_uint64)]


class rk_npu_matmul_weight_config(Structure):
    _fields_ = [("K", c_int32), ("N", c_int32), ("k_tile", c_int32)]


class rk_npu_matmul_weight_requirements(Structure):
    _fields_ = [("bytes", c_uint64)]


class rk_npu_matmul_strategy(Structure):
    _fields_ = [("op_kind", c_uint32), ("M", c_int32), ("N", c_int32), ("K", c_int32),
                ("k_tile", c_int32), ("n_tile", c_int32), ("a_layout", c_uint32),
                ("c_layout", c_uint32), ("wave_count", c_int32), ("n_groups", c_int32),
                ("npu_core_mask", c_uint32), ("cpu_core_mask", c_uint64), ("cpu_threads", c_int32),
                ("total_us", c_double)]


class rk_npu_matmul_autotune_config(Structure):
    _fields_ = [("M", c_int32), ("N", c_int32), ("K", c_int32), ("required_k_tile", c_int32),
                ("allowed_npu_core_mask", c_uint32), ("allowed_cpu_core_mask", c_uint64),
                ("warmup", c_int32), ("loops", c_int32), ("repeats", c_int32), ("verbose", c_int32)]


class rk_npu_matmul_workspace_requirements(Structure):
    _fields_ = [("bytes", c_uint64)]


class rk_npu_i4_weight_config(Structure):
    _fields_ = [("K", c_int32), ("N", c_int32), ("k_tile", c_int32)]


class rk_npu_w4a8_weight_info(Structure):
    _fields_ = [("bound_relaxed", c_int32), ("multiplier", c_float),
                ("config", rk_npu_i4_weight_config)]


class rk_npu_w4a8_config(Structure):
    _fields_ = [("M", c_int32), ("N", c_int32), ("K", c_int32), ("k_tile", c_int32),
                ("m_tile", c_int32), ("n_tile", c_int32), ("npu_core_mask", c_uint32),
                ("cpu_threads", c_int32), ("pipeline", c_int32)]


class rk_npu_w4a8_options(Structure):
    _fields_ = [("reduce_backend", c_uint32)]


class rk_npu_w4a8_memory_info_ex(Structure):
    _fields_ = [("workspace_bytes", c_uint64)]


class rk_npu_w4a8_timings(Structure):
    _fields_ = [("upload_us", c_double), ("device_us", c_double), ("download_us", c_double),
                ("total_us", c_double)]


class rk_npu_w4a8_strategy(Structure):
    _fields_ = [("config", rk_npu_w4a8_config), ("cpu_core_mask", c_uint64), ("total_us", c_double)]


class rk_npu_w4a8_strategy_ex(Structure):
    _fields_ = [("base", rk_npu_w4a8_strategy), ("execution", rk_npu_w4a8_options)]


class rk_npu_w4a8_autotune_config(Structure):
    _fields_ = [("M", c_int32), ("N", c_int32), ("K", c_int32), ("required_k_tile", c_int32),
                ("k_tile_multiplier", c_double), ("allowed_npu_core_mask", c_uint32),
                ("allowed_cpu_core_mask", c_uint64), ("warmup", c_int32), ("loops", c_int32),
                ("repeats", c_int32), ("verbose", c_int32)]


class rk_npu_moe_w8_weight_config(Structure):
    _fields_ = [("hidden", c_int32), ("intermediate", c_int32), ("routed_experts", c_int32),
                ("shared_expert", c_int32)]


class rk_npu_moe_w8_config(Structure):
    _fields_ = [("weights", rk_npu_moe_w8_weight_config), ("top", c_int32), ("max_rows", c_int32),
                ("npu_cores", c_int32), ("cpu_threads", c_int32)]


class rk_npu_moe_w8_expert(Structure):
    _fields_ = [("gate_up", POINTER(c_int8)), ("gate_up_scales", POINTER(c_float)),
                ("down", POINTER(c_int8)), ("down_scales", POINTER(c_float))]


class rk_npu_moe_w8_timings(Structure):
    _fields_ = [(n, c_double) for n in (
        "input_us", "schedule_us", "build_us", "sync_us", "gather_us", "gate_us", "middle_npu_us",
        "middle_cpu_us", "down_us", "combine_us", "lut_load_us", "total_us")] + [
        ("gather_tasks", c_int32), ("middle_tasks", c_int32), ("gemm_tasks", c_int32)]


class rk_npu_moe_import_timings(Structure):
    _fields_ = [("copy_us", c_double), ("validate_us", c_double), ("gate_sync_us", c_double),
                ("down_sync_us", c_double), ("total_us", c_double)]


class rk_npu_hip_kernel_stat(Structure):
    _fields_ = [("kind", c_int32), ("bits", c_int32), ("epilogue", c_int32), ("rows", c_int32),
                ("K", c_int32), ("N", c_int32), ("launches", c_int32), ("total_ms", c_double),
                ("name", ctypes.c_char * 64)]


class rk_npu_hip_plan(Structure):
    _fields_ = [("kind", c_int32), ("block_m", c_int32), ("block_n", c_int32),
                ("k_splits", c_int32), ("grid", c_int32)]


class rk_npu_hip_checkpoint_part(Structure):
    _fields_ = [("data", c_void_p), ("scales", c_void_p), ("n", c_int32), ("format", c_int32)]


class rk_npu_attention_f16_config(Structure):
    _fields_ = [("query_heads", c_int32), ("kv_heads", c_int32), ("head_dim", c_int32), ("softmax_scale", c_float),
                ("max_query_rows", c_int32), ("max_capacity", c_int32), ("initial_capacity", c_int32),
                ("core_mask", c_uint32), ("kv_tile", c_int32), ("flags", c_uint32), ("mask_mode", c_uint32)]


class rk_npu_attention_f16_sizes(Structure):
    _fields_ = [("key_bytes", c_uint64), ("value_bytes", c_uint64), ("tail_bytes", c_uint64),
                ("workspace_bytes", c_uint64), ("active_core_mask", c_uint32)]


class rk_npu_attention_f16_cache_info(Structure):
    _fields_ = [("length", c_int32), ("capacity", c_int32), ("max_capacity", c_int32), ("generation", c_uint64),
                ("key_bytes", c_uint64), ("value_bytes", c_uint64), ("tail_bytes", c_uint64)]


class rk_npu_attention_f16_timings(Structure):
    _fields_ = [("upload_us", c_double), ("device_us", c_double), ("download_us", c_double),
                ("total_us", c_double)]


P = POINTER
i8p = P(c_int8)
f32p = P(c_float)
i32p = P(c_int32)

# name: (restype, argtypes)
SIGNATURES = {
    # non-hot operator families (rk_npu_mm_tune.h, rk_npu_mm_gelu.h,
    # rk_npu_mla_f16.h, rk_npu_gdn.h): report RK_NPU_ERR_UNSUPPORTED
    "rk_npu_mm_autotune_config_init": (None, [c_void_p, c_int32, c_int32, c_int32]),
    "rk_npu_mm_autotune_cache_load": (c_int, [c_void_p, c_void_p, c_char_p, c_void_p, c_void_p]),
    "rk_npu_mm_autotune_cached": (c_int, [c_void_p, c_void_p, c_char_p, c_int32, c_void_p, c_void_p, c_void_p]),
    "rk_npu_mm_autotune": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p]),
    "rk_npu_mm_strategy_default": (c_int, [c_void_p, c_void_p]),
    "rk_npu_mm_tuned_weights_match": (c_int, [c_void_p, c_void_p]),
    "rk_npu_mm_tuned_workspace_create": (c_int, [c_void_p, c_void_p, c_void_p]),
    "rk_npu_mm_tuned_workspace_free": (None, [c_void_p]),
    "rk_npu_mm_tuned_weights_create": (c_int, [c_void_p, c_void_p, c_void_p, c_uint64, c_char_p, c_void_p]),
    "rk_npu_mm_tuned_weights_free": (None, [c_void_p]),
    "rk_npu_mm_tuned_run_weights": (c_int, [c_void_p, c_void_p, c_uint64, c_void_p, c_void_p, c_void_p, c_uint64]),
    "rk_npu_mm_desc_init": (None, [c_void_p, c_int32, c_int32, c_int32, c_int32]),
    "rk_npu_mm_options_init": (None, [c_void_p]),
    "rk_npu_mm_plan_create": (c_int, [c_void_p, c_void_p, c_void_p]),
    "rk_npu_mm_plan_free": (None, [c_void_p]),
    "rk_npu_mm_workspace_create": (c_int, [c_void_p, c_void_p, c_uint32, c_void_p]),
    "rk_npu_mm_workspace_free": (None, [c_void_p]),
    "rk_npu_mm_packed_b_create": (c_int, [c_void_p, c_void_p, c_void_p, c_uint64, c_void_p]),
    "rk_npu_mm_packed_b_free": (None, [c_void_p]),
    "rk_npu_mm_run_packed_b": (c_int, [c_void_p, c_void_p, c_uint64, c_void_p, c_void_p, c_uint64]),
    "rk_npu_mm_gelu_config_init": (None, [c_void_p, c_int32, c_int32, c_int32]),
    "rk_npu_mm_gelu_prepare": (c_int, [c_void_p, c_void_p, c_void_p]),
    "rk_npu_mm_gelu_free": (None, [c_void_p]),
    "rk_npu_mm_gelu_run_weights": (c_int, [c_void_p, c_void_p, c_uint64, c_void_p, c_void_p, c_void_p]),
    "rk_npu_mla_f16_config_init": (None, [c_void_p]),
    "rk_npu_mla_f16_weights_create": (c_int, [c_void_p, c_void_p, c_void_p]),
    "rk_npu_mla_f16_weights_free": (None, [c_void_p]),
    "rk_npu_mla_f16_cache_create": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p]),
    "rk_npu_mla_f16_cache_free": (None, [c_void_p]),
    "rk_npu_mla_f16_prepare": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p]),
    "rk_npu_mla_f16_workspace_free": (None, [c_void_p]),
    "rk_npu_mla_f16_cache_get_info": (c_int, [c_void_p, c_void_p]),
    "rk_npu_mla_f16_cache_reserve": (c_int, [c_void_p, c_void_p, c_int32]),
    "rk_npu_mla_f16_cache_load": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32]),
    "rk_npu_mla_f16_cache_truncate": (c_int, [c_void_p, c_int32]),
    "rk_npu_mla_f16_cache_append": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32]),
    "rk_npu_mla_f16_run": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p,
                                   c_void_p, c_void_p]),
    "rk_npu_gdn_config_init": (None, [c_void_p, c_int32]),
    "rk_npu_gdn_prepare": (c_int, [c_void_p, c_void_p, c_void_p]),
    "rk_npu_gdn_workspace_free": (None, [c_void_p]),
    "rk_npu_gdn_run_projected_strided": (c_int, [c_void_p, c_void_p, c_uint64, c_void_p, c_void_p, c_void_p,
                                                 c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "rk_npu_strerror": (c_char_p, [c_int]),
    "rk_npu_open": (c_void_p, [c_char_p]),
    "rk_npu_close": (None, [c_void_p]),
    "rk_npu_iommu_domain_create": (c_void_p, [c_void_p, c_uint32]),
    "rk_npu_iommu_domain_free": (None, [c_void_p]),
    "rk_npu_iommu_domain_set_reclaim": (None, [c_void_p, c_void_p, c_void_p]),
    "rk_npu_iommu_domain_memory_stats": (c_int, [c_void_p, P(rk_npu_domain_memory_stats)]),
    "rk_npu_f32i8f32_weights_create": (c_void_p, [c_void_p, P(rk_npu_matmul_weight_config), i8p, f32p]),
    "rk_npu_f32i8f32_weights_create_compress": (c_void_p, [c_void_p, P(rk_npu_matmul_weight_config), i8p, f32p]),
    "rk_npu_f32i8f32_weights_free": (None, [c_void_p]),
    "rk_npu_f32i8f32_weights_memory_query": (c_int, [P(rk_npu_matmul_weight_config),
                                                     P(rk_npu_matmul_weight_requirements)]),
    "rk_npu_f32i8f32_weights_compressed_layout_generation": (c_uint64, [c_void_p]),
    "rk_npu_matmul_k_partition_query": (c_int, [c_int, c_int, c_int]),
    "rk_npu_matmul_autotune_config_init": (None, [P(rk_npu_matmul_autotune_config), c_int, c_int, c_int]),
    "rk_npu_matmul_autotune_cache_load": (c_int, [c_void_p, c_char_p, c_uint32, P(rk_npu_matmul_autotune_config),
                                                  P(rk_npu_matmul_strategy), P(rk_npu_matmul_strategy)]),
    "rk_npu_matmul_autotune_cached": (c_int, [c_void_p, P(rk_npu_matmul_autotune_config), c_uint32, c_char_p,
                                              c_int, P(rk_npu_matmul_strategy), P(rk_npu_matmul_strategy),
                                              P(c_int)]),
    "rk_npu_matmul_workspace_memory_query": (c_int, [P(rk_npu_matmul_strategy),
                                                     P(rk_npu_matmul_workspace_requirements)]),
    "rk_npu_matmul_workspace_create": (c_void_p, [c_void_p, P(rk_npu_matmul_strategy)]),
    "rk_npu_matmul_workspace_free": (None, [c_void_p]),
    "rk_npu_f32i8f32_run_dynamic": (c_int, [c_void_p, c_void_p, f32p, f32p]),
    "rk_npu_w4a8_weights_create": (c_void_p, [c_void_p, P(rk_npu_i4_weight_config), i8p, f32p]),
    "rk_npu_w4a8_weights_free": (None, [c_void_p]),
    "rk_npu_w4a8_weights_query": (c_int, [c_void_p, P(rk_npu_w4a8_weight_info)]),
    "rk_npu_i4_weights_memory_query": (c_int, [P(rk_npu_i4_weight_config), P(c_uint64)]),
    "rk_npu_w4a8_config_init": (None, [P(rk_npu_w4a8_config), c_int, c_int, c_int]),
    "rk_npu_w4a8_options_init": (None, [P(rk_npu_w4a8_options)]),
    "rk_npu_w4a8_memory_query_ex": (c_int, [P(rk_npu_w4a8_config), P(rk_npu_w4a8_options),
                                            P(rk_npu_w4a8_memory_info_ex)]),
    "rk_npu_w4a8_workspace_create_ex": (c_void_p, [c_void_p, P(rk_npu_w4a8_config), P(rk_npu_w4a8_options)]),
    "rk_npu_w4a8_workspace_free": (None, [c_void_p]),
    "rk_npu_w4a8_run_f32": (c_int, [c_void_p, c_void_p, f32p, f32p, P(rk_npu_w4a8_timings)]),
    "rk_npu_w4a8_run_swiglu_f32": (c_int, [c_void_p, c_void_p, f32p, f32p, P(rk_npu_w4a8_timings)]),
    "rk_npu_w4a8_run_ffn_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, f32p, f32p,
                                        P(rk_npu_w4a8_timings)]),
    "rk_npu_w4a8_tuning_profile_from_weights": (c_void_p, [c_void_p]),
    "rk_npu_w4a8_tuning_profile_free": (None, [c_void_p]),
    "rk_npu_w4a8_tuning_profile_fingerprint": (c_uint64, [c_void_p]),
    "rk_npu_w4a8_autotune_config_init": (None, [P(rk_npu_w4a8_autotune_config), c_int, c_int, c_int]),
    "rk_npu_w4a8_autotune_cache_load_profile_ex": (c_int, [c_void_p, P(rk_npu_w4a8_autotune_config), c_void_p,
                                                           c_char_p, P(rk_npu_w4a8_strategy_ex),
                                                           P(rk_npu_w4a8_strategy_ex)]),
    "rk_npu_w4a8_autotune_cached_ex": (c_int, [c_void_p, P(rk_npu_w4a8_autotune_config), i8p, f32p, c_char_p,
                                               c_int, P(rk_npu_w4a8_strategy_ex), P(rk_npu_w4a8_strategy_ex),
                                               P(c_int)]),
    "rk_npu_w4a8_autotune_ex": (c_int, [c_void_p, P(rk_npu_w4a8_autotune_config), i8p, f32p,
                                        P(rk_npu_w4a8_strategy_ex), P(rk_npu_w4a8_strategy_ex)]),
    "rk_npu_moe_w8_config_init": (None, [P(rk_npu_moe_w8_config), c_int, c_int, c_int, c_int, c_int, c_int]),
    "rk_npu_moe_quant_weights_create": (c_void_p, [c_void_p, P(rk_npu_moe_w8_weight_config),
                                                   P(rk_npu_moe_w8_expert)]),
    "rk_npu_moe_quant_weights_create_full_k": (c_void_p, [c_void_p, P(rk_npu_moe_w8_weight_config),
                                                          P(rk_npu_moe_w8_expert)]),
    "rk_npu_moe_w4_weights_create": (c_void_p, [c_void_p, P(rk_npu_moe_w8_weight_config),
                                                P(rk_npu_moe_w8_expert)]),
    "rk_npu_moe_w4w8_weights_create": (c_void_p, [c_void_p, P(rk_npu_moe_w8_weight_config),
                                                  P(rk_npu_moe_w8_expert)]),
    "rk_npu_moe_quant_slots_create": (c_void_p, [c_void_p, P(rk_npu_moe_w8_weight_config)]),
    "rk_npu_moe_w4_slots_create": (c_void_p, [c_void_p, P(rk_npu_moe_w8_weight_config),
                                              P(rk_npu_moe_w8_expert)]),
    "rk_npu_moe_w8_weights_free": (None, [c_void_p]),
    "rk_npu_moe_w8_weights_device_bytes": (c_uint64, [c_void_p]),
    "rk_npu_moe_quant_workspace_create": (c_void_p, [c_void_p, P(rk_npu_moe_w8_config)]),
    "rk_npu_moe_w4_workspace_create": (c_void_p, [c_void_p, P(rk_npu_moe_w8_config)]),
    "rk_npu_moe_w4w8_workspace_create": (c_void_p, [c_void_p, P(rk_npu_moe_w8_config)]),
    "rk_npu_moe_w8_workspace_free": (None, [c_void_p]),
    "rk_npu_moe_w8_workspace_device_bytes": (c_uint64, [c_void_p]),
    "rk_npu_moe_w8_run_f32": (c_int, [c_void_p, c_void_p, c_int, f32p, i32p, f32p, f32p,
                                      P(rk_npu_moe_w8_timings)]),
    "rk_npu_moe_quant_expert_blob_bytes": (c_uint64, [c_void_p]),
    "rk_npu_moe_quant_export_expert": (c_int, [c_void_p, c_int, c_void_p, c_uint64]),
    "rk_npu_moe_quant_import_expert": (c_int, [c_void_p, c_int, c_void_p, c_uint64]),
    "rk_npu_moe_quant_import_expert_timed": (c_int, [c_void_p, c_int, c_void_p, c_uint64,
                                                     P(rk_npu_moe_import_timings)]),
    "rk_npu_moe_quant_swap_slots": (c_int, [c_void_p, c_int, c_void_p, c_int]),
    "rk_npu_hip_linear_run": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p, c_int, c_int, c_int,
                                      c_void_p]),
    "rk_npu_hip_linear_run_static": (c_int, [c_void_p, c_int, c_void_p, c_int, c_void_p, c_int, c_int, c_int,
                                             c_void_p]),
    "rk_npu_hip_ffn_run": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p, c_int,
                                   c_void_p, c_int, c_int, c_void_p]),
    "rk_npu_hip_moe_run": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "rk_npu_hip_moe_status": (c_int, [c_void_p]),
    "rk_npu_hip_f32i8f32_weights_create_device": (c_void_p, [c_void_p, P(rk_npu_matmul_weight_config), c_void_p,
                                                             c_void_p]),
    "rk_npu_hip_w4a8_weights_create_device": (c_void_p, [c_void_p, P(rk_npu_i4_weight_config), c_void_p,
                                                         c_void_p]),
    "rk_npu_hip_weights_create_checkpoint": (c_void_p, [c_void_p, c_int, c_int, P(rk_npu_hip_checkpoint_part),
                                                        c_int]),
    "rk_npu_hip_workspace_codes": (c_int, [c_void_p, c_int, c_int, i8p, f32p, i32p]),
    "rk_npu_hip_inject_alloc_failures": (c_int, [c_int]),
    "rk_npu_hip_ffn_status": (c_int, [c_void_p, c_int]),
    "rk_npu_hip_set_switch": (c_int, [c_char_p, c_int, POINTER(c_int)]),
    "rk_npu_hip_linear_plan": (c_int, [c_int, c_int, c_int, c_int, P(rk_npu_hip_plan)]),
    "rk_npu_hip_profile_begin": (c_int, [c_int]),
    "rk_npu_hip_profile_end": (c_int, []),
    "rk_npu_hip_profile_read": (c_int, [P(rk_npu_hip_kernel_stat), c_int, P(c_int)]),
    "rk_npu_attention_f16_config_init": (None, [P(rk_npu_attention_f16_config)]),
    "rk_npu_attention_f16_query": (c_int, [P(rk_npu_attention_f16_config), c_int32, c_int32, c_int32,
                                           P(rk_npu_attention_f16_sizes)]),
    "rk_npu_attention_f16_prepare": (c_int, [c_void_p, P(rk_npu_attention_f16_config), P(c_void_p)]),
    "rk_npu_attention_f16_workspace_free": (None, [c_void_p]),
    "rk_npu_attention_f16_cache_create": (c_int, [c_void_p, P(rk_npu_attention_f16_config), P(c_void_p)]),
    "rk_npu_attention_f16_cache_free": (None, [c_void_p]),
    "rk_npu_attention_f16_cache_reserve": (c_int, [c_void_p, c_void_p, c_int32]),
    "rk_npu_attention_f16_cache_load": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32]),
    "rk_npu_attention_f16_cache_append": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32]),
    "rk_npu_attention_f16_cache_truncate": (c_int, [c_void_p, c_int32]),
    "rk_npu_attention_f16_cache_get_info": (c_int, [c_void_p, P(rk_npu_attention_f16_cache_info)]),
    "rk_npu_attention_f16_run": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p,
                                         P(rk_npu_attention_f16_timings), c_void_p]),
    "rk_npu_attention_f16_run_half": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p,
                                              P(rk_npu_attention_f16_timings), c_void_p]),
    "rk_npu_hip_attention_cache_append": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_void_p]),
    "rk_npu_hip_attention_run": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_int32,
                                         c_void_p]),
}

# Measurement-only library (libhip_probes.so, csrc/probes.hip): the roofline
# probes bench.py --probes runs. Not part of the product library or its ABI.
PROBE_LIB_PATH = os.path.join(PKG_DIR, "libhip_probes.so")
PROBE_SIGNATURES = {
    "rk_npu_hip_stream_probe": (c_int, [c_void_p, c_uint64, c_int, c_int, c_int, c_void_p, c_void_p]),
    "rk_npu_hip_mfma_probe": (c_int, [c_int, c_int, c_void_p, c_void_p]),
    "rk_npu_hip_mfma_rand_probe": (c_int, [c_int, c_int, c_void_p, c_void_p]),
    "rk_npu_hip_lds_probe": (c_int, [c_int, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "rk_npu_hip_wave_place_probe": (c_int, [c_int, c_int, c_void_p, c_void_p]),
    "rk_npu_hip_load_probe": (c_int, [c_int, c_int, c_int, c_int, c_void_p, c_uint64, c_int, c_void_p, c_void_p,
                                      c_void_p]),
}

RECLAIM_CALLBACK = ctypes.CFUNCTYPE(None, c_void_p)

_lib = None


class LibraryMissing(RuntimeError):
    pass


def lib():
    """Load libhip_matmul.so; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(
                f"{LIB_PATH} is missing: build it with `python -m open_rknpu2_lm_infer_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


_probe_lib = None


def probe_lib():
    """Load libhip_probes.so (measurement only); raise if it has not been built."""
    global _probe_lib
    if _probe_lib is None:
        if not os.path.exists(PROBE_LIB_PATH):
            raise LibraryMissing(
                f"{PROBE_LIB_PATH} is missing: build it with `python -m open_rknpu2_lm_infer_amd.build`")
        L = ctypes.CDLL(PROBE_LIB_PATH)
        for name, (res, args) in PROBE_SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _probe_lib = L
    return _probe_lib


def strerror(rc: int) -> str:
    return lib().rk_npu_strerror(rc).decode()


def exported_symbols() -> list:
    return sorted(SIGNATURES)

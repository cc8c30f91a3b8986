/*
 * rk_npu_mm_tune.h — the floating-point (FP16/BF16/TF32) matrix-multiply ABI
 * the reference's Rust layer binds for its non-quantized projections
 * (src/npu/floating.rs: FloatBackend/FloatLinear for vision and decoder
 * auxiliary matrices; src/npu/tf32.rs: Tf32Linear for routers). These are
 * not on the quantized-linear path this library implements: every entry
 * point that would create a plan, workspace or weights returns
 * RK_NPU_ERR_UNSUPPORTED (creating nothing), every run returns
 * RK_NPU_ERR_UNSUPPORTED, the *_init calls fill defaults and the *_free calls
 * accept what the creators return (NULL). They exist so that the reference's
 * crate, whose src/npu.rs compiles these modules unconditionally
 * (src/npu.rs:28-49), builds and links unchanged; a model that needs them
 * fails at load with "unsupported operation".
 *
 * Names, argument order and field names follow the call sites cited below;
 * integer constants are enumerators, so bindgen gives them the type of the
 * fields and parameters they are assigned to or passed as.
 */
#ifndef RK_NPU_MM_TUNE_H
#define RK_NPU_MM_TUNE_H

#include <stdint.h>

#include "rk_npu_quant_matmul.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (src/npu/floating.rs:138-157, 312; src/npu/tf32.rs:40-42). */
typedef enum rk_npu_mm_dtype {
    RK_NPU_MM_F16 = 0,
    RK_NPU_MM_BF16 = 1,
    RK_NPU_MM_F32 = 2,
    RK_NPU_MM_TF32 = 3
} rk_npu_mm_dtype;

/* Host-side representation of A/C (src/npu/floating.rs:151, 387, 396;
 * src/npu/tf32.rs:72). */
typedef enum rk_npu_mm_host_type {
    RK_NPU_MM_HOST_F32 = 0,
    RK_NPU_MM_HOST_STORAGE = 1,
    RK_NPU_MM_HOST_PACKED_B = 2
} rk_npu_mm_host_type;

/* Operand layouts (src/npu/tf32.rs:46-47). */
typedef enum rk_npu_mm_layout { RK_NPU_MM_LAYOUT_NATIVE = 0 } rk_npu_mm_layout;

/* Execution options (src/npu/tf32.rs:44-51; src/npu/floating.rs:237, 260,
 * 296-298). */
typedef struct rk_npu_mm_options {
    int32_t n_tile;
    int32_t split_k;
    rk_npu_mm_layout a_layout;
    rk_npu_mm_layout c_layout;
    uint32_t allowed_npu_core_mask;
} rk_npu_mm_options;

/* Tuning request (src/npu/floating.rs:54-74, 224). */
typedef struct rk_npu_mm_autotune_config {
    int32_t M;
    int32_t N;
    int32_t K;
    rk_npu_mm_dtype dtype;
    rk_npu_mm_host_type host_type;
    int32_t with_bias;
    uint32_t allowed_npu_core_mask;
    uint64_t allowed_cpu_core_mask;
    int32_t warmup;
    int32_t loops;
    int32_t repeats;
    int32_t verbose;
} rk_npu_mm_autotune_config;

/* A tuned (or default) strategy with its measured costs
 * (src/npu/floating.rs:286-303). */
typedef struct rk_npu_mm_strategy {
    int32_t M;
    int32_t N;
    int32_t K;
    rk_npu_mm_dtype dtype;
    rk_npu_mm_host_type host_type;
    int32_t m_tile;
    int32_t task_m_tile;
    int32_t fused_io;
    int32_t k_tile;
    rk_npu_mm_options options;
    uint64_t cpu_core_mask;
    int32_t cpu_threads;
    int32_t tuning_revision;
    double total_us;
    double robust_us;
    double jitter_pct;
    double workspace_us;
    double weight_us;
    double max_abs_error;
} rk_npu_mm_strategy;

/* Problem description of a planned multiply (src/npu/tf32.rs:34-43). */
typedef struct rk_npu_mm_desc {
    int32_t M;
    int32_t N;
    int32_t K;
    int32_t batch;
    rk_npu_mm_dtype a_type;
    rk_npu_mm_dtype b_type;
    rk_npu_mm_dtype c_type;
    int32_t trans_a;
    int32_t trans_b;
} rk_npu_mm_desc;

typedef struct rk_npu_mm_tuned_weights rk_npu_mm_tuned_weights;
typedef struct rk_npu_mm_tuned_workspace rk_npu_mm_tuned_workspace;
typedef struct rk_npu_mm_plan rk_npu_mm_plan;
typedef struct rk_npu_mm_workspace rk_npu_mm_workspace;
typedef struct rk_npu_mm_packed_b rk_npu_mm_packed_b;

/* ---- tuned FP16/BF16 linear (src/npu/floating.rs) ------------------------ */
/* Defaults for an M x K x N problem (floating.rs:63). */
void rk_npu_mm_autotune_config_init(rk_npu_mm_autotune_config* config, int32_t M, int32_t N, int32_t K);
/* Tuning-cache lookup (floating.rs:183-192): RK_NPU_ERR_CACHE_MISS. */
int rk_npu_mm_autotune_cache_load(rk_npu_ctx* ctx, const rk_npu_mm_autotune_config* config, const char* path,
                                  rk_npu_mm_strategy* fastest, rk_npu_mm_strategy* stable);
/* Searches (floating.rs:209-221): RK_NPU_ERR_UNSUPPORTED. */
int rk_npu_mm_autotune_cached(rk_npu_iommu_domain* domain, const rk_npu_mm_autotune_config* config,
                              const char* path, int32_t force, rk_npu_mm_strategy* fastest,
                              rk_npu_mm_strategy* stable, int32_t* hit);
int rk_npu_mm_autotune(rk_npu_iommu_domain* domain, const rk_npu_mm_autotune_config* config,
                       rk_npu_mm_strategy* fastest, rk_npu_mm_strategy* stable);
/* Library baseline strategy (floating.rs:251): RK_NPU_ERR_UNSUPPORTED. */
int rk_npu_mm_strategy_default(const rk_npu_mm_autotune_config* config, rk_npu_mm_strategy* strategy);
/* Whether resident weights suit a strategy (floating.rs:168, 237): nonzero. */
int rk_npu_mm_tuned_weights_match(const rk_npu_mm_tuned_weights* weights, const rk_npu_mm_strategy* strategy);
/* (floating.rs:265, 334-343): RK_NPU_ERR_UNSUPPORTED, *out = NULL. */
int rk_npu_mm_tuned_workspace_create(rk_npu_iommu_domain* domain, const rk_npu_mm_strategy* strategy,
                                     rk_npu_mm_tuned_workspace** out);
void rk_npu_mm_tuned_workspace_free(rk_npu_mm_tuned_workspace* workspace);
int rk_npu_mm_tuned_weights_create(rk_npu_iommu_domain* domain, const rk_npu_mm_autotune_config* config,
                                   const uint16_t* weights, uint64_t weight_bytes, const char* cache_path,
                                   rk_npu_mm_tuned_weights** out);
void rk_npu_mm_tuned_weights_free(rk_npu_mm_tuned_weights* weights);
/* (floating.rs:483-493): RK_NPU_ERR_UNSUPPORTED. */
int rk_npu_mm_tuned_run_weights(rk_npu_mm_tuned_workspace* workspace, const void* input, uint64_t input_bytes,
                                const rk_npu_mm_tuned_weights* weights, const float* bias, void* output,
                                uint64_t output_bytes);

/* ---- planned TF32 multiply with packed B (src/npu/tf32.rs) --------------- */
void rk_npu_mm_desc_init(rk_npu_mm_desc* desc, int32_t M, int32_t N, int32_t K, int32_t batch);
void rk_npu_mm_options_init(rk_npu_mm_options* options);
/* (tf32.rs:52-57, 66-78, 121-131): RK_NPU_ERR_UNSUPPORTED, *out = NULL. */
int rk_npu_mm_plan_create(const rk_npu_mm_desc* desc, const rk_npu_mm_options* options, rk_npu_mm_plan** out);
void rk_npu_mm_plan_free(rk_npu_mm_plan* plan);
int rk_npu_mm_workspace_create(rk_npu_iommu_domain* domain, const rk_npu_mm_plan* plan, rk_npu_mm_host_type host,
                               rk_npu_mm_workspace** out);
void rk_npu_mm_workspace_free(rk_npu_mm_workspace* workspace);
int rk_npu_mm_packed_b_create(rk_npu_iommu_domain* domain, const rk_npu_mm_plan* plan, const void* b,
                              uint64_t b_bytes, rk_npu_mm_packed_b** out);
void rk_npu_mm_packed_b_free(rk_npu_mm_packed_b* packed);
/* (tf32.rs:152-162): RK_NPU_ERR_UNSUPPORTED. */
int rk_npu_mm_run_packed_b(rk_npu_mm_workspace* workspace, const void* a, uint64_t a_bytes,
                           const rk_npu_mm_packed_b* b, void* c, uint64_t c_bytes);

#ifdef __cplusplus
}
#endif
#endif

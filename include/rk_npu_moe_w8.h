/*
 * rk_npu_moe_w8.h — grouped routed-expert FFN of the MI355X hip_matmul
 * library. Names and fields follow the reference's Rust call sites
 * (src/npu/moe.rs:35-47, 121-126, 131-149, 160-162, 179-213, 245-256,
 * 270-319, 342-350, 373-384); see rk_npu_quant_matmul.h for conventions.
 *
 * Numerics of rk_npu_moe_w8_run_f32 (per token row r):
 *   1. the input row is quantized once: scale = max|x|/127 (1 for a zero
 *      row, no FLT_MIN floor), codes rounded to nearest-even, clamped to +-127;
 *   2. for every rank with route > 0: gate/up int32 GEMM, dequant
 *      (f32(acc) * row_scale) * scale[n], FP32 SwiGLU, requantization of the
 *      (token, expert) middle row with the rule of step 1, down int32 GEMM,
 *      dequant, and sum = fma(contribution, route, sum) in rank order;
 *   3. the shared expert (if any) is computed the same way and added after
 *      the routed sum.
 */
#ifndef RK_NPU_MOE_W8_H
#define RK_NPU_MOE_W8_H

#include "rk_npu_quant_matmul.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct rk_npu_moe_w8_weight_config {
    int32_t hidden;
    int32_t intermediate;
    int32_t routed_experts;
    int32_t shared_expert; /* 0 or 1 */
} rk_npu_moe_w8_weight_config;

typedef struct rk_npu_moe_w8_config {
    rk_npu_moe_w8_weight_config weights;
    int32_t top;      /* routes per token, 1..8 */
    int32_t max_rows; /* largest `rows` a run may pass */
    int32_t npu_cores;
    int32_t cpu_threads;
} rk_npu_moe_w8_config;

void rk_npu_moe_w8_config_init(rk_npu_moe_w8_config* config, int hidden, int intermediate,
                               int routed_experts, int shared_expert, int top, int max_rows);

/* One expert: gate_up codes [hidden][2*intermediate] (gate columns first),
 * down codes [intermediate][hidden], both [K][N] row-major int8, with f32
 * per-output-channel scales. Copied on creation. */
typedef struct rk_npu_moe_w8_expert {
    const int8_t* gate_up;
    const float* gate_up_scales;
    const int8_t* down;
    const float* down_scales;
} rk_npu_moe_w8_expert;

typedef struct rk_npu_moe_w8_weights rk_npu_moe_w8_weights;
typedef struct rk_npu_moe_w8_workspace rk_npu_moe_w8_workspace;

/* Routed experts with W4 gate_up and W4 down (src/npu/moe.rs:108-111, 131-137). */
rk_npu_moe_w8_weights* rk_npu_moe_quant_weights_create(rk_npu_iommu_domain* domain,
                                                       const rk_npu_moe_w8_weight_config* config,
                                                       const rk_npu_moe_w8_expert* experts);
/* Same numerics; kept for the caller's full-K bank (src/npu/moe.rs:133-135). */
rk_npu_moe_w8_weights* rk_npu_moe_quant_weights_create_full_k(
    rk_npu_iommu_domain* domain, const rk_npu_moe_w8_weight_config* config,
    const rk_npu_moe_w8_expert* experts);
/* Routed W4 experts plus a shared W8 expert at experts[routed_experts]
 * (src/npu/moe.rs:131-133, 222-240). */
rk_npu_moe_w8_weights* rk_npu_moe_w4_weights_create(rk_npu_iommu_domain* domain,
                                                    const rk_npu_moe_w8_weight_config* config,
                                                    const rk_npu_moe_w8_expert* experts);
/* Routed W4 gate_up with W8 down (+ optional shared W8 expert), the mixed
 * bank of MINICPMV47_35A3_FUSED_MOE_20261019.md:76. */
rk_npu_moe_w8_weights* rk_npu_moe_w4w8_weights_create(rk_npu_iommu_domain* domain,
                                                      const rk_npu_moe_w8_weight_config* config,
                                                      const rk_npu_moe_w8_expert* experts);
/* Empty W4 banks whose experts arrive through import (src/npu/moe.rs:141-149). */
rk_npu_moe_w8_weights* rk_npu_moe_quant_slots_create(rk_npu_iommu_domain* domain,
                                                     const rk_npu_moe_w8_weight_config* config);
rk_npu_moe_w8_weights* rk_npu_moe_w4_slots_create(rk_npu_iommu_domain* domain,
                                                  const rk_npu_moe_w8_weight_config* config,
                                                  const rk_npu_moe_w8_expert* shared);
void rk_npu_moe_w8_weights_free(rk_npu_moe_w8_weights* weights);
uint64_t rk_npu_moe_w8_weights_device_bytes(const rk_npu_moe_w8_weights* weights);

rk_npu_moe_w8_workspace* rk_npu_moe_quant_workspace_create(rk_npu_iommu_domain* domain,
                                                           const rk_npu_moe_w8_config* config);
rk_npu_moe_w8_workspace* rk_npu_moe_w4_workspace_create(rk_npu_iommu_domain* domain,
                                                        const rk_npu_moe_w8_config* config);
rk_npu_moe_w8_workspace* rk_npu_moe_w4w8_workspace_create(rk_npu_iommu_domain* domain,
                                                          const rk_npu_moe_w8_config* config);
void rk_npu_moe_w8_workspace_free(rk_npu_moe_w8_workspace* workspace);
uint64_t rk_npu_moe_w8_workspace_device_bytes(const rk_npu_moe_w8_workspace* workspace);

typedef struct rk_npu_moe_w8_timings {
    double input_us;
    double schedule_us;
    double build_us;
    double sync_us;
    double gather_us;
    double gate_us;
    double middle_npu_us;
    double middle_cpu_us;
    double down_us;
    double combine_us;
    double lut_load_us;
    double total_us;
    int32_t gather_tasks;
    int32_t middle_tasks;
    int32_t gemm_tasks;
} rk_npu_moe_w8_timings;

/* input f32 [rows][hidden]; ids i32 [rows][top] in [0, routed_experts);
 * routes f32 [rows][top]; output f32 [rows][hidden]; 1 <= rows <= max_rows.
 * Replaces the call at src/npu/moe.rs:373-384. timings may be NULL. */
int rk_npu_moe_w8_run_f32(rk_npu_moe_w8_workspace* workspace, const rk_npu_moe_w8_weights* weights,
                          int rows, const float* input, const int32_t* ids, const float* routes,
                          float* output, rk_npu_moe_w8_timings* timings);

/* ---- expert records for streaming (src/npu/moe.rs:243-320) --------------- */
#define RK_NPU_MOE_QUANT_BLOB_VERSION 1u

typedef struct rk_npu_moe_import_timings {
    double copy_us;
    double validate_us;
    double gate_sync_us;
    double down_sync_us;
    double total_us;
} rk_npu_moe_import_timings;

/* Bytes of one routed expert record (header + device-layout payload). */
uint64_t rk_npu_moe_quant_expert_blob_bytes(const rk_npu_moe_w8_weights* weights);
int rk_npu_moe_quant_export_expert(const rk_npu_moe_w8_weights* weights, int expert, void* data,
                                   uint64_t bytes);
int rk_npu_moe_quant_import_expert(rk_npu_moe_w8_weights* weights, int slot, const void* data,
                                   uint64_t bytes);
int rk_npu_moe_quant_import_expert_timed(rk_npu_moe_w8_weights* weights, int slot,
                                         const void* data, uint64_t bytes,
                                         rk_npu_moe_import_timings* timings);
/* Exchanges routed expert `slot` of `weights` with expert `staged` of `bank`
 * (same geometry) without copying payloads. */
int rk_npu_moe_quant_swap_slots(rk_npu_moe_w8_weights* weights, int slot,
                                rk_npu_moe_w8_weights* bank, int staged);

#ifdef __cplusplus
}
#endif
#endif

/*
 * rk_npu_gdn.h — the gated-delta-network (linear attention) prefill ABI the
 * reference's Rust layer binds for Qwen3.5-style recurrent layers
 * (src/npu/gated_delta.rs). Not on the quantized-linear path this library
 * implements: rk_npu_gdn_prepare and the run return RK_NPU_ERR_UNSUPPORTED
 * and create or change nothing, the init call fills defaults and the free call
 * accepts NULL. Present so the reference's crate, whose src/npu.rs compiles
 * the gated_delta module unconditionally (src/npu.rs:28-49), builds and links
 * unchanged; its callers then keep their CPU path.
 */
#ifndef RK_NPU_GDN_H
#define RK_NPU_GDN_H

#include <stdint.h>

#include "rk_npu_quant_matmul.h"

#ifdef __cplusplus
extern "C" {
#endif

/* (src/npu/gated_delta.rs:122-126) */
typedef enum rk_npu_gdn_precision {
    RK_NPU_GDN_TF32 = 0,
    RK_NPU_GDN_COMPENSATED_TF32 = 1
} rk_npu_gdn_precision;
/* (src/npu/gated_delta.rs:130) */
typedef enum rk_npu_gdn_head_mapping { RK_NPU_GDN_HEAD_GROUPED = 1 } rk_npu_gdn_head_mapping;

/* (src/npu/gated_delta.rs:119-130) */
typedef struct rk_npu_gdn_config {
    int32_t rows;
    int32_t chunk_size;
    rk_npu_gdn_precision precision;
    int32_t cpu_threads;
    uint32_t core_mask;
    rk_npu_gdn_head_mapping head_mapping;
} rk_npu_gdn_config;

/* (src/npu/gated_delta.rs:170, 197-204) */
typedef struct rk_npu_gdn_timings {
    double total_us;
    double hardware_us;
    double prepare_us;
    double coefficients_us;
    double solve_us;
    double collect_us;
} rk_npu_gdn_timings;

typedef struct rk_npu_gdn_workspace rk_npu_gdn_workspace;

void rk_npu_gdn_config_init(rk_npu_gdn_config* config, int32_t rows);
/* (gated_delta.rs:131-139): RK_NPU_ERR_UNSUPPORTED, *out = NULL. */
int rk_npu_gdn_prepare(rk_npu_iommu_domain* domain, const rk_npu_gdn_config* config, rk_npu_gdn_workspace** out);
void rk_npu_gdn_workspace_free(rk_npu_gdn_workspace* workspace);
/* (gated_delta.rs:173-188): RK_NPU_ERR_UNSUPPORTED, outputs, state and
 * history unchanged. */
int rk_npu_gdn_run_projected_strided(rk_npu_gdn_workspace* workspace, const float* projected,
                                     uint64_t projected_stride, const float* conv_weights, const float* history,
                                     const float* log_decay, const float* beta, const float* state, float* output,
                                     float* state_out, float* history_out, rk_npu_gdn_timings* timings);

#ifdef __cplusplus
}
#endif
#endif

/*
 * rk_npu_mm_gelu.h — the fused FP16 GEMM + bias + tanh-GELU ABI the
 * reference's Rust layer binds for vision FFNs (src/npu/floating.rs:400-460,
 * src/npu/floating_gelu.rs). Not on the quantized-linear path this library
 * implements: rk_npu_mm_gelu_prepare and rk_npu_mm_gelu_run_weights return
 * RK_NPU_ERR_UNSUPPORTED (creating nothing), the init call fills defaults and
 * the free call accepts NULL. Present so the reference's crate builds and
 * links unchanged (src/npu.rs:28-49 compiles the floating module
 * unconditionally).
 */
#ifndef RK_NPU_MM_GELU_H
#define RK_NPU_MM_GELU_H

#include <stdint.h>

#include "rk_npu_mm_tune.h"

#ifdef __cplusplus
extern "C" {
#endif

/* (src/npu/floating.rs:429-433) */
typedef struct rk_npu_mm_gelu_config {
    int32_t M;
    int32_t N;
    int32_t K;
    uint32_t core_mask;
    int32_t verbose;
} rk_npu_mm_gelu_config;

/* The mapped FP32 result panel of a fused run, read by the caller
 * (src/npu/floating_gelu.rs:52-76): `rows` x `columns` logical values stored
 * in `storage_rows` x `storage_columns` panels, `elements` floats at `data`,
 * each to be multiplied by `scale`. */
typedef struct rk_npu_mm_gelu_view {
    int32_t rows;
    int32_t columns;
    int32_t storage_rows;
    int32_t storage_columns;
    uint64_t elements;
    const float* data;
    float scale;
} rk_npu_mm_gelu_view;

typedef struct rk_npu_mm_gelu_workspace rk_npu_mm_gelu_workspace;

void rk_npu_mm_gelu_config_init(rk_npu_mm_gelu_config* config, int32_t M, int32_t N, int32_t K);
/* (floating.rs:436-439): RK_NPU_ERR_UNSUPPORTED, *out = NULL. */
int rk_npu_mm_gelu_prepare(rk_npu_iommu_domain* domain, const rk_npu_mm_gelu_config* config,
                           rk_npu_mm_gelu_workspace** out);
void rk_npu_mm_gelu_free(rk_npu_mm_gelu_workspace* workspace);
/* (floating.rs:447-458): RK_NPU_ERR_UNSUPPORTED, the view left untouched. */
int rk_npu_mm_gelu_run_weights(rk_npu_mm_gelu_workspace* workspace, const uint16_t* input, uint64_t input_bytes,
                               const rk_npu_mm_tuned_weights* weights, const float* bias,
                               rk_npu_mm_gelu_view* view);

#ifdef __cplusplus
}
#endif
#endif

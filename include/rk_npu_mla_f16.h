/*
 * rk_npu_mla_f16.h — the absorbed multi-head latent attention (MLA) ABI the
 * reference's Rust layer binds for Ling-style models (src/npu/mla.rs). Not on
 * the quantized-linear path this library implements: the weight, cache and
 * workspace creators return RK_NPU_ERR_UNSUPPORTED and create nothing, the
 * cache and run calls return RK_NPU_ERR_UNSUPPORTED, the init call fills
 * defaults and the free calls accept NULL. Present so the reference's crate,
 * whose src/npu.rs compiles the mla module unconditionally (src/npu.rs:28-49),
 * builds and links unchanged; an MLA model fails at load.
 */
#ifndef RK_NPU_MLA_F16_H
#define RK_NPU_MLA_F16_H

#include <stdint.h>

#include "rk_npu_quant_matmul.h"

#ifdef __cplusplus
extern "C" {
#endif

/* (src/npu/mla.rs:27) */
typedef enum rk_npu_mla_f16_mode { RK_NPU_MLA_F16_ABSORBED = 1 } rk_npu_mla_f16_mode;
/* flags bits (src/npu/mla.rs:33) */
#define RK_NPU_MLA_F16_STABLE_SOFTMAX 1u

/* (src/npu/mla.rs:25-33) */
typedef struct rk_npu_mla_f16_config {
    rk_npu_mla_f16_mode mode;
    int32_t max_query_rows;
    int32_t kv_tile;
    int32_t initial_capacity;
    int32_t max_capacity;
    uint32_t core_mask;
    uint32_t flags;
} rk_npu_mla_f16_config;

/* (src/npu/mla.rs:68-79) */
typedef struct rk_npu_mla_f16_cache_info {
    int32_t length;
    int32_t capacity;
    int32_t max_capacity;
    uint64_t key_bytes;
    uint64_t value_bytes;
    uint64_t tail_bytes;
} rk_npu_mla_f16_cache_info;

typedef struct rk_npu_mla_f16_timings {
    double total_us;
} rk_npu_mla_f16_timings;

typedef struct rk_npu_mla_f16_weights rk_npu_mla_f16_weights;
typedef struct rk_npu_mla_f16_cache rk_npu_mla_f16_cache;
typedef struct rk_npu_mla_f16_workspace rk_npu_mla_f16_workspace;

void rk_npu_mla_f16_config_init(rk_npu_mla_f16_config* config);
/* (mla.rs:39-56): RK_NPU_ERR_UNSUPPORTED, *out = NULL. */
int rk_npu_mla_f16_weights_create(rk_npu_iommu_domain* domain, const uint16_t* kv_b, rk_npu_mla_f16_weights** out);
void rk_npu_mla_f16_weights_free(rk_npu_mla_f16_weights* weights);
int rk_npu_mla_f16_cache_create(rk_npu_iommu_domain* domain, const rk_npu_mla_f16_config* config,
                                const rk_npu_mla_f16_weights* weights, rk_npu_mla_f16_cache** out);
void rk_npu_mla_f16_cache_free(rk_npu_mla_f16_cache* cache);
int rk_npu_mla_f16_prepare(rk_npu_iommu_domain* domain, const rk_npu_mla_f16_config* config,
                           const rk_npu_mla_f16_weights* weights, rk_npu_mla_f16_workspace** out);
void rk_npu_mla_f16_workspace_free(rk_npu_mla_f16_workspace* workspace);
/* (mla.rs:68-160): RK_NPU_ERR_UNSUPPORTED. */
int rk_npu_mla_f16_cache_get_info(const rk_npu_mla_f16_cache* cache, rk_npu_mla_f16_cache_info* info);
int rk_npu_mla_f16_cache_reserve(rk_npu_ctx* ctx, rk_npu_mla_f16_cache* cache, int32_t capacity);
int rk_npu_mla_f16_cache_load(rk_npu_ctx* ctx, rk_npu_mla_f16_cache* cache, const uint16_t* latent,
                              const uint16_t* rotary, int32_t rows);
int rk_npu_mla_f16_cache_truncate(rk_npu_mla_f16_cache* cache, int32_t length);
int rk_npu_mla_f16_cache_append(rk_npu_ctx* ctx, rk_npu_mla_f16_cache* cache, const uint16_t* latent,
                                const uint16_t* rotary, int32_t rows);
/* (mla.rs:163-177): RK_NPU_ERR_UNSUPPORTED. */
int rk_npu_mla_f16_run(rk_npu_ctx* ctx, rk_npu_mla_f16_workspace* workspace, rk_npu_mla_f16_cache* cache,
                       const uint16_t* query, const float* gates, int32_t rows, int32_t position, float* output,
                       rk_npu_mla_f16_timings* timings, const void* reserved);

#ifdef __cplusplus
}
#endif
#endif

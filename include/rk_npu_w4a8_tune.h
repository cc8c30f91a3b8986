/*
 * rk_npu_w4a8_tune.h — W4A8 strategy / tuning entry points bound by the
 * reference (src/npu.rs:927, 1093-1193). The GPU library keeps no tuning
 * cache: cache loads report RK_NPU_ERR_CACHE_MISS and "tuning" returns the
 * library's own launch plan without measuring or writing files.
 */
#ifndef RK_NPU_W4A8_TUNE_H
#define RK_NPU_W4A8_TUNE_H

#include "rk_npu_w4a8.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct rk_npu_w4a8_tuning_profile rk_npu_w4a8_tuning_profile;

/* A profile identifies a weight set for cache keys (src/npu.rs:574-578,
 * 921-928). The fingerprint is a 64-bit hash of shape, codes and scales. */
rk_npu_w4a8_tuning_profile* rk_npu_w4a8_tuning_profile_from_weights(
    const rk_npu_w4a8_weights* weights);
void rk_npu_w4a8_tuning_profile_free(rk_npu_w4a8_tuning_profile* profile);
uint64_t rk_npu_w4a8_tuning_profile_fingerprint(const rk_npu_w4a8_tuning_profile* profile);

typedef struct rk_npu_w4a8_strategy {
    rk_npu_w4a8_config config;
    uint64_t cpu_core_mask;
    double total_us;
} rk_npu_w4a8_strategy;

typedef struct rk_npu_w4a8_strategy_ex {
    rk_npu_w4a8_strategy base;
    rk_npu_w4a8_options execution;
} rk_npu_w4a8_strategy_ex;

typedef struct rk_npu_w4a8_autotune_config {
    int32_t M;
    int32_t N;
    int32_t K;
    int32_t required_k_tile;
    double k_tile_multiplier;
    uint32_t allowed_npu_core_mask;
    uint64_t allowed_cpu_core_mask;
    int32_t warmup;
    int32_t loops;
    int32_t repeats;
    int32_t verbose;
} rk_npu_w4a8_autotune_config;

void rk_npu_w4a8_autotune_config_init(rk_npu_w4a8_autotune_config* config, int M, int N, int K);

/* Always RK_NPU_ERR_CACHE_MISS (src/npu.rs:1110-1131). */
int rk_npu_w4a8_autotune_cache_load_profile_ex(rk_npu_ctx* ctx,
                                               const rk_npu_w4a8_autotune_config* config,
                                               const rk_npu_w4a8_tuning_profile* profile,
                                               const char* path,
                                               rk_npu_w4a8_strategy_ex* fastest,
                                               rk_npu_w4a8_strategy_ex* stable);
/* Fills both strategies with the library's plan; *hit = 0; no file written. */
int rk_npu_w4a8_autotune_cached_ex(rk_npu_ctx* ctx, const rk_npu_w4a8_autotune_config* config,
                                   const int8_t* codes, const float* scales, const char* path,
                                   int force, rk_npu_w4a8_strategy_ex* fastest,
                                   rk_npu_w4a8_strategy_ex* stable, int* hit);
/* Same without a cache path (src/npu/ubatch_probe.rs:147). */
int rk_npu_w4a8_autotune_ex(rk_npu_ctx* ctx, const rk_npu_w4a8_autotune_config* config,
                            const int8_t* codes, const float* scales,
                            rk_npu_w4a8_strategy_ex* fastest, rk_npu_w4a8_strategy_ex* stable);

#ifdef __cplusplus
}
#endif
#endif

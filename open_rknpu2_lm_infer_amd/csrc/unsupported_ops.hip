// Entry points of the reference's non-quantized operator families (FP16/BF16
// and TF32 matrix multiplies, fused GELU, MLA attention, gated-delta prefill)
// that its Rust crate binds and links unconditionally (src/npu.rs:28-49,
// build.rs:138-145). They are outside this library's hot path: the creators
// report RK_NPU_ERR_UNSUPPORTED and create nothing, the runs report
// RK_NPU_ERR_UNSUPPORTED and write nothing, the *_init calls give defaults,
// and the *_free calls accept the NULL handles the creators leave.
#include <cstring>

#include "../../include/rk_npu_gdn.h"
#include "../../include/rk_npu_mla_f16.h"
#include "../../include/rk_npu_mm_gelu.h"
#include "../../include/rk_npu_mm_tune.h"

template <typename T>
static int unsupported_create(T** out) {
    if (out) *out = nullptr;
    return RK_NPU_ERR_UNSUPPORTED;
}

extern "C" {

// ---- rk_npu_mm_tune.h ----------------------------------------------------------

void rk_npu_mm_autotune_config_init(rk_npu_mm_autotune_config* config, int32_t M, int32_t N, int32_t K) {
    if (!config) return;
    std::memset(config, 0, sizeof(*config));
    config->M = M;
    config->N = N;
    config->K = K;
    config->dtype = RK_NPU_MM_F16;
    config->host_type = RK_NPU_MM_HOST_F32;
    config->allowed_npu_core_mask = 1;
    config->warmup = 1;
    config->loops = 3;
    config->repeats = 3;
}

int rk_npu_mm_autotune_cache_load(rk_npu_ctx*, const rk_npu_mm_autotune_config* config, const char*,
                                  rk_npu_mm_strategy*, rk_npu_mm_strategy*) {
    return config ? RK_NPU_ERR_CACHE_MISS : RK_NPU_ERR_PARAM;
}

int rk_npu_mm_autotune_cached(rk_npu_iommu_domain*, const rk_npu_mm_autotune_config*, const char*, int32_t,
                              rk_npu_mm_strategy*, rk_npu_mm_strategy*, int32_t* hit) {
    if (hit) *hit = 0;
    return RK_NPU_ERR_UNSUPPORTED;
}

int rk_npu_mm_autotune(rk_npu_iommu_domain*, const rk_npu_mm_autotune_config*, rk_npu_mm_strategy*,
                       rk_npu_mm_strategy*) {
    return RK_NPU_ERR_UNSUPPORTED;
}

int rk_npu_mm_strategy_default(const rk_npu_mm_autotune_config*, rk_npu_mm_strategy*) {
    return RK_NPU_ERR_UNSUPPORTED;
}

int rk_npu_mm_tuned_weights_match(const rk_npu_mm_tuned_weights*, const rk_npu_mm_strategy*) {
    return RK_NPU_ERR_UNSUPPORTED;
}

int rk_npu_mm_tuned_workspace_create(rk_npu_iommu_domain*, const rk_npu_mm_strategy*,
                                     rk_npu_mm_tuned_workspace** out) {
    return unsupported_create(out);
}

void rk_npu_mm_tuned_workspace_free(rk_npu_mm_tuned_workspace*) {}

int rk_npu_mm_tuned_weights_create(rk_npu_iommu_domain*, const rk_npu_mm_autotune_config*, const uint16_t*,
                                   uint64_t, const char*, rk_npu_mm_tuned_weights** out) {
    return unsupported_create(out);
}

void rk_npu_mm_tuned_weights_free(rk_npu_mm_tuned_weights*) {}

int rk_npu_mm_tuned_run_weights(rk_npu_mm_tuned_workspace*, const void*, uint64_t, const rk_npu_mm_tuned_weights*,
                                const float*, void*, uint64_t) {
    return RK_NPU_ERR_UNSUPPORTED;
}

void rk_npu_mm_desc_init(rk_npu_mm_desc* desc, int32_t M, int32_t N, int32_t K, int32_t batch) {
    if (!desc) return;
    std::memset(desc, 0, sizeof(*desc));
    desc->M = M;
    desc->N = N;
    desc->K = K;
    desc->batch = batch;
    desc->a_type = desc->b_type = RK_NPU_MM_F16;
    desc->c_type = RK_NPU_MM_F32;
}

void rk_npu_mm_options_init(rk_npu_mm_options* options) {
    if (!options) return;
    std::memset(options, 0, sizeof(*options));
    options->a_layout = options->c_layout = RK_NPU_MM_LAYOUT_NATIVE;
    options->allowed_npu_core_mask = 1;
}

int rk_npu_mm_plan_create(const rk_npu_mm_desc*, const rk_npu_mm_options*, rk_npu_mm_plan** out) {
    return unsupported_create(out);
}

void rk_npu_mm_plan_free(rk_npu_mm_plan*) {}

int rk_npu_mm_workspace_create(rk_npu_iommu_domain*, const rk_npu_mm_plan*, rk_npu_mm_host_type,
                               rk_npu_mm_workspace** out) {
    return unsupported_create(out);
}

void rk_npu_mm_workspace_free(rk_npu_mm_workspace*) {}

int rk_npu_mm_packed_b_create(rk_npu_iommu_domain*, const rk_npu_mm_plan*, const void*, uint64_t,
                              rk_npu_mm_packed_b** out) {
    return unsupported_create(out);
}

void rk_npu_mm_packed_b_free(rk_npu_mm_packed_b*) {}

int rk_npu_mm_run_packed_b(rk_npu_mm_workspace*, const void*, uint64_t, const rk_npu_mm_packed_b*, void*,
                           uint64_t) {
    return RK_NPU_ERR_UNSUPPORTED;
}

// ---- rk_npu_mm_gelu.h ----------------------------------------------------------

void rk_npu_mm_gelu_config_init(rk_npu_mm_gelu_config* config, int32_t M, int32_t N, int32_t K) {
    if (!config) return;
    std::memset(config, 0, sizeof(*config));
    config->M = M;
    config->N = N;
    config->K = K;
    config->core_mask = 1;
}

int rk_npu_mm_gelu_prepare(rk_npu_iommu_domain*, const rk_npu_mm_gelu_config*, rk_npu_mm_gelu_workspace** out) {
    return unsupported_create(out);
}

void rk_npu_mm_gelu_free(rk_npu_mm_gelu_workspace*) {}

int rk_npu_mm_gelu_run_weights(rk_npu_mm_gelu_workspace*, const uint16_t*, uint64_t, const rk_npu_mm_tuned_weights*,
                               const float*, rk_npu_mm_gelu_view*) {
    return RK_NPU_ERR_UNSUPPORTED;
}

// ---- rk_npu_mla_f16.h ----------------------------------------------------------

void rk_npu_mla_f16_config_init(rk_npu_mla_f16_config* config) {
    if (!config) return;
    std::memset(config, 0, sizeof(*config));
    config->mode = RK_NPU_MLA_F16_ABSORBED;
    config->max_query_rows = 32;
    config->initial_capacity = 32;
    config->max_capacity = 4096;
    config->core_mask = 1;
    config->flags = RK_NPU_MLA_F16_STABLE_SOFTMAX;
}

int rk_npu_mla_f16_weights_create(rk_npu_iommu_domain*, const uint16_t*, rk_npu_mla_f16_weights** out) {
    return unsupported_create(out);
}

void rk_npu_mla_f16_weights_free(rk_npu_mla_f16_weights*) {}

int rk_npu_mla_f16_cache_create(rk_npu_iommu_domain*, const rk_npu_mla_f16_config*, const rk_npu_mla_f16_weights*,
                                rk_npu_mla_f16_cache** out) {
    return unsupported_create(out);
}

void rk_npu_mla_f16_cache_free(rk_npu_mla_f16_cache*) {}

int rk_npu_mla_f16_prepare(rk_npu_iommu_domain*, const rk_npu_mla_f16_config*, const rk_npu_mla_f16_weights*,
                           rk_npu_mla_f16_workspace** out) {
    return unsupported_create(out);
}

void rk_npu_mla_f16_workspace_free(rk_npu_mla_f16_workspace*) {}

int rk_npu_mla_f16_cache_get_info(const rk_npu_mla_f16_cache*, rk_npu_mla_f16_cache_info*) {
    return RK_NPU_ERR_UNSUPPORTED;
}

int rk_npu_mla_f16_cache_reserve(rk_npu_ctx*, rk_npu_mla_f16_cache*, int32_t) { return RK_NPU_ERR_UNSUPPORTED; }

int rk_npu_mla_f16_cache_load(rk_npu_ctx*, rk_npu_mla_f16_cache*, const uint16_t*, const uint16_t*, int32_t) {
    return RK_NPU_ERR_UNSUPPORTED;
}

int rk_npu_mla_f16_cache_truncate(rk_npu_mla_f16_cache*, int32_t) { return RK_NPU_ERR_UNSUPPORTED; }

int rk_npu_mla_f16_cache_append(rk_npu_ctx*, rk_npu_mla_f16_cache*, const uint16_t*, const uint16_t*, int32_t) {
    return RK_NPU_ERR_UNSUPPORTED;
}

int rk_npu_mla_f16_run(rk_npu_ctx*, rk_npu_mla_f16_workspace*, rk_npu_mla_f16_cache*, const uint16_t*, const float*,
                       int32_t, int32_t, float*, rk_npu_mla_f16_timings*, const void*) {
    return RK_NPU_ERR_UNSUPPORTED;
}

// ---- rk_npu_gdn.h --------------------------------------------------------------

void rk_npu_gdn_config_init(rk_npu_gdn_config* config, int32_t rows) {
    if (!config) return;
    std::memset(config, 0, sizeof(*config));
    config->rows = rows;
    config->chunk_size = 64;
    config->precision = RK_NPU_GDN_TF32;
    config->cpu_threads = 1;
    config->core_mask = 1;
    config->head_mapping = RK_NPU_GDN_HEAD_GROUPED;
}

int rk_npu_gdn_prepare(rk_npu_iommu_domain*, const rk_npu_gdn_config*, rk_npu_gdn_workspace** out) {
    return unsupported_create(out);
}

void rk_npu_gdn_workspace_free(rk_npu_gdn_workspace*) {}

int rk_npu_gdn_run_projected_strided(rk_npu_gdn_workspace*, const float*, uint64_t, const float*, const float*,
                                     const float*, const float*, const float*, float*, float*, float*,
                                     rk_npu_gdn_timings*) {
    return RK_NPU_ERR_UNSUPPORTED;
}

}  // extern "C"

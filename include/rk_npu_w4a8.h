/*
 * rk_npu_w4a8.h — W4A8 (int4 weight codes in [-8, 7], dynamic per-token int8
 * activation) entry points of the MI355X hip_matmul library. Names and field
 * names follow the reference's Rust call sites (src/npu.rs:539-579,
 * 1093-1193, 1243-1266, 1296-1304, 1402-1410); see rk_npu_quant_matmul.h for
 * the shared conventions.
 */
#ifndef RK_NPU_W4A8_H
#define RK_NPU_W4A8_H

#include "rk_npu_quant_matmul.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct rk_npu_i4_weight_config {
    int32_t K;
    int32_t N;
    int32_t k_tile; /* 0 = let the library choose (it reports K) */
} rk_npu_i4_weight_config;

typedef struct rk_npu_w4a8_weights rk_npu_w4a8_weights;

/* codes: int8 [K][N] row-major holding values in [-8, 7]; scales f32 [N] > 0.
 * Copied on creation. Out-of-range codes make the call return NULL.
 * Replaces the call at src/npu.rs:545-556. */
rk_npu_w4a8_weights* rk_npu_w4a8_weights_create(rk_npu_iommu_domain* domain,
                                                const rk_npu_i4_weight_config* config,
                                                const int8_t* codes, const float* scales);
void rk_npu_w4a8_weights_free(rk_npu_w4a8_weights* weights);

typedef struct rk_npu_w4a8_weight_info {
    int32_t bound_relaxed; /* always 0: int32 accumulation is exact for any K */
    float multiplier;      /* always 1 */
    rk_npu_i4_weight_config config;
} rk_npu_w4a8_weight_info;

/* src/npu.rs:558-566 */
int rk_npu_w4a8_weights_query(const rk_npu_w4a8_weights* weights, rk_npu_w4a8_weight_info* info);
/* Device bytes of W4 weights of this shape (src/npu.rs:569-573). */
int rk_npu_i4_weights_memory_query(const rk_npu_i4_weight_config* config, uint64_t* bytes);

typedef enum rk_npu_w4a8_pipeline_mode {
    RK_NPU_W4A8_SERIAL = 0,
    RK_NPU_W4A8_PIPELINED = 1
} rk_npu_w4a8_pipeline_mode;

typedef enum rk_npu_w4a8_reduce_backend {
    RK_NPU_W4A8_REDUCE_DEVICE = 0,
    RK_NPU_W4A8_REDUCE_CPU = 1
} rk_npu_w4a8_reduce_backend;

typedef struct rk_npu_w4a8_config {
    int32_t M; /* rows per call */
    int32_t N;
    int32_t K;
    int32_t k_tile;
    int32_t m_tile;
    int32_t n_tile;
    uint32_t npu_core_mask;
    int32_t cpu_threads;
    int32_t pipeline;
} rk_npu_w4a8_config;

typedef struct rk_npu_w4a8_options {
    rk_npu_w4a8_reduce_backend reduce_backend; /* accepted; the GPU always reduces in int32 */
} rk_npu_w4a8_options;

void rk_npu_w4a8_config_init(rk_npu_w4a8_config* config, int M, int N, int K);
void rk_npu_w4a8_options_init(rk_npu_w4a8_options* options);

typedef struct rk_npu_w4a8_memory_info_ex {
    uint64_t workspace_bytes;
} rk_npu_w4a8_memory_info_ex;

int rk_npu_w4a8_memory_query_ex(const rk_npu_w4a8_config* config,
                                const rk_npu_w4a8_options* options,
                                rk_npu_w4a8_memory_info_ex* info);

typedef struct rk_npu_w4a8_workspace rk_npu_w4a8_workspace;

rk_npu_w4a8_workspace* rk_npu_w4a8_workspace_create_ex(rk_npu_iommu_domain* domain,
                                                       const rk_npu_w4a8_config* config,
                                                       const rk_npu_w4a8_options* options);
void rk_npu_w4a8_workspace_free(rk_npu_w4a8_workspace* workspace);

/* Optional per-call timing (microseconds, wall clock of the whole call and of
 * the device part). */
typedef struct rk_npu_w4a8_timings {
    double upload_us;
    double device_us;
    double download_us;
    double total_us;
} rk_npu_w4a8_timings;

/* C[M][N] = dequant(Q(A[M][K]) x W) with the rule of rk_npu_f32i8f32_run_dynamic.
 * Replaces the call at src/npu.rs:1402-1410. timings may be NULL. */
int rk_npu_w4a8_run_f32(rk_npu_w4a8_workspace* workspace, const rk_npu_w4a8_weights* weights,
                        const float* A, float* C, rk_npu_w4a8_timings* timings);

/* C[M][N/2]: out[m][j] = silu(Y[m][j]) * Y[m][N/2 + j] for the full product Y;
 * silu(g) = g / (1 + exp(-g)) in FP32 with the exponent argument saturated
 * to [-80, 80] and a signed zero for g < -80. Requires N % 64 == 0, else
 * RK_NPU_ERR_PARAM. Replaces the call at src/npu.rs:1402-1408. */
int rk_npu_w4a8_run_swiglu_f32(rk_npu_w4a8_workspace* workspace,
                               const rk_npu_w4a8_weights* weights, const float* A, float* C,
                               rk_npu_w4a8_timings* timings);

/* Fused FFN: gate_up (K = H, N = 2F, N % 64 == 0) -> SwiGLU -> per-row
 * requantization of the middle with the dense rule over all F columns ->
 * down (K = F, N = H). `down` may be W4 (rk_npu_w4a8_weights) or W8
 * (rk_npu_f32i8f32_weights) as given by down_bits. down_workspace must be a
 * workspace of the matching kind and the same M. Output C[M][H]. The
 * reference library's rk_npu_w4a8_run_ffn_f32 (library-only there,
 * QWEN3_W4A8_SWIGLU_MAXABS_FUSION_20261022.md:84-106). */
int rk_npu_w4a8_run_ffn_f32(rk_npu_w4a8_workspace* gate_up_workspace,
                            const rk_npu_w4a8_weights* gate_up, void* down_workspace,
                            const void* down, int down_bits, const float* A, float* C,
                            rk_npu_w4a8_timings* timings);

#ifdef __cplusplus
}
#endif
#endif

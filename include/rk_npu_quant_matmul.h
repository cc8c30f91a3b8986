/*
 * rk_npu_quant_matmul.h — context, domain, error and W8A8 (int8 weight,
 * dynamic per-token int8 activation) entry points of the MI355X hip_matmul
 * library. Names, argument meaning and field names follow what the
 * reference's Rust layer binds through bindgen (build.rs:138-145, allowlist
 * rk_npu_.* / RK_NPU_.*); layouts behind the opaque handles are this
 * library's own.
 *
 * Conventions (src/npu.rs:177-200):
 *  - *_create returns an owning pointer or NULL; the matching *_free releases.
 *  - every other call returns 0 on success or a negative RK_NPU_ERR_* code,
 *    described by rk_npu_strerror().
 *  - A and C buffers of the *_run* calls are caller-owned HOST f32 arrays,
 *    fully consumed / produced when the call returns.
 *  - weights are immutable after creation and may be shared by concurrent
 *    calls on distinct workspaces; calls on one workspace are serialized by
 *    the caller, and an overlapping call returns RK_NPU_ERR_BUSY.
 */
#ifndef RK_NPU_QUANT_MATMUL_H
#define RK_NPU_QUANT_MATMUL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- errors (src/npu.rs:187-200, 909-914) -------------------------------- */
#define RK_NPU_OK 0
#define RK_NPU_ERR_PARAM (-1)
#define RK_NPU_ERR_NOMEM (-2)
#define RK_NPU_ERR_DEVICE (-3)
#define RK_NPU_ERR_CACHE_MISS (-4)
#define RK_NPU_ERR_BUSY (-5)
#define RK_NPU_ERR_UNSUPPORTED (-6)
#define RK_NPU_ERR_FORMAT (-7)

/* Replaces the reference library's error table (bound at src/npu.rs:189). */
const char* rk_npu_strerror(int rc);

/* ---- context and allocation domains (src/npu.rs:483-501) ----------------- */
typedef struct rk_npu_ctx rk_npu_ctx;
typedef struct rk_npu_iommu_domain rk_npu_iommu_domain;

/* Number of allocation domains a context offers (src/npu.rs:479). */
#define RK_NPU_IOMMU_DOMAIN_COUNT 16u

/* Opens the GPU named by `device` (a decimal HIP ordinal; NULL or "" = the
 * current device). Replaces rk_npu_open at src/npu.rs:487. */
rk_npu_ctx* rk_npu_open(const char* device);
void rk_npu_close(rk_npu_ctx* ctx);

/* A domain is an accounting scope for device allocations (the reference's
 * IOMMU domain, src/npu.rs:492-501). */
rk_npu_iommu_domain* rk_npu_iommu_domain_create(rk_npu_ctx* ctx, uint32_t id);
void rk_npu_iommu_domain_free(rk_npu_iommu_domain* domain);

/* Called (without library locks held) when a device allocation in the
 * domain fails, before one retry (src/npu.rs:234-260). */
void rk_npu_iommu_domain_set_reclaim(rk_npu_iommu_domain* domain, void (*reclaim)(void* cookie),
                                     void* cookie);

typedef struct rk_npu_domain_memory_stats {
    uint64_t live_bytes;
    uint64_t peak_bytes;
    uint64_t creates;
    uint64_t destroys;
} rk_npu_domain_memory_stats;

/* src/npu.rs:909-914 */
int rk_npu_iommu_domain_memory_stats(const rk_npu_iommu_domain* domain,
                                     rk_npu_domain_memory_stats* stats);

/* ---- W8A8 weights (src/npu.rs:580-616) ----------------------------------- */
typedef struct rk_npu_matmul_weight_config {
    int32_t K;
    int32_t N;
    int32_t k_tile; /* accepted for compatibility; the GPU reduces all of K in int32 */
} rk_npu_matmul_weight_config;

typedef struct rk_npu_matmul_weight_requirements {
    uint64_t bytes;
} rk_npu_matmul_weight_requirements;

typedef struct rk_npu_f32i8f32_weights rk_npu_f32i8f32_weights;

/* codes: int8 [K][N] row-major (codes[k*N + n]); scales: f32 [N] > 0.
 * Both are copied; the caller may free them on return (src/npu.rs:619-621). */
rk_npu_f32i8f32_weights* rk_npu_f32i8f32_weights_create(rk_npu_iommu_domain* domain,
                                                        const rk_npu_matmul_weight_config* config,
                                                        const int8_t* codes, const float* scales);
/* Lossless variant (src/npu.rs:597-601). Device storage is the raw layout. */
rk_npu_f32i8f32_weights* rk_npu_f32i8f32_weights_create_compress(
    rk_npu_iommu_domain* domain, const rk_npu_matmul_weight_config* config, const int8_t* codes,
    const float* scales);
void rk_npu_f32i8f32_weights_free(rk_npu_f32i8f32_weights* weights);
int rk_npu_f32i8f32_weights_memory_query(const rk_npu_matmul_weight_config* config,
                                         rk_npu_matmul_weight_requirements* requirements);
/* Always 0: the GPU layout is never re-encoded after creation (src/npu.rs:636-641). */
uint64_t rk_npu_f32i8f32_weights_compressed_layout_generation(
    const rk_npu_f32i8f32_weights* weights);

/* K-partition legality used by the caller's W8 planning (src/npu.rs:944-986,
 * test table src/npu.rs:1568-1595). Returns 0 when legal, RK_NPU_ERR_PARAM
 * otherwise. */
int rk_npu_matmul_k_partition_query(int rows, int K, int k_tile);

/* ---- W8A8 strategy, tuning and workspaces (src/npu.rs:987-1079, 1268-1279) */
typedef enum rk_npu_matmul_op_kind {
    RK_NPU_MATMUL_F32I8F32_DYNAMIC = 1
} rk_npu_matmul_op_kind;
typedef enum rk_npu_matmul_a_layout { RK_NPU_MATMUL_A_LAYOUT_NORMAL = 0 } rk_npu_matmul_a_layout;
typedef enum rk_npu_matmul_c_layout { RK_NPU_MATMUL_C_LAYOUT_NATIVE = 0 } rk_npu_matmul_c_layout;

typedef struct rk_npu_matmul_strategy {
    rk_npu_matmul_op_kind op_kind;
    int32_t M; /* rows per call (the caller's bucket) */
    int32_t N;
    int32_t K;
    int32_t k_tile;
    int32_t n_tile;
    rk_npu_matmul_a_layout a_layout;
    rk_npu_matmul_c_layout c_layout;
    int32_t wave_count;
    int32_t n_groups;
    uint32_t npu_core_mask;
    uint64_t cpu_core_mask;
    int32_t cpu_threads;
    double total_us;
} rk_npu_matmul_strategy;

typedef struct rk_npu_matmul_autotune_config {
    int32_t M;
    int32_t N;
    int32_t K;
    int32_t required_k_tile;
    uint32_t allowed_npu_core_mask;
    uint64_t allowed_cpu_core_mask;
    int32_t warmup;
    int32_t loops;
    int32_t repeats;
    int32_t verbose;
} rk_npu_matmul_autotune_config;

void rk_npu_matmul_autotune_config_init(rk_npu_matmul_autotune_config* config, int M, int N, int K);
/* There is no persistent tuning cache on the GPU: always RK_NPU_ERR_CACHE_MISS
 * (the caller then uses its fallback strategy, src/npu.rs:1060-1077). */
int rk_npu_matmul_autotune_cache_load(rk_npu_ctx* ctx, const char* path, rk_npu_matmul_op_kind op,
                                      const rk_npu_matmul_autotune_config* config,
                                      rk_npu_matmul_strategy* fastest,
                                      rk_npu_matmul_strategy* stable);
/* Fills both strategies with the library's launch plan for the shape; writes
 * no file; *hit = 0. */
int rk_npu_matmul_autotune_cached(rk_npu_ctx* ctx, const rk_npu_matmul_autotune_config* config,
                                  rk_npu_matmul_op_kind op, const char* path, int force,
                                  rk_npu_matmul_strategy* fastest, rk_npu_matmul_strategy* stable,
                                  int* hit);

typedef struct rk_npu_matmul_workspace_requirements {
    uint64_t bytes;
} rk_npu_matmul_workspace_requirements;

typedef struct rk_npu_matmul_workspace rk_npu_matmul_workspace;

int rk_npu_matmul_workspace_memory_query(const rk_npu_matmul_strategy* strategy,
                                         rk_npu_matmul_workspace_requirements* requirements);
/* A workspace serves calls of exactly strategy->M rows for weights of
 * strategy->K x strategy->N. */
rk_npu_matmul_workspace* rk_npu_matmul_workspace_create(rk_npu_iommu_domain* domain,
                                                        const rk_npu_matmul_strategy* strategy);
void rk_npu_matmul_workspace_free(rk_npu_matmul_workspace* workspace);

/* Y[M][N] = dequant(Q(A[M][K]) x W): per-row dynamic int8 quantization of A
 * (scale = max|a|/127 floored at FLT_MIN, 1 for a zero row; codes rounded
 * half away from zero, clamped to +-127), exact int32 accumulation and
 * y = (f32(acc) * row_scale) * scales[n]. Replaces the call at
 * src/npu.rs:1412-1417. */
int rk_npu_f32i8f32_run_dynamic(rk_npu_matmul_workspace* workspace,
                                const rk_npu_f32i8f32_weights* weights, const float* A, float* C);

#ifdef __cplusplus
}
#endif
#endif

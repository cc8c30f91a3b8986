/*
 * rk_npu_attention_f16.h — FP16 grouped-query attention with a device KV
 * cache: the entry points the reference's Rust layer binds for its native
 * attention (src/npu.rs:295-345 workspace, 420-440 config, 662-760 cache
 * creation; src/npu/attention.rs cache load / append / truncate / reserve /
 * info and the causal and no-mask runs). Names, argument meaning and field
 * names follow those call sites; the layouts behind the opaque handles are
 * this library's own.
 *
 * Semantics. A cache holds, per KV head, `length` rows of K and V (head_dim
 * fp16 values each). rk_npu_attention_f16_run takes `rows` query rows per
 * query head, the first at absolute position `position`, and computes for
 * query head h (KV head h / (query_heads / kv_heads)) and row r:
 *     s_j = softmax_scale * (q_r . k_j)            (fp16 inputs, f32 math)
 *     out_r = sum_j p_j v_j / sum_j p_j,  p_j = exp(s_j - max_j s_j)
 * over keys j < length, and with the causal mask (mask_mode
 * RK_NPU_ATTENTION_F16_CAUSAL) only j <= position + r. Host arrays are
 * head-major: q and out [query_heads][rows][head_dim], K/V appended as
 * [kv_heads][rows][head_dim] (src/npu/attention.rs:240-262, 325-351).
 */
#ifndef RK_NPU_ATTENTION_F16_H
#define RK_NPU_ATTENTION_F16_H

#include <stdint.h>

#include "rk_npu_quant_matmul.h"

#ifdef __cplusplus
extern "C" {
#endif

/* mask_mode values (src/npu.rs:680, 734, 744) */
#define RK_NPU_ATTENTION_F16_CAUSAL 0
#define RK_NPU_ATTENTION_F16_NO_MASK 1
/* flags bits (src/npu.rs:437): the softmax subtracts the row max; it always
 * does here, the flag is accepted for compatibility. */
#define RK_NPU_ATTENTION_F16_STABLE_SOFTMAX 1u

typedef struct rk_npu_attention_f16_config {
    int32_t query_heads;      /* multiple of kv_heads */
    int32_t kv_heads;         /* 1..32 */
    int32_t head_dim;         /* multiple of 32, at most 256 */
    float softmax_scale;      /* finite, > 0 (usually 1/sqrt(head_dim)) */
    int32_t max_query_rows;   /* rows per run call, 1..256 */
    int32_t max_capacity;     /* KV rows a cache may grow to (multiple of 32) */
    int32_t initial_capacity; /* KV rows allocated at creation (multiple of 32) */
    uint32_t core_mask;       /* accepted and ignored (one GPU) */
    int32_t kv_tile;          /* accepted and ignored: the kernel tiles by itself */
    uint32_t flags;           /* RK_NPU_ATTENTION_F16_STABLE_SOFTMAX */
    uint32_t mask_mode;       /* RK_NPU_ATTENTION_F16_CAUSAL or _NO_MASK */
} rk_npu_attention_f16_config;

typedef struct rk_npu_attention_f16_sizes {
    uint64_t key_bytes;       /* K storage for the queried capacity */
    uint64_t value_bytes;     /* V storage for the queried capacity */
    uint64_t tail_bytes;      /* bookkeeping beyond K/V (0 here) */
    uint64_t workspace_bytes; /* device workspace for the queried query rows */
    uint32_t active_core_mask;
} rk_npu_attention_f16_sizes;

typedef struct rk_npu_attention_f16_cache_info {
    int32_t length;       /* rows held */
    int32_t capacity;     /* rows allocated */
    int32_t max_capacity; /* rows the cache may grow to: config max_capacity rounded up to 32
                             (src/npu/vision_tests.rs:201) */
    uint64_t generation;  /* changes whenever the K/V storage is reallocated or reloaded, not on
                             append or truncate (src/npu.rs:1789) */
    uint64_t key_bytes;
    uint64_t value_bytes;
    uint64_t tail_bytes;
} rk_npu_attention_f16_cache_info;

/* Host-clock intervals of one run call (optional). */
typedef struct rk_npu_attention_f16_timings {
    double upload_us;
    double device_us;
    double download_us;
    double total_us;
} rk_npu_attention_f16_timings;

typedef struct rk_npu_attention_f16_cache rk_npu_attention_f16_cache;
typedef struct rk_npu_attention_f16_workspace rk_npu_attention_f16_workspace;

/* Defaults: scale 1/sqrt(128), causal, STABLE_SOFTMAX, 128 query rows,
 * capacity 4096 (src/npu.rs:425). */
void rk_npu_attention_f16_config_init(rk_npu_attention_f16_config* config);

/* Storage for a cache of `capacity` rows and a workspace for `query_rows`
 * (src/npu.rs:310-319, 454-465; the fourth argument is the KV capacity the
 * workspace serves and only validated). */
int rk_npu_attention_f16_query(const rk_npu_attention_f16_config* config, int32_t capacity, int32_t query_rows,
                               int32_t kv_capacity, rk_npu_attention_f16_sizes* sizes);

/* Workspace for run calls of this geometry (src/npu.rs:321-326). */
int rk_npu_attention_f16_prepare(rk_npu_iommu_domain* domain, const rk_npu_attention_f16_config* config,
                                 rk_npu_attention_f16_workspace** workspace);
void rk_npu_attention_f16_workspace_free(rk_npu_attention_f16_workspace* workspace);

/* An empty cache of initial_capacity rows (src/npu.rs:686, 749). */
int rk_npu_attention_f16_cache_create(rk_npu_iommu_domain* domain, const rk_npu_attention_f16_config* config,
                                      rk_npu_attention_f16_cache** cache);
void rk_npu_attention_f16_cache_free(rk_npu_attention_f16_cache* cache);

/* Grow to at least `capacity` rows (at most max_capacity), keeping the rows
 * held (src/npu/attention.rs:226-244). */
int rk_npu_attention_f16_cache_reserve(rk_npu_ctx* ctx, rk_npu_attention_f16_cache* cache, int32_t capacity);
/* Replace the contents by `rows` rows ([kv_heads][rows][head_dim] fp16 host
 * arrays); rows == 0 (k, v may be NULL) empties the cache
 * (src/npu/attention.rs:80-90, 203-217). */
int rk_npu_attention_f16_cache_load(rk_npu_ctx* ctx, rk_npu_attention_f16_cache* cache, const uint16_t* k,
                                    const uint16_t* v, int32_t rows);
/* Append `rows` rows after the ones held (src/npu/attention.rs:286-297). */
int rk_npu_attention_f16_cache_append(rk_npu_ctx* ctx, rk_npu_attention_f16_cache* cache, const uint16_t* k,
                                      const uint16_t* v, int32_t rows);
/* Keep the first `length` rows (src/npu/attention.rs:192-201). */
int rk_npu_attention_f16_cache_truncate(rk_npu_attention_f16_cache* cache, int32_t length);
int rk_npu_attention_f16_cache_get_info(const rk_npu_attention_f16_cache* cache,
                                        rk_npu_attention_f16_cache_info* info);

/* Attention of `rows` query rows ([query_heads][rows][head_dim] fp16 host
 * array), the first at `position`, over the cache; f32 output
 * [query_heads][rows][head_dim] (src/npu/attention.rs:339-352). `timings`
 * may be NULL; `reserved` must be NULL. */
int rk_npu_attention_f16_run(rk_npu_ctx* ctx, rk_npu_attention_f16_workspace* workspace,
                             rk_npu_attention_f16_cache* cache, const uint16_t* q, int32_t rows, int32_t position,
                             float* output, rk_npu_attention_f16_timings* timings, const void* reserved);
/* Same with fp16 output, the f32 result rounded to nearest
 * (src/npu/attention.rs:100-113). */
int rk_npu_attention_f16_run_half(rk_npu_ctx* ctx, rk_npu_attention_f16_workspace* workspace,
                                  rk_npu_attention_f16_cache* cache, const uint16_t* q, int32_t rows,
                                  int32_t position, uint16_t* output, rk_npu_attention_f16_timings* timings,
                                  const void* reserved);

/* ---- device-resident entry points (no reference counterpart) ------------
 * For callers whose K/V/Q/output already live in HBM (same layouts as the
 * host calls), on the caller's HIP stream (NULL: the null stream); nothing
 * is synchronized. out_f16 selects fp16 output. */
int rk_npu_hip_attention_cache_append(rk_npu_attention_f16_cache* cache, const void* k_dev, const void* v_dev,
                                      int32_t rows, void* stream);
int rk_npu_hip_attention_run(rk_npu_attention_f16_workspace* workspace, rk_npu_attention_f16_cache* cache,
                             const void* q_dev, int32_t rows, int32_t position, void* out_dev, int32_t out_f16,
                             void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RK_NPU_ATTENTION_F16_H */

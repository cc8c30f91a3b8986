/*
 * CPU oracle for the quantized-linear hot path — TEST INFRASTRUCTURE ONLY.
 *
 * This library restates, in plain C, the CPU semantics the reference pins for
 * its dynamic-int8-activation linear, fused SwiGLU, fused FFN and routed MoE.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only as the checker (or the timed CPU baseline). The product
 * library never links or calls it.
 *
 * Each function cites the reference lines it restates; tests/ pins every one
 * of them with known answers, closed forms or brute force.
 */
#ifndef RK_ORACLE_H
#define RK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/npu.rs:201-211 */
int orc_bucket(int rows);

/* src/npu.rs:1537-1547 (dense rule: FLT_MIN floor, ties away from zero). */
void orc_quant_dense_row(const float* x, int k, int8_t* codes, float* scale);
/* MOE_CPU_FUSION_20261023.md:13 (MoE rule: no floor, ties to even). */
void orc_quant_moe_row(const float* x, int k, int8_t* codes, float* scale);

/* src/npu.rs:1548-1552: acc[m][n] = sum_k a[m][k] * w[k][n], w is [K][N]. */
void orc_gemm_i8(const int8_t* a, const int8_t* w, int m, int k, int n, int32_t* acc);

/* src/npu.rs:1553: y = (f32(acc) * row_scale) * col_scale. */
float orc_dequant(int32_t acc, float row_scale, float col_scale);

/* The whole Linear oracle of src/npu.rs:1533-1557 (dense quant rule).
 * codes [K][N], scales [N], input [rows][K], output [rows][N]. Optional
 * q_out [rows][K], s_out [rows] and acc_out [rows][N] expose intermediates. */
void orc_linear(const int8_t* codes, const float* scales, int k, int n,
                const float* input, int rows, float* output,
                int8_t* q_out, float* s_out, int32_t* acc_out);

/* Project-owned FP32 exp, Cody–Waite reduction + degree-7 Taylor. Defined
 * for |x| <= 80 (callers clamp). */
float orc_expf(float x);
/* SwiGLU with the reference's fused-path range handling
 * (QWEN3_W4A8_SWIGLU_MAXABS_FUSION_20261022.md:102; formula
 * native/cpu_kernels/swiglu.cpp:23-26). */
float orc_swiglu(float gate, float up);

/* src/npu.rs:1651-1657: out[r][j] = swiglu(Y[r][j], Y[r][N/2+j]), j < N/2. */
void orc_linear_swiglu(const int8_t* codes, const float* scales, int k, int n,
                       const float* input, int rows, float* output);

/* Fused FFN (QWEN3_W4A8_SWIGLU_MAXABS_FUSION_20261022.md:48-50,84,106):
 * gate_up [H][2F] -> SwiGLU -> dense requant of the middle row -> down [F][H].
 * mid_out [rows][F] optional. */
void orc_ffn(const int8_t* gu_codes, const float* gu_scales,
             const int8_t* dn_codes, const float* dn_scales, int h, int f,
             const float* input, int rows, float* output, float* mid_out);

/* Routed MoE (src/npu/moe.rs:353-387 contract, numerics per
 * MOE_CPU_FUSION_20261023.md:13, MOE_ROUTED_SHARED_JOINT_20261023.md:19,
 * combine per src/model/experts/paged.rs:494-507).
 * gu_codes[e] [h][2I], dn_codes[e] [I][h]; shared_* may be NULL. */
void orc_moe(const int8_t* const* gu_codes, const float* const* gu_scales,
             const int8_t* const* dn_codes, const float* const* dn_scales,
             int experts, int h, int inter,
             const int8_t* sh_gu_codes, const float* sh_gu_scales,
             const int8_t* sh_dn_codes, const float* sh_dn_scales, int sh_inter,
             const float* input, int rows, const int32_t* ids, const float* routes,
             int top, float* output);

/* src/model/qwen35/moe.rs:51-67: top-k by descending logit (total order,
 * ties to the lower id), softmax over the selected k. Returns 0 or -1. */
int orc_routes(const float* logits, int count, int top, int32_t* ids, float* weights);

/* src/model/checkpoint.rs:558-571: I32 words [N][ceil(K*bits/32)] -> codes [K][N]. */
void orc_unpack_codes(const uint32_t* words, int bits, int n, int k, int8_t* codes);

/* src/model/checkpoint.rs:573-604: concatenate [K][N_i] matrices along N. */
void orc_concatenate(const int8_t* const* codes, const int* ns, int count, int k, int8_t* out);

/* SplitMix64 stream used to synthesise seeded inputs. */
uint64_t orc_splitmix64(uint64_t* state);

/* Thread count the OpenMP loops use. */
int orc_threads(void);

#ifdef __cplusplus
}
#endif
#endif

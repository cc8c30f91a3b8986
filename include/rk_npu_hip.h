/*
 * rk_npu_hip.h — device-resident entry points of the MI355X hip_matmul
 * library. These have NO counterpart in the reference: its C ABI only takes
 * host f32 buffers. They serve callers whose activations already live in HBM
 * (HIP graph capture, serving loops, benchmarks) and share every kernel with
 * the host-buffer entry points, so their results are bit-identical.
 *
 * All A/C/ids/routes pointers are DEVICE pointers on the context's GPU.
 * `stream` is the hipStream_t the work is enqueued on, used as given (NULL is
 * the HIP null stream, so work stays ordered with a caller that uses it); the
 * call only enqueues work and returns without synchronizing. The workspace stays
 * busy until that work completes on the stream: the caller must not issue a
 * second call on the same workspace from another stream before that.
 */
#ifndef RK_NPU_HIP_H
#define RK_NPU_HIP_H

#include "rk_npu_moe_w8.h"
#include "rk_npu_quant_matmul.h"
#include "rk_npu_w4a8.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Activation element types of device buffers. */
#define RK_NPU_HIP_F32 0
#define RK_NPU_HIP_F16 1

/* Epilogues. */
#define RK_NPU_HIP_PLAIN 0
#define RK_NPU_HIP_SWIGLU 1

/* Linear on device buffers. weights is a rk_npu_f32i8f32_weights* (bits 8)
 * or a rk_npu_w4a8_weights* (bits 4); workspace the matching workspace kind.
 * A [rows][K] of a_type, C [rows][N] (PLAIN) or [rows][N/2] (SWIGLU, needs
 * N % 64 == 0) of c_type. 1 <= rows <= the workspace's M. */
int rk_npu_hip_linear_run(void* workspace, const void* weights, int bits, const void* A, int a_type,
                          void* C, int c_type, int rows, int epilogue, void* stream);

/* Allocation-free linear. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Arguments, semantics and
 * results are those of rk_npu_hip_linear_run without the workspace: the
 * call's scratch (activation codes, row scales, code sums and maxima, partial
 * sums) is a slice of one RK_NPU_HIP_STATIC_SCRATCH_BYTES array per GPU inside
 * the library, set up by rk_npu_open for its device (RK_NPU_ERR_DEVICE if that
 * failed). The call allocates nothing and calls no allocating routine.
 * Limits: 1 <= rows <= RK_NPU_HIP_STATIC_MAX_ROWS, and the shape's buffers,
 * about 256 * round_up(K, 64) + 12 * round_up(N, 256) + 4 KiB bytes, must fit
 * the array (K up to about 60000 at small N); otherwise RK_NPU_ERR_PARAM and
 * nothing is enqueued. Every such call on one GPU shares that GPU's array,
 * which keeps the last call's contents: calls that overlap on one GPU (other
 * streams or threads) race and give wrong results, so serialize them (e.g. on
 * one stream). */
#define RK_NPU_HIP_STATIC_SCRATCH_BYTES (16u << 20)
#define RK_NPU_HIP_STATIC_MAX_ROWS 256
int rk_npu_hip_linear_run_static(const void* weights, int bits, const void* A, int a_type, void* C,
                                 int c_type, int rows, int epilogue, void* stream);

/* Fused FFN on device buffers: gate_up (bits gu_bits, N = 2F) -> SwiGLU ->
 * dense requant of the middle -> down (bits dn_bits). Semantics of
 * rk_npu_w4a8_run_ffn_f32. */
int rk_npu_hip_ffn_run(void* gate_up_workspace, const void* gate_up, int gu_bits,
                       void* down_workspace, const void* down, int dn_bits, const void* A,
                       int a_type, void* C, int c_type, int rows, void* stream);

/* With the switch HM_FFN_FUSED set to 1, a one-row call of
 * rk_npu_hip_ffn_run whose shapes allow it (W4 gate_up with K up to 3072,
 * such as 2560 -> 2 x 9728) runs as ONE launch whose down pieces wait on the
 * device, with a bounded spin, for the gate_up blocks of the same launch (the
 * launch runs only when the GPU can hold all of its blocks at once). If that
 * wait ever gives up (another workload holding the CUs for milliseconds), the
 * output is not valid and the down workspace records it: rk_npu_hip_ffn_status
 * synchronizes the device and returns RK_NPU_ERR_DEVICE once for such calls
 * (clearing the record), else 0. The host-buffer rk_npu_w4a8_run_ffn_f32
 * checks it itself. Off by default: slower than two launches here. */
int rk_npu_hip_ffn_status(void* down_workspace, int dn_bits);

/* Routed MoE on device buffers, semantics of rk_npu_moe_w8_run_f32. ids must
 * lie in [0, routed_experts): they are checked on the device and an
 * out-of-range id makes the call return RK_NPU_ERR_PARAM at the next
 * rk_npu_hip_moe_status() (the row is skipped, nothing is read out of bounds). */
int rk_npu_hip_moe_run(rk_npu_moe_w8_workspace* workspace, const rk_npu_moe_w8_weights* weights,
                       int rows, const float* input, const int32_t* ids, const float* routes,
                       float* output, void* stream);
/* Synchronizes the workspace's last device MoE call and reports whether it
 * saw an out-of-range expert id (RK_NPU_ERR_PARAM) or not (0). */
int rk_npu_hip_moe_status(rk_npu_moe_w8_workspace* workspace);

/* Weights from DEVICE-resident codes [K][N] int8 and scales [N] f32. */
rk_npu_f32i8f32_weights* rk_npu_hip_f32i8f32_weights_create_device(
    rk_npu_iommu_domain* domain, const rk_npu_matmul_weight_config* config,
    const int8_t* codes, const float* scales);
rk_npu_w4a8_weights* rk_npu_hip_w4a8_weights_create_device(rk_npu_iommu_domain* domain,
                                                           const rk_npu_i4_weight_config* config,
                                                           const int8_t* codes,
                                                           const float* scales);

/* Weights built on the GPU straight from checkpoint storage, replacing the
 * host path QuantLoader::load -> unpack_codes / transpose_codes -> concatenate
 * (src/model/checkpoint.rs:505-527, 558-571, 266-280, 573-604): no [K][N]
 * code matrix is formed on the host or the device. The parts are the fused
 * projection's matrices along N in order (q||k||v, gate||up), all with the
 * same k; each part's data and scales are DEVICE pointers:
 *   RK_NPU_HIP_PACK_QUANTIZED: int32 words [n][ceil(k * bits / 32)]; the value
 *     of (row n, column k) is bits (k % (32/bits)) * bits .. of word
 *     k / (32/bits), code = value - 2^(bits-1) (compressed-tensors
 *     pack-quantized, little-endian words);
 *   RK_NPU_HIP_INT_QUANTIZED (bits 8 only): int8 codes [n][k].
 * scales: [n] f32, all > 0. Returns a rk_npu_w4a8_weights* (bits 4) or a
 * rk_npu_f32i8f32_weights* (bits 8) to cast to, freed with the matching
 * *_weights_free; NULL on bad arguments (at most 8 parts), a nonpositive
 * scale, or allocation failure. Weights are identical to creating them from
 * the unpacked, concatenated [K][N] codes. */
#define RK_NPU_HIP_PACK_QUANTIZED 0
#define RK_NPU_HIP_INT_QUANTIZED 1
typedef struct rk_npu_hip_checkpoint_part {
    const void* data;
    const float* scales;
    int32_t n;
    int32_t format;
} rk_npu_hip_checkpoint_part;
void* rk_npu_hip_weights_create_checkpoint(rk_npu_iommu_domain* domain, int bits, int k,
                                           const rk_npu_hip_checkpoint_part* parts, int count);

/* Diagnostics: copies what the workspace's last call left on the device for
 * its first `rows` rows: the int8 activation codes as [rows][K] row-major,
 * the per-row scales and the per-row code sums (any output may be NULL).
 * Synchronizes the device first. */
int rk_npu_hip_workspace_codes(void* workspace, int bits, int rows, int8_t* codes, float* scales,
                               int32_t* rowsums);

/* Test hook for failure paths: the next `count` device allocations made by
 * the library fail as if the GPU were out of memory (the domain's reclaim
 * callback still runs first). Returns the previous count. */
int rk_npu_hip_inject_alloc_failures(int count);

/* Plan switches for tests and measurements. Each starts from the environment
 * variable of the same name, read once per process; this call sets one for
 * the rest of the process (later plans and workspace sizing use it) and
 * stores the value it replaces in *previous (may be NULL). Names and values:
 *   HM_GEMM_VARIANT  -1 by shape; 0..5 forces the 256x256, 256x128, 128x128,
 *                    64x128, 32x128 or 192x256 GEMM tile
 *   HM_SPLITS        0 by shape; n > 0 forces n K pieces per GEMM tile
 *   HM_FORCE_GEMM    1: rows <= 8 take the MFMA GEMM instead of the GEMV
 *   HM_GEMV_QW       -1 by shape; 0 never, 1 always (when the rows fit) a
 *                    quantization wave in the GEMV blocks
 *   HM_GEMV_SPLITS   0 by shape; n > 0 forces n K pieces of the one-row GEMV
 *                    after a SwiGLU
 *   HM_FFN_FUSED     0: a one-row FFN runs as two launches (gate_up, then
 *                    down); 1: as one launch when its shapes allow
 *   HM_FFN_SPIN      polls a one-launch FFN's down blocks make for their
 *                    gate_up blocks before giving up (65536); negative: they
 *                    give up at once (tests of the failure report)
 *   HM_GEMV_PREQ     -1: 4 rows are quantized by a launch before the GEMV;
 *                    0: inside the GEMV blocks wherever the rows fit
 *   HM_GEMV_COMBINE  1: a one-token MoE call with a shared expert runs the
 *                    combine in the shared down GEMV's epilogue where that
 *                    GEMV allows; 0: always as a separate launch
 *   HM_HOST_FLAG     1: a host-buffer call (rk_npu_*_run_f32, _run_dynamic,
 *                    the MoE run) whose input and output each fit 64 KB
 *                    runs on the compute queue: a kernel fetches its inputs
 *                    from the workspace's pinned stage, and a copy kernel
 *                    writes C and a completion word into the stage, which
 *                    the CPU polls; 0: copies in and out and a wait on the
 *                    stream (HM_HOST_SPIN), as larger calls always do
 *   HM_HOST_POLL     microseconds a host-buffer call on the kernel path
 *                    polls its completion word before it waits on its
 *                    stream instead (2000; 0: after the first 256 polls)
 *   HM_HOST_SPIN     0: a host-buffer call that waits on its stream does so
 *                    in hipStreamSynchronize; 1: by polling its stream
 *                    (slower here)
 * Unknown names return RK_NPU_ERR_PARAM. */
int rk_npu_hip_set_switch(const char* name, int value, int* previous);

/* Kernel timing for measurement tools. Between profile_begin and
 * profile_end every GEMM/GEMV/quantization launch of the library is
 * bracketed by two HIP events recorded on the stream it is launched on (at
 * most max_launches launches; later ones are not recorded). Not for use under
 * graph capture. profile_read synchronizes the device and returns one entry
 * per distinct (kind, bits, epilogue, rows, K, N) with its launch count and
 * summed event time. kind: 0 GEMV, 1 MFMA GEMM, 2 quantization, 3 grouped GEMM. */
typedef struct rk_npu_hip_kernel_stat {
    int32_t kind;
    int32_t bits;
    int32_t epilogue;
    int32_t rows;
    int32_t K;
    int32_t N;
    int32_t launches;
    double total_ms;
    char name[64];
} rk_npu_hip_kernel_stat;
int rk_npu_hip_profile_begin(int max_launches);
int rk_npu_hip_profile_end(void);
int rk_npu_hip_profile_read(rk_npu_hip_kernel_stat* stats, int capacity, int* count);

/* Launch plan the library uses for a linear of this shape, for diagnostics:
 * kind 0 = GEMV (no MFMA), 1 = MFMA GEMM; tile sizes and K splits. */
typedef struct rk_npu_hip_plan {
    int32_t kind;
    int32_t block_m;
    int32_t block_n;
    int32_t k_splits;
    int32_t grid;
} rk_npu_hip_plan;
int rk_npu_hip_linear_plan(int rows, int K, int N, int bits, rk_npu_hip_plan* plan);

#ifdef __cplusplus
}
#endif
#endif

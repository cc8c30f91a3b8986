// Kernel launch entry points the runtime calls (hip_matmul.hip), defined in
// the launch_*.hip translation units: the GEMM tiles by weight width, the
// GEMVs by activation type and weight width, the one-launch FFN. Splitting
// the template instantiations over these units lets them compile in
// parallel.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

#include "kernels.hpp"

namespace hm {

int device_cus();  // compute units of the current device (hip_matmul.hip)

// GEMM block tiles (rows x columns), indexed by the plan (kBM / kBN in
// hip_matmul.hip).
enum GemmVariant { V256x256 = 0, V256x128 = 1, V128x128 = 2, V64x128 = 3, V32x128 = 4, V192x256 = 5 };

// GEMM of one weight width: epi EPI_PLAIN / EPI_SWIGLU_MAX, tile variant v,
// staged (16-byte aligned output) or not, G.splits K pieces.
void launch_gemm_w8(int epi, int v, bool staged, const GemmParams& G, int tiles, hipStream_t s);
void launch_gemm_w4(int epi, int v, bool staged, const GemmParams& G, int tiles, hipStream_t s);

// GEMV of `mr` rows (1, 2, 4, 8), rows quantized beforehand (preq), by a
// quantization wave (qwn = 1) or by the block; split-K pieces; the one-row
// plain GEMV with the MoE combine (f32 activations only).
#define HM_DECLARE_GEMV(X, B)                                                                               \
    void launch_gemv_##X##_w##B(int epi, int mr, const GemvParams& V, int grid, size_t lds, hipStream_t s,   \
                                bool preq, int qwn);                                                       \
    void launch_gemv_split_##X##_w##B(const GemvParams& V, int grid, int rounds, size_t lds, hipStream_t s);
HM_DECLARE_GEMV(f32, 8)
HM_DECLARE_GEMV(f32, 4)
HM_DECLARE_GEMV(f16, 8)
HM_DECLARE_GEMV(f16, 4)
#undef HM_DECLARE_GEMV
void launch_gemv_combine_w8(const GemvParams& V, int groups, int rounds, size_t lds, hipStream_t s);
void launch_gemv_combine_w4(const GemvParams& V, int groups, int rounds, size_t lds, hipStream_t s);

// The one-launch FFN; false (nothing enqueued) when its blocks cannot all be
// resident on this GPU at once.
bool launch_ffn_fused_any(int a_type, int dn_bits, int rwg, const GemvParams& Pg, const GemvParams& Pd, int grid,
                          size_t lds, hipStream_t s);

inline void launch_gemm_any(int bits, int epi, int v, bool staged, const GemmParams& G, int tiles, hipStream_t s) {
    if (bits == 8)
        launch_gemm_w8(epi, v, staged, G, tiles, s);
    else
        launch_gemm_w4(epi, v, staged, G, tiles, s);
}

inline void launch_gemv_any(int x_type, int bits, int epi, int mr, const GemvParams& V, int grid, size_t lds,
                            hipStream_t s, bool preq, int qwn) {
    if (x_type == DT_F32) {
        if (bits == 8)
            launch_gemv_f32_w8(epi, mr, V, grid, lds, s, preq, qwn);
        else
            launch_gemv_f32_w4(epi, mr, V, grid, lds, s, preq, qwn);
    } else {
        if (bits == 8)
            launch_gemv_f16_w8(epi, mr, V, grid, lds, s, preq, qwn);
        else
            launch_gemv_f16_w4(epi, mr, V, grid, lds, s, preq, qwn);
    }
}

inline void launch_gemv_split_any(int x_type, int bits, const GemvParams& V, int grid, int rounds, size_t lds,
                                  hipStream_t s) {
    if (x_type == DT_F32) {
        if (bits == 8)
            launch_gemv_split_f32_w8(V, grid, rounds, lds, s);
        else
            launch_gemv_split_f32_w4(V, grid, rounds, lds, s);
    } else {
        if (bits == 8)
            launch_gemv_split_f16_w8(V, grid, rounds, lds, s);
        else
            launch_gemv_split_f16_w4(V, grid, rounds, lds, s);
    }
}

inline void launch_gemv_combine_any(int bits, const GemvParams& V, int groups, int rounds, size_t lds,
                                    hipStream_t s) {
    if (bits == 8)
        launch_gemv_combine_w8(V, groups, rounds, lds, s);
    else
        launch_gemv_combine_w4(V, groups, rounds, lds, s);
}

}  // namespace hm

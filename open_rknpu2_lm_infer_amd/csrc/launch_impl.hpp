// Launch templates of the GEMM and GEMV kernels (tile and register-window
// variants chosen at run time), instantiated by the launch_*.hip translation
// units, one per activation type and weight width, which compile in
// parallel; launch.hpp declares what they define.
#pragma once

#include <hip/hip_runtime.h>

#include "kernels.hpp"
#include "launch.hpp"

namespace hm {

// Outputs without a 16-byte aligned base and row pitch take the 128x128
// tile with per-lane stores (staged = false); all other launches stage rows
// through LDS. A split plan (64x128 / 128x128 tiles, staged) is two launches:
// the K pieces' partials, then the per-tile sum and epilogue.
template <int BM, int BN, int WGM, int WGN, int BITS, int EPI>
static void launch_split(const GemmParams& G, int tiles, hipStream_t s) {
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WGM, WGN, BITS, EPI_PLAIN, true, SPLIT_PART>), dim3(tiles * G.splits),
                       dim3(WGM * WGN * 64), 0, s, G);
    if constexpr (BM == 128 && BN == 128 && WGM == 2 && WGN == 2)
        hipLaunchKernelGGL((gemm_split_finish_kernel<BITS, EPI>), dim3(tiles * 4), dim3(64), 0, s, G);
    else
        hipLaunchKernelGGL((gemm_kernel<BM, BN, WGM, WGN, BITS, EPI, true, SPLIT_FINISH>), dim3(tiles),
                           dim3(WGM * WGN * 64), 0, s, G);
}

template <int BITS, int EPI>
static void launch_gemm(int v, bool staged, const GemmParams& G, int tiles, hipStream_t s) {
    if (!staged) {
        hipLaunchKernelGGL((gemm_kernel<128, 128, 2, 2, BITS, EPI, false>), dim3(tiles), dim3(256), 0, s, G);
        return;
    }
    if (G.splits > 1) {
        if (v == V64x128)
            launch_split<64, 128, 2, 2, BITS, EPI>(G, tiles, s);
        else
            launch_split<128, 128, 2, 2, BITS, EPI>(G, tiles, s);
        return;
    }
    switch (v) {
        case V256x256:
            hipLaunchKernelGGL((gemm_kernel<256, 256, 2, 4, BITS, EPI, true>), dim3(tiles), dim3(512), 0, s, G);
            break;
        case V192x256:
            hipLaunchKernelGGL((gemm_kernel<192, 256, 2, 4, BITS, EPI, true>), dim3(tiles), dim3(512), 0, s, G);
            break;
        case V256x128:
            hipLaunchKernelGGL((gemm_kernel<256, 128, 2, 2, BITS, EPI, true>), dim3(tiles), dim3(256), 0, s, G);
            break;
        case V128x128:
            hipLaunchKernelGGL((gemm_kernel<128, 128, 2, 2, BITS, EPI, true>), dim3(tiles), dim3(256), 0, s, G);
            break;
        case V64x128:
            hipLaunchKernelGGL((gemm_kernel<64, 128, 2, 2, BITS, EPI, true>), dim3(tiles), dim3(256), 0, s, G);
            break;
        default:
            hipLaunchKernelGGL((gemm_kernel<32, 128, 1, 2, BITS, EPI, true>), dim3(tiles), dim3(128), 0, s, G);
            break;
    }
}

template <typename T, int MR, int BITS, int EPI, bool PREQ, int QWN>
static void launch_gemv_w(const GemvParams& V, int groups, size_t lds, hipStream_t s) {
    // Register windows sized to the group (rounds of 256 16-byte chunks), so
    // no thread loads a chunk past the group's end and no registers hold one:
    // fewer registers, more resident blocks, no wasted load issue. Groups of
    // more than 8 rounds (the 9728-long down projection) take 512-thread
    // blocks: half the serial loads, quantization and dot products per thread
    // on the few blocks such a matrix has.
    const int planes = BITS == 8 ? V.K_pad / 16 : V.K_pad / 32;
    const int chunks = planes * 8 * (EPI == EPI_PLAIN ? 1 : 2);
    const int rounds = (chunks + 255) / 256;
    if constexpr (QWN == 1) {  // groups of 5 to 8 rounds (shorter ones, forced by HM_GEMV_QW, take 5)
        if (rounds <= 5)
            hipLaunchKernelGGL((gemv_kernel<T, MR, BITS, EPI, 5, 1, PREQ, 1, 256, false, 1>), dim3(groups), dim3(320),
                               lds, s, V);
        else if (rounds <= 6)
            hipLaunchKernelGGL((gemv_kernel<T, MR, BITS, EPI, 6, 1, PREQ, 1, 256, false, 1>), dim3(groups), dim3(320),
                               lds, s, V);
        else
            hipLaunchKernelGGL((gemv_kernel<T, MR, BITS, EPI, 8, 1, PREQ, 1, 256, false, 1>), dim3(groups), dim3(320),
                               lds, s, V);
        return;
    }
    if (rounds <= 3)
        hipLaunchKernelGGL((gemv_kernel<T, MR, BITS, EPI, 3, 1, PREQ>), dim3(groups), dim3(256), lds, s, V);
    else if (rounds <= 4)
        hipLaunchKernelGGL((gemv_kernel<T, MR, BITS, EPI, 4, 1, PREQ>), dim3(groups), dim3(256), lds, s, V);
    else if (rounds <= 5)
        hipLaunchKernelGGL((gemv_kernel<T, MR, BITS, EPI, 5, 1, PREQ>), dim3(groups), dim3(256), lds, s, V);
    else if (rounds <= 6)
        hipLaunchKernelGGL((gemv_kernel<T, MR, BITS, EPI, 6, 1, PREQ>), dim3(groups), dim3(256), lds, s, V);
    else if (rounds <= 8)
        hipLaunchKernelGGL((gemv_kernel<T, MR, BITS, EPI, 8, 1, PREQ>), dim3(groups), dim3(256), lds, s, V);
    else if (chunks <= 512 * 5)
        hipLaunchKernelGGL((gemv_kernel<T, MR, BITS, EPI, 5, 1, PREQ, 1, 512>), dim3(groups), dim3(512), lds, s, V);
    else if (chunks <= 512 * 6)
        hipLaunchKernelGGL((gemv_kernel<T, MR, BITS, EPI, 6, 1, PREQ, 1, 512>), dim3(groups), dim3(512), lds, s, V);
    else if (chunks <= 512 * 10)
        hipLaunchKernelGGL((gemv_kernel<T, MR, BITS, EPI, 5, 2, PREQ, 1, 512>), dim3(groups), dim3(512), lds, s, V);
    else
        hipLaunchKernelGGL((gemv_kernel<T, MR, BITS, EPI, 8, 2, PREQ, 1, 512>), dim3(groups), dim3(512), lds, s, V);
}

// The one-row plain GEMV with the MoE combine in its epilogue.
template <int BITS>
static void launch_gemv_combine(const GemvParams& V, int groups, int rounds, size_t lds, hipStream_t s) {
    if (rounds <= 3)
        hipLaunchKernelGGL((gemv_combine_kernel<BITS, 3>), dim3(groups), dim3(256), lds, s, V);
    else if (rounds <= 4)
        hipLaunchKernelGGL((gemv_combine_kernel<BITS, 4>), dim3(groups), dim3(256), lds, s, V);
    else if (rounds <= 5)
        hipLaunchKernelGGL((gemv_combine_kernel<BITS, 5>), dim3(groups), dim3(256), lds, s, V);
    else if (rounds <= 6)
        hipLaunchKernelGGL((gemv_combine_kernel<BITS, 6>), dim3(groups), dim3(256), lds, s, V);
    else
        hipLaunchKernelGGL((gemv_combine_kernel<BITS, 8>), dim3(groups), dim3(256), lds, s, V);
}

// Split-K GEMV (one row, plain epilogue): rounds of the largest piece.
template <typename T, int BITS>
static void launch_gemv_split(const GemvParams& V, int grid, int rounds, size_t lds, hipStream_t s) {
    if (rounds <= 3)
        hipLaunchKernelGGL((gemv_kernel<T, 1, BITS, EPI_PLAIN, 3, 1, false, 1, 256, false, 0, true>), dim3(grid),
                           dim3(256), lds, s, V);
    else if (rounds <= 4)
        hipLaunchKernelGGL((gemv_kernel<T, 1, BITS, EPI_PLAIN, 4, 1, false, 1, 256, false, 0, true>), dim3(grid),
                           dim3(256), lds, s, V);
    else if (rounds <= 5)
        hipLaunchKernelGGL((gemv_kernel<T, 1, BITS, EPI_PLAIN, 5, 1, false, 1, 256, false, 0, true>), dim3(grid),
                           dim3(256), lds, s, V);
    else if (rounds <= 6)
        hipLaunchKernelGGL((gemv_kernel<T, 1, BITS, EPI_PLAIN, 6, 1, false, 1, 256, false, 0, true>), dim3(grid),
                           dim3(256), lds, s, V);
    else
        hipLaunchKernelGGL((gemv_kernel<T, 1, BITS, EPI_PLAIN, 8, 1, false, 1, 256, false, 0, true>), dim3(grid),
                           dim3(256), lds, s, V);
}

// Rows quantized beforehand (preq), by a quantization wave of the block
// (qwn = 1), or by every thread of the block.
template <typename T, int MR, int BITS, int EPI>
static void launch_gemv_mr(const GemvParams& V, int groups, size_t lds, hipStream_t s, bool preq, int qwn) {
    if constexpr (MR > 4) {
        (void)preq;  // more than 4 rows are always quantized beforehand (enqueue_linear)
        (void)qwn;
        launch_gemv_w<float, MR, BITS, EPI, true, 0>(V, groups, lds, s);
    } else if constexpr (MR == 4) {
        (void)qwn;  // 4 rows: beforehand, or by every thread of the block (HM_GEMV_PREQ=0)
        if (preq)
            launch_gemv_w<float, MR, BITS, EPI, true, 0>(V, groups, lds, s);
        else
            launch_gemv_w<T, MR, BITS, EPI, false, 0>(V, groups, lds, s);
    } else {
        if (preq)
            launch_gemv_w<float, MR, BITS, EPI, true, 0>(V, groups, lds, s);  // activations unused
        else if (qwn == 1)
            launch_gemv_w<T, MR, BITS, EPI, false, 1>(V, groups, lds, s);
        else
            launch_gemv_w<T, MR, BITS, EPI, false, 0>(V, groups, lds, s);
    }
}

template <typename T, int BITS, int EPI>
static void launch_gemv(int mr, const GemvParams& V, int grid, size_t lds, hipStream_t s, bool preq, int qwn) {
    switch (mr) {
        case 1:
            launch_gemv_mr<T, 1, BITS, EPI>(V, grid, lds, s, preq, qwn);
            break;
        case 2:
            launch_gemv_mr<T, 2, BITS, EPI>(V, grid, lds, s, preq, qwn);
            break;
        case 4:
            launch_gemv_mr<T, 4, BITS, EPI>(V, grid, lds, s, preq, qwn);
            break;
        default:
            launch_gemv_mr<T, 8, BITS, EPI>(V, grid, lds, s, preq, qwn);
            break;
    }
}

template <typename T, int BITS>
static void launch_gemv_epi(int epi, int mr, const GemvParams& V, int grid, size_t lds, hipStream_t s, bool preq,
                            int qwn) {
    if (epi == EPI_PLAIN)
        launch_gemv<T, BITS, EPI_PLAIN>(mr, V, grid, lds, s, preq, qwn);
    else
        launch_gemv<T, BITS, EPI_SWIGLU_MAX>(mr, V, grid, lds, s, preq, qwn);
}

}  // namespace hm

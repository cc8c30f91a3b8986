// HIP kernels of the routed-expert (MoE) FFN: device-side token
// permutation, ragged grouped GEMM over the permutation, rank-ordered combine.
#pragma once

#include "kernels.hpp"

namespace hm {

constexpr int MOE_MAX_EXPERTS = 512;

// ---------------------------------------------------------------------------
// Counting sort of the (token, rank) assignments by expert. Assignments with
// route <= 0 are skipped (they contribute nothing to the combine); an expert id
// outside [0, experts) raises the error flag and is skipped as well. Each
// expert's assignments get a contiguous run of slots; every run is cut into
// m-tiles of BM slots for the grouped GEMM. Within a run the slot order is
// arbitrary: every slot is computed independently and the combine reads
// slots through pos[] in rank order, so results do not depend on it.
// ---------------------------------------------------------------------------
struct RouteParams {
    const int* ids;
    const float* routes;
    int rows, top, experts;
    int* pos;       // [rows*top] slot or -1
    int* perm;      // [rows*top] slot -> assignment
    int4* tiles;    // [max_tiles] {expert, slot_begin, slot_end, 0}
    int* counts;    // [0] slots used, [1] tiles
    unsigned* rowmax_mid;
    int rowmax_count;
    unsigned* error;
};

template <int BM>
__global__ __launch_bounds__(1024) void moe_route_kernel(RouteParams P) {
    __shared__ int cnt[MOE_MAX_EXPERTS];
    __shared__ int fill[MOE_MAX_EXPERTS];
    __shared__ int off[MOE_MAX_EXPERTS];
    __shared__ int toff[MOE_MAX_EXPERTS];
    const int tid = threadIdx.x;
    const int A = P.rows * P.top;
    for (int e = tid; e < P.experts; e += 1024) {
        cnt[e] = 0;
        fill[e] = 0;
    }
    for (int i = tid; i < P.rowmax_count; i += 1024) P.rowmax_mid[i] = 0u;
    __syncthreads();
    // Each thread's first RC assignments are requested at once (one memory
    // round trip instead of one per assignment; indices past A re-read the
    // last assignment and are masked) and their experts stay in registers
    // for the second pass (-1 for a skipped route); later ones are read again.
    constexpr int RC = 8;
    int ce[RC], idv[RC];
    float rv[RC];
#pragma unroll
    for (int i = 0; i < RC; ++i) {
        const int a = min(tid + 1024 * i, A - 1);
        idv[i] = P.ids[a];
        rv[i] = P.routes[a];
    }
#pragma unroll
    for (int i = 0; i < RC; ++i) {
        ce[i] = -1;
        if (tid + 1024 * i < A) {
            const int e = idv[i];
            const bool in_range = e >= 0 && e < P.experts;
            if (!in_range) atomicOr(P.error, 1u);
            const bool live = in_range && rv[i] > 0.0f;
            if (live) atomicAdd(&cnt[e], 1);
            ce[i] = live ? e : -1;
        }
    }
    for (int a = tid + 1024 * RC; a < A; a += 1024) {
        const int e = P.ids[a];
        const bool in_range = e >= 0 && e < P.experts;
        if (!in_range) atomicOr(P.error, 1u);
        if (in_range && P.routes[a] > 0.0f) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // Exclusive prefix sums of slots and tiles over the experts: wave 0, each
    // lane owns MOE_MAX_EXPERTS / 64 consecutive experts, then a wave scan.
    if (tid < 64) {
        constexpr int PER = MOE_MAX_EXPERTS / 64;
        int ls = 0, lt = 0;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = tid * PER + i;
            const int c = e < P.experts ? cnt[e] : 0;
            ls += c;
            lt += (c + BM - 1) / BM;
        }
        int is = ls, it = lt;  // inclusive scans over lanes
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int us = __shfl_up(is, d), ut = __shfl_up(it, d);
            if (tid >= d) {
                is += us;
                it += ut;
            }
        }
        int run = is - ls, tiles = it - lt;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = tid * PER + i;
            if (e < P.experts) {
                off[e] = run;
                toff[e] = tiles;
                run += cnt[e];
                tiles += (cnt[e] + BM - 1) / BM;
            }
        }
        if (tid == 63) {
            P.counts[0] = is;
            P.counts[1] = it;
        }
    }
    __syncthreads();
    for (int a = tid, i = 0; a < A; a += 1024, ++i) {
        int e = -1;
        if (i < RC) {
#pragma unroll
            for (int j = 0; j < RC; ++j)
                if (i == j) e = ce[j];
        } else {
            e = P.ids[a];
            if (!(e >= 0 && e < P.experts && P.routes[a] > 0.0f)) e = -1;
        }
        int slot = -1;
        if (e >= 0) {
            slot = off[e] + atomicAdd(&fill[e], 1);
            P.perm[slot] = a;
        }
        P.pos[a] = slot;
    }
    for (int e = tid; e < P.experts; e += 1024) {
        const int n = (cnt[e] + BM - 1) / BM;
        for (int t = 0; t < n; ++t) {
            const int b = off[e] + t * BM;
            P.tiles[toff[e] + t] = make_int4(e, b, min(off[e] + cnt[e], b + BM), 0);
        }
    }
}

// ---------------------------------------------------------------------------
// Grouped GEMM: block = (m-tile of one expert's slot run, n-tile). Gather mode
// (perm != nullptr) reads A row perm[slot] / top (the token's quantized input
// row); otherwise A row = slot (the requantized middle). Blocks past the
// device-side tile count exit at once.
// ---------------------------------------------------------------------------
struct MoeGemmParams {
    const int8_t* a;
    int a_alloc;
    const int* perm;
    int top;
    const float* rowscale;
    const int* rowsum;
    const uint8_t* const* b_tab;
    const float* const* s_tab;
    const int4* tiles;
    const int* counts;
    void* c;
    long ldc;
    int c_type;
    unsigned* rowmax;
    int N, K_pad, N_pad, half, tiles_n;
};

template <int BM, int BN, int WGM, int WGN, int BITS, int EPI, bool STAGED>
__global__ __launch_bounds__(WGM* WGN * 64, 1) void moe_gemm_kernel(MoeGemmParams P) {
    using C = TileCfg<BM, BN, WGM, WGN, BITS>;
    __shared__ __attribute__((aligned(16))) uint8_t smem[C::SMEM];
    __shared__ int s_rows[BM];
#ifndef MOE_XCD_ORDER
#define MOE_XCD_ORDER 1
#endif
#if MOE_XCD_ORDER
    // Blocks are dealt to the 8 XCDs round-robin: XCD x = block % 8 takes the
    // row tiles x, x + 8, ..., all N-tiles of one row tile in a row, so the
    // tile's activation rows are fetched into that XCD's L2 once and shared
    // by its N-tiles (the grid is 8 * ceil(max tiles / 8) * tiles_n blocks).
    const int i = blockIdx.x >> 3;
    const int t = (blockIdx.x & 7) + 8 * (i / P.tiles_n), tn = i % P.tiles_n;
#else
    const int t = blockIdx.x / P.tiles_n, tn = blockIdx.x % P.tiles_n;
#endif
    if (t >= P.counts[1]) return;
    const int4 tile = P.tiles[t];
    const int e = tile.x, begin = tile.y, end = tile.z;
    for (int i = threadIdx.x; i < BM; i += C::NT) {
        const int slot = begin + i < end ? begin + i : begin;
        s_rows[i] = P.perm ? P.perm[slot] / P.top : slot;
    }
    __syncthreads();
    size_t a_off[C::A_LOADS];
#pragma unroll
    for (int i = 0; i < C::A_LOADS; ++i) {
        const int c = threadIdx.x + i * C::NT;
        a_off[i] = (size_t)(c / BM) * P.a_alloc + s_rows[c % BM];
    }
    v16i acc[C::FM][C::FN];
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    const int n0 = tn * BN;
    auto row_of = [&](int local, int& out_row, int& src_row) {
        out_row = begin + local;
        src_row = s_rows[local];
        return begin + local < end;
    };
    const auto pre = epilogue_prefetch<BM, BN, WGM, WGN, BITS>(P.rowscale, P.rowsum, P.s_tab[e], n0, row_of);
    gemm_mainloop<BM, BN, WGM, WGN, BITS>(smem, P.a, (size_t)P.a_alloc, a_off, P.b_tab[e], P.K_pad, n0, P.K_pad >> 6,
                                          acc);
    gemm_epilogue<BM, BN, WGM, WGN, BITS, EPI, STAGED>(acc, n0, pre, P.N, P.half, P.c, P.ldc, P.c_type, P.rowmax,
                                                       row_of, smem);
}

// ---------------------------------------------------------------------------
// Combine: out[r][c] = sum over rank (in order, skipped slots excluded) of
// fma(contribution, route, sum), then + shared contribution.
// ---------------------------------------------------------------------------
struct CombineParams {
    const float* contrib;  // [slots][h]
    const int* pos;        // slot of each assignment (-1: skipped); nullptr: slot = assignment
    const float* routes;
    const float* shared;  // [rows][h] or nullptr
    int rows, top, h;
    float* out;
};

// VEC output columns per thread (4 when every row is 16-byte aligned): the
// ranks' slots and weights (uniform over the block: scalar loads) and the
// contributions are requested together, 8 ranks at a time (one memory round
// trip instead of one per rank), then added in rank order, so each sum is the
// same sequence of single-rounding fma as the reference's rank loop. A
// skipped rank reads a valid row and is not added.
constexpr int COMBINE_BATCH = 8;
template <int VEC>
static __global__ __launch_bounds__(256) void moe_combine_kernel(CombineParams P) {
    typedef float fv __attribute__((ext_vector_type(VEC)));
    const int r = blockIdx.y;
    const int c = (blockIdx.x * 256 + threadIdx.x) * VEC;
    if (c >= P.h) return;
    fv sum = fv(0.0f);
    for (int r0 = 0; r0 < P.top; r0 += COMBINE_BATCH) {
        const int a0 = r * P.top + r0;
        const int n = min(COMBINE_BATCH, P.top - r0);
        float w[COMBINE_BATCH];
        int slot[COMBINE_BATCH];
        fv v[COMBINE_BATCH];
        if (n == COMBINE_BATCH) {
#pragma unroll
            for (int i = 0; i < COMBINE_BATCH; ++i) w[i] = P.routes[a0 + i];
            if (P.pos) {
#pragma unroll
                for (int i = 0; i < COMBINE_BATCH; ++i) slot[i] = P.pos[a0 + i];
            } else {
#pragma unroll
                for (int i = 0; i < COMBINE_BATCH; ++i) slot[i] = w[i] > 0.0f ? a0 + i : -1;
            }
        } else {
#pragma unroll
            for (int i = 0; i < COMBINE_BATCH; ++i) {
                w[i] = i < n ? P.routes[a0 + i] : 0.0f;
                slot[i] = i >= n ? -1 : (P.pos ? P.pos[a0 + i] : (w[i] > 0.0f ? a0 + i : -1));
            }
        }
#pragma unroll
        for (int i = 0; i < COMBINE_BATCH; ++i)
            v[i] = *reinterpret_cast<const fv*>(P.contrib + (size_t)max(slot[i], 0) * P.h + c);
#pragma unroll
        for (int i = 0; i < COMBINE_BATCH; ++i)
            if (slot[i] >= 0) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) sum[e] = __builtin_fmaf(v[i][e], w[i], sum[e]);
            }
    }
    if (P.shared) {
        const fv sh = *reinterpret_cast<const fv*>(P.shared + (size_t)r * P.h + c);
#pragma unroll
        for (int e = 0; e < VEC; ++e) sum[e] = sum[e] + sh[e];
    }
    *reinterpret_cast<fv*>(P.out + (size_t)r * P.h + c) = sum;
}

}  // namespace hm

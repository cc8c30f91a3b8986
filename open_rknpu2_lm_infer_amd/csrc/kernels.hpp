// HIP kernels of the quantized-linear hot path, written for gfx950 (CDNA4).
//
// Device data layouts (all chosen so every global access is a coalesced
// 16-byte-per-lane load and every LDS fragment read is conflict free):
//   activation codes  A8 : [K_pad/16][M_alloc][16]  int8   ("k16 planes")
//   W8 weights           : [K_pad/16][N_pad][16]    int8
//   W4 weights           : [K_pad/32][N_pad][16]    bytes, two offset-binary
//                          nibbles (u = code + 8) per byte. Entry j of column
//                          p holds, with g = j/2 and h = j%2, the codes
//                          k = 64g + 16h + b in the low nibble of byte b and
//                          k = 64g + 32 + 16h + b in the high nibble.
//   column order         : when N % 64 == 0 the packed column p maps to the
//                          original column orig_col(p): 32 gate columns then
//                          the 32 matching up columns (N/2 + ...), so a
//                          SwiGLU pair always sits in one wave's registers.
// W4 products use u = code + 8 directly on the int8 datapath and subtract
// 8 * sum(activation codes of the row) in the epilogue, which is exact in int32.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cfloat>

namespace hm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

enum { QUANT_DENSE = 0, QUANT_MOE = 1 };
enum { EPI_PLAIN = 0, EPI_SWIGLU = 1, EPI_SWIGLU_MAX = 2 };
enum { DT_F32 = 0, DT_F16 = 1 };

// exp(x) for |x| <= 80: Cody–Waite reduction x = n*ln2 + r (ln2 split in a
// 12-bit-short high part and a low part), degree-7 Taylor polynomial of e^r
// (coefficients 1/j! rounded to f32) in Horner form, 2^n through the exponent
// field. Each step is a single IEEE operation, so the result is bit-identical
// to the same sequence evaluated on the host.
__device__ __forceinline__ float hm_expf(float x) {
    const float log2e = 0x1.715476p+0f;
    const float ln2_hi = 0x1.62ep-1f;
    const float ln2_lo = 0x1.0bfbe8p-15f;
    float kf = __builtin_rintf(x * log2e);
    float r = __builtin_fmaf(kf, -ln2_hi, x);
    r = __builtin_fmaf(kf, -ln2_lo, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0x1.0p-1f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    int n = (int)kf;
    return p * __int_as_float((n + 127) << 23);
}

// silu(g) * u with the exponent argument saturated to [-80, 80] and a signed
// zero for g < -80.
__device__ __forceinline__ float hm_swiglu(float g, float u) {
    float t = fminf(fmaxf(-g, -80.0f), 80.0f);
    float e = hm_expf(t);
    float silu = g / (1.0f + e);
    if (g < -80.0f) silu = __builtin_copysignf(0.0f, g);
    return silu * u;
}

__device__ __forceinline__ int orig_col(int p, int half) {
    if (!half) return p;
    int q = p >> 6, w = p & 63;
    return w < 32 ? (q << 5) + w : half + (q << 5) + (w - 32);
}

__device__ __forceinline__ void store_out(void* c, int c_type, size_t idx, float v) {
    if (c_type == DT_F32)
        static_cast<float*>(c)[idx] = v;
    else
        static_cast<__half*>(c)[idx] = __float2half_rn(v);
}

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
    return static_cast<float>(v);
}
template <>
__device__ __forceinline__ float to_f32<__half>(__half v) {
    return __half2float(v);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// ---------------------------------------------------------------------------
// Per-row dynamic int8 quantization.
// 16 rows per 256-thread block. Phase 1: one wave per row computes max|x| with
// a wave reduction (or takes a precomputed max from rowmax_in). Phase 2: each
// thread quantizes 16 consecutive k of one row and writes them as one 16-byte
// chunk of the k16-plane layout; 16 consecutive threads cover one 256-byte run.
// ---------------------------------------------------------------------------
struct QuantParams {
    const void* x;
    int x_type;
    long lda;
    int rows, K, K_pad, M_alloc;
    int vec;  // 1 when rows are 16-byte aligned and K % 16 == 0
    int8_t* codes;
    float* rowscale;
    int* rowsum;
    const unsigned* rowmax_in;
    unsigned* rowmax_clear;  // zeroed for the block's rows (next middle's max)
    const int* rows_dev;     // optional device-side row count (<= rows)
};

__device__ __forceinline__ void load16(const float* p, float (&v)[16]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 t = reinterpret_cast<const float4*>(p)[q];
        v[4 * q] = t.x;
        v[4 * q + 1] = t.y;
        v[4 * q + 2] = t.z;
        v[4 * q + 3] = t.w;
    }
}
__device__ __forceinline__ void load16(const __half* p, float (&v)[16]) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const v4u t = reinterpret_cast<const v4u*>(p)[q];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const unsigned bits = t[w];
            v[8 * q + 2 * w] = __half2float(__ushort_as_half((unsigned short)(bits & 0xffffu)));
            v[8 * q + 2 * w + 1] = __half2float(__ushort_as_half((unsigned short)(bits >> 16)));
        }
    }
}

template <typename T, int RULE>
__global__ __launch_bounds__(256) void quant_rows_kernel(QuantParams P) {
    __shared__ float s_inv[16];
    __shared__ int s_sum[4][16];
    const T* x = static_cast<const T*>(P.x);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r0 = blockIdx.x * 16;
    const int rows = P.rows_dev ? min(P.rows, *P.rows_dev) : P.rows;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int lr = wave * 4 + i, r = r0 + lr;
        float m = 0.0f;
        if (r < rows) {
            if (P.rowmax_in) {
                m = __uint_as_float(P.rowmax_in[r]);
            } else {
                const T* xr = x + (size_t)r * P.lda;
                for (int k = lane; k < P.K; k += 64) m = fmaxf(m, fabsf(to_f32(xr[k])));
                m = wave_max(m);
            }
        }
        if (lane == 0) {
            float s;
            if (RULE == QUANT_DENSE)
                s = (m == 0.0f) ? 1.0f : fmaxf(m / 127.0f, FLT_MIN);
            else
                s = (m == 0.0f) ? 1.0f : m / 127.0f;
            s_inv[lr] = 1.0f / s;
            if (r < rows) P.rowscale[r] = s;
        }
    }
    if (P.rowmax_clear && tid < 16 && r0 + tid < P.M_alloc) P.rowmax_clear[r0 + tid] = 0u;
    __syncthreads();
    const int lr = tid & 15, r = r0 + lr;
    const float inv = s_inv[lr];
    const int KG = P.K_pad >> 4;
    int sum = 0;
    for (int kg = tid >> 4; kg < KG; kg += 16) {
        float v[16];
        if (r < rows) {
            const T* xr = x + (size_t)r * P.lda + kg * 16;
            if (P.vec && kg * 16 + 16 <= P.K) {
                load16(xr, v);
            } else {
#pragma unroll
                for (int b = 0; b < 16; ++b) v[b] = (kg * 16 + b < P.K) ? to_f32(xr[b]) : 0.0f;
            }
        } else {
#pragma unroll
            for (int b = 0; b < 16; ++b) v[b] = 0.0f;
        }
        unsigned packed[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int b = 0; b < 16; ++b) {
            float q = v[b] * inv;
            q = (RULE == QUANT_DENSE) ? roundf(q) : __builtin_rintf(q);
            q = fminf(fmaxf(q, -127.0f), 127.0f);
            int qi = (int)q;
            sum += qi;
            packed[b >> 2] |= ((unsigned)qi & 0xffu) << ((b & 3) * 8);
        }
        v4u out = {packed[0], packed[1], packed[2], packed[3]};
        *reinterpret_cast<v4u*>(P.codes + ((size_t)kg * P.M_alloc + r0 + lr) * 16) = out;
    }
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);
    if (lane < 16) s_sum[wave][lane] = sum;
    __syncthreads();
    if (tid < 16 && r0 + tid < rows)
        P.rowsum[r0 + tid] = s_sum[0][tid] + s_sum[1][tid] + s_sum[2][tid] + s_sum[3][tid];
}

// ---------------------------------------------------------------------------
// Weight packing ([K][N] int8 codes -> device layouts) and column scales.
// One thread per 16-byte output entry; consecutive threads read consecutive
// columns of the same k, so the reads of a wave are contiguous runs.
// ---------------------------------------------------------------------------
struct PackParams {
    const int8_t* codes;
    const float* scales;
    int K, N, K_pad, N_pad, half;
    uint8_t* out;
    float* colscale;
    unsigned* bad;  // set when a W4 code lies outside [-8, 7]
};

static __global__ __launch_bounds__(256) void pack_w8_kernel(PackParams P) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t total = (size_t)(P.K_pad / 16) * P.N_pad;
    if (idx >= total) return;
    const int p = (int)(idx % P.N_pad), kg = (int)(idx / P.N_pad);
    const int n = p < P.N ? orig_col(p, P.half) : -1;
    unsigned w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int b = 0; b < 16; ++b) {
        const int k = kg * 16 + b;
        unsigned v = (n >= 0 && k < P.K) ? (unsigned)(uint8_t)P.codes[(size_t)k * P.N + n] : 0u;
        w[b >> 2] |= v << ((b & 3) * 8);
    }
    v4u out = {w[0], w[1], w[2], w[3]};
    *reinterpret_cast<v4u*>(P.out + idx * 16) = out;
    if (kg == 0) P.colscale[p] = n >= 0 ? P.scales[n] : 0.0f;
}

static __global__ __launch_bounds__(256) void pack_w4_kernel(PackParams P) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t total = (size_t)(P.K_pad / 32) * P.N_pad;
    if (idx >= total) return;
    const int p = (int)(idx % P.N_pad), j = (int)(idx / P.N_pad);
    const int n = p < P.N ? orig_col(p, P.half) : -1;
    const int klo = 64 * (j >> 1) + 16 * (j & 1), khi = klo + 32;
    unsigned w[4] = {0u, 0u, 0u, 0u};
    unsigned bad = 0u;
#pragma unroll
    for (int b = 0; b < 16; ++b) {
        int lo = 0, hi = 0;
        if (n >= 0 && klo + b < P.K) lo = P.codes[(size_t)(klo + b) * P.N + n];
        if (n >= 0 && khi + b < P.K) hi = P.codes[(size_t)(khi + b) * P.N + n];
        bad |= (unsigned)(lo < -8 || lo > 7 || hi < -8 || hi > 7);
        const unsigned byte = (unsigned)((lo + 8) & 15) | ((unsigned)((hi + 8) & 15) << 4);
        w[b >> 2] |= byte << ((b & 3) * 8);
    }
    v4u out = {w[0], w[1], w[2], w[3]};
    *reinterpret_cast<v4u*>(P.out + idx * 16) = out;
    if (j == 0) P.colscale[p] = n >= 0 ? P.scales[n] : 0.0f;
    if (bad) atomicOr(P.bad, 1u);
}

// ---------------------------------------------------------------------------
// Prefill GEMM on MFMA: v_mfma_i32_32x32x32_i8, int32 accumulation.
// Block tile BM x BN, K step 64, WGM x WGN waves, wave tile (BM/WGM) x (BN/WGN).
// A and B tiles go global -> registers -> LDS (two stages, one barrier per
// K step); every LDS fragment read is a 16-byte read at consecutive addresses
// for each half-wave. The W4 B tile stays packed in LDS (half the bytes) and
// is unpacked in registers: one 16-byte entry feeds both 32-k MFMA steps.
// Epilogue: optional W4 offset correction, dequant (f32(acc)*s_row)*s_col,
// and plain / SwiGLU / SwiGLU+row-max stores.
// ---------------------------------------------------------------------------
struct GemmParams {
    const int8_t* a;
    const uint8_t* b;
    const float* rowscale;
    const int* rowsum;
    const float* colscale;
    void* c;
    long ldc;
    int c_type;
    int M, N, K_pad, M_alloc, N_pad, half;
    unsigned* rowmax;
    int tiles_m, tiles_n;
};

// Main loop shared by the dense and the grouped GEMM: accumulates the
// (BM x BN) tile whose A rows are given per thread by a_off (the plane-0 chunk
// index of each of the thread's A loads) and whose B panel starts at column n0
// of gb. acc must be zero on entry.
template <int BM, int BN, int WGM, int WGN, int BITS>
struct TileCfg {
    static constexpr int NT = WGM * WGN * 64;
    static constexpr int TM = BM / WGM, TN = BN / WGN;
    static constexpr int FM = TM / 32, FN = TN / 32;
    static constexpr int A_STAGE = BM * 64;
    static constexpr int B_STAGE = (BITS == 8) ? BN * 64 : BN * 32;
    static constexpr int STAGE = A_STAGE + B_STAGE;
    static constexpr int A_LOADS = A_STAGE / 16 / NT;
    static constexpr int B_LOADS = B_STAGE / 16 / NT;
    static_assert(A_STAGE % (16 * NT) == 0 && B_STAGE % (16 * NT) == 0, "tile/thread mismatch");
};

template <int BM, int BN, int WGM, int WGN, int BITS>
__device__ __forceinline__ void gemm_mainloop(uint8_t* smem, const int8_t* __restrict__ ga, size_t a_plane,
                                              const size_t (&a_off)[TileCfg<BM, BN, WGM, WGN, BITS>::A_LOADS],
                                              const uint8_t* __restrict__ gb, int N_pad, int n0, int KT,
                                              v16i (&acc)[TileCfg<BM, BN, WGM, WGN, BITS>::FM]
                                                         [TileCfg<BM, BN, WGM, WGN, BITS>::FN]) {
    using C = TileCfg<BM, BN, WGM, WGN, BITS>;
    constexpr int NT = C::NT, TM = C::TM, TN = C::TN, FM = C::FM, FN = C::FN;
    constexpr int A_STAGE = C::A_STAGE, STAGE = C::STAGE, A_LOADS = C::A_LOADS, B_LOADS = C::B_LOADS;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int half_id = lane >> 5, l32 = lane & 31;

    v4i ra[A_LOADS], rb[B_LOADS];
    auto gload = [&](int kt) {
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i)
            ra[i] = *reinterpret_cast<const v4i*>(ga + ((size_t)kt * 4 * a_plane + a_off[i]) * 16);
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) {
            const int c = tid + i * NT;
            const int kg = c / BN, col = c % BN;
            const int plane = (BITS == 8) ? kt * 4 + kg : kt * 2 + kg;
            rb[i] = *reinterpret_cast<const v4i*>(gb + ((size_t)plane * N_pad + n0 + col) * 16);
        }
    };
    auto sstore = [&](int buf) {
        uint8_t* sa = smem + buf * STAGE;
        uint8_t* sb = sa + A_STAGE;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) *reinterpret_cast<v4i*>(sa + (tid + i * NT) * 16) = ra[i];
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) *reinterpret_cast<v4i*>(sb + (tid + i * NT) * 16) = rb[i];
    };

    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) gload(kt + 1);
        const uint8_t* sa = smem + cur * STAGE;
        const uint8_t* sb = sa + A_STAGE;
        if (BITS == 8) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                v4i af[FM], bf[FN];
#pragma unroll
                for (int i = 0; i < FM; ++i)
                    af[i] = *reinterpret_cast<const v4i*>(sa + ((2 * s + half_id) * BM + wm * TM + i * 32 + l32) * 16);
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    bf[j] = *reinterpret_cast<const v4i*>(sb + ((2 * s + half_id) * BN + wn * TN + j * 32 + l32) * 16);
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        } else {
            v4u bw[FN];
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bw[j] = *reinterpret_cast<const v4u*>(sb + (half_id * BN + wn * TN + j * 32 + l32) * 16);
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                v4i af[FM];
#pragma unroll
                for (int i = 0; i < FM; ++i)
                    af[i] = *reinterpret_cast<const v4i*>(sa + ((2 * s + half_id) * BM + wm * TM + i * 32 + l32) * 16);
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const v4u nib = (s == 0) ? (bw[j] & 0x0F0F0F0Fu) : ((bw[j] >> 4) & 0x0F0F0F0Fu);
                    const v4i bf = __builtin_bit_cast(v4i, nib);
#pragma unroll
                    for (int i = 0; i < FM; ++i)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf, acc[i][j], 0, 0, 0);
                }
            }
        }
        if (kt + 1 < KT) sstore(cur ^ 1);
        __syncthreads();
    }
}

// Epilogue of a finished tile. Fragment (i, j) register r holds row
// 8*(r/4) + 4*half_id + r%4 and column l32 of its 32x32 block. row_of maps the
// tile-local row to (output row, scale row, valid).
template <int BM, int BN, int WGM, int WGN, int BITS, int EPI, typename RowMap>
__device__ __forceinline__ void gemm_epilogue(
    const v16i (&acc)[TileCfg<BM, BN, WGM, WGN, BITS>::FM][TileCfg<BM, BN, WGM, WGN, BITS>::FN], int n0,
    const float* __restrict__ rowscale, const int* __restrict__ rowsum, const float* __restrict__ colscale, int N,
    int half, void* c, long ldc, int c_type, unsigned* rowmax, RowMap row_of) {
    using C = TileCfg<BM, BN, WGM, WGN, BITS>;
    constexpr int TM = C::TM, TN = C::TN, FM = C::FM, FN = C::FN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int half_id = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int local = wm * TM + i * 32 + (r >> 2) * 8 + half_id * 4 + (r & 3);
            int out_row, src_row;
            const bool row_ok = row_of(local, out_row, src_row);
            const float s_row = rowscale[src_row];
            const int corr = (BITS == 4) ? 8 * rowsum[src_row] : 0;
            if (EPI == EPI_PLAIN) {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const int p = n0 + wn * TN + j * 32 + l32;
                    const float y = ((float)(acc[i][j][r] - corr) * s_row) * colscale[p];
                    if (row_ok && p < N) store_out(c, c_type, (size_t)out_row * ldc + orig_col(p, half), y);
                }
            } else {
                float mx = 0.0f;
#pragma unroll
                for (int j = 0; j < FN; j += 2) {
                    const int p = n0 + wn * TN + j * 32 + l32;
                    const float g = ((float)(acc[i][j][r] - corr) * s_row) * colscale[p];
                    const float u = ((float)(acc[i][j + 1][r] - corr) * s_row) * colscale[p + 32];
                    const float o = hm_swiglu(g, u);
                    mx = fmaxf(mx, fabsf(o));
                    if (row_ok && p < N) store_out(c, c_type, (size_t)out_row * ldc + ((p >> 6) << 5) + l32, o);
                }
                if (EPI == EPI_SWIGLU_MAX) {
#pragma unroll
                    for (int off = 16; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
                    if (l32 == 0 && row_ok) atomicMax(rowmax + out_row, __float_as_uint(mx));
                }
            }
        }
    }
}

template <int BM, int BN, int WGM, int WGN, int BITS, int EPI>
__global__ __launch_bounds__(WGM* WGN * 64, 1) void gemm_kernel(GemmParams P) {
    using C = TileCfg<BM, BN, WGM, WGN, BITS>;
    static_assert(EPI == EPI_PLAIN || C::FN % 2 == 0, "SwiGLU pairs need an even fragment count");
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * C::STAGE];

    // Block -> tile: give each of the 8 XCDs (blocks are dealt round-robin)
    // a contiguous range of tile ids, then walk groups of 8 M-tiles so that
    // neighbouring tiles share weight panels in the XCD's L2.
    const int T = P.tiles_m * P.tiles_n;
    const int bid = blockIdx.x;
    const int per = T >> 3;
    const int tile = (bid < (per << 3)) ? ((bid & 7) * per + (bid >> 3)) : bid;
    constexpr int G = 8;
    const int group = tile / (G * P.tiles_n);
    const int first_m = group * G;
    const int gm = min(P.tiles_m - first_m, G);
    const int in_g = tile - group * G * P.tiles_n;
    const int tm = first_m + in_g % gm;
    const int tn = in_g / gm;
    const int m0 = tm * BM, n0 = tn * BN;

    size_t a_off[C::A_LOADS];
#pragma unroll
    for (int i = 0; i < C::A_LOADS; ++i) {
        const int c = threadIdx.x + i * C::NT;
        a_off[i] = (size_t)(c / BM) * P.M_alloc + m0 + c % BM;
    }
    v16i acc[C::FM][C::FN];
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    gemm_mainloop<BM, BN, WGM, WGN, BITS>(smem, P.a, (size_t)P.M_alloc, a_off, P.b, P.N_pad, n0, P.K_pad >> 6, acc);
    const int M = P.M;
    gemm_epilogue<BM, BN, WGM, WGN, BITS, EPI>(acc, n0, P.rowscale, P.rowsum, P.colscale, P.N, P.half, P.c, P.ldc,
                                               P.c_type, P.rowmax, [&](int local, int& out_row, int& src_row) {
                                                   const int row = m0 + local;
                                                   out_row = row;
                                                   src_row = row < M ? row : 0;
                                                   return row < M;
                                               });
}

// ---------------------------------------------------------------------------
// Decode GEMV / skinny GEMM (M <= 8) without MFMA: bandwidth bound.
// Block = 4 waves over 64 packed columns and one K split; lane = column, so a
// wave's weight load is 64 x 16 contiguous bytes. The block's activation codes
// sit in LDS and are read as broadcasts. Dot products use v_dot4_i32_i8.
// With several K splits the int32 partials are added atomically into a
// per-workspace buffer; the last block of a column group (arrival counter)
// finishes the epilogue and resets buffer and counter for the next call.
// ---------------------------------------------------------------------------
struct GemvParams {
    const int8_t* a;
    const uint8_t* b;
    const float* rowscale;
    const int* rowsum;
    const float* colscale;
    void* c;
    long ldc;
    int c_type;
    int M, N, K_pad, M_alloc, N_pad, half;
    unsigned* rowmax;
    int ksplit, kg_per_split;  // kg = 64-k groups
    int* acc;                  // [8][N_pad] int32, zero between calls
    unsigned* counters;        // [N_pad/64], zero between calls
};

constexpr int GEMV_LDS_BYTES = 16384;

template <int MR, int BITS, int EPI>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams P) {
    __shared__ __attribute__((aligned(16))) int8_t sa[GEMV_LDS_BYTES];
    __shared__ int red[4][MR][64];
    __shared__ int s_last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ncg = P.N_pad >> 6;
    const int cg = blockIdx.x % ncg, split = blockIdx.x / ncg;
    const int n0 = cg * 64, p = n0 + lane;
    const int KG = P.K_pad >> 6;
    const int kg_begin = split * P.kg_per_split;
    const int kg_end = min(KG, kg_begin + P.kg_per_split);

    // Activation codes of this K split, [kg16 - 4*kg_begin][MR][16].
    const int chunks = (kg_end - kg_begin) * 4 * MR;
    for (int c = tid; c < chunks; c += 256) {
        const int kgl = c / MR, m = c % MR;
        *reinterpret_cast<v4i*>(sa + c * 16) =
            *reinterpret_cast<const v4i*>(P.a + ((size_t)(4 * kg_begin + kgl) * P.M_alloc + m) * 16);
    }
    __syncthreads();

    int acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0;
    const uint8_t* __restrict__ gb = P.b;

    if (BITS == 8) {
        const int e_begin = 4 * kg_begin, e_end = 4 * kg_end;
        auto consume = [&](const v4i w, int e) {
            const int8_t* ab = sa + (e - e_begin) * MR * 16;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const v4i a = *reinterpret_cast<const v4i*>(ab + m * 16);
                int t = acc[m];
                t = __builtin_amdgcn_sdot4(a.x, w.x, t, false);
                t = __builtin_amdgcn_sdot4(a.y, w.y, t, false);
                t = __builtin_amdgcn_sdot4(a.z, w.z, t, false);
                t = __builtin_amdgcn_sdot4(a.w, w.w, t, false);
                acc[m] = t;
            }
        };
        int e = e_begin + wave;
        for (; e + 12 < e_end; e += 16) {
            const v4i w0 = *reinterpret_cast<const v4i*>(gb + ((size_t)e * P.N_pad + p) * 16);
            const v4i w1 = *reinterpret_cast<const v4i*>(gb + ((size_t)(e + 4) * P.N_pad + p) * 16);
            const v4i w2 = *reinterpret_cast<const v4i*>(gb + ((size_t)(e + 8) * P.N_pad + p) * 16);
            const v4i w3 = *reinterpret_cast<const v4i*>(gb + ((size_t)(e + 12) * P.N_pad + p) * 16);
            consume(w0, e);
            consume(w1, e + 4);
            consume(w2, e + 8);
            consume(w3, e + 12);
        }
        for (; e < e_end; e += 4) consume(*reinterpret_cast<const v4i*>(gb + ((size_t)e * P.N_pad + p) * 16), e);
    } else {
        const int j_begin = 2 * kg_begin, j_end = 2 * kg_end;
        auto consume = [&](const v4u w, int j) {
            const v4i lo = __builtin_bit_cast(v4i, w & 0x0F0F0F0Fu);
            const v4i hi = __builtin_bit_cast(v4i, (w >> 4) & 0x0F0F0F0Fu);
            const int kga = 4 * ((j >> 1) - kg_begin) + (j & 1);
            const int8_t* aa = sa + kga * MR * 16;
            const int8_t* ab = sa + (kga + 2) * MR * 16;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const v4i x0 = *reinterpret_cast<const v4i*>(aa + m * 16);
                const v4i x1 = *reinterpret_cast<const v4i*>(ab + m * 16);
                int t = acc[m];
                t = __builtin_amdgcn_sdot4(x0.x, lo.x, t, false);
                t = __builtin_amdgcn_sdot4(x0.y, lo.y, t, false);
                t = __builtin_amdgcn_sdot4(x0.z, lo.z, t, false);
                t = __builtin_amdgcn_sdot4(x0.w, lo.w, t, false);
                t = __builtin_amdgcn_sdot4(x1.x, hi.x, t, false);
                t = __builtin_amdgcn_sdot4(x1.y, hi.y, t, false);
                t = __builtin_amdgcn_sdot4(x1.z, hi.z, t, false);
                t = __builtin_amdgcn_sdot4(x1.w, hi.w, t, false);
                acc[m] = t;
            }
        };
        int j = j_begin + wave;
        for (; j + 12 < j_end; j += 16) {
            const v4u w0 = *reinterpret_cast<const v4u*>(gb + ((size_t)j * P.N_pad + p) * 16);
            const v4u w1 = *reinterpret_cast<const v4u*>(gb + ((size_t)(j + 4) * P.N_pad + p) * 16);
            const v4u w2 = *reinterpret_cast<const v4u*>(gb + ((size_t)(j + 8) * P.N_pad + p) * 16);
            const v4u w3 = *reinterpret_cast<const v4u*>(gb + ((size_t)(j + 12) * P.N_pad + p) * 16);
            consume(w0, j);
            consume(w1, j + 4);
            consume(w2, j + 8);
            consume(w3, j + 12);
        }
        for (; j < j_end; j += 4) consume(*reinterpret_cast<const v4u*>(gb + ((size_t)j * P.N_pad + p) * 16), j);
    }

#pragma unroll
    for (int m = 0; m < MR; ++m) red[wave][m][lane] = acc[m];
    __syncthreads();
    // Wave w finishes rows w and w + 4 (every lane holds one column).
    constexpr int RPW = (MR + 3) / 4;
    int total[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int m = wave + 4 * i;
        total[i] = (m < MR) ? red[0][m][lane] + red[1][m][lane] + red[2][m][lane] + red[3][m][lane] : 0;
    }
    if (P.ksplit > 1) {
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int m = wave + 4 * i;
            if (m < MR)
                __hip_atomic_fetch_add(P.acc + (size_t)m * P.N_pad + p, total[i], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
        __threadfence();
        __syncthreads();
        if (tid == 0) {
            const unsigned prev =
                __hip_atomic_fetch_add(P.counters + cg, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            s_last = (prev == (unsigned)(P.ksplit - 1));
        }
        __syncthreads();
        if (!s_last) return;
        __threadfence();
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int m = wave + 4 * i;
            if (m < MR)
                total[i] = __hip_atomic_exchange(P.acc + (size_t)m * P.N_pad + p, 0, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
        }
        if (tid == 0) __hip_atomic_store(P.counters + cg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int m = wave + 4 * i;
        if (m >= MR) break;  // wave-uniform
        const bool row_ok = m < P.M;
        const int corr = (BITS == 4 && row_ok) ? 8 * P.rowsum[m] : 0;
        const float y = ((float)(total[i] - corr) * P.rowscale[m]) * P.colscale[p];
        if (EPI == EPI_PLAIN) {
            if (row_ok && p < P.N) store_out(P.c, P.c_type, (size_t)m * P.ldc + orig_col(p, P.half), y);
        } else {
            const float u = __shfl_xor(y, 32);
            const float o = hm_swiglu(y, u);
            if (lane < 32 && row_ok && p < P.N) store_out(P.c, P.c_type, (size_t)m * P.ldc + (n0 >> 1) + lane, o);
            if (EPI == EPI_SWIGLU_MAX) {
                float mx = lane < 32 ? fabsf(o) : 0.0f;
                mx = wave_max(mx);
                if (lane == 0 && row_ok) atomicMax(P.rowmax + m, __float_as_uint(mx));
            }
        }
    }
}

}  // namespace hm

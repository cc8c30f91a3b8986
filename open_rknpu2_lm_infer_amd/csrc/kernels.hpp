// HIP kernels of the quantized-linear hot path, written for gfx950 (CDNA4).
//
// Device data layouts (all chosen so every global access is a coalesced
// 16-byte-per-lane load and every LDS fragment read is conflict free):
//   activation codes  A8 : [K_pad/16][M_alloc][16]  int8   ("k16 planes")
//   weights              : 8-column tiles, [N_pad/8][planes][8][16] bytes,
//                          so one tile's whole K is one contiguous stream
//                          (decode) and a K step of a tile is a 512-byte
//                          (W8) or 256-byte (W4) contiguous run (prefill).
//   W8 plane             : 16 k of one column (planes = K_pad/16)
//   W4 plane j           : two offset-binary nibbles (u = code + 8) per byte;
//                          with g = j/2 and h = j%2 byte b holds
//                          k = 64g + 16h + b in the low nibble and
//                          k = 64g + 32 + 16h + b in the high nibble
//                          (planes = K_pad/32).
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

// f32 -> f16 (RNE) of a value already rounded to f32. The empty asm keeps
// the compiler from fusing the conversion with the multiply that produced v
// into one mixed-precision instruction (one rounding straight to f16, which
// differs from rounding to f32 and then to f16) where it can see the type.
__device__ __forceinline__ __half f32_to_f16(float v) {
    asm volatile("" : "+v"(v));
    return __float2half_rn(v);
}

template <int V>
struct IntTag {
    static constexpr int value = V;
};

__device__ __forceinline__ void store_out(void* c, int c_type, size_t idx, float v) {
    if (c_type == DT_F32)
        static_cast<float*>(c)[idx] = v;
    else
        static_cast<__half*>(c)[idx] = f32_to_f16(v);
}

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
    return static_cast<float>(v);
}
template <>
__device__ __forceinline__ float to_f32<__half>(__half v) {
    return __half2float(v);
}

// Cross-lane reductions on DPP moves (no LDS round trip): quad_perm
// [1,0,3,2] and [2,3,0,1] reduce lanes within a quad, row_half_mirror within
// 8 lanes, row_mirror within a 16-lane row, row_bcast:15 / row_bcast:31 carry
// row results upward so lane 63 ends with the whole wave's; lanes a move does
// not write keep their own value (the operation's identity on itself).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ int dpp_move(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, ROW_MASK, 0xf, false);
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_move(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v),
                                                                 CTRL, ROW_MASK, 0xf, false));
}
constexpr int DPP_QUAD_XOR1 = 0xB1, DPP_QUAD_XOR2 = 0x4E, DPP_ROW_HALF_MIRROR = 0x141, DPP_ROW_MIRROR = 0x140,
              DPP_ROW_BCAST15 = 0x142, DPP_ROW_BCAST31 = 0x143;

// Sum over the 8 lanes of the wave that share lane % 8, in each of them:
// row_ror:8 pairs lanes 8 apart within a 16-lane row; v_permlane16_swap /
// v_permlane32_swap exchange odd with even rows / the upper with the lower
// half, so the two halves of each swap add to the pair's sum.
__device__ __forceinline__ int sum_mod8(int v) {
    v += __builtin_amdgcn_update_dpp(v, v, 0x128, 0xf, 0xf, false);  // row_ror:8
    const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = (int)a[0] + (int)a[1];
    const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (int)b[0] + (int)b[1];
}

// max over each aligned group of 8 lanes, in every lane of the group
// A non-negative row maximum as the bits an unsigned atomic max combines
// (for non-negative floats the integer order is the float order). A NaN group
// maximum (all of its values NaN) becomes 0, as fmaxf(0, NaN) does where the
// partial maxima are combined with fmaxf instead: bits 0x7FC00000 would beat
// every finite value and +inf.
__device__ __forceinline__ unsigned max_bits(float m) { return __float_as_uint(fmaxf(m, 0.0f)); }

__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, dpp_move<DPP_QUAD_XOR1>(v));
    v = fmaxf(v, dpp_move<DPP_QUAD_XOR2>(v));
    return fmaxf(v, dpp_move<DPP_ROW_HALF_MIRROR>(v));
}

__device__ __forceinline__ int wave_sum(int v) {
    v += dpp_move<DPP_QUAD_XOR1>(v);
    v += dpp_move<DPP_QUAD_XOR2>(v);
    v += dpp_move<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_move<DPP_ROW_MIRROR>(v);
    // rows 1 and 3 add the row below; then rows 2 and 3 add row 1's total
    v += __builtin_amdgcn_update_dpp(0, v, DPP_ROW_BCAST15, 0xa, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, DPP_ROW_BCAST31, 0xc, 0xf, false);
    return __builtin_amdgcn_readlane(v, 63);
}

__device__ __forceinline__ float wave_max(float v) {
    v = max8(v);
    v = fmaxf(v, dpp_move<DPP_ROW_MIRROR>(v));
    v = fmaxf(v, dpp_move<DPP_ROW_BCAST15, 0xa>(v));
    v = fmaxf(v, dpp_move<DPP_ROW_BCAST31, 0xc>(v));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// ---------------------------------------------------------------------------
// Per-row dynamic int8 quantization: a row is owned by TPR threads (the
// whole 256-thread block, or one wave for rows of at most 64 * QUANT_CHUNKS
// chunks). Thread t owns the 16-element chunks kg = t + TPR*j of the row; every chunk load (and
// every precomputed row-max partial) is issued before the first wait, the
// row max reduces over the block (wave shuffles, then LDS), and each chunk is
// quantized from registers into one 16-byte entry of the k16-plane layout.
// ---------------------------------------------------------------------------
// 16-element chunks per thread the quantization kernel keeps in registers
// (rows up to 256 * 16 * QUANT_CHUNKS elements take no second pass).
constexpr int QUANT_CHUNKS = 3;

struct QuantParams {
    const void* x;
    int x_type;
    long lda;
    int rows, K, K_pad, M_alloc;
    int vec;  // 1 when rows are 16-byte aligned and K % 16 == 0
    int8_t* codes;
    float* rowscale;
    int* rowsum;
    const float* part_in;    // optional precomputed row maxima: max over part_in[r*part_count + i]
    int part_count;
    unsigned* rowmax_clear;  // zeroed for the block's rows (next middle's max)
    const int* rows_dev;     // optional device-side row count (<= rows)
    const int* row_map;      // optional: output row r quantizes input row row_map[r] / map_div
    int map_div;
};

// Input row of output row r (the MoE slot order: the slot's token).
__device__ __forceinline__ int quant_src_row(const QuantParams& P, int r) {
    return P.row_map ? P.row_map[r] / P.map_div : r;
}

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
// Loads through a pointer into global memory (HBM or mapped host memory),
// which every activation, weight, scale and partial pointer here is. Said at
// the load itself because a pointer the kernel reads from a device table (the
// MoE expert weights and scales) is otherwise generic: loads through it, and
// through every address selected between it and another, become flat loads,
// which count on both the vector-memory and the LDS counters, so a wait for
// any one result becomes a wait for every load in flight (the grouped decode
// GEMV waited for its rows before requesting its weights).
template <typename V>
__device__ __forceinline__ V gload(const void* p) {
    return *(const __attribute__((address_space(1))) V*)p;
}
template <typename V>
__device__ __forceinline__ V gload_nt(const void* p) {
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) V*)p);
}

// 16 activations as raw 16-byte words (2 for fp16, 4 for f32), so a load can
// be issued now and converted later without waiting on anything else.
template <typename T>
__device__ __forceinline__ void load16_raw(const T* p, v4u (&r)[4]) {
#pragma unroll
    for (int q = 0; q < (int)(16 * sizeof(T) / 16); ++q) r[q] = gload<v4u>(reinterpret_cast<const v4u*>(p) + q);
}
__device__ __forceinline__ void cvt16_raw(const v4u (&r)[4], float (&v)[16], float) {
#pragma unroll
    for (int b = 0; b < 16; ++b) v[b] = __uint_as_float(r[b >> 2][b & 3]);
}
__device__ __forceinline__ void cvt16_raw(const v4u (&r)[4], float (&v)[16], __half) {
#pragma unroll
    for (int b = 0; b < 16; ++b) {
        const unsigned bits = r[b >> 3][(b >> 1) & 3];
        v[b] = __half2float(__ushort_as_half((unsigned short)((b & 1) ? (bits >> 16) : (bits & 0xffffu))));
    }
}

// Code of one scaled value, q = clamp(round(s), +-127) with the dense rule's
// rounding (half away from zero) or the MoE rule's (half to even). Clamping
// first is equivalent (the bounds are integers). For a value already in
// [-127, 127], trunc(q + copysign(0x1.fffffep-2, q)) is exactly roundf(q):
// the sum is exact or rounds within the integer interval except at q = n - 0.5,
// where it reaches n; adding 0.5 instead would send 0x1.fffffep-2 to 1. (The
// identity is checked over every float of the range by the test suite.)
template <int RULE>
__device__ __forceinline__ int quant_code(float s) {
    const float q = fminf(fmaxf(s, -127.0f), 127.0f);
    if (RULE == QUANT_DENSE) return (int)(q + __builtin_copysignf(0x1.fffffep-2f, q));
    return (int)__builtin_rintf(q);
}

// Low bytes of four codes as one word (v_perm_b32: byte i of the result is
// byte sel_i of {second operand bytes 0-3, first operand bytes 4-7}, 0x0c
// gives zero), and the sum of a word's four signed bytes (v_dot4 with ones).
__device__ __forceinline__ unsigned pack4(int a, int b, int c, int d) {
    const unsigned ab = __builtin_amdgcn_perm((unsigned)b, (unsigned)a, 0x0c0c0400u);
    const unsigned cd = __builtin_amdgcn_perm((unsigned)d, (unsigned)c, 0x0c0c0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}
__device__ __forceinline__ int sum4(unsigned w, int acc) {
    return __builtin_amdgcn_sdot4((int)w, 0x01010101, acc, false);
}

// 16 already scaled values -> 16 int8 codes, sum += codes.
template <int RULE>
__device__ __forceinline__ v4u quant_scaled(const float (&sv)[16], int& sum) {
    unsigned packed[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        packed[w] = pack4(quant_code<RULE>(sv[4 * w]), quant_code<RULE>(sv[4 * w + 1]), quant_code<RULE>(sv[4 * w + 2]),
                          quant_code<RULE>(sv[4 * w + 3]));
        sum = sum4(packed[w], sum);
    }
    return v4u{packed[0], packed[1], packed[2], packed[3]};
}

// 16 values -> 16 int8 codes of v * inv, sum += codes.
template <int RULE>
__device__ __forceinline__ v4u quant_chunk(const float (&v)[16], float inv, int& sum) {
    float sv[16];
#pragma unroll
    for (int b = 0; b < 16; ++b) sv[b] = v[b] * inv;
    return quant_scaled<RULE>(sv, sum);
}

// v * inv for 16 raw activations: f32 as is; fp16 through v_fma_mix_f32, the
// conversion folded into the multiply: fma(h, inv, -0) is the product rounded
// once, exactly h * inv (the -0 addend keeps signed zeros; it is held in a
// register the compiler cannot see through, or it would fold the fma back
// into a convert and a multiply).
__device__ __forceinline__ void scale16_raw(const v4u (&r)[4], float inv, float (&sv)[16], float) {
#pragma unroll
    for (int b = 0; b < 16; ++b) sv[b] = __uint_as_float(r[b >> 2][b & 3]) * inv;
}
__device__ __forceinline__ void scale16_raw(const v4u (&r)[4], float inv, float (&sv)[16], __half) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    float nz;
    asm volatile("v_mov_b32 %0, 0x80000000" : "=v"(nz));
#pragma unroll
    for (int b = 0; b < 16; ++b) {
        // (the word is copied out first: __builtin_bit_cast of a vector-element
        // lvalue reads the vector's first word whatever the element index)
        const unsigned word = r[b >> 3][(b >> 1) & 3];
        const h2 pair = __builtin_bit_cast(h2, word);
        sv[b] = __builtin_fmaf((float)pair[b & 1], inv, nz);
    }
}

template <int RULE>
__device__ __forceinline__ float quant_scale(float m) {
    if (RULE == QUANT_DENSE) return (m == 0.0f) ? 1.0f : fmaxf(m / 127.0f, FLT_MIN);
    return (m == 0.0f) ? 1.0f : m / 127.0f;
}

template <typename T, int RULE, int TPR>
__global__ __launch_bounds__(256) void quant_rows_kernel(QuantParams P) {
    constexpr int J = QUANT_CHUNKS;  // chunks per thread held in registers
    constexpr int PV = 8;            // row-max partials per thread held in registers
    __shared__ float s_max[4];
    __shared__ int s_sum[4];
    const T* x = static_cast<const T*>(P.x);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tid = threadIdx.x % TPR;  // thread within its row
    const int r = blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
    const int rows = P.rows_dev ? min(P.rows, *P.rows_dev) : P.rows;
    if (P.rowmax_clear && tid == 0 && r < P.M_alloc) P.rowmax_clear[r] = 0u;
    if (r >= rows) return;  // uniform over the row's threads (a block or a wave)
    const int KG = P.K_pad >> 4;
    const T* xr = x + (size_t)quant_src_row(P, r) * P.lda;
    // 1. Issue every load (no branches around them: masked-off lanes re-read
    // the row start), then reduce.
    // (a masked-off chunk re-reads the row's first chunk, which aligned rows
    // always have; unaligned rows read a 16-byte-aligned workspace word)
    const T* dummy = P.vec ? xr : reinterpret_cast<const T*>(P.rowscale);
    v4u raw[J][4];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int kg = tid + TPR * j;
        const bool ok = P.vec && kg * 16 < P.K;
        load16_raw(ok ? xr + kg * 16 : dummy, raw[j]);
    }
    float pv[PV];
    const float* pr = P.part_in ? P.part_in + (size_t)r * P.part_count : P.rowscale;
#pragma unroll
    for (int i = 0; i < PV; ++i) {
        const int idx = tid + TPR * i;
        pv[i] = pr[(P.part_in && idx < P.part_count) ? idx : 0];  // masked at use
    }
    asm volatile("" ::: "memory");
    // Chunk j as 16 floats (zero past K; scalar reads when rows are unaligned).
    auto chunk = [&](int j, float (&v)[16]) {
        const int kg = tid + TPR * j;
        if (P.vec) {
            cvt16_raw(raw[j], v, T());
#pragma unroll
            for (int b = 0; b < 16; ++b) v[b] = (kg * 16 < P.K) ? v[b] : 0.0f;
        } else {
#pragma unroll
            for (int b = 0; b < 16; ++b) v[b] = (kg * 16 + b < P.K) ? to_f32(xr[kg * 16 + b]) : 0.0f;
        }
    };
    float m = 0.0f;
    if (P.part_in) {
#pragma unroll
        for (int i = 0; i < PV; ++i)
            if (tid + TPR * i < P.part_count) m = fmaxf(m, pv[i]);
        for (int i = tid + TPR * PV; i < P.part_count; i += TPR) m = fmaxf(m, pr[i]);
    } else {
#pragma unroll
        for (int j = 0; j < J; ++j) {
            if (tid + TPR * j >= KG) continue;
            float v[16];
            chunk(j, v);
#pragma unroll
            for (int b = 0; b < 16; ++b) m = fmaxf(m, fabsf(v[b]));
        }
        for (int kg = tid + TPR * J; kg < KG; kg += TPR)  // rows longer than 16 * TPR * J elements
#pragma unroll
            for (int b = 0; b < 16; ++b)
                if (kg * 16 + b < P.K) m = fmaxf(m, fabsf(to_f32(xr[kg * 16 + b])));
    }
    m = wave_max(m);
    if (TPR == 256) {
        if (lane == 0) s_max[wave] = m;
        __syncthreads();
        m = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
    }
    const float sc = quant_scale<RULE>(m);
    const float inv = 1.0f / sc;
    if (tid == 0) P.rowscale[r] = sc;

    // 2. Quantize each chunk into its 16-byte entry.
    int sum = 0;
    auto quantize = [&](int kg, const float (&v)[16]) {
        *reinterpret_cast<v4u*>(P.codes + ((size_t)kg * P.M_alloc + r) * 16) = quant_chunk<RULE>(v, inv, sum);
    };
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int kg = tid + TPR * j;
        if (kg >= KG) continue;
        float v[16];
        chunk(j, v);
        quantize(kg, v);
    }
    for (int kg = tid + TPR * J; kg < KG; kg += TPR) {
        float v[16];
#pragma unroll
        for (int b = 0; b < 16; ++b) v[b] = (kg * 16 + b < P.K) ? to_f32(xr[kg * 16 + b]) : 0.0f;
        quantize(kg, v);
    }
    sum = wave_sum(sum);
    if (TPR == 256) {
        if (lane == 0) s_sum[wave] = sum;
        __syncthreads();
        sum = s_sum[0] + s_sum[1] + s_sum[2] + s_sum[3];
    }
    if (tid == 0) P.rowsum[r] = sum;
}

// Row-tiled quantization for many rows: a block quantizes RB rows, 256/RB
// threads per row, and writes the code planes [K_pad/16][M_alloc][16] as
// RB*16-byte runs (one plane of its RB rows) through an LDS transpose, instead
// of one 16-byte entry per cache line. Loads stay contiguous along each row.
// The row max comes from precomputed maxima (HAS_MAX, any K: one streaming
// pass, NI groups of loads in flight) or from the row itself, held in
// registers (at most NI groups of 256/RB chunks). Values and rounding are
// those of quant_rows_kernel. Needs 16-byte aligned rows with K % 16 == 0.
template <typename T, int RULE, int RB, int NI, bool HAS_MAX>
__global__ __launch_bounds__(256) void quant_tile_kernel(QuantParams P) {
    constexpr int TW = 256 / RB;    // threads (chunk columns) per row
    constexpr int PITCH = RB + 1;   // LDS entries per chunk column (padding against bank conflicts)
    __shared__ v4u s_codes[2][TW * PITCH];
    const T* x = static_cast<const T*>(P.x);
    const int t = threadIdx.x;
    const int ri = t / TW, cg = t % TW;  // row in block, chunk column
    const int r0 = blockIdx.x * RB, r = r0 + ri;
    const int rows = P.rows_dev ? min(P.rows, *P.rows_dev) : P.rows;
    if (r0 >= rows) {
        if (P.rowmax_clear && cg == 0 && r < P.M_alloc) P.rowmax_clear[r] = 0u;
        return;  // uniform over the block
    }
    const bool live = r < rows;
    const int KG = P.K_pad >> 4;
    const int groups = (KG + TW - 1) / TW;
    const T* xr = x + (size_t)quant_src_row(P, live ? r : r0) * P.lda;
    auto ok = [&](int kg) { return live && kg * 16 < P.K; };

    float m = 0.0f;
    v4u raw[NI][4];
    if (HAS_MAX) {
        const float* pr = P.part_in + (size_t)(live ? r : r0) * P.part_count;
        for (int i = cg; i < P.part_count; i += TW) m = fmaxf(m, pr[i]);
    } else {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int kg = i * TW + cg;
            load16_raw(ok(kg) ? xr + kg * 16 : xr, raw[i]);
        }
        asm volatile("" ::: "memory");
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int kg = i * TW + cg;
            if (!ok(kg)) continue;
            float v[16];
            cvt16_raw(raw[i], v, T());
#pragma unroll
            for (int b = 0; b < 16; ++b) m = fmaxf(m, fabsf(v[b]));
        }
    }
    if constexpr (TW == 64) {
        m = wave_max(m);
    } else {
#pragma unroll
        for (int off = TW / 2; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    }
    if (P.rowmax_clear && cg == 0) P.rowmax_clear[r] = 0u;
    const float sc = quant_scale<RULE>(m);
    const float inv = 1.0f / sc;
    int sum = 0;
    // Group g: chunk g*TW+cg of every row -> LDS -> TW planes of RB rows.
    auto emit = [&](int g, float (&v)[16]) {
        const int kg = g * TW + cg;
        if (!ok(kg)) {
#pragma unroll
            for (int b = 0; b < 16; ++b) v[b] = 0.0f;
        }
        v4u* buf = s_codes[g & 1];
        buf[cg * PITCH + ri] = quant_chunk<RULE>(v, inv, sum);
        __syncthreads();
        // thread t stores plane t / RB of row t % RB
        const int pk = g * TW + t / RB;
        if (pk < KG)
            *reinterpret_cast<v4u*>(P.codes + ((size_t)pk * P.M_alloc + r0 + t % RB) * 16) =
                buf[(t / RB) * PITCH + t % RB];
    };
    if constexpr (HAS_MAX) {
        // batches of NI groups: all of a batch's loads are issued first
        for (int g0 = 0; g0 < groups; g0 += NI) {
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int kg = (g0 + i) * TW + cg;
                load16_raw(ok(kg) ? xr + kg * 16 : xr, raw[i]);
            }
            asm volatile("" ::: "memory");
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                if (g0 + i >= groups) break;
                float v[16];
                cvt16_raw(raw[i], v, T());
                emit(g0 + i, v);
            }
        }
    } else {
#pragma unroll
        for (int g = 0; g < NI; ++g) {
            if (g >= groups) break;
            float v[16];
            cvt16_raw(raw[g], v, T());
            emit(g, v);
        }
    }
    if constexpr (TW == 64) {
        sum = wave_sum(sum);
    } else {
#pragma unroll
        for (int off = TW / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    }
    if (live && cg == 0) {
        P.rowscale[r] = sc;
        P.rowsum[r] = sum;
    }
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

// Thread i handles plane pl of packed column p (consecutive threads walk
// consecutive columns of one plane, so the [K][N] reads are contiguous) and
// stores that 16-byte entry at its tile position.
static __global__ __launch_bounds__(256) void pack_w8_kernel(PackParams P) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int planes = P.K_pad / 16;
    const size_t total = (size_t)planes * P.N_pad;
    if (idx >= total) return;
    const int p = (int)(idx % P.N_pad), pl = (int)(idx / P.N_pad);
    const int n = p < P.N ? orig_col(p, P.half) : -1;
    unsigned w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int b = 0; b < 16; ++b) {
        const int k = pl * 16 + b;
        unsigned v = (n >= 0 && k < P.K) ? (unsigned)(uint8_t)P.codes[(size_t)k * P.N + n] : 0u;
        w[b >> 2] |= v << ((b & 3) * 8);
    }
    v4u out = {w[0], w[1], w[2], w[3]};
    const size_t dst = (((size_t)(p >> 3) * planes + pl) * 8 + (p & 7)) * 16;
    *reinterpret_cast<v4u*>(P.out + dst) = out;
    if (pl == 0) P.colscale[p] = n >= 0 ? P.scales[n] : 0.0f;
}

static __global__ __launch_bounds__(256) void pack_w4_kernel(PackParams P) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int planes = P.K_pad / 32;
    const size_t total = (size_t)planes * P.N_pad;
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
    const size_t dst = (((size_t)(p >> 3) * planes + j) * 8 + (p & 7)) * 16;
    *reinterpret_cast<v4u*>(P.out + dst) = out;
    if (j == 0) P.colscale[p] = n >= 0 ? P.scales[n] : 0.0f;
    if (bad) atomicOr(P.bad, 1u);
}

// Packing straight from checkpoint storage (the fused matrix's parts along
// N): pack-quantized int32 words [n][ceil(k*bits/32)] holding code + 2^(bits-1)
// in consecutive bit fields, or int-quantized int8 codes [n][k]. Column n of
// the fused matrix is column n - start of the part containing it.
constexpr int CKPT_MAX_PARTS = 8;
struct CkptPart {
    const void* data;
    const float* scales;
    int start, n, format, words;  // words per row (pack-quantized)
};
struct CkptParams {
    CkptPart part[CKPT_MAX_PARTS];
    int count, bits, K, N, K_pad, N_pad, half;
    uint8_t* out;
    float* colscale;
};

// Code field of (k, column n) in the unpacked offset form u = code + 2^(bits-1).
__device__ __forceinline__ unsigned ckpt_field(const CkptParams& P, const CkptPart& q, int n, int k) {
    if (q.format == 1) return (unsigned)((int)static_cast<const int8_t*>(q.data)[(size_t)n * P.K + k] + 128) & 0xffu;
    const int f = 32 / P.bits;
    const unsigned w = static_cast<const unsigned*>(q.data)[(size_t)n * q.words + k / f];
    return (w >> ((k % f) * P.bits)) & ((1u << P.bits) - 1u);
}

// One thread per 16-byte tile entry, as pack_w8_kernel / pack_w4_kernel:
// W8 stores codes (u - 128), W4 the offset nibbles u as they are.
static __global__ __launch_bounds__(256) void pack_ckpt_kernel(CkptParams P) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int planes = P.bits == 8 ? P.K_pad / 16 : P.K_pad / 32;
    if (idx >= (size_t)planes * P.N_pad) return;
    const int p = (int)(idx % P.N_pad), j = (int)(idx / P.N_pad);
    const int n = p < P.N ? orig_col(p, P.half) : -1;
    int qi = 0;
    for (int i = 1; i < P.count; ++i) qi = (n >= P.part[i].start) ? i : qi;
    const CkptPart& q = P.part[qi];
    const int ln = n - q.start;
    unsigned w[4] = {0u, 0u, 0u, 0u};
    if (P.bits == 8) {
#pragma unroll
        for (int b = 0; b < 16; ++b) {
            const int k = j * 16 + b;
            const unsigned v = (n >= 0 && k < P.K) ? ((ckpt_field(P, q, ln, k) - 128u) & 0xffu) : 0u;
            w[b >> 2] |= v << ((b & 3) * 8);
        }
    } else {
        const int klo = 64 * (j >> 1) + 16 * (j & 1), khi = klo + 32;
#pragma unroll
        for (int b = 0; b < 16; ++b) {
            const unsigned lo = (n >= 0 && klo + b < P.K) ? ckpt_field(P, q, ln, klo + b) : 8u;
            const unsigned hi = (n >= 0 && khi + b < P.K) ? ckpt_field(P, q, ln, khi + b) : 8u;
            w[b >> 2] |= (lo | (hi << 4)) << ((b & 3) * 8);
        }
    }
    const size_t dst = (((size_t)(p >> 3) * planes + j) * 8 + (p & 7)) * 16;
    *reinterpret_cast<v4u*>(P.out + dst) = v4u{w[0], w[1], w[2], w[3]};
    if (j == 0) P.colscale[p] = n >= 0 ? q.scales[ln] : 0.0f;
}

// ---------------------------------------------------------------------------
// Prefill GEMM on MFMA: v_mfma_i32_32x32x32_i8, int32 accumulation.
// Block tile BM x BN, K step 64, WGM x WGN waves, wave tile (BM/WGM) x (BN/WGN).
// The W4 B tile stays packed in LDS (half the bytes) and is unpacked in
// registers: one 16-byte entry feeds both 32-k MFMA steps.
// Epilogue: optional W4 offset correction, dequant (f32(acc)*s_row)*s_col,
// and plain / SwiGLU / SwiGLU+row-max stores.
// Split-K (see gemm_kernel's SPLIT modes): integer sums are exact, so the
// output does not depend on the split.
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
    int splits;       // K pieces per tile (1: no split)
    int* split_part;  // [splits][tiles][BM*BN] int32 partials
};

// Main loop shared by the dense and the grouped GEMM: accumulates the
// (BM x BN) tile whose A rows are given per thread by a_off (the plane-0 chunk
// index of each of the thread's A loads) and whose B panel starts at column n0
// of gb. acc must be zero on entry.
//
// Pipeline: STAGES LDS buffers filled by direct global->LDS loads
// (global_load_lds_dwordx4: each lane's 16 bytes land at base + 16*lane, no
// staging registers), STAGES-1 of them in flight while one stage is
// multiplied. Each wave waits only for its own loads of the next stage (vmcnt
// counts the later stages still in flight) and one barrier per stage makes
// every wave's loads visible. Fragments are double-buffered in registers: the
// next stage is read from LDS while the MFMAs of the current one run. LDS
// keeps the fragment order A [k16 plane][BM][16] and B [plane][BN][16], so
// every fragment read is 16 consecutive bytes per lane for 32 consecutive
// lanes.
template <int BM, int BN, int WGM, int WGN, int BITS>
struct TileCfg {
    static constexpr int NT = WGM * WGN * 64;
    static constexpr int TM = BM / WGM, TN = BN / WGN;
    static constexpr int FM = TM / 32, FN = TN / 32;
    static constexpr int A_STAGE = BM * 64;
    static constexpr int B_STAGE = (BITS == 8) ? BN * 64 : BN * 32;
    static constexpr int STAGE = A_STAGE + B_STAGE;
    // A rounds of NT 16-byte chunks; when BM * 4 chunks are not a whole
    // number of rounds (BM = 192), only the first A_LAST_WAVES waves load in
    // the last A round, so those waves issue LPS loads per stage and the
    // others LPS - 1.
    static constexpr int A_CHUNKS = A_STAGE / 16;
    static constexpr int A_LOADS = (A_CHUNKS + NT - 1) / NT;
    static constexpr bool A_SPLIT = A_CHUNKS % NT != 0;
    static constexpr int A_LAST_WAVES = (A_CHUNKS - (A_LOADS - 1) * NT) / 64;
    static constexpr int B_LOADS = B_STAGE / 16 / NT;
    static constexpr int LPS = A_LOADS + B_LOADS;
    static constexpr int LPS_LO = A_SPLIT ? LPS - 1 : LPS;
    // as many stages as fit in 128 KB of LDS, at most 4
    static constexpr int STAGES = (4 * STAGE <= 131072) ? 4 : (3 * STAGE <= 131072 ? 3 : 2);
    static constexpr int LDS = STAGES * STAGE;
    // Shared memory of a block: the stage ring, or the epilogue's staging of
    // 32 rows per wave (f32, worst case) when that is larger.
    static constexpr int EPI_ROW = TN * 4 + 16;
    static constexpr int SMEM = LDS > WGM * WGN * 32 * EPI_ROW ? LDS : WGM * WGN * 32 * EPI_ROW;
    static_assert(A_CHUNKS % 64 == 0 && B_STAGE % (16 * NT) == 0, "tile/thread mismatch");
    static_assert(BN % 64 == 0, "a wave's B loads must cover one plane");
    static_assert(LPS * (STAGES - 1) <= 63, "vmcnt range");
};

// 16-byte direct global->LDS load: lane l's bytes land at lds + 16*l.
__device__ __forceinline__ void lds_dma16(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// s_waitcnt through the builtin (not inline asm) so that the compiler's own
// wait insertion sees it. gfx9 encoding: vmcnt[3:0] bits 3:0, expcnt bits 6:4,
// lgkmcnt bits 11:8, vmcnt[5:4] bits 15:14; a field at its maximum waits for
// nothing.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4)); }

template <int BM, int BN, int WGM, int WGN, int BITS>
__device__ __forceinline__ void gemm_mainloop(uint8_t* smem, const int8_t* __restrict__ ga, size_t a_plane,
                                              const size_t (&a_off)[TileCfg<BM, BN, WGM, WGN, BITS>::A_LOADS],
                                              const uint8_t* __restrict__ gb, int K_pad, int n0, int KT,
                                              v16i (&acc)[TileCfg<BM, BN, WGM, WGN, BITS>::FM]
                                                         [TileCfg<BM, BN, WGM, WGN, BITS>::FN]) {
    using C = TileCfg<BM, BN, WGM, WGN, BITS>;
    constexpr int NT = C::NT, TM = C::TM, TN = C::TN, FM = C::FM, FN = C::FN;
    constexpr int A_STAGE = C::A_STAGE, STAGE = C::STAGE, A_LOADS = C::A_LOADS, B_LOADS = C::B_LOADS;
    constexpr int S = C::STAGES, LPS = C::LPS;
    constexpr int PPS = (BITS == 8) ? 4 : 2;  // weight planes per 64-k step
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int half_id = lane >> 5, l32 = lane & 31;
    const int planes = (BITS == 8) ? K_pad / 16 : K_pad / 32;

    // B chunk c (LDS order [plane][BN][16]) of this thread's i-th load.
    size_t b_src[B_LOADS];
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
        const int c = tid + i * NT;
        const int pl = c / BN, n = c % BN;
        b_src[i] = ((size_t)(n0 / 8 + n / 8) * planes + pl) * 128 + (n % 8) * 16;
    }

    // Fragment registers of one stage, flattened: f < 2*FM is A[s][i] (32-k
    // half s, row block i); then B[h][j] for both halves (W8) or the packed
    // plane whose two nibbles give both halves (W4).
    constexpr int BH = (BITS == 8) ? 2 : 1;
    constexpr int NF = 2 * FM + BH * FN;
    constexpr int T = 2 * FM * FN;           // MFMAs per stage
    // issue groups per stage: one per 2 MFMAs on the 16-MFMA stages of the
    // 256x256 tile (o 4096x2560 63.6 -> 60.9 us, down 9728x2560 154.7 ->
    // 148.6 us at M=4096 against one per 4), one per 4 MFMAs otherwise
    // (finer groups left the 128x128 tiles unchanged or slower)
    constexpr int G = T >= 16 ? T / 2 : (T >= 4 ? T / 4 : 1);
    const int a_lane = (half_id * BM + wm * TM + l32) * 16;
    const int b_lane = (half_id * BN + wn * TN + l32) * 16;

    // Load d of a stage (A loads first), fragment read f, MFMA t: all indices
    // are compile-time constants after unrolling. In the last A round of a
    // split A stage the waves past A_LAST_WAVES have no chunk (a uniform
    // branch), and wait_own waits for each wave's own count.
    auto issue1 = [&](int d, int kt_, int buf) {
        uint8_t* sa = smem + buf * STAGE;
        if (d < A_LOADS) {
            if (!C::A_SPLIT || d < A_LOADS - 1 || wave < C::A_LAST_WAVES)
                lds_dma16(ga + ((size_t)kt_ * 4 * a_plane + a_off[d]) * 16, sa + (d * NT + wave * 64) * 16);
        } else
            lds_dma16(gb + b_src[d - A_LOADS] + (size_t)kt_ * (PPS * 128),
                      sa + A_STAGE + ((d - A_LOADS) * NT + wave * 64) * 16);
    };
    auto wait_own = [&](auto stages) {
        constexpr int n = decltype(stages)::value;
        if constexpr (C::A_SPLIT) {
            if (wave < C::A_LAST_WAVES)
                wait_vmcnt<LPS * n>();
            else
                wait_vmcnt<C::LPS_LO * n>();
        } else {
            wait_vmcnt<LPS * n>();
        }
    };
    auto read1 = [&](int f, int buf) -> v4i {
        const uint8_t* r = smem + buf * STAGE;
        if (f < 2 * FM) return *reinterpret_cast<const v4i*>(r + a_lane + (2 * (f / FM) * BM + (f % FM) * 32) * 16);
        const int h = (f - 2 * FM) / FN, j = (f - 2 * FM) % FN;
        return *reinterpret_cast<const v4i*>(r + A_STAGE + b_lane + (2 * h * BN + j * 32) * 16);
    };
    auto mfma1 = [&](int t, const v4i(&c)[NF]) {
        const int s2 = t / (FM * FN), i = (t / FN) % FM, j = t % FN;
        v4i bf;
        if (BITS == 8) {
            bf = c[2 * FM + s2 * FN + j];
        } else {
            const v4u raw = __builtin_bit_cast(v4u, c[2 * FM + j]);
            bf = __builtin_bit_cast(v4i, s2 == 0 ? (raw & 0x0F0F0F0Fu) : ((raw >> 4) & 0x0F0F0F0Fu));
        }
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(c[s2 * FM + i], bf, acc[i][j], 0, 0, 0);
    };

    // Prologue: stages 0..S-1 in flight, stage 0 read into registers.
#pragma unroll
    for (int st = 0; st < S; ++st)
        if (st < KT)
#pragma unroll
            for (int d = 0; d < LPS; ++d) issue1(d, st, st);
    if (KT >= S)
        wait_own(IntTag<S - 1>{});
    else
        wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    v4i cur[NF], nxt[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) cur[f] = read1(f, 0);

    // Iteration kt: stage kt is in registers (or arriving). Once every wave
    // holds its fragments and its own loads of stage kt+1 have landed, one
    // barrier frees buffer kt%S for stage kt+S and publishes stage kt+1. The
    // loads of stage kt+S and the fragment reads of stage kt+1 (into the other
    // register set) are then spread over G groups of the stage's MFMAs, so
    // the load path and the LDS stay busy while the matrix cores run. Past the
    // last stage the read is stale and unused.
#define HM_STAGE(kt_, C_, N_)                                                                     \
    do {                                                                                          \
        wait_lgkmcnt0();                                                                          \
        if ((kt_) + 1 < KT) {                                                                     \
            if ((kt_) + S - 1 < KT)                                                               \
                wait_own(IntTag<S - 2>{});                                                        \
            else                                                                                  \
                wait_vmcnt<0>();                                                                  \
        }                                                                                         \
        __builtin_amdgcn_s_barrier();                                                             \
        asm volatile("" ::: "memory");                                                            \
        const bool iss_ = (kt_) + S < KT;                                                         \
        const int nbuf_ = ((kt_) + 1) % S, ibuf_ = (kt_) % S;                                     \
        _Pragma("unroll") for (int g = 0; g < G; ++g) {                                           \
            __builtin_amdgcn_sched_barrier(0);                                                    \
            if (iss_)                                                                             \
                _Pragma("unroll") for (int d = g * LPS / G; d < (g + 1) * LPS / G; ++d)           \
                    issue1(d, (kt_) + S, ibuf_);                                                  \
            _Pragma("unroll") for (int f = g * NF / G; f < (g + 1) * NF / G; ++f)                 \
                N_[f] = read1(f, nbuf_);                                                          \
            __builtin_amdgcn_sched_barrier(0);                                                    \
            _Pragma("unroll") for (int t = g * T / G; t < (g + 1) * T / G; ++t) mfma1(t, C_);     \
        }                                                                                         \
        __builtin_amdgcn_sched_barrier(0);                                                        \
    } while (0)

    // Pairs of stages ping-pong between the two register sets; an odd last
    // stage runs after the loop (a conditional second stage inside the loop
    // makes the compiler spill the accumulators).
    int kt = 0;
    for (; kt + 1 < KT; kt += 2) {
        HM_STAGE(kt, cur, nxt);
        HM_STAGE(kt + 1, nxt, cur);
    }
    if (kt < KT) HM_STAGE(kt, cur, nxt);
#undef HM_STAGE
}

// Per-thread values the epilogue needs from HBM, requested before the main
// loop so they have long arrived when it ends: the row scale and W4 code-sum
// correction of tile row threadIdx.x, and the column scales of this lane's
// fragment columns.
template <int BM, int BN, int WGM, int WGN, int BITS>
struct EpiPre {
    float rs;
    int rc;
    float cs[TileCfg<BM, BN, WGM, WGN, BITS>::FN];
};

template <int BM, int BN, int WGM, int WGN, int BITS, typename RowMap>
__device__ __forceinline__ EpiPre<BM, BN, WGM, WGN, BITS> epilogue_prefetch(const float* __restrict__ rowscale,
                                                                         const int* __restrict__ rowsum,
                                                                         const float* __restrict__ colscale, int n0,
                                                                         RowMap row_of) {
    using C = TileCfg<BM, BN, WGM, WGN, BITS>;
    static_assert(BM <= C::NT, "one tile row per thread");
    EpiPre<BM, BN, WGM, WGN, BITS> pre;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wn = wave % WGN;
    int out_row, src_row;
    const int local = threadIdx.x < BM ? threadIdx.x : 0;
    row_of(local, out_row, src_row);
    pre.rs = rowscale[src_row];
    pre.rc = (BITS == 4) ? 8 * rowsum[src_row] : 0;
#pragma unroll
    for (int j = 0; j < C::FN; ++j) pre.cs[j] = colscale[n0 + wn * C::TN + j * 32 + (lane & 31)];
    return pre;
}

// Epilogue of a finished tile: dequantize (two RNE multiplies, row scale then
// column scale), optional SwiGLU with the row max of |out| for the next
// quantization, and the store.
template <int BM, int BN, int WGM, int WGN, int BITS, int EPI, bool STAGED, typename RowMap>
__device__ __forceinline__ void gemm_epilogue(
    const v16i (&acc)[TileCfg<BM, BN, WGM, WGN, BITS>::FM][TileCfg<BM, BN, WGM, WGN, BITS>::FN], int n0,
    const EpiPre<BM, BN, WGM, WGN, BITS>& pre, int N, int half, void* c, long ldc, int c_type, unsigned* rowmax,
    RowMap row_of, uint8_t* smem) {
    using C = TileCfg<BM, BN, WGM, WGN, BITS>;
    constexpr int TM = C::TM, TN = C::TN, FM = C::FM, FN = C::FN, NW = WGM * WGN;
    __shared__ float s_rs[BM];
    __shared__ int s_rc[BM];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int half_id = lane >> 5, l32 = lane & 31;
    // Output columns this wave owns (SwiGLU: TN/2, contiguous from out0).
    constexpr int OUTC = (EPI == EPI_PLAIN) ? TN : TN / 2;
    const int out0 = (EPI == EPI_PLAIN) ? n0 + wn * TN : (n0 + wn * TN) >> 1;
    const int n_out = (EPI == EPI_PLAIN) ? N : N / 2;

    // STAGED (the output has a 16-byte aligned base and row pitch): rows are
    // staged through LDS in f32 (SwiGLU: the row max is taken on exact
    // values) and written as 16-byte runs, fp16 outputs converted from the
    // staged f32 values there. Otherwise each lane stores its own elements.
    // Values and rounding (f32, then f32 -> fp16) are identical either way.
    // Where registers allow (W8, or one row fragment per wave) a fragment's
    // 16 row scales (and W4 corrections) are read from LDS at once, so no
    // value waits on its own LDS read; with one block per CU (small M)
    // nothing else hides those waits. (The W4 tiles of two row fragments per
    // wave would lose a resident block to the registers; their epilogue runs
    // under other blocks' main loops.)
    constexpr bool staged = STAGED;
    constexpr bool BATCH = (BITS == 8) || (FM == 1);
    constexpr int WAVE_LDS = C::SMEM / NW;
    constexpr int FIT = WAVE_LDS / (32 * (OUTC * 4 + 16));
    static_assert(FIT >= 1, "epilogue staging does not fit in LDS");
    constexpr int FPI = FIT >= FM ? FM : ((FIT >= 2 && FM % 2 == 0) ? 2 : 1);
    constexpr int pitch = OUTC * 4 + 16;
    uint8_t* wl = smem + wave * WAVE_LDS;
    if (threadIdx.x < BM) {
        s_rs[threadIdx.x] = pre.rs;
        s_rc[threadIdx.x] = pre.rc;
    }
    __syncthreads();

#pragma unroll
    for (int i0 = 0; i0 < FM; i0 += FPI) {
#pragma unroll
        for (int ii = 0; ii < FPI; ++ii) {
            const int i = i0 + ii;
            float srow[BATCH ? 16 : 1];
            int scorr[BATCH ? 16 : 1];
            if constexpr (BATCH) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int local = wm * TM + i * 32 + (r >> 2) * 8 + half_id * 4 + (r & 3);
                    srow[r] = s_rs[local];
                    scorr[r] = (BITS == 4) ? s_rc[local] : 0;
                }
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rr = (r >> 2) * 8 + half_id * 4 + (r & 3);
                const int local = wm * TM + i * 32 + rr;
                uint8_t* lrow = wl + (ii * 32 + rr) * pitch;
                const float s_row = BATCH ? srow[BATCH ? r : 0] : s_rs[local];
                const int corr = BATCH ? scorr[BATCH ? r : 0] : s_rc[local];
                if (EPI == EPI_PLAIN) {
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        const float y = ((float)(acc[i][j][r] - corr) * s_row) * pre.cs[j];
                        if constexpr (staged) {
                            reinterpret_cast<float*>(lrow)[j * 32 + l32] = y;
                        } else {
                            const int p = n0 + wn * TN + j * 32 + l32;
                            int out_row, src_row;
                            if (row_of(local, out_row, src_row) && p < N)
                                store_out(c, c_type, (size_t)out_row * ldc + orig_col(p, half), y);
                        }
                    }
                } else {
                    float mx = 0.0f;
#pragma unroll
                    for (int j = 0; j < FN; j += 2) {
                        const float g = ((float)(acc[i][j][r] - corr) * s_row) * pre.cs[j];
                        const float u = ((float)(acc[i][j + 1][r] - corr) * s_row) * pre.cs[j + 1];
                        const float o = hm_swiglu(g, u);
                        if constexpr (staged) {
                            reinterpret_cast<float*>(lrow)[(j >> 1) * 32 + l32] = o;
                        } else {
                            const int p = n0 + wn * TN + j * 32 + l32;
                            mx = fmaxf(mx, fabsf(o));
                            int out_row, src_row;
                            if (row_of(local, out_row, src_row) && p < N)
                                store_out(c, c_type, (size_t)out_row * ldc + ((p >> 6) << 5) + l32, o);
                        }
                    }
                    if constexpr (EPI == EPI_SWIGLU_MAX && !staged) {
#pragma unroll
                        for (int off = 16; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
                        int out_row, src_row;
                        if (l32 == 0 && row_of(local, out_row, src_row)) atomicMax(rowmax + out_row, max_bits(mx));
                    }
                }
            }
        }
        if constexpr (!staged) continue;
        __syncthreads();
        if (EPI == EPI_PLAIN) {
            // 16-byte runs: chunk q of the staged rows -> (row, 16/esz columns).
            auto runs = [&](auto per_tag) {
                constexpr int per = decltype(per_tag)::value, cpr = OUTC / per;
                for (int q = lane; q < FPI * 32 * cpr; q += 64) {
                    const int lr = q / cpr, cc = (q - lr * cpr) * per;
                    int out_row, src_row;
                    if (!row_of(wm * TM + i0 * 32 + lr, out_row, src_row)) continue;
                    const int p = out0 + cc;
                    const int col = orig_col(p, half), valid = N - p;
                    const float* src = reinterpret_cast<const float*>(wl + lr * pitch) + cc;
                    const size_t at = (size_t)out_row * ldc + col;
                    if (valid >= per) {
                        if constexpr (per == 4) {
                            *reinterpret_cast<float4*>(static_cast<float*>(c) + at) =
                                *reinterpret_cast<const float4*>(src);
                        } else {
                            const float4 lo = reinterpret_cast<const float4*>(src)[0];
                            const float4 hi = reinterpret_cast<const float4*>(src)[1];
                            const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                            unsigned w[4];
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                w[e] = (unsigned)__half_as_ushort(f32_to_f16(v[2 * e])) |
                                       ((unsigned)__half_as_ushort(f32_to_f16(v[2 * e + 1])) << 16);
                            *reinterpret_cast<uint4*>(static_cast<__half*>(c) + at) = uint4{w[0], w[1], w[2], w[3]};
                        }
                    } else {
                        for (int t = 0; t < valid; ++t) store_out(c, c_type, at + t, src[t]);
                    }
                }
            };
            if (c_type == DT_F32)
                runs(IntTag<4>{});
            else
                runs(IntTag<8>{});
        } else {
            // 4 staged f32 values per lane: max |o| over the row's lanes (CPR
            // consecutive lanes), conversion to the output type, one store.
            constexpr int CPR = OUTC / 4;
            static_assert((FPI * 32 * CPR) % 64 == 0 && 64 % CPR == 0, "rows must not straddle waves");
            for (int q = lane; q < FPI * 32 * CPR; q += 64) {
                const int lr = q / CPR, cc = (q % CPR) * 4;
                int out_row, src_row;
                const bool row_ok = row_of(wm * TM + i0 * 32 + lr, out_row, src_row);
                const float4 v = *reinterpret_cast<const float4*>(wl + lr * pitch + cc * 4);
                const int col = out0 + cc, valid = row_ok ? n_out - col : 0;
                float mx = 0.0f;
                if (valid > 0) mx = fabsf(v.x);
                if (valid > 1) mx = fmaxf(mx, fabsf(v.y));
                if (valid > 2) mx = fmaxf(mx, fabsf(v.z));
                if (valid > 3) mx = fmaxf(mx, fabsf(v.w));
                if (valid >= 4) {
                    if (c_type == DT_F32) {
                        *reinterpret_cast<float4*>(static_cast<float*>(c) + (size_t)out_row * ldc + col) = v;
                    } else {
                        const __half2 h01 = __floats2half2_rn(v.x, v.y), h23 = __floats2half2_rn(v.z, v.w);
                        uint2 pk;
                        pk.x = *reinterpret_cast<const unsigned*>(&h01);
                        pk.y = *reinterpret_cast<const unsigned*>(&h23);
                        *reinterpret_cast<uint2*>(static_cast<__half*>(c) + (size_t)out_row * ldc + col) = pk;
                    }
                } else {
                    const float vv[4] = {v.x, v.y, v.z, v.w};
                    for (int t = 0; t < valid; ++t) store_out(c, c_type, (size_t)out_row * ldc + col + t, vv[t]);
                }
                if (EPI == EPI_SWIGLU_MAX) {
                    if constexpr (CPR == 8) {
                        mx = max8(mx);
                    } else {
#pragma unroll
                        for (int off = 1; off < CPR; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
                    }
                    if ((lane % CPR) == 0 && row_ok) atomicMax(rowmax + out_row, max_bits(mx));
                }
            }
        }
        __syncthreads();
    }
}

// Split-K in two launches: SPLIT_PART blocks compute K piece b / tiles of
// tile b % tiles and store the int32 accumulators (16 bytes per lane,
// fragment order, [piece][tile][BM*BN]); one SPLIT_FINISH block per tile then
// sums the pieces (exact integer sums, in piece order) and runs the epilogue.
// The launch boundary orders the two, so no block waits for another and no
// device-scope fence is needed.
enum { SPLIT_NONE = 0, SPLIT_PART = 1, SPLIT_FINISH = 2 };

template <int FM, int FN, int NT>
__device__ __forceinline__ v4i* part_slot(int* part, size_t tile_ints, int q, int T, int tile, int i, int j, int h) {
    return reinterpret_cast<v4i*>(part + ((size_t)q * T + tile) * tile_ints +
                                  ((size_t)((i * FN + j) * 4 + h) * NT + threadIdx.x) * 4);
}

template <int BM, int BN, int WGM, int WGN, int BITS, int EPI, bool STAGED, int SPLIT = SPLIT_NONE>
__global__ __launch_bounds__(WGM* WGN * 64, 1) void gemm_kernel(GemmParams P) {
    using C = TileCfg<BM, BN, WGM, WGN, BITS>;
    static_assert(EPI == EPI_PLAIN || C::FN % 2 == 0, "SwiGLU pairs need an even fragment count");
    constexpr int FM = C::FM, FN = C::FN, NT = C::NT;
    constexpr size_t TILE_INTS = (size_t)BM * BN;
    __shared__ __attribute__((aligned(16))) uint8_t smem[C::SMEM];

    // Block -> (K piece, tile). Tiles: give each of the 8 XCDs (blocks are
    // dealt round-robin) a contiguous range of tile ids, then walk groups of
    // 8 M-tiles so that neighbouring tiles share weight panels in the XCD's
    // L2. Pieces are the outer index, so blocks of one piece share K ranges.
    const int T = P.tiles_m * P.tiles_n;
    const int piece = SPLIT == SPLIT_PART ? blockIdx.x / T : 0;
    const int bid = blockIdx.x - piece * T;
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

    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    const int M = P.M;
    auto row_of = [&](int local, int& out_row, int& src_row) {
        const int row = m0 + local;
        out_row = row;
        src_row = row < M ? row : 0;
        return row < M;
    };

    if constexpr (SPLIT == SPLIT_FINISH) {
        const auto pre = epilogue_prefetch<BM, BN, WGM, WGN, BITS>(P.rowscale, P.rowsum, P.colscale, n0, row_of);
        for (int q = 0; q < P.splits; ++q) {
            v4i v[FM][FN][4];
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int h = 0; h < 4; ++h)
                        v[i][j][h] = *part_slot<FM, FN, NT>(P.split_part, TILE_INTS, q, T, tile, i, j, h);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] += v[i][j][r >> 2][r & 3];
        }
        gemm_epilogue<BM, BN, WGM, WGN, BITS, EPI, STAGED>(acc, n0, pre, P.N, P.half, P.c, P.ldc, P.c_type, P.rowmax,
                                                           row_of, smem);
        return;
    }

    const int KT_all = P.K_pad >> 6;
    const int splits = SPLIT == SPLIT_PART ? P.splits : 1;
    const int k0 = (int)((long)KT_all * piece / splits);
    const int k1 = (int)((long)KT_all * (piece + 1) / splits);
    constexpr int PPS = (BITS == 8) ? 4 : 2;  // weight planes per 64-k step
    size_t a_off[C::A_LOADS];
#pragma unroll
    for (int i = 0; i < C::A_LOADS; ++i) {
        // (tile rows past the code buffer's rows, which a 192-row tile of the
        // last M-tile reaches, read its last row; their outputs are masked)
        const int c = min((int)threadIdx.x + i * NT, C::A_CHUNKS - 1);
        a_off[i] = (size_t)(c / BM) * P.M_alloc + min(m0 + c % BM, P.M_alloc - 1);
    }
    EpiPre<BM, BN, WGM, WGN, BITS> pre;
    if constexpr (SPLIT == SPLIT_NONE)
        pre = epilogue_prefetch<BM, BN, WGM, WGN, BITS>(P.rowscale, P.rowsum, P.colscale, n0, row_of);
    gemm_mainloop<BM, BN, WGM, WGN, BITS>(smem, P.a + (size_t)k0 * 64 * P.M_alloc, (size_t)P.M_alloc, a_off,
                                          P.b + (size_t)k0 * PPS * 128, P.K_pad, n0, k1 - k0, acc);
    if constexpr (SPLIT == SPLIT_PART) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int h = 0; h < 4; ++h)
                    *part_slot<FM, FN, NT>(P.split_part, TILE_INTS, piece, T, tile, i, j, h) =
                        v4i{acc[i][j][4 * h], acc[i][j][4 * h + 1], acc[i][j][4 * h + 2], acc[i][j][4 * h + 3]};
    } else {
        gemm_epilogue<BM, BN, WGM, WGN, BITS, EPI, STAGED>(acc, n0, pre, P.N, P.half, P.c, P.ldc, P.c_type, P.rowmax,
                                                           row_of, smem);
    }
}

// Finish of a split 128x128 tile (2x2 waves) by four one-wave blocks: block b
// sums the K pieces' partials of wave b % 4 of tile b / 4 (the part kernel's
// layout, read as it lies: 1 KB runs per fragment quarter) and runs that
// wave's 64x64 epilogue, which is the same dequantization and store as the
// tile's, so the finish spreads over four times the blocks (the 80 tiles of
// a 512-row 9728x2560 down projection ran on 80 of 256 CUs; FFN M=512 call
// 79.6 -> 78.8 us).
template <int BITS, int EPI>
__global__ __launch_bounds__(64) void gemm_split_finish_kernel(GemmParams P) {
    using C = TileCfg<128, 128, 2, 2, BITS>;  // the partials' layout
    using W = TileCfg<64, 64, 1, 1, BITS>;    // one wave's sub-tile
    static_assert(C::FM == W::FM && C::FN == W::FN, "a wave tile of the split tile is the sub-tile");
    constexpr int FM = C::FM, FN = C::FN, NT = C::NT;
    constexpr size_t TILE_INTS = (size_t)128 * 128;
    __shared__ __attribute__((aligned(16))) uint8_t smem[W::SMEM];
    const int T = P.tiles_m * P.tiles_n;
    const int tile = blockIdx.x >> 2, w = blockIdx.x & 3, wm = w / 2, wn = w % 2;
    const int lane = threadIdx.x;
    // tile -> (tm, tn) as in gemm_kernel
    constexpr int G = 8;
    const int group = tile / (G * P.tiles_n);
    const int first_m = group * G;
    const int gm = min(P.tiles_m - first_m, G);
    const int in_g = tile - group * G * P.tiles_n;
    const int tm = first_m + in_g % gm, tn = in_g / gm;
    const int m0 = tm * 128 + wm * 64, n0 = tn * 128 + wn * 64;
    const int M = P.M;
    auto row_of = [&](int local, int& out_row, int& src_row) {
        const int row = m0 + local;
        out_row = row;
        src_row = row < M ? row : 0;
        return row < M;
    };
    const auto pre = epilogue_prefetch<64, 64, 1, 1, BITS>(P.rowscale, P.rowsum, P.colscale, n0, row_of);
    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    for (int q = 0; q < P.splits; ++q) {
        const int* base = P.split_part + ((size_t)q * T + tile) * TILE_INTS;
        v4i v[FM][FN][4];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int h = 0; h < 4; ++h)
                    v[i][j][h] = *reinterpret_cast<const v4i*>(base + ((size_t)((i * FN + j) * 4 + h) * NT + w * 64 + lane) * 4);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] += v[i][j][r >> 2][r & 3];
    }
    gemm_epilogue<64, 64, 1, 1, BITS, EPI, true>(acc, n0, pre, P.N, P.half, P.c, P.ldc, P.c_type, P.rowmax, row_of,
                                                 smem);
}

// ---------------------------------------------------------------------------
// Decode GEMV / skinny GEMM (M <= 8) without MFMA: bandwidth bound, one launch.
// A block owns one tile group for the whole K: one 8-column weight tile, or
// (SwiGLU) a gate tile and its up tile, so no reduction crosses blocks and
// one block is launched per group (enough blocks are resident that every
// weight byte of a decode-sized matrix is requested at once). The group's
// bytes are a flat stream of 16-byte chunks (chunk q = plane q/8, column q%8
// of its tile); thread tid of the NTHR takes chunks tid + NTHR*r, so every
// wave load is 1 KB contiguous and the column of a thread is fixed (tid % 8). All chunks
// (up to NW register windows of RW rounds each) are requested first; the block then
// quantizes the activation rows itself (row max from x or from precomputed
// partial maxima, the dense or MoE rule) into LDS while they are in flight.
// Dot products use v_dot4_i32_i8; partials reduce over threads of the same
// column with cross-lane shuffles and over waves through LDS. SwiGLU+max
// writes one partial max per block.
// ---------------------------------------------------------------------------
// Activation chunks (16 elements) each GEMV thread quantizes from registers;
// rows with K_pad/16 * rows above 256 * GEMV_XMAX are quantized beforehand.
constexpr int GEMV_XMAX = 3;

struct GemvParams {
    const void* x;
    long lda;
    int rule;             // QUANT_DENSE or QUANT_MOE
    int vec;              // rows are 16-element aligned and K % 16 == 0
    const float* part_in; // optional row maxima as partials [row][part_count]
    int part_count;
    float* part_out;      // SwiGLU+max: per-block max |out|, [row][gridDim.x]
    const uint8_t* b;
    const float* colscale;
    void* c;
    long ldc;
    int c_type;
    int M, K, N, K_pad, N_pad, half;
    // Quantized rows [K_pad/16][M_alloc][16] with their scales and code sums:
    // written by block 0 when the kernel quantizes (diagnostics), read when
    // the rows were quantized beforehand (PREQ).
    int8_t* diag_codes;
    float* diag_scale;
    int* diag_rowsum;
    int M_alloc;
    // Grouped mode (routed experts, one row per slot): block row s = slot s <
    // slot_count[0] of assignment perm[s] (token perm[s] / top, expert
    // ids[perm[s]]): weights and column scales of that expert, activation row
    // s (or the token's pre-quantized row), output row s, partial maxima row s.
    // perm == nullptr: slot s is assignment s itself (no routing launch); its
    // blocks return at once when routes[s] is not positive, and when ids[s]
    // is outside [0, experts) after setting bit 0 of *error.
    const uint8_t* const* b_tab;
    const float* const* s_tab;
    const int* perm;
    const int* ids;
    const int* slot_count;
    int top;
    const float* routes;
    int experts;
    unsigned* error;
    int x_by_token;  // grouped, rows quantized in the block: activation row = token, not slot
    // Split K (one row, plain epilogue, row maxima as partials): block b is
    // piece b % ksplit of group b / ksplit over its share of the 64-k units.
    // Each piece adds (1 << 40) + (its exact int32 column sum + 2^31) into the
    // column's 64-bit slot kacc[col]: bits 40 and up count the pieces, the
    // low 40 bits hold the biased sum (below ksplit * 2^32 <= 2^35). The piece
    // that sees ksplit - 1 earlier pieces finishes the column and clears the
    // slot; kacc[N_pad] collects the row's code sum for diagnostics the same
    // way.
    int ksplit;
    unsigned long long* kacc;
    // One-launch FFN (ffn_m1_kernel): the gate_up blocks (producers) publish
    // the middle row and its maxima to the down blocks (consumers) of the same
    // launch through `sync` (FfnSync layout); fuse_block / fuse_blocks are the
    // block's index in the whole launch and the launch's block count.
    unsigned* sync;
    int producers, consumers;
    int spin_limit;
    int fuse_block, fuse_blocks;
    // MoE combine in the epilogue (FUSE_COMBINE: one token row, routes of its
    // top <= GEMV_COMB_TOP ranks, slot = assignment): the output column is
    // sum_rank fma(comb_contrib[rank][col], routes[rank], .) + this GEMV's
    // value, the moe_combine_kernel arithmetic, stored as f32.
    const float* comb_contrib;
    const float* comb_routes;
    int comb_top, comb_h;
};
constexpr int GEMV_COMB_TOP = 8;

// Synchronisation words of a one-launch FFN, kept zero between launches (the
// launch's last block clears them). Arrivals are spread over SLOTS counters
// so that no address takes more than a few dozen atomics, and every word has
// its own 64-byte line:
//   cnt[s]   producers with index % SLOTS == s that published their middle
//            values and block max (counted after those stores completed)
//   mx[s]    max |middle| over those producers (float bits, atomic max)
//   ready    producer slots that are complete; the producer completing the
//            last one sets the flags
//   flag[r]  SLOTS replicas of the all-published flag (64-bit), so the down
//            blocks each poll one line of their own residue class
//   done[s]  blocks with launch index % SLOTS == s that finished
//   top      done slots that completed; the block completing the last clears all
//   err      bit 0: a down block gave up waiting (its spin limit ran out)
constexpr int FFN_SLOTS = 32;
constexpr int FFN_LINE = 16;  // words per line (64 bytes)
constexpr int FFN_SYNC_WORDS = (4 * FFN_SLOTS + 3) * FFN_LINE;
struct FfnSync {
    unsigned* base;
    __device__ unsigned* cnt(int s) const { return base + s * FFN_LINE; }
    __device__ unsigned* mx(int s) const { return base + (FFN_SLOTS + s) * FFN_LINE; }
    __device__ unsigned* done(int s) const { return base + (2 * FFN_SLOTS + s) * FFN_LINE; }
    __device__ unsigned long long* flag(int r) const {
        return reinterpret_cast<unsigned long long*>(base + (3 * FFN_SLOTS + r) * FFN_LINE);
    }
    __device__ unsigned* top() const { return base + 4 * FFN_SLOTS * FFN_LINE; }
    __device__ unsigned* ready() const { return base + (4 * FFN_SLOTS + 1) * FFN_LINE; }
    __device__ unsigned* err() const { return base + (4 * FFN_SLOTS + 2) * FFN_LINE; }
};
// Blocks i < n with i % FFN_SLOTS == s.
__device__ __forceinline__ unsigned ffn_slot_count(int n, int s) {
    return (unsigned)(n / FFN_SLOTS + (s < n % FFN_SLOTS ? 1 : 0));
}

enum { FUSE_NONE = 0, FUSE_PRODUCER = 1, FUSE_CONSUMER = 2, FUSE_COMBINE = 3 };

__device__ __forceinline__ unsigned ld_agent(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A block of a one-launch FFN has finished everything that touches the
// synchronisation words or the middle row (called by one lane, after its
// wave's memory operations completed): count it, and let the last block of
// the launch clear the words for the next launch.
__device__ __forceinline__ void ffn_block_done(const GemvParams& P) {
    const FfnSync S{P.sync};
    const int s = P.fuse_block % FFN_SLOTS;
    const unsigned was = __hip_atomic_fetch_add(S.done(s), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (was + 1 != ffn_slot_count(P.fuse_blocks, s)) return;
    const unsigned t = __hip_atomic_fetch_add(S.top(), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((int)t + 1 != min(P.fuse_blocks, FFN_SLOTS)) return;
    for (int i = 0; i < FFN_SLOTS; ++i) {
        st_agent(S.cnt(i), 0u);
        st_agent(S.mx(i), 0u);
        st_agent(S.done(i), 0u);
        __hip_atomic_store(S.flag(i), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    st_agent(S.ready(), 0u);
    st_agent(S.top(), 0u);
}

// A producer has published (its stores and max completed): count it; the
// producer that completes the last slot publishes the row max to the flags.
__device__ __forceinline__ void ffn_producer_arrive(const GemvParams& P, int producer) {
    const FfnSync S{P.sync};
    const int s = producer % FFN_SLOTS;
    const unsigned was = __hip_atomic_fetch_add(S.cnt(s), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (was + 1 != ffn_slot_count(P.producers, s)) return;
    const unsigned r = __hip_atomic_fetch_add(S.ready(), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((int)r + 1 != min(P.producers, FFN_SLOTS)) return;
    for (int i = 0; i < FFN_SLOTS; ++i)
        __hip_atomic_store(S.flag(i), 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A consumer wave waits (one lane polls its flag replica, bounded: past
// P.spin_limit polls, or at once when it is negative, it flags the error word
// and goes on) until every producer has published, then returns the row max,
// the max of the slot maxima (each producer's max completed before its slot
// did, and every slot before the flag was set).
__device__ __forceinline__ float ffn_wait_row_max(const GemvParams& P, int lane) {
    const FfnSync S{P.sync};
    if (lane == 0) {
        const unsigned long long* f = S.flag(P.fuse_block % FFN_SLOTS);
        for (int it = 0;; ++it) {
            if (P.spin_limit >= 0 && __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0ull) break;
            if (it >= P.spin_limit) {
                __hip_atomic_fetch_or(S.err(), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const unsigned m = lane < FFN_SLOTS ? ld_agent(S.mx(lane)) : 0u;
    return wave_max(__uint_as_float(m));
}


// Activation chunks per lane of the quantization wave (QWN = 1 blocks): rows
// of at most 64 * gemv_qb<T>() chunks in all (M * K / 16) take that path.
template <typename T>
constexpr int gemv_qb() { return sizeof(T) == 2 ? 4 : 3; }

// The quantization wave of a block with QWN = 1 (threads 0-63): it loads the
// block's activation rows (chunk c = lane + 64*j, in registers), takes each
// row's max from them or from the precomputed partial maxima, and writes the
// codes [k16][row][16] to LDS, the row scales to s_scale and the code sums to
// s_sum[0]. It runs beside the weight waves, which only issue their weight
// loads and then wait at the block barrier, so the quantization chain overlaps
// the weight stream instead of following the weight waves' load issue. (The
// code keeps QWN general; four such waves in front of the 512-thread down
// projection were slower than its in-block quantization: 7.3 -> 7.8 us, the
// partial-maxima batches of each wave running in series.)
template <typename T, int MR, int QWN>
__device__ __forceinline__ void gemv_quant_waves(const GemvParams& P, int8_t* sa, float* s_scale,
                                                 int (*s_sum)[MR], int qt, bool diag) {
    constexpr int QB = gemv_qb<T>();
    constexpr int QT = 64 * QWN;
    constexpr int PB = 8;  // precomputed partial maxima per lane per batch
    const int lane = qt & 63, qwave = qt >> 6;
    const int chunks = (P.K_pad >> 4) * MR;
    const T* x = static_cast<const T*>(P.x);
    // a masked lane reads its own chunk of row 0 (never one shared address)
    const T* spare = x + (size_t)min(qt, (P.K >> 4) - 1) * 16;
    v4u xr[QB][4];
    {
#pragma unroll
        for (int j = 0; j < QB; ++j) {
            if (QT * j >= chunks) break;
            const int c = qt + QT * j, kg = c / MR, m = c % MR;
            const bool ok = c < chunks && m < P.M && kg * 16 < P.K;
            load16_raw(ok ? x + (size_t)m * P.lda + kg * 16 : spare, xr[j]);
        }
    }
    // words of a chunk the lane does not own (it read its spare chunk) are
    // zeroed once, before both passes
#pragma unroll
    for (int j = 0; j < QB; ++j) {
        if (QT * j >= chunks) break;
        const int c = qt + QT * j, kg = c / MR, m = c % MR;
        const bool ok = c < chunks && m < P.M && kg * 16 < P.K;
#pragma unroll
        for (int q = 0; q < (int)sizeof(T); ++q)  // (sizeof(T) 16-byte words per chunk)
            xr[j][q] = ok ? xr[j][q] : v4u{0u, 0u, 0u, 0u};
    }
    float mx[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) mx[m] = 0.0f;
    if (QWN > 1 || P.part_in) {
        const int spare_idx = lane < P.part_count ? lane : 0;
        for (int base = 0; base < P.part_count; base += 64 * PB) {
            float pv[MR][PB];
#pragma unroll
            for (int i = 0; i < PB; ++i)
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    const int idx = base + lane + 64 * i;
                    const bool ok = m < P.M && idx < P.part_count;
                    pv[m][i] = P.part_in[ok ? (size_t)m * P.part_count + idx : (size_t)spare_idx];
                }
#pragma unroll
            for (int i = 0; i < PB; ++i)
#pragma unroll
                for (int m = 0; m < MR; ++m)
                    if (m < P.M && base + lane + 64 * i < P.part_count) mx[m] = fmaxf(mx[m], pv[m][i]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < QB; ++j) {
            if (qt + QT * j >= chunks) continue;
            float v[16];
            cvt16_raw(xr[j], v, T());
            float lm = 0.0f;
#pragma unroll
            for (int b = 0; b < 16; ++b) lm = fmaxf(lm, fabsf(v[b]));
            const int m = (qt + QT * j) % MR;
#pragma unroll
            for (int r = 0; r < MR; ++r) mx[r] = (r == m) ? fmaxf(mx[r], lm) : mx[r];
        }
    }
    float scale[MR], inv[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const float v = wave_max(mx[m]);
        if (P.rule == QUANT_DENSE)
            scale[m] = (v == 0.0f) ? 1.0f : fmaxf(v / 127.0f, FLT_MIN);
        else
            scale[m] = (v == 0.0f) ? 1.0f : v / 127.0f;
        inv[m] = 1.0f / scale[m];
    }
    diag = diag && P.diag_codes;
    int psum[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) psum[m] = 0;
#pragma unroll
    for (int j = 0; j < QB; ++j) {
        const int c = qt + QT * j, m = c % MR;
        if (c >= chunks) continue;
        float iv = inv[0];
#pragma unroll
        for (int r = 1; r < MR; ++r) iv = (r == m) ? inv[r] : iv;
        float sv[16];
        scale16_raw(xr[j], iv, sv, T());
        int sum = 0;
        const v4u pk = (P.rule == QUANT_DENSE) ? quant_scaled<QUANT_DENSE>(sv, sum) : quant_scaled<QUANT_MOE>(sv, sum);
#pragma unroll
        for (int r = 0; r < MR; ++r) psum[r] += (r == m) ? sum : 0;
        *reinterpret_cast<v4u*>(sa + c * 16) = pk;
        if (diag) *reinterpret_cast<v4u*>(P.diag_codes + ((size_t)(c / MR) * P.M_alloc + m) * 16) = pk;
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const int isum = wave_sum(psum[m]);
        if (lane == 0) {
            if (qwave == 0) s_scale[m] = scale[m];
            s_sum[qwave][m] = isum;
        }
    }
}

// QWN = 1: the block has a quantization wave (gemv_quant_waves) before its
// NTHR weight threads; the rows must fit it (at most 64 * gemv_qb<T>() chunks).
// SPLITK: the block is one K piece of a group (GemvParams::ksplit).
// One block of the GEMV: block `bid` of `nblk` along x. FUSE_PRODUCER /
// FUSE_CONSUMER are the gate_up and down roles in a one-launch FFN
// (ffn_m1_kernel); FUSE_NONE is the standalone GEMV (gemv_kernel).
template <typename T, int MR, int BITS, int EPI, int RW, int NW, bool PREQ, int GPB = 1, int NTHR = 256,
          bool GROUPED = false, int QWN = 0, bool SPLITK = false, int FUSE = FUSE_NONE>
__device__ __forceinline__ void gemv_block(GemvParams P, const int bid, const int nblk, int8_t* sa) {
    // sa: [K_pad/16][MR][16] codes (the piece's K) in dynamic shared memory
    // Split K: this block's piece of the 64-k units, the row slice, and where
    // its planes start in the tile.
    int plane_off = 0, grp = bid;
    const int K_pad_full = P.K_pad;
    static_assert(FUSE == FUSE_NONE || (MR == 1 && GPB == 1 && !PREQ && !GROUPED), "the one-launch FFN runs one row");
    static_assert(FUSE != FUSE_PRODUCER || (EPI == EPI_SWIGLU_MAX && QWN == 1), "producers: the SwiGLU GEMV, quantization wave");
    static_assert(FUSE != FUSE_CONSUMER || (SPLITK && QWN == 0), "consumers: split-K pieces quantized by the whole block");
    static_assert(FUSE != FUSE_COMBINE || (EPI == EPI_PLAIN && !SPLITK && QWN == 0), "combine: the plain one-row GEMV");
    if constexpr (SPLITK) {
        static_assert(MR == 1 && GPB == 1 && EPI == EPI_PLAIN && !PREQ && !GROUPED && QWN == 0,
                      "split K: one row, plain epilogue, in-block quantization");
        const int piece = bid % P.ksplit;
        grp = bid / P.ksplit;
        const int U = P.K_pad >> 6;
        const int u0 = U * piece / P.ksplit, u1 = U * (piece + 1) / P.ksplit;
        plane_off = u0 * (BITS == 8 ? 4 : 2);
        P.x = static_cast<const T*>(P.x) + 64 * u0;
        P.K = max(0, min(P.K - 64 * u0, 64 * (u1 - u0)));
        P.K_pad = 64 * (u1 - u0);
        if (P.diag_codes) P.diag_codes += (size_t)4 * u0 * P.M_alloc * 16;
    }
    if constexpr (GROUPED) {
        static_assert(MR == 1 && GPB == 1, "one slot row per block");
        const int s = blockIdx.y;
        int a = s;
        if (P.perm) {
            if (s >= P.slot_count[0]) return;  // uniform over the block
            a = P.perm[s];
        } else {
            // Every id is checked, a skipped route's too (as the routing
            // kernel of larger batches and the host entry do), before a
            // skipped route returns without a contribution.
            const int e0 = P.ids[s];
            if (e0 < 0 || e0 >= P.experts) {
                if (threadIdx.x == 0) atomicOr(P.error, 1u);
                return;
            }
            if (!(P.routes[s] > 0.0f)) return;
        }
        const int tok = a / P.top, e = P.ids[a];
        P.b = P.b_tab[e];
        P.colscale = P.s_tab[e];
        // Both table loads have returned before the rows are requested (their
        // masked-off address needs the weight pointer anyway); a table load
        // still pending at the join of the rows' uniform branches made the
        // compiler wait there for every row load before the weight stream.
        asm volatile("" ::: "memory");
        wait_vmcnt<0>();
        P.x = static_cast<const T*>(P.x) + (size_t)(P.x_by_token ? tok : s) * P.lda;
        if (P.part_in) P.part_in += (size_t)s * P.part_count;
        P.c = static_cast<uint8_t*>(P.c) + (size_t)s * P.ldc * (P.c_type == DT_F32 ? 4 : 2);
        if (P.part_out) P.part_out += (size_t)s * gridDim.x;
        if (PREQ) {
            P.diag_codes += (size_t)tok * 16;
            P.diag_scale += tok;
            P.diag_rowsum += tok;
        }
    }
    constexpr int TPG = (EPI == EPI_PLAIN) ? 1 : 2;  // tiles per group
    constexpr int TPB = TPG * GPB;                   // tiles per block (GPB groups)
    constexpr int XMAX = GEMV_XMAX;  // 16-element activation chunks per thread
    constexpr int PV = 5;            // precomputed row-max partials per thread
    constexpr int NWV = NTHR / 64;   // waves per block
    __shared__ float s_red[NWV][MR];
    __shared__ int s_isum[NWV][MR];
    __shared__ int red[NWV][TPB][MR][8];
    auto block_isum = [&](int m) {
        int v = 0;
#pragma unroll
        for (int w = 0; w < NWV; ++w) v += s_isum[w][m];
        return v;
    };
    // (QWN > 0: the first QWN hardware waves quantize; the weight threads are
    // numbered from the next wave on)
    constexpr bool QW = QWN > 0;
    static_assert(QWN <= 1, "one quantization wave (more were slower)");
    const int tid = (int)threadIdx.x - 64 * QWN, lane = threadIdx.x & 63, wave = tid >> 6;
    if constexpr (QW) {
        static_assert(!PREQ, "the quantization waves quantize the rows");
        if (threadIdx.x < 64 * QWN) {
            // First waves of the block and the highest issue priority: their
            // row loads and quantization chain go ahead of the weight waves'
            // load issue (which stalls on the memory pipeline's back-pressure)
            // instead of queuing behind it (gate/up 2560x19456 W4 M=1: 8.7 us
            // with the wave last at normal priority, 6.5 us first at priority 3).
            __builtin_amdgcn_s_setprio(3);
            gemv_quant_waves<T, MR, QWN>(P, sa, s_red[0], s_isum, threadIdx.x, grp == 0);
            wait_lgkmcnt0();
            __builtin_amdgcn_s_barrier();  // codes, scales and code sums are in LDS
            __builtin_amdgcn_s_barrier();  // (the weight waves' partial sums)
            return;
        }
    }
    const int c8 = tid & 7;
    const int KG16 = P.K_pad >> 4;
    const int PL = (BITS == 8) ? KG16 : (P.K_pad >> 5);
    const int CPT = PL * 8;                  // chunks per tile
    const int CPG = CPT * TPB;               // chunks per group
    const int NWIN = (CPG + NTHR * RW - 1) / (NTHR * RW);
    const int chunks = KG16 * MR;            // activation chunks (<= NTHR * XMAX unless PREQ)
    const int g0 = grp * GPB;  // first group of the block
    const int groups = SPLITK ? nblk / P.ksplit : nblk * GPB;
    // (a tile's planes span the whole K even when the block takes a piece)
    const int CPT_full = (BITS == 8 ? K_pad_full >> 4 : K_pad_full >> 5) * 8;

    // Tile group g: one 8-column tile, or (SwiGLU) a gate tile and its up
    // tile; the block's GPB groups are consecutive and their tiles form one
    // stream of TPB tiles.
    int tile[TPB];
    const uint8_t* tb[TPB];
#pragma unroll
    for (int gp = 0; gp < GPB; ++gp) {
        const int g = g0 + gp;
        if (TPG == 1) {
            tile[gp] = g;
        } else {
            tile[2 * gp] = 8 * (g >> 2) + (g & 3);
            tile[2 * gp + 1] = tile[2 * gp] + 4;
        }
    }
#pragma unroll
    for (int t = 0; t < TPB; ++t) tb[t] = P.b + ((size_t)tile[t] * CPT_full + (size_t)plane_off * 8) * 16;
    // Stream position q -> (tile t of the block, chunk within the tile).
    auto locate = [&](int q, int& t, int& r) {
        t = 0;
#pragma unroll
        for (int i = 1; i < TPB; ++i) t += (q >= i * CPT) ? 1 : 0;
        r = q - t * CPT;
    };
    const uint8_t* tb0 = tb[0];

    // 1. Requests go out in the order they are needed, because a wait for a
    // load also waits for every load issued before it: this thread's
    // activation chunks (raw) or code chunks and the precomputed row maxima
    // first, then every weight chunk of the group (up to NW windows) and the
    // column scales. No load sits under a branch (addresses are clamped and
    // results masked at use): a load that may be skipped makes every later
    // wait of the compiler assume it was, and a register written on only one
    // side of a branch makes it wait for everything at the join.
    // Rounds of activation chunks (and of partial maxima) that hold work for
    // some thread of the block are requested; the others are not issued at
    // all (every vector-memory instruction costs the CU's load path, masked
    // or not). These branches are uniform and precede the weight stream; the
    // row-max reduction below starts from an opaque zero so that the compiler
    // cannot hoist its first step to their join, where it waited for every
    // load before the weights were requested. Within an issued round a
    // masked-off lane reads bytes it loads anyway (its first weight chunk or
    // its column scale), never one shared address: thousands of requests to
    // one line would queue on one cache channel.
    // Blocks without a quantization wave request their rows (or the rows'
    // codes) at raised issue priority and drop it for the weight stream, so
    // the rows' loads of the CU's later blocks are issued ahead of its
    // earlier blocks' pending weight loads (decode M=1 W4: qkv 2560x6144
    // 4.56 -> 4.34 us, down 9728x2560
    // 7.31 -> 7.21 us, o 4096x2560 3.75 -> 3.80 us, step 0.815 -> 0.806 ms,
    // the same box, the two builds alternated).
    if constexpr (!QW) {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(3);
        __builtin_amdgcn_sched_barrier(0);
    }
    const uint8_t* own = tb0 + (size_t)min(tid, CPT - 4) * 16;  // 64 readable bytes (CPT >= 16)
    v4u xraw[XMAX][4];
    const T* x = static_cast<const T*>(P.x);
#pragma unroll
    for (int j = 0; j < XMAX; ++j) {
        // (QW: the quantization wave loads the rows; a one-launch FFN's down
        // block loads its middle slice after the producers have published)
        if (QW || FUSE == FUSE_CONSUMER || NTHR * j >= chunks) break;
        const int c = tid + NTHR * j, kg = c / MR, m = c % MR;
        if (PREQ) {
            const bool ok = c < chunks && m < P.M;
            xraw[j][0] = gload<v4u>(ok ? P.diag_codes + ((size_t)kg * P.M_alloc + m) * 16
                                       : reinterpret_cast<const int8_t*>(own));
        } else {
            const bool ok = c < chunks && m < P.M && kg * 16 < P.K;
            load16_raw(ok ? x + (size_t)m * P.lda + kg * 16 : reinterpret_cast<const T*>(own), xraw[j]);
        }
    }
    float pv[MR][PV];
    const float* own_cs = P.colscale + 8 * tile[0] + c8;
    if (!PREQ && !QW && P.part_in) {
#pragma unroll
        for (int i = 0; i < PV; ++i) {
            if (NTHR * i >= P.part_count) break;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const int idx = tid + NTHR * i;
                const bool ok = m < P.M && idx < P.part_count;
                pv[m][i] = gload<float>(ok ? P.part_in + (size_t)m * P.part_count + idx : own_cs);  // masked at use
            }
        }
    }
    // MoE combine: the routes and this thread's column of every routed
    // contribution (written by an earlier launch), requested with the rows.
    float comb_r[FUSE == FUSE_COMBINE ? GEMV_COMB_TOP : 1], comb_c[FUSE == FUSE_COMBINE ? GEMV_COMB_TOP : 1];
    if constexpr (FUSE == FUSE_COMBINE) {
        const int p = 8 * tile[0] + c8;
        const int col = p < P.N ? orig_col(p, P.half) : 0;
#pragma unroll
        for (int r = 0; r < GEMV_COMB_TOP; ++r) {
            const int a = r < P.comb_top ? r : 0;
            comb_r[r] = P.comb_routes[a];
            comb_c[r] = P.comb_contrib[(size_t)a * P.comb_h + col];
        }
    }
    // (the empty asm statements keep the compiler from sinking these loads
    // to their first use, which would put them behind the weight stream)
    asm volatile("" ::: "memory");
    auto load_window = [&](int w, auto& buf) {
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const int q = (tid + NTHR * (w * RW + i)) % CPG;  // past the block's tiles: a re-read, skipped
            int t, r;
            locate(q, t, r);
            const uint8_t* base = tb[0];
#pragma unroll
            for (int u = 1; u < TPB; ++u) base = (t == u) ? tb[u] : base;
            // (streamed once: non-temporal)
            buf[i] = gload_nt<v4u>(base + (size_t)r * 16);
        }
    };
    v4u wa[RW], wb[NW == 2 ? RW : 1];
    if constexpr (!QW) {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
    }
    load_window(0, wa);
    if (NW == 2 && NWIN > 1) load_window(1, wb);
    float cs[TPB];
#pragma unroll
    for (int t = 0; t < TPB; ++t) cs[t] = gload<float>(P.colscale + 8 * tile[t] + c8);
    asm volatile("" ::: "memory");

    float scale[MR];
    int corr[MR];
    int row_isum[MR];  // the block's code sum of each row (its K piece when split)
    if (PREQ) {
        // 2-3. Rows quantized beforehand: codes to LDS, scales and sums from HBM.
#pragma unroll
        for (int j = 0; j < XMAX; ++j) {
            const int c = tid + NTHR * j, m = c % MR;
            if (c < chunks) *reinterpret_cast<v4u*>(sa + c * 16) = (m < P.M) ? xraw[j][0] : v4u{0u, 0u, 0u, 0u};
        }
        for (int c = tid + NTHR * XMAX; c < chunks; c += NTHR) {  // long rows: after the weights
            const int m = c % MR;
            *reinterpret_cast<v4u*>(sa + c * 16) =
                (m < P.M) ? *reinterpret_cast<const v4u*>(P.diag_codes + ((size_t)(c / MR) * P.M_alloc + m) * 16)
                          : v4u{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            scale[m] = m < P.M ? P.diag_scale[m] : 1.0f;
            corr[m] = (BITS == 4 && m < P.M) ? 8 * P.diag_rowsum[m] : 0;
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) row_isum[m] = 0;
        wait_lgkmcnt0();
        __builtin_amdgcn_s_barrier();
    } else if (QW) {
        // 2-3. Codes, scales and code sums from the quantization waves.
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            scale[m] = s_red[0][m];
            int isum = 0;
#pragma unroll
            for (int w = 0; w < QWN; ++w) isum += s_isum[w][m];
            corr[m] = BITS == 4 ? 8 * isum : 0;
            row_isum[m] = isum;
            if (grp == 0 && P.diag_codes && tid == m && m < P.M) {
                P.diag_scale[m] = scale[m];
                if (!SPLITK) P.diag_rowsum[m] = isum;  // (split: summed over pieces below)
            }
        }
    } else {
        // 2. Row maxima (from the activations or the precomputed partials),
        // block max through LDS, row scales.
        // (from a zero the compiler cannot see through: with a literal 0 it
        // took the first partial's max right after the partials' loads, before
        // the weight stream, and waited there for every load in flight)
        float zero;
        asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
        float mx[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) mx[m] = zero;
        if constexpr (FUSE == FUSE_CONSUMER) {
            // every wave waits for the producers and takes the row max from
            // their slot maxima; then its threads load their middle chunks
            // with ordinary loads: no cache can hold a stale copy of the row
            // (no block of this launch reads it before the flag, the producers
            // stored it at agent scope before counting themselves, and a
            // launch never starts with another launch's stale lines, by the
            // runtime's kernel-boundary ordering), and each XCD's L2 fetches it
            // once for all the pieces it runs.
            mx[0] = ffn_wait_row_max(P, lane);
#pragma unroll
            for (int j = 0; j < XMAX; ++j) {
                if (NTHR * j >= chunks) break;
                const int c = tid + NTHR * j;
                const bool ok = c < chunks && c * 16 < P.K;
                load16_raw(ok ? x + (size_t)c * 16 : reinterpret_cast<const T*>(own), xraw[j]);
            }
        }
        // words of a chunk the thread does not own (it read its own weight
        // bytes) are zeroed once, before both passes
#pragma unroll
        for (int j = 0; j < XMAX; ++j) {
            if (NTHR * j >= chunks) break;
            const int c = tid + NTHR * j, kg = c / MR, m = c % MR;
            const bool ok = c < chunks && m < P.M && kg * 16 < P.K;
#pragma unroll
            for (int q = 0; q < (int)sizeof(T); ++q)  // (sizeof(T) 16-byte words per chunk)
                xraw[j][q] = ok ? xraw[j][q] : v4u{0u, 0u, 0u, 0u};
        }
        if (FUSE == FUSE_CONSUMER) {
            // (the row max is already known)
        } else if (P.part_in) {
#pragma unroll
            for (int m = 0; m < MR; ++m) {
#pragma unroll
                for (int i = 0; i < PV; ++i)
                    if (m < P.M && tid + NTHR * i < P.part_count) mx[m] = fmaxf(mx[m], pv[m][i]);
                if (m < P.M)
                    for (int i = tid + NTHR * PV; i < P.part_count; i += NTHR)
                        mx[m] = fmaxf(mx[m], P.part_in[(size_t)m * P.part_count + i]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < XMAX; ++j) {
                if (tid + NTHR * j >= chunks) continue;  // (pure arithmetic: no load under the branch)
                float v[16];
                cvt16_raw(xraw[j], v, T());
                float lm = 0.0f;
#pragma unroll
                for (int b = 0; b < 16; ++b) lm = fmaxf(lm, fabsf(v[b]));
                const int m = (tid + NTHR * j) % MR;
#pragma unroll
                for (int r = 0; r < MR; ++r) mx[r] = (r == m) ? fmaxf(mx[r], lm) : mx[r];
            }
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float v = wave_max(mx[m]);
            if (lane == 0) s_red[wave][m] = v;
        }
        wait_lgkmcnt0();
        __builtin_amdgcn_s_barrier();
        float inv[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float v = s_red[0][m];
#pragma unroll
            for (int w = 1; w < NWV; ++w) v = fmaxf(v, s_red[w][m]);
            if (P.rule == QUANT_DENSE)
                scale[m] = (v == 0.0f) ? 1.0f : fmaxf(v / 127.0f, FLT_MIN);
            else
                scale[m] = (v == 0.0f) ? 1.0f : v / 127.0f;
            inv[m] = 1.0f / scale[m];
        }

        // 3. Quantize this thread's chunks into LDS, chunk c = (k16 group, row).
        int psum[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) psum[m] = 0;
#pragma unroll
        for (int j = 0; j < XMAX; ++j) {
            const int c = tid + NTHR * j, m = c % MR;
            if (c >= chunks) continue;
            float iv = inv[0];
#pragma unroll
            for (int r = 1; r < MR; ++r) iv = (r == m) ? inv[r] : iv;
            float sv[16];
            scale16_raw(xraw[j], iv, sv, T());
            int sum = 0;
            const v4u pk = (P.rule == QUANT_DENSE) ? quant_scaled<QUANT_DENSE>(sv, sum) : quant_scaled<QUANT_MOE>(sv, sum);
            const unsigned packed[4] = {pk[0], pk[1], pk[2], pk[3]};
#pragma unroll
            for (int r = 0; r < MR; ++r) psum[r] += (r == m) ? sum : 0;
            *reinterpret_cast<v4u*>(sa + c * 16) = v4u{packed[0], packed[1], packed[2], packed[3]};
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const int v = wave_sum(psum[m]);
            if (lane == 0) s_isum[wave][m] = v;
        }
        wait_lgkmcnt0();
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            row_isum[m] = block_isum(m);
            corr[m] = (BITS == 4) ? 8 * row_isum[m] : 0;
        }
        if (grp == 0 && P.diag_codes) {
            for (int c = tid; c < chunks; c += NTHR)
                *reinterpret_cast<v4u*>(P.diag_codes + ((size_t)(c / MR) * P.M_alloc + c % MR) * 16) =
                    *reinterpret_cast<const v4u*>(sa + c * 16);
            if (tid < MR && tid < P.M) {
                P.diag_scale[tid] = scale[tid];
                if (!SPLITK) P.diag_rowsum[tid] = block_isum(tid);  // (split: summed over pieces below)
            }
        }
    }

    // 4. Dots: chunk q = tid + NTHR*r of the group's stream. One row:
    // v_dot4 per chunk. 2 to 8 rows, on the matrix cores (the plan requires
    // chunks per tile to be a multiple of 64, K_pad % 128 == 0 for W8 and
    // % 256 for W4, so that a wave's round lies in one tile): a wave's 64 chunks of a round are
    // planes p0..p0+7 (p0 a multiple of 8) of one tile, lane L holding plane
    // p0 + (L >> 3), column L & 7. Read as the B operand of
    // v_mfma_i32_16x16x64_i8 (lane L: column n = L & 15, k = 16 * (L >> 4) +
    // 0..15), column n takes plane p0 + 2g + (n >> 3) for k chunk g: columns
    // n < 8 see the even planes, n >= 8 the odd ones. One MFMA against the
    // even planes' activation codes (A lane L: row L & 15, the same k chunk)
    // and one against the odd planes' give, in columns 0-7 of the first and
    // 8-15 of the second, exact partial sums of the 8 tile columns; W4 planes
    // hold two 16-k chunks (low and high nibbles), so four MFMAs. Rows past
    // MR read row (L & 15) % MR; their outputs are not used.
    v4i accE[TPB], accO[TPB];
    if constexpr (MR >= 2) {
#pragma unroll
        for (int t = 0; t < TPB; ++t) accE[t] = accO[t] = v4i{0, 0, 0, 0};
    }
    auto consume_mf = [&](int w, const auto& buf) {
        const int mrow = lane & (MR - 1), g = lane >> 4;
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const int q0 = wave * 64 + NTHR * (w * RW + i);  // the wave's first chunk (uniform)
            if (q0 >= CPG) continue;
            int tq, rq;
            locate(q0, tq, rq);
            const int p0 = rq >> 3;
            const v4i wv = __builtin_bit_cast(v4i, buf[i]);
            auto codes = [&](int kg) { return *reinterpret_cast<const v4i*>(sa + (kg * MR + mrow) * 16); };
            v4i e = tq == 0 ? accE[0] : accE[TPB - 1];
            v4i o = tq == 0 ? accO[0] : accO[TPB - 1];
            if constexpr (BITS == 8) {
                const v4i ae = codes(p0 + 2 * g), ao = codes(p0 + 2 * g + 1);
                e = __builtin_amdgcn_mfma_i32_16x16x64_i8(ae, wv, e, 0, 0, 0);
                o = __builtin_amdgcn_mfma_i32_16x16x64_i8(ao, wv, o, 0, 0, 0);
            } else {
                const int kb = 4 * ((p0 >> 1) + g);
                const v4i a0 = codes(kb), a1 = codes(kb + 1), a2 = codes(kb + 2), a3 = codes(kb + 3);
                const v4i lo = wv & 0x0F0F0F0F, hi = (wv >> 4) & 0x0F0F0F0F;
                e = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, lo, e, 0, 0, 0);
                o = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, lo, o, 0, 0, 0);
                e = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, hi, e, 0, 0, 0);
                o = __builtin_amdgcn_mfma_i32_16x16x64_i8(a3, hi, o, 0, 0, 0);
            }
            if (tq == 0) {
                accE[0] = e;
                accO[0] = o;
            } else {
                accE[TPB - 1] = e;
                accO[TPB - 1] = o;
            }
        }
    };
    int acc[TPB][MR];
#pragma unroll
    for (int t = 0; t < TPB; ++t)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[t][m] = 0;
    auto consume = [&](int w, const auto& buf) {
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const int q = tid + NTHR * (w * RW + i);
            if (q >= CPG) continue;
            int tq, rq;
            locate(q, tq, rq);
            const int pl = rq >> 3;
            const v4u wv = buf[i];
            int d[MR];
            if (BITS == 8) {
                const int8_t* ab = sa + pl * MR * 16;
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    const v4i a = *reinterpret_cast<const v4i*>(ab + m * 16);
                    int v = __builtin_amdgcn_sdot4(a.x, (int)wv.x, 0, false);
                    v = __builtin_amdgcn_sdot4(a.y, (int)wv.y, v, false);
                    v = __builtin_amdgcn_sdot4(a.z, (int)wv.z, v, false);
                    d[m] = __builtin_amdgcn_sdot4(a.w, (int)wv.w, v, false);
                }
            } else {
                const int kga = 4 * (pl >> 1) + (pl & 1);
                const int8_t* aa = sa + kga * MR * 16;
                const int8_t* ab = sa + (kga + 2) * MR * 16;
                const v4u lo = wv & 0x0F0F0F0Fu, hi = (wv >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    const v4i x0 = *reinterpret_cast<const v4i*>(aa + m * 16);
                    const v4i x1 = *reinterpret_cast<const v4i*>(ab + m * 16);
                    int v = __builtin_amdgcn_sdot4(x0.x, (int)lo.x, 0, false);
                    v = __builtin_amdgcn_sdot4(x0.y, (int)lo.y, v, false);
                    v = __builtin_amdgcn_sdot4(x0.z, (int)lo.z, v, false);
                    v = __builtin_amdgcn_sdot4(x0.w, (int)lo.w, v, false);
                    v = __builtin_amdgcn_sdot4(x1.x, (int)hi.x, v, false);
                    v = __builtin_amdgcn_sdot4(x1.y, (int)hi.y, v, false);
                    v = __builtin_amdgcn_sdot4(x1.z, (int)hi.z, v, false);
                    d[m] = __builtin_amdgcn_sdot4(x1.w, (int)hi.w, v, false);
                }
            }
#pragma unroll
            for (int t = 0; t < TPB; ++t)
#pragma unroll
                for (int m = 0; m < MR; ++m) acc[t][m] += (tq == t) ? d[m] : 0;
        }
    };
    // Windows ping-pong between the two register sets (longer K only); with
    // one set, a further window is requested after the previous one is used.
    auto run_windows = [&](auto&& use) {
        if constexpr (NW == 2) {
            for (int w = 0; w < NWIN; w += 2) {
                use(w, wa);
                if (w + 2 < NWIN) load_window(w + 2, wa);
                if (w + 1 < NWIN) {
                    use(w + 1, wb);
                    if (w + 3 < NWIN) load_window(w + 3, wb);
                }
            }
        } else {
            for (int w = 0; w < NWIN; ++w) {
                if (w > 0) load_window(w, wa);
                use(w, wa);
            }
        }
    };
    constexpr bool mfd = MR >= 2;
    if constexpr (mfd)
        run_windows(consume_mf);
    else
        run_windows(consume);

    // 5. Reduce over threads of the same column: lane moves within a wave, LDS
    // across waves; wave 0 finishes the 8 columns. (Matrix-core dots: lane L
    // holds rows 4 * (L >> 4) + 0..3 of column L & 15; column c < 8 is the
    // even-plane sum of lane c plus the odd-plane sum of lane c + 8.)
    if constexpr (mfd) {
#pragma unroll
        for (int t = 0; t < TPB; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int v = accE[t][i] + __shfl_down(accO[t][i], 8, 16);
                const int m = 4 * (lane >> 4) + i;
                if ((lane & 15) < 8 && m < MR) red[wave][t][m][lane & 7] = v;
            }
    } else {
#pragma unroll
        for (int t = 0; t < TPB; ++t)
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                int v = acc[t][m];
                v = sum_mod8(v);
                if (lane < 8) red[wave][t][m][c8] = v;
            }
    }
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    if constexpr (SPLITK) {
        // One device-scope 64-bit add per column returns the slot as it was:
        // the piece that finds ksplit - 1 pieces counted holds the whole sum
        // (earlier adds are performed before it, being atomics on the same
        // slot), writes the column and clears the slot for the next call.
        if (wave == 0) {
            constexpr unsigned long long ONE = 1ull << 40, BIAS = 1ull << 31, LOW = ONE - 1;
            int tot = 0;
#pragma unroll
            for (int w = 0; w < NWV; ++w) tot += red[w][0][0][c8];
            const unsigned long long mine = ONE + (unsigned long long)((long long)(tot - corr[0]) + (long long)BIAS);
            unsigned long long* slot = P.kacc + 8 * tile[0] + c8;
            const unsigned long long last = (unsigned long long)(P.ksplit - 1);
            if (lane < 8) {
                const unsigned long long was = __hip_atomic_fetch_add(slot, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if ((was >> 40) == last) {
                    const long long total = (long long)((was + mine) & LOW) - (long long)(P.ksplit * BIAS);
                    // every piece has added: clear the slot for the next call
                    __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    const float y = ((float)(int)total * scale[0]) * cs[0];
                    const int p = 8 * tile[0] + c8;
                    if (P.M > 0 && p < P.N) store_out(P.c, P.c_type, orig_col(p, P.half), y);
                }
            }
            if (lane == 0 && grp == 0 && P.diag_codes) {
                const unsigned long long sm = ONE + (unsigned long long)((long long)row_isum[0] + (long long)BIAS);
                unsigned long long* row_slot = P.kacc + P.N_pad;
                const unsigned long long was = __hip_atomic_fetch_add(row_slot, sm, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if ((was >> 40) == last) {
                    P.diag_rowsum[0] = (int)((long long)((was + sm) & LOW) - (long long)(P.ksplit * BIAS));
                    __hip_atomic_store(row_slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }

        }
        return;
    }
    if (wave == 0) {
#pragma unroll
        for (int gp = 0; gp < GPB; ++gp) {
            const int g = g0 + gp;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const bool row_ok = m < P.M;
                float y[TPG];
#pragma unroll
                for (int t = 0; t < TPG; ++t) {
                    const int tt = gp * TPG + t;
                    int tot = 0;
#pragma unroll
                    for (int w = 0; w < NWV; ++w) tot += red[w][tt][m][c8];
                    y[t] = ((float)(tot - corr[m]) * scale[m]) * cs[tt];
                }
                const int p = 8 * tile[gp * TPG] + c8;
                if (EPI == EPI_PLAIN) {
                    if constexpr (FUSE == FUSE_COMBINE) {
                        // ranks in order, single-rounding fma, then the add
                        float sum = 0.0f;
#pragma unroll
                        for (int r = 0; r < GEMV_COMB_TOP; ++r)
                            if (r < P.comb_top && comb_r[r] > 0.0f) sum = __builtin_fmaf(comb_c[r], comb_r[r], sum);
                        if (lane < 8 && row_ok && p < P.N)
                            static_cast<float*>(P.c)[(size_t)m * P.ldc + orig_col(p, P.half)] = sum + y[0];
                    } else {
                        if (lane < 8 && row_ok && p < P.N)
                            store_out(P.c, P.c_type, (size_t)m * P.ldc + orig_col(p, P.half), y[0]);
                    }
                } else {
                    const float o = hm_swiglu(y[0], y[TPG - 1]);
                    const size_t oi = (size_t)m * P.ldc + ((p >> 6) << 5) + (p & 31);
                    if constexpr (FUSE == FUSE_PRODUCER) {
                        // f32 middle, stored at agent scope for the consumers
                        if (lane < 8 && row_ok && p < P.N)
                            __hip_atomic_store(static_cast<float*>(P.c) + oi, o, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                    } else {
                        if (lane < 8 && row_ok && p < P.N) store_out(P.c, P.c_type, oi, o);
                    }
                    if (EPI == EPI_SWIGLU_MAX) {
                        float mxo = (lane < 8 && p < P.N) ? fabsf(o) : 0.0f;
                        mxo = max8(mxo);
                        if constexpr (FUSE == FUSE_PRODUCER) {
                            if (lane == 0 && row_ok)
                                __hip_atomic_fetch_max(FfnSync{P.sync}.mx(bid % FFN_SLOTS), max_bits(mxo),
                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        } else {
                            if (lane == 0) P.part_out[(size_t)m * groups + g] = row_ok ? mxo : 0.0f;
                        }
                    }
                }
            }
        }
        if constexpr (FUSE == FUSE_PRODUCER) {
            // Publish: the middle values and the max have completed at agent
            // scope before the arrival is counted.
            wait_vmcnt<0>();
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            if (lane == 0) ffn_producer_arrive(P, bid);
        }
    }
}

template <typename T, int MR, int BITS, int EPI, int RW, int NW, bool PREQ, int GPB = 1, int NTHR = 256,
          bool GROUPED = false, int QWN = 0, bool SPLITK = false>
__global__ __launch_bounds__(NTHR + 64 * QWN) void gemv_kernel(GemvParams P) {
    extern __shared__ __attribute__((aligned(16))) int8_t sa[];
    gemv_block<T, MR, BITS, EPI, RW, NW, PREQ, GPB, NTHR, GROUPED, QWN, SPLITK>(P, blockIdx.x, gridDim.x, sa);
}

// The plain one-row GEMV whose epilogue also combines a token's routed
// expert contributions with its value (the MoE shared expert's down
// projection at one token; GemvParams::comb_*).
template <int BITS, int RW>
__global__ __launch_bounds__(256) void gemv_combine_kernel(GemvParams P) {
    extern __shared__ __attribute__((aligned(16))) int8_t sa[];
    gemv_block<float, 1, BITS, EPI_PLAIN, RW, 1, false, 1, 256, false, 0, false, FUSE_COMBINE>(P, blockIdx.x, gridDim.x,
                                                                                             sa);
}

// The FFN of one row in one launch. Block b first computes gate/up tile pair
// b (b < G.producers: a quantization wave and 192 weight threads, `RWG`
// rounds of weights, the SwiGLU middle values published at agent scope),
// then K piece b of the down projection (b < Dn.consumers: 256 threads,
// `RWD` rounds): it requests that piece's weights at once, waits (bounded)
// until every producer has published, quantizes its slice of the middle with
// the row's max and adds its split-K sums. Every block's down weights stream
// right after its own gate/up work, and no block holds a CU slot idle. The
// launch must be resident as a whole (the plan checks the occupancy), since a
// block waits for producers that may run later in launch order; if it is not
// (another workload holding CUs), the wait runs out and the error word says
// so. Results are bit-identical to the two-launch FFN: the same quantization,
// products and epilogues, with the middle's max taken over the producers'
// block maxima.
// Blocks of 256 threads, one wave per SIMD (five-wave blocks fit four, not
// five, to a CU here).
constexpr int FFN_WEIGHT_THREADS = 192;
constexpr int FFN_THREADS = FFN_WEIGHT_THREADS + 64;
template <typename TX, int BG, int RWG, int BD, int RWD>
__global__ __launch_bounds__(FFN_THREADS) void ffn_m1_kernel(GemvParams G, GemvParams Dn) {
    extern __shared__ __attribute__((aligned(16))) int8_t sa[];
    const int b = blockIdx.x;
    G.fuse_block = Dn.fuse_block = b;
    G.fuse_blocks = Dn.fuse_blocks = gridDim.x;
    if (b < G.producers)
        gemv_block<TX, 1, BG, EPI_SWIGLU_MAX, RWG, 1, false, 1, FFN_WEIGHT_THREADS, false, 1, false, FUSE_PRODUCER>(
            G, b, G.producers, sa);
    // (the producers' codes stay in the first K_pad bytes: some of its waves
    // may still read them while others start on the piece)
    if (b < Dn.consumers)
        gemv_block<float, 1, BD, EPI_PLAIN, RWD, 1, false, 1, FFN_THREADS, false, 0, true, FUSE_CONSUMER>(
            Dn, b, Dn.consumers, sa + G.K_pad);
    __syncthreads();
    if (threadIdx.x == 0) ffn_block_done(G);
}

}  // namespace hm

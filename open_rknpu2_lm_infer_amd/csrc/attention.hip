// FP16 grouped-query attention over a device KV cache: the rk_npu_attention_f16
// C ABI (include/rk_npu_attention_f16.h) and its kernels.
//
// Layout in HBM: a cache holds K and V as [kv_heads][capacity][head_dim] fp16
// (one contiguous head_dim row per key). A run takes Q as
// [query_heads][rows][head_dim] fp16 and writes [query_heads][rows][head_dim]
// f32 or fp16. Math is f32: q is scaled by softmax_scale on load, scores are
// f32 dot products, the softmax is online (running max and sum, the
// accumulators rescaled when the max grows), and the output is the
// accumulated sum of p * v divided by the sum of p.
//
// Work split: block = (key split, tile of RT query rows, KV head). The query
// rows of one KV head are its (query head of the group, query row) pairs, so
// the group's heads share every K/V tile read. A block streams 64-key tiles
// of K then V through LDS; a decode-sized call (few rows) spreads the keys
// over many splits whose partial (max, sum, accumulators) a second launch
// combines.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>

#include "../../include/rk_npu_attention_f16.h"
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wunused-function"  // (the header's other kernels)
#include "kernels.hpp"
#pragma clang diagnostic pop
#include "runtime.hpp"

namespace hm {

constexpr uint32_t MAGIC_ATTN_CACHE = 0x43414841u;
constexpr uint32_t MAGIC_ATTN_WORK = 0x57414841u;
constexpr int ATTN_KT = 64;              // keys per tile
constexpr int ATTN_MAX_SPLITS = 256;     // key splits per (KV head, row tile)
// Partial rows a workspace holds: plan_attention launches at most 2048
// blocks when it splits the keys, each with at most 128 query rows (head_dim
// 64 and 128, MFMA tiles) or 16 (head_dim 256).
static inline size_t attn_partial_rows(int head_dim) { return (size_t)2048 * (head_dim <= 128 ? 64 : 16); }

struct AttnParams {
    const __half* q;  // [qh][m][D]
    const __half* k;  // [kh][cap][D]
    const __half* v;
    void* out;        // [qh][m][D], f32 or fp16
    int out_f16;
    float* part;      // [kh][row_tiles*RT][splits][D + 2]: max, sum, accumulators
    int qh, kh, m, cap, len, pos, causal;
    float scale;
    int splits, keys_per_split, row_tiles, key_end;
    int rows_pad;     // row_tiles * RT: partial rows per KV head
};

// max / sum over the N consecutive lanes (N = 16 or 64) that share a query row
template <int N>
__device__ __forceinline__ float group_max(float v) {
    v = fmaxf(v, dpp_move<DPP_QUAD_XOR1>(v));
    v = fmaxf(v, dpp_move<DPP_QUAD_XOR2>(v));
    v = fmaxf(v, dpp_move<DPP_ROW_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_move<DPP_ROW_MIRROR>(v));
    if constexpr (N == 64) {
        v = fmaxf(v, dpp_move<DPP_ROW_BCAST15, 0xa>(v));
        v = fmaxf(v, dpp_move<DPP_ROW_BCAST31, 0xc>(v));
        v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    }
    return v;
}
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    v = v + dpp_move<DPP_QUAD_XOR1>(v);
    v = v + dpp_move<DPP_QUAD_XOR2>(v);
    v = v + dpp_move<DPP_ROW_HALF_MIRROR>(v);
    v = v + dpp_move<DPP_ROW_MIRROR>(v);
    if constexpr (N == 64) {
        v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), DPP_ROW_BCAST15,
                                                                      0xa, 0xf, false));
        v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), DPP_ROW_BCAST31,
                                                                      0xc, 0xf, false));
        v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    }
    return v;
}

// Block: 256 threads; RT query rows (RT = 4: 64 threads per row, RT = 16: 16
// threads per row). Thread (row, sub) scores keys sub + RPT*i of each tile
// and owns output dims [sub*DPT, sub*DPT + DPT) of its row. K/V tiles (64
// keys, 32 at head_dim 256) go through two LDS buffers; the next tile's loads
// are in flight (registers) while the current tile is computed. Scores are
// v_dot2_f32_f16 sums over the fp16 q and k pairs (exact products, f32
// accumulation) times the scale; p * v folds the fp16 conversion into the
// multiply-add.
template <int D, int RT>
__global__ __launch_bounds__(256) void attn_split_kernel(AttnParams P) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    constexpr int KT = D == 256 ? 32 : ATTN_KT;      // keys per tile
    constexpr int RPT = 256 / RT;                    // threads per row
    constexpr int SPT = KT >= RPT ? KT / RPT : 1;    // scores per thread per tile
    constexpr int DPT = D / RPT;                     // output dims per thread
    constexpr int KP = D + 8;                        // LDS row pitch of a K/V tile (halves)
    constexpr int PER = (KT * (D / 8) + 255) / 256;  // 16-byte K (and V) pieces per thread per tile
    constexpr int QPT = RT * D / 256;                // q halves per thread (2..16)
    static_assert(DPT >= 1 && D % RPT == 0 && D % 8 == 0 && (QPT == 1 || QPT % 2 == 0),
                  "head_dim must split over the threads");
    constexpr int QW = QPT >= 2 ? QPT / 2 : 1;  // q words per thread (QPT = 1: one half)
    __shared__ __attribute__((aligned(16))) __half qs[RT][D];
    __shared__ __attribute__((aligned(16))) __half ks[KT][KP];
    __shared__ __attribute__((aligned(16))) __half vs[KT][KP];
    __shared__ float ps[RT][KT];
    const int split = blockIdx.x, rt = blockIdx.y, g = blockIdx.z;
    const int G = P.qh / P.kh, R = G * P.m;
    const int tid = threadIdx.x, row = tid / RPT, sub = tid % RPT;
    const int rr = rt * RT + row;
    const bool row_ok = rr < R;
    const int gi = row_ok ? rr / P.m : 0, qr = row_ok ? rr % P.m : 0;
    int klimit = P.len;  // keys [0, klimit) are visible to this row
    if (P.causal) klimit = min(klimit, P.pos + qr + 1);
    const int k0 = split * P.keys_per_split;
    const int k1 = min(k0 + P.keys_per_split, P.key_end);
    const __half* kbase = P.k + (size_t)g * P.cap * D;
    const __half* vbase = P.v + (size_t)g * P.cap * D;
    // q: thread's QPT halves of the [RT][D] tile, one load (rows past R: 0)
    const int qe = tid * QPT, qrow = qe / D, qcol = qe % D, qrr = rt * RT + qrow;
    const bool q_ok = qrr < R;
    const __half* qsrc = P.q + ((size_t)(g * G + (q_ok ? qrr / P.m : 0)) * P.m + (q_ok ? qrr % P.m : 0)) * D + qcol;
    unsigned qv[QW];
#pragma unroll
    for (int i = 0; i < QW; ++i)
        qv[i] = QPT == 1 ? (unsigned)reinterpret_cast<const unsigned short*>(qsrc)[0]
                         : reinterpret_cast<const unsigned*>(qsrc)[i];
    v4u kr[PER], vr[PER];
    auto issue = [&](int kb) {
#pragma unroll
        for (int t = 0; t < PER; ++t) {
            const int i = tid + 256 * t, j = i / (D / 8), c = i % (D / 8), key = kb + j;
            const bool ok = i < KT * (D / 8) && key < k1;
            const size_t off = ok ? (size_t)key * D + c * 8 : 0;  // (masked: a valid row, zeroed at the store)
            kr[t] = *reinterpret_cast<const v4u*>(kbase + off);
            vr[t] = *reinterpret_cast<const v4u*>(vbase + off);
        }
    };
    auto store = [&](int kb) {
#pragma unroll
        for (int t = 0; t < PER; ++t) {
            const int i = tid + 256 * t, j = i / (D / 8), c = i % (D / 8), key = kb + j;
            if (i < KT * (D / 8)) {
                const bool ok = key < k1;
                *reinterpret_cast<v4u*>(&ks[j][c * 8]) = ok ? kr[t] : v4u{0u, 0u, 0u, 0u};
                *reinterpret_cast<v4u*>(&vs[j][c * 8]) = ok ? vr[t] : v4u{0u, 0u, 0u, 0u};
            }
        }
    };
    if (k0 < k1) issue(k0);
    if constexpr (QPT == 1) {
        reinterpret_cast<unsigned short*>(&qs[qrow][qcol])[0] = q_ok ? (unsigned short)qv[0] : (unsigned short)0;
    } else {
#pragma unroll
        for (int i = 0; i < QW; ++i) reinterpret_cast<unsigned*>(&qs[qrow][qcol])[i] = q_ok ? qv[i] : 0u;
    }
    float mrun = -INFINITY, lrun = 0.0f;
    float acc[DPT];
#pragma unroll
    for (int e = 0; e < DPT; ++e) acc[e] = 0.0f;
    for (int kb = k0; kb < k1; kb += KT) {
        __syncthreads();  // (the previous tile's reads are done)
        store(kb);
        __syncthreads();
        if (kb + KT < k1) issue(kb + KT);  // next tile in flight during this one
        float s[SPT];
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const int j = sub + RPT * i;
            float a = 0.0f;
            if (j < KT) {
#pragma unroll 4
                for (int c = 0; c < D; c += 8) {
                    const v4u kw = *reinterpret_cast<const v4u*>(&ks[j][c]);
                    const v4u qw = *reinterpret_cast<const v4u*>(&qs[row][c]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const unsigned qu = qw[e], ku = kw[e];  // (copied out before the bit casts)
                        a = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, qu), __builtin_bit_cast(h2, ku), a, false);
                    }
                }
            }
            const int key = kb + j;
            s[i] = (row_ok && j < KT && key < klimit && key < k1) ? a * P.scale : -INFINITY;
            tmax = fmaxf(tmax, s[i]);
        }
        tmax = group_max<RPT>(tmax);
        const float mnew = fmaxf(mrun, tmax);
        // (a row with no visible key yet keeps max -inf, sum 0, scale 1)
        const float alpha = (mnew == -INFINITY) ? 1.0f : __expf(mrun - mnew);
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const float p = (s[i] == -INFINITY) ? 0.0f : __expf(s[i] - mnew);
            if (sub + RPT * i < KT) ps[row][sub + RPT * i] = p;
            psum += p;
        }
        psum = group_sum<RPT>(psum);
        lrun = lrun * alpha + psum;
        mrun = mnew;
#pragma unroll
        for (int e = 0; e < DPT; ++e) acc[e] *= alpha;
        __syncthreads();  // (p written)
#pragma unroll 4
        for (int j = 0; j < KT; ++j) {
            const float p = ps[row][j];
#pragma unroll
            for (int e = 0; e < DPT; ++e) acc[e] = __builtin_fmaf(p, __half2float(vs[j][sub * DPT + e]), acc[e]);
        }
    }
    if (!row_ok) return;
    const int h = g * G + gi;
    if (P.splits == 1) {
        const float inv = 1.0f / lrun;
        const size_t o = ((size_t)h * P.m + qr) * D + sub * DPT;
#pragma unroll
        for (int e = 0; e < DPT; ++e) {
            const float y = acc[e] * inv;
            if (P.out_f16)
                static_cast<__half*>(P.out)[o + e] = __float2half_rn(y);
            else
                static_cast<float*>(P.out)[o + e] = y;
        }
        return;
    }
    float* part = P.part + (((size_t)g * P.rows_pad + rr) * P.splits + split) * (D + 2);
    if (sub == 0) {
        part[0] = mrun;
        part[1] = lrun;
    }
#pragma unroll
    for (int e = 0; e < DPT; ++e) part[2 + sub * DPT + e] = acc[e];
}

// Matrix-core variant for 16 or more query rows per KV head (head_dim 64 or
// 128). Block = NW waves (4 or 8), each owning 16 query rows of one KV head, over
// 64-key tiles of its key split; the K/V tile is shared by the block. Per
// tile, with v_mfma_f32_16x16x32_f16 (fp16 operands, f32 accumulation):
//   S^T = K Q^T   A = K rows from LDS, B = Q fragments held in registers;
//                 the accumulator gives lane l the raw scores of query row
//                 l%16 for keys 4(l/16)..+3 of each 16-key block,
//   softmax       weights p = 2^(s c - m) with c = scale * log2(e) and m the
//                 row's running max in those units, rounded to fp16 in place;
//                 m moves only when a row's max grows by more than ATTN_LAZY
//                 (so p <= 2^ATTN_LAZY, which fp16 holds), and only then are
//                 the accumulators and sums rescaled: each lane compares the
//                 max of its own 16 scores with that bound, and the row max
//                 over the row's 4 lanes is formed only when one passes it,
//   O^T += V^T P^T  A = V^T fragments, B = the weights as they lie (the
//                 accumulator layout of S^T is the B layout of P^T once each
//                 lane's 8 k-slots name keys {4(l/16)..+3, 16+4(l/16)..+3} of
//                 a 32-key step, which the A fragments are read to match),
// so a lane's O^T accumulators all belong to its own query row and every
// rescale is lane-local; each lane keeps a partial sum of its own weights
// (v_dot2 against ones: the fp16 weights summed exactly in f32), added over
// the row's 4 lanes at the end. Masks (causal, keys past the split) apply
// only on tiles that cross them.
// Tiles reach LDS in one of two ways:
//   8 waves (one block per CU): direct global->LDS loads into three tile
//     buffers, K and V row-major (key, dim) in 16-byte slots permuted within
//     each row against bank conflicts; tile t + 2 is requested after tile t's
//     last LDS reads, into the buffer of tile t - 1 (every wave has passed
//     tile t's barrier, so it is free), one barrier per tile; V^T fragments
//     come from transposing LDS reads (ds_read_b64_tr_b16);
//   4 waves (several blocks per CU, where 96 KB of tile buffers would leave
//     one): the next tile's K/V in registers while this one is used, stored
//     between two barriers, V transposed on the way in (each 32-key chunk's
//     4-key groups in the order 0 4 1 5 2 6 3 7, so a lane's 8 k-slots are
//     one 16-byte read).
// Operand layouts (16x16x32, wave64): A lane l = row l%16, k-slots
// 8(l/16)..+7; B lane l = column l%16, same k-slots; C lane l = rows
// 4(l/16)..+3 of column l%16.
constexpr float ATTN_LAZY = 8.0f;

// Max / sum over the 4 lanes l % 16 + 16 j (a query row's lanes in the
// accumulator layout), in each of them: v_permlane16_swap exchanges odd with
// even 16-lane rows and v_permlane32_swap the upper with the lower half, so
// each swap's two results are a lane pair 16 (then 32) apart, without an LDS
// round trip.
__device__ __forceinline__ float max_rows4(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_rows4(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int D, int NW>
__global__ __launch_bounds__(64 * NW) void attn_mfma_kernel(AttnParams P) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    typedef _Float16 hh2 __attribute__((ext_vector_type(2)));
    typedef float f4 __attribute__((ext_vector_type(4)));
    typedef unsigned u2 __attribute__((ext_vector_type(2)));
    typedef short s4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s4 lds_s4;
    constexpr int KT = ATTN_KT, KS = D / 32, NB = D / 16;
    constexpr int NT = 64 * NW;
    constexpr bool DMA = NW == 8;
    static_assert(D == 64 || D == 128, "MFMA attention: head_dim 64 or 128");
    static_assert(KT == 64, "tile shape");
    // direct loads: 16-byte slots per row, bytes of one matrix of a tile,
    // slots per thread per matrix, tile buffers
    constexpr int SPR = D / 8, MAT = KT * D * 2, DPT = KT * SPR / NT, NBUF = 3;
    static_assert(!DMA || KT * SPR % NT == 0, "tile shape");
    // register path: row pads against LDS bank conflicts in the fragment
    // reads (pads of 16 halves measured fastest), 16-byte K pieces per tile,
    // V pieces of 4 keys x 8 dims per tile
    constexpr int KP = D + 16, VP = KT + 16;
    constexpr int KPIECES = KT * (D / 8), VPIECES = (KT / 4) * (D / 8), KPT = KPIECES / NT;
    static_assert(DMA || (KPIECES % NT == 0 && VPIECES <= NT), "tile shape");
    constexpr int SMEM = DMA ? NBUF * 2 * MAT : (KT * KP + D * VP) * 2;
    __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];
    auto ks = reinterpret_cast<__half (*)[KP]>(smem);
    auto vt = reinterpret_cast<__half (*)[VP]>(smem + KT * KP * 2);

    const int split = blockIdx.x, rt = blockIdx.y, g = blockIdx.z;
    const int G = P.qh / P.kh, R = G * P.m;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lo = lane & 15, hi = lane >> 4;
    const int k0 = split * P.keys_per_split;
    const int k1 = min(k0 + P.keys_per_split, P.key_end);
    const float c = P.scale * 1.4426950408889634f;
    const __half* kbase = P.k + (size_t)g * P.cap * D;
    const __half* vbase = P.v + (size_t)g * P.cap * D;
    // this lane's query row, its key limit and Q fragments
    const int rr = rt * (16 * NW) + wave * 16 + lo;
    const bool row_ok = rr < R;
    int lim = 0;
    if (row_ok) {
        lim = P.len;
        if (P.causal) lim = min(lim, P.pos + rr % P.m + 1);
    }
    // keys below `open` are visible to every row of this wave (rows past R
    // are discarded, so they do not count)
    int open = row_ok ? lim : 0x7fffffff;
    open = min(open, __shfl_xor(open, 1));
    open = min(open, __shfl_xor(open, 2));
    open = min(open, __shfl_xor(open, 4));
    open = min(open, __shfl_xor(open, 8));
    open = __builtin_amdgcn_readfirstlane(min(open, k1));  // (uniform: a scalar branch below)
    h8 qf[KS];
    {
        const __half* qp = P.q + ((size_t)(g * G + (row_ok ? rr / P.m : 0)) * P.m + (row_ok ? rr % P.m : 0)) * D;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const v4u x = row_ok ? *reinterpret_cast<const v4u*>(qp + 32 * k + 8 * hi) : v4u{0u, 0u, 0u, 0u};
            qf[k] = __builtin_bit_cast(h8, x);
        }
    }

    // --- direct loads. Slot c of row r lies at c ^ swk(r) (K: 16 consecutive
    // rows take 16 distinct slots of one logical column, which the score
    // fragments read per 16 lanes) or c ^ swv(r) (V: 8 consecutive rows take
    // distinct slot pairs 2c, 2c + 1, the 32 bytes of each of 8 rows a half
    // wave's transposing reads take).
    auto swk = [](int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); };
    auto swv = [](int r) { return D == 128 ? 2 * (r & 7) : 2 * ((r >> 1) & 3); };
    // this thread's slots: physical slot t * NT + tid of each matrix -> row,
    // and the logical slot (16-byte column) it holds
    int drow[DMA ? DPT : 1], dkc[DMA ? DPT : 1], dvc[DMA ? DPT : 1];
    if constexpr (DMA) {
#pragma unroll
        for (int t = 0; t < DPT; ++t) {
            const int pslot = t * NT + tid, r = pslot / SPR, ps = pslot % SPR;
            drow[t] = r;
            dkc[t] = ps ^ swk(r);
            dvc[t] = ps ^ swv(r);
        }
    }
    // keys past the split read the split's last key (finite data; masked)
    auto issue_dma = [&](int kb, int buf) {
        const char* kt = reinterpret_cast<const char*>(kbase + (size_t)kb * D);
        const char* vtp = reinterpret_cast<const char*>(vbase + (size_t)kb * D);
        const int last = k1 - 1 - kb;
        uint8_t* dst = smem + buf * 2 * MAT + (wave * 64) * 16;
#pragma unroll
        for (int t = 0; t < DPT; ++t) {
            const int r = min(drow[t], last);
            lds_dma16(kt + (r * D + dkc[t] * 8) * 2, dst + t * NT * 16);
            lds_dma16(vtp + (r * D + dvc[t] * 8) * 2, dst + MAT + t * NT * 16);
        }
    };

    // --- register path. K piece i: key i / (D/8), dims 8 (i % (D/8)); V
    // piece (tid): keys 4 (tid % 16)..+3, dims 8 (tid / 16)..+7
    const bool vthread = tid < VPIECES;
    const int vj = tid & 15, vc = tid >> 4;
    // byte offsets within a tile (the tile base is uniform): K piece t, V row t
    unsigned koff[DMA ? 1 : KPT], voff[4];
    v4u kr[DMA ? 1 : KPT], vr[4];
    if constexpr (!DMA) {
#pragma unroll
        for (int t = 0; t < KPT; ++t) {
            const int i = tid + NT * t;
            koff[t] = (unsigned)((i / (D / 8)) * D + (i % (D / 8)) * 8) * 2u;
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) voff[t] = (unsigned)((4 * vj + t) * D + vc * 8) * 2u;
    }
    auto issue_regs = [&](int kb) {
        const char* kt = reinterpret_cast<const char*>(kbase + (size_t)kb * D);
        const char* vtp = reinterpret_cast<const char*>(vbase + (size_t)kb * D);
        if (kb + KT <= k1) {  // (uniform) whole tile inside the split
#pragma unroll
            for (int t = 0; t < KPT; ++t) kr[t] = *reinterpret_cast<const v4u*>(kt + koff[t]);
            if (vthread) {
#pragma unroll
                for (int t = 0; t < 4; ++t) vr[t] = *reinterpret_cast<const v4u*>(vtp + voff[t]);
            }
        } else {  // keys past the split read the tile's first row (zeroed in store)
#pragma unroll
            for (int t = 0; t < KPT; ++t) {
                const int key = kb + (tid + NT * t) / (D / 8);
                kr[t] = *reinterpret_cast<const v4u*>(kt + (key < k1 ? koff[t] : 0u));
            }
            if (vthread) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int key = kb + 4 * vj + t;
                    vr[t] = *reinterpret_cast<const v4u*>(vtp + (key < k1 ? voff[t] : 0u));
                }
            }
        }
    };
    auto store_regs = [&](int kb) {
        if (kb + KT > k1) {  // (block-uniform) zero the keys past the split
#pragma unroll
            for (int t = 0; t < KPT; ++t)
                if (kb + (tid + NT * t) / (D / 8) >= k1) kr[t] = v4u{0u, 0u, 0u, 0u};
#pragma unroll
            for (int t = 0; t < 4; ++t)
                if (kb + 4 * vj + t >= k1) vr[t] = v4u{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int t = 0; t < KPT; ++t) {
            const int i = tid + NT * t;
            *reinterpret_cast<v4u*>(&ks[i / (D / 8)][(i % (D / 8)) * 8]) = kr[t];
        }
        if (vthread) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int cw = e >> 1;
                u2 x;
                if (e & 1) {
                    x[0] = (vr[0][cw] >> 16) | (vr[1][cw] & 0xffff0000u);
                    x[1] = (vr[2][cw] >> 16) | (vr[3][cw] & 0xffff0000u);
                } else {
                    x[0] = (vr[0][cw] & 0xffffu) | (vr[1][cw] << 16);
                    x[1] = (vr[2][cw] & 0xffffu) | (vr[3][cw] << 16);
                }
                const int lg = vj & 7, pos = lg < 4 ? 2 * lg : 2 * lg - 7;
                *reinterpret_cast<u2*>(&vt[vc * 8 + e][32 * (vj >> 3) + 4 * pos]) = x;
            }
        }
    };

    f4 o[NB];
#pragma unroll
    for (int n = 0; n < NB; ++n) o[n] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    float mrun = -INFINITY, lpart = 0.0f;
    const hh2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    if constexpr (DMA) {
        if (k0 < k1) issue_dma(k0, 0);
        if (k0 + KT < k1) issue_dma(k0 + KT, 1);
    } else {
        if (k0 < k1) issue_regs(k0);
    }
    int buf = 0;
    for (int kb = k0; kb < k1; kb += KT) {
        const uint8_t* kst = smem + buf * 2 * MAT;
        const uint8_t* vst = kst + MAT;
        if constexpr (DMA) {
            if (kb + KT < k1)
                wait_vmcnt<2 * DPT>();  // (this thread's loads of the tile have landed; the next tile's may not)
            else
                wait_vmcnt<0>();
            __syncthreads();  // (every thread's have)
        } else {
            __syncthreads();  // (the previous tile's LDS reads are done)
            store_regs(kb);
            __syncthreads();
            if (kb + KT < k1) issue_regs(kb + KT);
        }
        // (k outermost: the 4 key blocks' products are independent, so they
        // issue back to back instead of waiting on each other)
        f4 sacc[4];
        h8 ka[4][KS];
#pragma unroll
        for (int k = 0; k < KS; ++k)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                const void* src = DMA ? static_cast<const void*>(kst + (cb * 16 + lo) * (D * 2) +
                                                                ((4 * k + hi) ^ swk(lo)) * 16)
                                      : static_cast<const void*>(&ks[cb * 16 + lo][32 * k + 8 * hi]);
                ka[cb][k] = __builtin_bit_cast(h8, *reinterpret_cast<const v4u*>(src));
            }
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) sacc[cb] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < KS; ++k)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
                sacc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[cb][k], qf[k], sacc[cb], 0, 0, 0);
        if (__builtin_expect(kb + KT > open, 0)) {  // (uniform) the tile crosses a mask
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = kb + cb * 16 + 4 * hi + r;
                    if (!(key < lim && key < k1)) sacc[cb][r] = -INFINITY;
                }
        }
        // the lane's max of its 16 scores (3-input maxima); the row max only
        // when some lane's max passes its row's bound
        float lmax = -INFINITY;
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
            lmax = __builtin_elementwise_maximum(
                __builtin_elementwise_maximum(lmax, __builtin_elementwise_maximum(sacc[cb][0], sacc[cb][1])),
                __builtin_elementwise_maximum(sacc[cb][2], sacc[cb][3]));
        if (__builtin_expect(__builtin_amdgcn_ballot_w64(lmax * c > mrun + ATTN_LAZY) != 0, 0)) {  // (uniform)
            const float tm = max_rows4(lmax) * c;
            float alpha = 1.0f;
            if (tm > mrun + ATTN_LAZY) {
                alpha = __builtin_amdgcn_exp2f(mrun - tm);  // (0 from -inf)
                mrun = tm;
            }
            lpart *= alpha;
#pragma unroll
            for (int n = 0; n < NB; ++n) o[n] *= alpha;
        }
        const float msub = (mrun == -INFINITY) ? 0.0f : mrun;  // (no visible key yet: all scores -inf)
        h8 pb[2];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
#pragma unroll
            for (int r = 0; r < 4; r += 2) {
                const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[cb][r], c, -msub));
                const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[cb][r + 1], c, -msub));
                const hh2 ph = {(_Float16)p0, (_Float16)p1};
                pb[cb >> 1][(cb & 1) * 4 + r] = ph[0];
                pb[cb >> 1][(cb & 1) * 4 + r + 1] = ph[1];
                lpart = __builtin_amdgcn_fdot2(ph, ones, lpart, false);
            }
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {  // (k outermost: the NB products are independent)
            h8 va[NB];
#pragma unroll
            for (int n = 0; n < NB; ++n) {
                if constexpr (DMA) {
                    // transposing reads: lane j of a 16-lane group names dims
                    // 4 (j % 4)..+3 of key row 4 (j / 4) of the group's 16
                    // keys; lane i receives dim i of the rows named by lanes
                    // i / 4, 4 + i / 4, 8 + i / 4, 12 + i / 4: its dim of keys
                    // 4 hi..+3 (then of keys 16 + 4 hi..+3) of the step
                    const int vr0 = 32 * k + 4 * hi + (lo >> 2);
                    const uint8_t* p =
                        vst + vr0 * (D * 2) + (((2 * n + ((lo & 3) >> 1)) ^ swv(vr0)) * 16) + (lo & 1) * 8;
                    const s4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)p);
                    const s4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p + 16 * (D * 2)));
                    const u2 ua = __builtin_bit_cast(u2, a), ub = __builtin_bit_cast(u2, b);
                    va[n] = __builtin_bit_cast(h8, v4u{ua[0], ua[1], ub[0], ub[1]});
                } else {
                    va[n] = __builtin_bit_cast(h8, *reinterpret_cast<const v4u*>(&vt[16 * n + lo][32 * k + 8 * hi]));
                }
            }
#pragma unroll
            for (int n = 0; n < NB; ++n) o[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[n], pb[k], o[n], 0, 0, 0);
        }
        if constexpr (DMA) {
            // (the compiler waits for every direct load in flight before a
            // transposing read, so the request comes after this tile's)
            if (kb + 2 * KT < k1) issue_dma(kb + 2 * KT, buf == 0 ? NBUF - 1 : buf - 1);
            buf = buf == NBUF - 1 ? 0 : buf + 1;
        }
    }
    float l = lpart;
    l = sum_rows4(l);
    if (!row_ok) return;
    const int h = g * G + rr / P.m, qr = rr % P.m;
    if (P.splits == 1) {
        const float inv = 1.0f / l;
        const size_t o0 = ((size_t)h * P.m + qr) * D + 4 * hi;
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const f4 y = o[n] * inv;
            if (P.out_f16) {
                const unsigned short b0 = __half_as_ushort(__float2half_rn(y[0]));
                const unsigned short b1 = __half_as_ushort(__float2half_rn(y[1]));
                const unsigned short b2 = __half_as_ushort(__float2half_rn(y[2]));
                const unsigned short b3 = __half_as_ushort(__float2half_rn(y[3]));
                *reinterpret_cast<u2*>(static_cast<__half*>(P.out) + o0 + 16 * n) =
                    u2{b0 | ((unsigned)b1 << 16), b2 | ((unsigned)b3 << 16)};
            } else {
                *reinterpret_cast<f4*>(static_cast<float*>(P.out) + o0 + 16 * n) = y;
            }
        }
    } else {
        // partial: running max in natural-log units as the combine expects
        float* part = P.part + (((size_t)g * P.rows_pad + rr) * P.splits + split) * (D + 2);
        if (hi == 0) {
            part[0] = (mrun == -INFINITY) ? -INFINITY : mrun * 0.6931471805599453f;
            part[1] = l;
        }
#pragma unroll
        for (int n = 0; n < NB; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) part[2 + 16 * n + 4 * hi + r] = o[n][r];
    }
}

// Combine the key splits of one (KV head, row): block = (row, KV head).
// Thread t takes split t for the max M and the weight w_t = exp(m_t - M) (0
// for a split that saw no key) and the denominator sum_t w_t l_t; then wave w
// takes splits w, w + 4, ... for all head dims (lane + 64 j), loading up to 16
// splits at once so their latencies overlap; the 4 waves' sums meet in LDS:
// out = sum_s w_s acc_s / sum_s w_s l_s.
template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnParams P) {
    constexpr int ND = D / 64;  // dims per lane
    constexpr int B = 16;       // splits loaded at once per wave
    constexpr size_t STRIDE = D + 2;
    static_assert(ATTN_MAX_SPLITS <= 256, "one thread per split");
    __shared__ float w_s[256];
    __shared__ float red[2][4];
    __shared__ float sums[4][D];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rr = blockIdx.x, g = blockIdx.y;
    const int G = P.qh / P.kh, R = G * P.m;
    if (rr >= R) return;  // (block-uniform)
    const int h = g * G + rr / P.m, qr = rr % P.m;
    const int S = P.splits;
    const float* p0 = P.part + ((size_t)g * P.rows_pad + rr) * S * STRIDE;
    // the first batch of accumulators is requested with the maxima and sums
    // (its addresses do not depend on them: one memory round trip)
    float v[B][ND];
#pragma unroll
    for (int u = 0; u < B; ++u) {
        const int sp = min(wave + 4 * u, S - 1);
#pragma unroll
        for (int d = 0; d < ND; ++d) v[u][d] = p0[sp * STRIDE + 2 + lane + 64 * d];
    }
    const float m = tid < S ? p0[tid * STRIDE] : -INFINITY;
    const float l = tid < S ? p0[tid * STRIDE + 1] : 0.0f;
    float mx = group_max<64>(m);
    if (lane == 0) red[0][wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    const float w = (m == -INFINITY) ? 0.0f : __expf(m - mx);
    w_s[tid] = w;
    const float den = group_sum<64>(w * l);
    if (lane == 0) red[1][wave] = den;
    __syncthreads();
    float num[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d) num[d] = 0.0f;
    for (int s0 = wave; s0 < S; s0 += 4 * B) {
        if (s0 != wave) {
#pragma unroll
            for (int u = 0; u < B; ++u) {
                const int sp = min(s0 + 4 * u, S - 1);
#pragma unroll
                for (int d = 0; d < ND; ++d) v[u][d] = p0[sp * STRIDE + 2 + lane + 64 * d];
            }
        }
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int sp = s0 + 4 * u;
            const float wi = sp < S ? w_s[sp] : 0.0f;
#pragma unroll
            for (int d = 0; d < ND; ++d) num[d] = __builtin_fmaf(wi, v[u][d], num[d]);
        }
    }
#pragma unroll
    for (int d = 0; d < ND; ++d) sums[wave][lane + 64 * d] = num[d];
    __syncthreads();
    if (wave == 0) {
        const float inv = 1.0f / ((red[1][0] + red[1][1]) + (red[1][2] + red[1][3]));
        const size_t o = ((size_t)h * P.m + qr) * D + lane;
#pragma unroll
        for (int d = 0; d < ND; ++d) {
            const int dd = lane + 64 * d;
            const float y = ((sums[0][dd] + sums[1][dd]) + (sums[2][dd] + sums[3][dd])) * inv;
            if (P.out_f16)
                static_cast<__half*>(P.out)[o + 64 * d] = __float2half_rn(y);
            else
                static_cast<float*>(P.out)[o + 64 * d] = y;
        }
    }
}

// The same combine for few splits (at most 64) over many rows: one wave per
// row, lane s holds split s's weight; the splits' accumulators are loaded B
// (8 or 16) at a time (dims lane + 64 j) and each weight is broadcast from
// its lane.
template <int D, int B>
__global__ __launch_bounds__(256) void attn_combine_rows_kernel(AttnParams P) {
    constexpr int ND = D / 64;
    constexpr size_t STRIDE = D + 2;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rr = blockIdx.x * 4 + wave, g = blockIdx.y;
    const int G = P.qh / P.kh, R = G * P.m;
    if (rr >= R) return;  // (wave-uniform; no barrier below)
    const int h = g * G + rr / P.m, qr = rr % P.m;
    const int S = P.splits;
    const float* p0 = P.part + ((size_t)g * P.rows_pad + rr) * S * STRIDE;
    // the first 16 splits' accumulators are loaded together with the maxima
    // and sums (one memory round trip for up to 16 splits)
    float v[B][ND];
#pragma unroll
    for (int u = 0; u < B; ++u) {
        const int sp = min(u, S - 1);
#pragma unroll
        for (int d = 0; d < ND; ++d) v[u][d] = p0[sp * STRIDE + 2 + lane + 64 * d];
    }
    const float m = lane < S ? p0[lane * STRIDE] : -INFINITY;
    const float l = lane < S ? p0[lane * STRIDE + 1] : 0.0f;
    const float mx = group_max<64>(m);
    const float w = (m == -INFINITY) ? 0.0f : __expf(m - mx);
    const float den = group_sum<64>(w * l);
    float num[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d) num[d] = 0.0f;
    for (int s0 = 0; s0 < S; s0 += B) {
        if (s0 > 0) {
#pragma unroll
            for (int u = 0; u < B; ++u) {
                const int sp = min(s0 + u, S - 1);
#pragma unroll
                for (int d = 0; d < ND; ++d) v[u][d] = p0[sp * STRIDE + 2 + lane + 64 * d];
            }
        }
#pragma unroll
        for (int u = 0; u < B; ++u) {
            // (lanes past S hold weight 0)
            const float wi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), s0 + u));
#pragma unroll
            for (int d = 0; d < ND; ++d) num[d] = __builtin_fmaf(wi, v[u][d], num[d]);
        }
    }
    const float inv = 1.0f / den;
    const size_t o = ((size_t)h * P.m + qr) * D + lane;
#pragma unroll
    for (int d = 0; d < ND; ++d) {
        const float y = num[d] * inv;
        if (P.out_f16)
            static_cast<__half*>(P.out)[o + 64 * d] = __float2half_rn(y);
        else
            static_cast<float*>(P.out)[o + 64 * d] = y;
    }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
// Device-path work (rk_npu_hip_attention_cache_append / _run, enqueued on the
// caller's streams) that a later host call on the same cache or workspace must
// wait for: an event recorded after that work on its stream. The host call
// waits for the event only, not for the whole device. Work from a second
// stream while the first's is still pending, or work under graph capture
// (whose replays the host cannot see), makes the next wait a device-wide
// synchronize instead.
struct DevFence {
    std::mutex mu;
    hipEvent_t ev = nullptr;
    hipStream_t last = nullptr;
    bool used = false;   // ev holds the last device-path work
    bool broad = false;  // wait for the whole device next time

    // Note device-path work just enqueued on stream s.
    void note(hipStream_t s) {
        std::lock_guard<std::mutex> lock(mu);
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(s, &st) != hipSuccess || st != hipStreamCaptureStatusNone) {
            (void)hipGetLastError();
            broad = true;
            return;
        }
        if (used && s != last) {
            const hipError_t q = hipEventQuery(ev);
            (void)hipGetLastError();  // (not-ready is an answer, not an error)
            if (q != hipSuccess) broad = true;
        }
        if (!ev && hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            ev = nullptr;
            broad = true;
            return;
        }
        if (hipEventRecord(ev, s) != hipSuccess) {
            (void)hipGetLastError();
            broad = true;
            return;
        }
        used = true;
        last = s;
    }
    // Order stream s after the noted work (s == nullptr: the host waits).
    hipError_t wait(hipStream_t s) {
        std::lock_guard<std::mutex> lock(mu);
        if (broad) {
            const hipError_t e = hipDeviceSynchronize();
            if (e == hipSuccess) broad = used = false;
            return e;
        }
        if (!used) return hipSuccess;
        return s ? hipStreamWaitEvent(s, ev, 0) : hipEventSynchronize(ev);
    }
    void destroy() {
        if (ev) (void)hipEventDestroy(ev);
        ev = nullptr;
    }
};

struct AttnCache {
    uint32_t magic;
    Domain* domain;
    rk_npu_attention_f16_config cfg;
    __half* k;
    __half* v;
    int length, capacity;
    size_t bytes_each;  // of k and of v
    uint64_t generation;  // bumped whenever the K/V storage is replaced or reloaded
    DevFence fence;       // device-path appends (writes) and runs (reads) of the rows
    hipStream_t stream = nullptr;  // host-buffer appends (created on the first)
    HostStage hs;                  // their pinned staging
};

struct AttnWork {
    uint32_t magic;
    Domain* domain;
    rk_npu_attention_f16_config cfg;
    __half* q;     // host-call staging [qh][max_query_rows][D]
    float* out;    // host-call staging (f32; fp16 output uses the first half)
    float* part;   // split partials
    size_t q_bytes, out_bytes, part_bytes;
    hipStream_t stream;
    std::atomic<bool> busy;
    DevFence fence;  // device-path runs writing this workspace's partials
    HostStage hs;    // pinned staging of host-buffer runs
};

// The reference's checks (src/npu.rs:714-728) plus this library's limits.
static bool valid_config(const rk_npu_attention_f16_config* c) {
    if (!c) return false;
    const int d = c->head_dim;
    return c->kv_heads >= 1 && c->kv_heads <= 32 && c->query_heads >= c->kv_heads &&
           c->query_heads % c->kv_heads == 0 && c->query_heads <= 256 && d > 0 && d % 32 == 0 && d <= 256 &&
           std::isfinite(c->softmax_scale) && c->softmax_scale > 0.0f && c->max_query_rows >= 1 &&
           c->max_query_rows <= 256 && c->max_capacity >= 1 && c->initial_capacity >= 0 &&
           c->initial_capacity <= c->max_capacity &&
           (c->mask_mode == RK_NPU_ATTENTION_F16_CAUSAL || c->mask_mode == RK_NPU_ATTENTION_F16_NO_MASK);
}

// Head dims with a kernel instantiation.
static bool supported_dim(int d) { return d == 64 || d == 128 || d == 256; }

static size_t kv_bytes(const rk_npu_attention_f16_config* c, int capacity) {
    return (size_t)c->kv_heads * (size_t)capacity * c->head_dim * sizeof(__half);
}

static size_t part_bytes(const rk_npu_attention_f16_config* c) {
    return attn_partial_rows(c->head_dim) * (size_t)(c->head_dim + 2) * sizeof(float);
}

static AttnCache* as_cache(void* p) {
    AttnCache* c = static_cast<AttnCache*>(p);
    return (c && c->magic == MAGIC_ATTN_CACHE) ? c : nullptr;
}
static AttnWork* as_attn_work(void* p) {
    AttnWork* w = static_cast<AttnWork*>(p);
    return (w && w->magic == MAGIC_ATTN_WORK) ? w : nullptr;
}

// Grow to `capacity` rows (multiple of 32), keeping the rows held.
static int cache_grow(AttnCache* c, int capacity) {
    capacity = round_up(capacity, 32);
    if (capacity <= c->capacity) return RK_NPU_OK;
    if (capacity > round_up(c->cfg.max_capacity, 32)) return RK_NPU_ERR_PARAM;
    const size_t nb = kv_bytes(&c->cfg, capacity);
    __half* nk = static_cast<__half*>(domain_alloc(c->domain, nb));
    __half* nv = nk ? static_cast<__half*>(domain_alloc(c->domain, nb)) : nullptr;
    if (!nk || !nv) {
        domain_free(c->domain, nk, nb);
        return RK_NPU_ERR_NOMEM;
    }
    const size_t row = (size_t)c->cfg.head_dim * sizeof(__half);
    bool ok = true;
    if (c->length > 0) {
        ok = hipMemcpy2D(nk, capacity * row, c->k, (size_t)c->capacity * row, (size_t)c->length * row,
                         c->cfg.kv_heads, hipMemcpyDeviceToDevice) == hipSuccess &&
             hipMemcpy2D(nv, capacity * row, c->v, (size_t)c->capacity * row, (size_t)c->length * row,
                         c->cfg.kv_heads, hipMemcpyDeviceToDevice) == hipSuccess;
    }
    if (!ok) {
        domain_free(c->domain, nk, nb);
        domain_free(c->domain, nv, nb);
        return RK_NPU_ERR_DEVICE;
    }
    domain_free(c->domain, c->k, c->bytes_each);
    domain_free(c->domain, c->v, c->bytes_each);
    c->k = nk;
    c->v = nv;
    c->capacity = capacity;
    c->generation += 1;
    c->bytes_each = nb;
    return RK_NPU_OK;
}

// Copy `rows` rows per KV head ([kv_heads][rows][D]) after the rows held.
static int cache_put(AttnCache* c, const void* k, const void* v, int rows, hipMemcpyKind kind, hipStream_t s,
                     bool async) {
    const size_t row = (size_t)c->cfg.head_dim * sizeof(__half);
    const size_t dpitch = (size_t)c->capacity * row, spitch = (size_t)rows * row;
    __half* dk = c->k + (size_t)c->length * c->cfg.head_dim;
    __half* dv = c->v + (size_t)c->length * c->cfg.head_dim;
    hipError_t e1, e2;
    if (async) {
        e1 = hipMemcpy2DAsync(dk, dpitch, k, spitch, spitch, c->cfg.kv_heads, kind, s);
        e2 = hipMemcpy2DAsync(dv, dpitch, v, spitch, spitch, c->cfg.kv_heads, kind, s);
    } else {
        e1 = hipMemcpy2D(dk, dpitch, k, spitch, spitch, c->cfg.kv_heads, kind);
        e2 = hipMemcpy2D(dv, dpitch, v, spitch, spitch, c->cfg.kv_heads, kind);
    }
    if (e1 != hipSuccess || e2 != hipSuccess) return RK_NPU_ERR_DEVICE;
    c->length += rows;
    return RK_NPU_OK;
}

// Host-buffer append: rows of K and V ([kv_heads][rows][D] each, V at
// byte offset voff of the stage) copied into the cache rows [length, length +
// rows) of every head, 16 bytes per thread and step.
__global__ __launch_bounds__(256) void attn_append_kernel(const v4u* __restrict__ src, size_t voff_pieces,
                                                          v4u* __restrict__ k, v4u* __restrict__ v, int rows,
                                                          int row_pieces, size_t head_pieces, int length,
                                                          size_t total) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        const size_t per_head = (size_t)rows * row_pieces;
        const size_t h = i / per_head, r = i % per_head;
        const size_t at = h * head_pieces + (size_t)length * row_pieces + r;
        k[at] = src[i];
        v[at] = src[voff_pieces + i];
    }
}

// Appends host rows through the cache's pinned stage and stream, returning
// once they are in the cache (the stage's completion word); false when the
// stage path is not available (the caller copies directly).
static bool cache_put_staged(AttnCache* c, const void* k, const void* v, int rows, int& rc) {
    const int kh = c->cfg.kv_heads, D = c->cfg.head_dim;
    const size_t each = (size_t)kh * rows * D * sizeof(__half), voff = round_up_z(each, 256);
    if (!host_kernels_enabled()) return false;
    if (!c->stream && hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        (void)hipGetLastError();
        c->stream = nullptr;
        return false;
    }
    void* st = stage_reserve(c->hs, voff + each);
    if (!st) return false;
    std::memcpy(st, k, each);
    std::memcpy(static_cast<uint8_t*>(st) + voff, v, each);
    const int row_pieces = D / 8;
    const size_t total = (size_t)kh * rows * row_pieces;
    const int blocks = (int)std::min<size_t>(1024, (total + 255) / 256);
    hipLaunchKernelGGL(attn_append_kernel, dim3(blocks), dim3(256), 0, c->stream, static_cast<const v4u*>(c->hs.dev),
                       voff / 16, reinterpret_cast<v4u*>(c->k), reinterpret_cast<v4u*>(c->v), rows, row_pieces,
                       (size_t)c->capacity * row_pieces, c->length, total);
    if (hipGetLastError() != hipSuccess || !stage_download(c->hs, true, st, nullptr, nullptr, 0, c->stream)) {
        (void)hipStreamSynchronize(c->stream);
        rc = RK_NPU_ERR_DEVICE;
        return true;
    }
    c->length += rows;
    rc = RK_NPU_OK;
    return true;
}

struct AttnPlan {
    bool mfma;  // attn_mfma_kernel (64- or 128-row tiles) instead of attn_split_kernel
    int rt, row_tiles, splits, keys_per_split, key_end;
};

// Rows per tile: VALU kernel 4 when a KV head has at most 4 query rows
// (decode: one row of a 4-head group), else 16; MFMA kernel (16 or more rows
// per KV head) 64, or 128 from 128 rows on. Keys: enough splits that about
// 512 blocks run (256 of the 8-wave 128-row blocks, one per CU), each split
// a whole number of 64-key tiles; with more than one split the blocks write
// partials (enqueue_attention checks that the workspace holds them).
// Overrides for measurement: HM_ATTN_BLOCKS, HM_ATTN_WIDE_BLOCKS (the block
// counts the key splits aim at).
static int attn_env(const char* name, int fallback) {
    const char* v = std::getenv(name);
    return v ? std::atoi(v) : fallback;
}

static AttnPlan plan_attention(const rk_npu_attention_f16_config& c, int rows, int len, int pos) {
    AttnPlan p;
    const int G = c.query_heads / c.kv_heads, R = G * rows;
    p.mfma = R >= 16 && (c.head_dim == 64 || c.head_dim == 128);
    static const int env_blocks = attn_env("HM_ATTN_BLOCKS", 512);
    static const int env_wide = attn_env("HM_ATTN_WIDE_BLOCKS", 256);
    // 128 or more rows per KV head: 8-wave blocks of 128 rows, one per CU
    // (a K/V tile shared by twice the waves, and the two waves on a SIMD
    // belong to one block), aiming at HM_ATTN_WIDE_BLOCKS blocks
    p.rt = p.mfma ? (R >= 128 ? 128 : 64) : (R <= 4 ? 4 : 16);
    p.row_tiles = (R + p.rt - 1) / p.rt;
    p.key_end = (c.mask_mode == RK_NPU_ATTENTION_F16_CAUSAL) ? std::min(len, pos + rows) : len;
    const int kt = c.head_dim == 256 ? 32 : ATTN_KT;  // keys per tile of the kernel
    const int tiles = (p.key_end + kt - 1) / kt;
    const int base = p.row_tiles * c.kv_heads;
    const int target = std::min(std::max(p.rt == 128 ? env_wide : env_blocks, 64), 1024);
    int want = base >= target ? 1 : (target + base - 1) / base;
    want = std::max(1, std::min(std::min(want, tiles), ATTN_MAX_SPLITS));
    const int tiles_per_split = (tiles + want - 1) / want;
    p.keys_per_split = tiles_per_split * kt;
    p.splits = (p.key_end + p.keys_per_split - 1) / p.keys_per_split;
    if (p.splits < 1) p.splits = 1;
    return p;
}

template <int D, int RT>
static void launch_attn(const AttnParams& P, const AttnPlan& pl, int kh, hipStream_t s) {
    hipLaunchKernelGGL((attn_split_kernel<D, RT>), dim3(pl.splits, pl.row_tiles, kh), dim3(256), 0, s, P);
}

static int enqueue_attention(AttnWork* w, AttnCache* c, const __half* q, int rows, int pos, void* out, int out_f16,
                             hipStream_t s) {
    const rk_npu_attention_f16_config& cfg = c->cfg;
    const bool causal = cfg.mask_mode == RK_NPU_ATTENTION_F16_CAUSAL;
    if (rows < 1 || rows > w->cfg.max_query_rows || pos < 0 || c->length < 1) return RK_NPU_ERR_PARAM;
    if (causal && (long)pos + rows > c->length) return RK_NPU_ERR_PARAM;
    const AttnPlan pl = plan_attention(cfg, rows, c->length, pos);
    if (pl.splits > 1 && (size_t)pl.row_tiles * pl.rt * cfg.kv_heads * pl.splits > attn_partial_rows(cfg.head_dim))
        return RK_NPU_ERR_UNSUPPORTED;
    AttnParams P;
    P.q = q;
    P.k = c->k;
    P.v = c->v;
    P.out = out;
    P.out_f16 = out_f16;
    P.part = w->part;
    P.qh = cfg.query_heads;
    P.kh = cfg.kv_heads;
    P.m = rows;
    P.cap = c->capacity;
    P.len = c->length;
    P.pos = pos;
    P.causal = causal ? 1 : 0;
    P.scale = cfg.softmax_scale;
    P.splits = pl.splits;
    P.keys_per_split = pl.keys_per_split;
    P.row_tiles = pl.row_tiles;
    P.key_end = pl.key_end;
    P.rows_pad = pl.row_tiles * pl.rt;
    const int D = cfg.head_dim;
#define HM_ATTN(DD)                                                    \
    if (pl.rt == 4)                                                    \
        launch_attn<DD, 4>(P, pl, cfg.kv_heads, s);                    \
    else                                                               \
        launch_attn<DD, 16>(P, pl, cfg.kv_heads, s);
    const dim3 grid(pl.splits, pl.row_tiles, cfg.kv_heads);
    if (pl.mfma && D == 64) {
        if (pl.rt == 128)
            hipLaunchKernelGGL((attn_mfma_kernel<64, 8>), grid, dim3(512), 0, s, P);
        else
            hipLaunchKernelGGL((attn_mfma_kernel<64, 4>), grid, dim3(256), 0, s, P);
    } else if (pl.mfma && D == 128) {
        if (pl.rt == 128)
            hipLaunchKernelGGL((attn_mfma_kernel<128, 8>), grid, dim3(512), 0, s, P);
        else
            hipLaunchKernelGGL((attn_mfma_kernel<128, 4>), grid, dim3(256), 0, s, P);
    } else if (D == 64) {
        HM_ATTN(64)
    } else if (D == 128) {
        HM_ATTN(128)
    } else {
        HM_ATTN(256)
    }
#undef HM_ATTN
    if (pl.splits > 1) {
        const int G = cfg.query_heads / cfg.kv_heads;
        // few splits: a wave per row; many: a block per row (measured: 8
        // splits over 4096 rows 2 us faster by wave, 64 splits over 32 rows
        // 14 us faster by block)
        const bool by_wave = pl.splits <= 16;
        const dim3 cgrid(by_wave ? (G * rows + 3) / 4 : G * rows, cfg.kv_heads);
        if (by_wave) {
            // (splits loaded per batch: 8 when there are at most 8, else 16)
#define HM_COMB_ROWS(DD)                                                                            \
    if (pl.splits <= 8)                                                                             \
        hipLaunchKernelGGL((attn_combine_rows_kernel<DD, 8>), cgrid, dim3(256), 0, s, P);           \
    else                                                                                            \
        hipLaunchKernelGGL((attn_combine_rows_kernel<DD, 16>), cgrid, dim3(256), 0, s, P);
            if (D == 64) {
                HM_COMB_ROWS(64)
            } else if (D == 128) {
                HM_COMB_ROWS(128)
            } else {
                HM_COMB_ROWS(256)
            }
#undef HM_COMB_ROWS
        } else if (D == 64) {
            hipLaunchKernelGGL(attn_combine_kernel<64>, cgrid, dim3(256), 0, s, P);
        } else if (D == 128) {
            hipLaunchKernelGGL(attn_combine_kernel<128>, cgrid, dim3(256), 0, s, P);
        } else {
            hipLaunchKernelGGL(attn_combine_kernel<256>, cgrid, dim3(256), 0, s, P);
        }
    }
    return hipGetLastError() == hipSuccess ? RK_NPU_OK : RK_NPU_ERR_DEVICE;
}

static int run_host(rk_npu_attention_f16_workspace* workspace, rk_npu_attention_f16_cache* cache, const uint16_t* q,
                    int rows, int pos, void* out, int out_f16, rk_npu_attention_f16_timings* t, const void* reserved) {
    AttnWork* w = as_attn_work(workspace);
    AttnCache* c = as_cache(cache);
    if (!w || !c || !q || !out || reserved) return RK_NPU_ERR_PARAM;
    if (w->cfg.query_heads != c->cfg.query_heads || w->cfg.kv_heads != c->cfg.kv_heads ||
        w->cfg.head_dim != c->cfg.head_dim || w->cfg.mask_mode != c->cfg.mask_mode ||
        w->cfg.softmax_scale != c->cfg.softmax_scale)
        return RK_NPU_ERR_PARAM;
    if (rows < 1 || rows > w->cfg.max_query_rows) return RK_NPU_ERR_PARAM;
    bool expected = false;
    if (!w->busy.compare_exchange_strong(expected, true)) return RK_NPU_ERR_BUSY;
    const double t0 = now_us();
    const size_t n = (size_t)c->cfg.query_heads * rows * c->cfg.head_dim;
    int rc = RK_NPU_OK;
    // Device-path appends and runs (rk_npu_hip_attention_cache_append / _run)
    // are enqueued on the caller's streams and may still be writing the
    // cache's rows or this workspace's partials: this call's stream waits for
    // them first. q comes in and the output goes out through the workspace's
    // pinned stage (the kernel path of small calls, else copies and a wait).
    const size_t qb = n * sizeof(__half), ob = n * (out_f16 ? sizeof(__half) : sizeof(float));
    void* st = nullptr;
    bool small = false;
    if (hipSetDevice(device_of(w->domain)) != hipSuccess || c->fence.wait(w->stream) != hipSuccess ||
        w->fence.wait(w->stream) != hipSuccess) {
        rc = RK_NPU_ERR_DEVICE;
    } else {
        st = stage_reserve(w->hs, std::max(qb, ob));
        small = stage_small(w->hs, st, qb, ob);
        const HostSeg seg{q, w->q, qb, 0};
        if (!stage_upload(w->hs, small, st, &seg, 1, w->stream) ||
            (t && hipStreamSynchronize(w->stream) != hipSuccess))
            rc = RK_NPU_ERR_DEVICE;
    }
    const double t1 = now_us();
    if (rc == RK_NPU_OK) rc = enqueue_attention(w, c, w->q, rows, pos, w->out, out_f16, w->stream);
    if (rc == RK_NPU_OK && t && hipStreamSynchronize(w->stream) != hipSuccess) rc = RK_NPU_ERR_DEVICE;
    const double t2 = now_us();
    if (rc == RK_NPU_OK && !stage_download(w->hs, small, st, out, w->out, ob, w->stream)) rc = RK_NPU_ERR_DEVICE;
    if (rc != RK_NPU_OK) (void)hipStreamSynchronize(w->stream);
    const double t3 = now_us();
    if (t) {
        t->upload_us = t1 - t0;
        t->device_us = t2 - t1;
        t->download_us = t3 - t2;
        t->total_us = t3 - t0;
    }
    w->busy.store(false);
    return rc;
}

}  // namespace hm

using namespace hm;

extern "C" {

void rk_npu_attention_f16_config_init(rk_npu_attention_f16_config* c) {
    if (!c) return;
    std::memset(c, 0, sizeof(*c));
    c->query_heads = 32;
    c->kv_heads = 8;
    c->head_dim = 128;
    c->softmax_scale = 1.0f / std::sqrt(128.0f);
    c->max_query_rows = 128;
    c->max_capacity = 4096;
    c->initial_capacity = 128;
    c->kv_tile = 512;
    c->flags = RK_NPU_ATTENTION_F16_STABLE_SOFTMAX;
    c->mask_mode = RK_NPU_ATTENTION_F16_CAUSAL;
}

int rk_npu_attention_f16_query(const rk_npu_attention_f16_config* c, int32_t capacity, int32_t query_rows,
                               int32_t kv_capacity, rk_npu_attention_f16_sizes* sizes) {
    if (!valid_config(c) || !sizes || capacity < 0 || query_rows < 1 || query_rows > 256 || kv_capacity < 0)
        return RK_NPU_ERR_PARAM;
    const int cap = round_up(capacity, 32);
    sizes->key_bytes = kv_bytes(c, cap);
    sizes->value_bytes = kv_bytes(c, cap);
    sizes->tail_bytes = 0;
    sizes->workspace_bytes = (uint64_t)c->query_heads * query_rows * c->head_dim * (sizeof(__half) + sizeof(float)) +
                             part_bytes(c);
    sizes->active_core_mask = 1u;
    return RK_NPU_OK;
}

int rk_npu_attention_f16_prepare(rk_npu_iommu_domain* domain, const rk_npu_attention_f16_config* config,
                                 rk_npu_attention_f16_workspace** out) {
    if (out) *out = nullptr;
    Domain* d = static_cast<Domain*>(domain);
    if (!d || !out || !valid_config(config)) return RK_NPU_ERR_PARAM;
    if (!supported_dim(config->head_dim)) return RK_NPU_ERR_UNSUPPORTED;
    if (hipSetDevice(device_of(d)) != hipSuccess) return RK_NPU_ERR_DEVICE;
    AttnWork* w = new (std::nothrow) AttnWork();
    if (!w) return RK_NPU_ERR_NOMEM;
    w->magic = MAGIC_ATTN_WORK;
    w->domain = d;
    w->cfg = *config;
    w->busy.store(false);
    w->stream = nullptr;
    const size_t n = (size_t)config->query_heads * config->max_query_rows * config->head_dim;
    w->q_bytes = n * sizeof(__half);
    w->out_bytes = n * sizeof(float);
    w->part_bytes = part_bytes(config);
    w->q = static_cast<__half*>(domain_alloc(d, w->q_bytes));
    w->out = static_cast<float*>(domain_alloc(d, w->out_bytes));
    w->part = static_cast<float*>(domain_alloc(d, w->part_bytes));
    if (!w->q || !w->out || !w->part || hipStreamCreateWithFlags(&w->stream, hipStreamNonBlocking) != hipSuccess) {
        rk_npu_attention_f16_workspace_free(reinterpret_cast<rk_npu_attention_f16_workspace*>(w));
        return RK_NPU_ERR_NOMEM;
    }
    *out = reinterpret_cast<rk_npu_attention_f16_workspace*>(w);
    return RK_NPU_OK;
}

void rk_npu_attention_f16_workspace_free(rk_npu_attention_f16_workspace* workspace) {
    AttnWork* w = as_attn_work(workspace);
    if (!w) return;
    (void)hipSetDevice(device_of(w->domain));
    if (w->stream) {
        (void)hipStreamSynchronize(w->stream);
        (void)hipStreamDestroy(w->stream);
    }
    (void)w->fence.wait(nullptr);
    w->fence.destroy();
    stage_release(w->hs);
    domain_free(w->domain, w->q, w->q_bytes);
    domain_free(w->domain, w->out, w->out_bytes);
    domain_free(w->domain, w->part, w->part_bytes);
    w->magic = 0;
    delete w;
}

int rk_npu_attention_f16_cache_create(rk_npu_iommu_domain* domain, const rk_npu_attention_f16_config* config,
                                      rk_npu_attention_f16_cache** out) {
    if (out) *out = nullptr;
    Domain* d = static_cast<Domain*>(domain);
    if (!d || !out || !valid_config(config)) return RK_NPU_ERR_PARAM;
    if (!supported_dim(config->head_dim)) return RK_NPU_ERR_UNSUPPORTED;
    if (hipSetDevice(device_of(d)) != hipSuccess) return RK_NPU_ERR_DEVICE;
    AttnCache* c = new (std::nothrow) AttnCache();
    if (!c) return RK_NPU_ERR_NOMEM;
    c->magic = MAGIC_ATTN_CACHE;
    c->domain = d;
    c->cfg = *config;
    c->length = 0;
    c->generation = 0;
    c->capacity = std::max(32, round_up(config->initial_capacity, 32));
    c->bytes_each = kv_bytes(config, c->capacity);
    c->k = static_cast<__half*>(domain_alloc(d, c->bytes_each));
    c->v = c->k ? static_cast<__half*>(domain_alloc(d, c->bytes_each)) : nullptr;
    if (!c->k || !c->v) {
        rk_npu_attention_f16_cache_free(reinterpret_cast<rk_npu_attention_f16_cache*>(c));
        return RK_NPU_ERR_NOMEM;
    }
    *out = reinterpret_cast<rk_npu_attention_f16_cache*>(c);
    return RK_NPU_OK;
}

void rk_npu_attention_f16_cache_free(rk_npu_attention_f16_cache* cache) {
    AttnCache* c = as_cache(cache);
    if (!c) return;
    (void)hipSetDevice(device_of(c->domain));
    (void)c->fence.wait(nullptr);
    c->fence.destroy();
    if (c->stream) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipStreamDestroy(c->stream);
    }
    stage_release(c->hs);
    domain_free(c->domain, c->k, c->bytes_each);
    domain_free(c->domain, c->v, c->bytes_each);
    c->magic = 0;
    delete c;
}

int rk_npu_attention_f16_cache_reserve(rk_npu_ctx* ctx, rk_npu_attention_f16_cache* cache, int32_t capacity) {
    AttnCache* c = as_cache(cache);
    if (!ctx || !c || capacity < 0) return RK_NPU_ERR_PARAM;
    if (hipSetDevice(device_of(c->domain)) != hipSuccess || c->fence.wait(nullptr) != hipSuccess)
        return RK_NPU_ERR_DEVICE;
    return cache_grow(c, capacity);
}

int rk_npu_attention_f16_cache_load(rk_npu_ctx* ctx, rk_npu_attention_f16_cache* cache, const uint16_t* k,
                                    const uint16_t* v, int32_t rows) {
    AttnCache* c = as_cache(cache);
    if (!ctx || !c || rows < 0 || (rows > 0 && (!k || !v))) return RK_NPU_ERR_PARAM;
    if (hipSetDevice(device_of(c->domain)) != hipSuccess || c->fence.wait(nullptr) != hipSuccess)
        return RK_NPU_ERR_DEVICE;
    c->length = 0;
    c->generation += 1;  // the contents are replaced (a reset when rows == 0)
    if (rows == 0) return RK_NPU_OK;
    int rc = cache_grow(c, rows);
    if (rc != RK_NPU_OK) return rc;
    return cache_put(c, k, v, rows, hipMemcpyHostToDevice, nullptr, false);
}

int rk_npu_attention_f16_cache_append(rk_npu_ctx* ctx, rk_npu_attention_f16_cache* cache, const uint16_t* k,
                                      const uint16_t* v, int32_t rows) {
    AttnCache* c = as_cache(cache);
    if (!ctx || !c || rows < 1 || !k || !v) return RK_NPU_ERR_PARAM;
    if ((long)c->length + rows > round_up(c->cfg.max_capacity, 32)) return RK_NPU_ERR_PARAM;
    if (hipSetDevice(device_of(c->domain)) != hipSuccess || c->fence.wait(nullptr) != hipSuccess)
        return RK_NPU_ERR_DEVICE;
    if (c->length + rows > c->capacity) {
        const int grown = std::min(round_up(c->cfg.max_capacity, 32), std::max(c->length + rows, 2 * c->capacity));
        int rc = cache_grow(c, grown);
        if (rc != RK_NPU_OK) return rc;
    }
    int rc = RK_NPU_OK;
    if (cache_put_staged(c, k, v, rows, rc)) return rc;
    return cache_put(c, k, v, rows, hipMemcpyHostToDevice, nullptr, false);
}

int rk_npu_attention_f16_cache_truncate(rk_npu_attention_f16_cache* cache, int32_t length) {
    AttnCache* c = as_cache(cache);
    if (!c || length < 0 || length > c->length) return RK_NPU_ERR_PARAM;
    c->length = length;
    return RK_NPU_OK;
}

int rk_npu_attention_f16_cache_get_info(const rk_npu_attention_f16_cache* cache,
                                        rk_npu_attention_f16_cache_info* info) {
    AttnCache* c = as_cache(const_cast<rk_npu_attention_f16_cache*>(cache));
    if (!c || !info) return RK_NPU_ERR_PARAM;
    info->length = c->length;
    info->capacity = c->capacity;
    info->max_capacity = round_up(c->cfg.max_capacity, 32);
    info->generation = c->generation;
    info->key_bytes = c->bytes_each;
    info->value_bytes = c->bytes_each;
    info->tail_bytes = 0;
    return RK_NPU_OK;
}

int rk_npu_attention_f16_run(rk_npu_ctx* ctx, rk_npu_attention_f16_workspace* workspace,
                             rk_npu_attention_f16_cache* cache, const uint16_t* q, int32_t rows, int32_t position,
                             float* output, rk_npu_attention_f16_timings* timings, const void* reserved) {
    if (!ctx) return RK_NPU_ERR_PARAM;
    return run_host(workspace, cache, q, rows, position, output, 0, timings, reserved);
}

int rk_npu_attention_f16_run_half(rk_npu_ctx* ctx, rk_npu_attention_f16_workspace* workspace,
                                  rk_npu_attention_f16_cache* cache, const uint16_t* q, int32_t rows,
                                  int32_t position, uint16_t* output, rk_npu_attention_f16_timings* timings,
                                  const void* reserved) {
    if (!ctx) return RK_NPU_ERR_PARAM;
    return run_host(workspace, cache, q, rows, position, output, 1, timings, reserved);
}

int rk_npu_hip_attention_cache_append(rk_npu_attention_f16_cache* cache, const void* k_dev, const void* v_dev,
                                      int32_t rows, void* stream) {
    AttnCache* c = as_cache(cache);
    if (!c || rows < 1 || !k_dev || !v_dev) return RK_NPU_ERR_PARAM;
    if ((long)c->length + rows > c->capacity) return RK_NPU_ERR_PARAM;  // (reserve first: no allocation here)
    if (hipSetDevice(device_of(c->domain)) != hipSuccess) return RK_NPU_ERR_DEVICE;
    const int rc = cache_put(c, k_dev, v_dev, rows, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream), true);
    if (rc == RK_NPU_OK) c->fence.note(static_cast<hipStream_t>(stream));
    return rc;
}

int rk_npu_hip_attention_run(rk_npu_attention_f16_workspace* workspace, rk_npu_attention_f16_cache* cache,
                             const void* q_dev, int32_t rows, int32_t position, void* out_dev, int32_t out_f16,
                             void* stream) {
    AttnWork* w = as_attn_work(workspace);
    AttnCache* c = as_cache(cache);
    if (!w || !c || !q_dev || !out_dev) return RK_NPU_ERR_PARAM;
    if (w->cfg.query_heads != c->cfg.query_heads || w->cfg.kv_heads != c->cfg.kv_heads ||
        w->cfg.head_dim != c->cfg.head_dim || w->cfg.mask_mode != c->cfg.mask_mode ||
        w->cfg.softmax_scale != c->cfg.softmax_scale)
        return RK_NPU_ERR_PARAM;
    if (hipSetDevice(device_of(w->domain)) != hipSuccess) return RK_NPU_ERR_DEVICE;
    const int rc = enqueue_attention(w, c, static_cast<const __half*>(q_dev), rows, position, out_dev,
                                     out_f16 ? 1 : 0, static_cast<hipStream_t>(stream));
    if (rc == RK_NPU_OK) {
        c->fence.note(static_cast<hipStream_t>(stream));
        w->fence.note(static_cast<hipStream_t>(stream));
    }
    return rc;
}

}  // extern "C"

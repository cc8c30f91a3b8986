// Roofline probes (rk_npu_hip_stream_probe, rk_npu_hip_mfma_probe): kernels
// that measure the two ceilings the hot path is judged against on the GPU
// it runs on, so the floors quoted for each projection come from committed
// code. They compute nothing the library uses and are built into a
// measurement-only library of their own (libhip_probes.so), not into the
// product library or its ABI headers. Both only enqueue on `stream`.
//   rk_npu_hip_stream_probe(src, bytes, blocks, threads, read, sink, stream):
//     one launch of `blocks` x `threads` (a multiple of 64 up to 512)
//     threads; sink holds one uint32 per block;
//   rk_npu_hip_mfma_probe(blocks, iters, sink, stream): `blocks` x 256
//     threads, each wave `iters` rounds of 8 MFMAs (65536 int8 ops each);
//     sink holds one int32 per thread. rk_npu_hip_mfma_rand_probe: the same
//     with full-range operand bytes, a different operand pair per MFMA.
//   rk_npu_hip_lds_probe(blocks, threads, iters, sink, clocks, stream):
//     `blocks` x `threads` threads with 64 KB of LDS each, every wave reading
//     iters x 8 KB from LDS; sink holds one uint32 per wave, clocks two
//     uint64 per block (shader-clock cycles, 100 MHz ticks of the loop).
//   rk_npu_hip_load_probe(blocks, threads, depth, to_lds, src, span, iters,
//     sink, clocks, stream): every wave of `blocks` x `threads` threads
//     streams `iters` 1-KB chunks (16 bytes per lane) of a `span`-byte source
//     region, keeping `depth` (4, 8 or 16) loads in flight: into LDS through
//     the LDS DMA load the GEMM ring uses (global_load_lds_dwordx4, to_lds =
//     1; waves x depth KB of LDS) or into registers (0; depth-load batches);
//     clocks two uint64 per block as above, sink one uint32 per wave.
//   rk_npu_hip_wave_place_probe(blocks, threads, out, stream): every wave
//     of `blocks` x `threads` stores its hardware id register (SIMD, CU) at
//     out[block * waves + wave].
//   stream: read `bytes` of device memory once with 16-byte non-temporal
//     loads (the GEMV's load instruction) in one launch of a chosen grid, or
//     launch the same grid with no loads (the launch's fixed cost);
//   mfma: back-to-back independent v_mfma_i32_32x32x32_i8 from registers
//     (no memory traffic): the dense int8 matrix-core rate the clock allows.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/rk_npu_quant_matmul.h"  // error codes

namespace hm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Thread t of the grid reads chunks t, t + T, t + 2T, ... (T = all threads):
// every wave load is one contiguous KB. The xor of the words is reduced per
// block and stored, so the loads cannot be removed.
__global__ __launch_bounds__(512) void stream_probe_kernel(const v4u* __restrict__ src, size_t chunks, int read,
                                                           unsigned* __restrict__ sink) {
    __shared__ unsigned s_x[8];
    const size_t T = (size_t)gridDim.x * blockDim.x;
    unsigned x = 0;
    if (read) {
        size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
        // four loads in flight per thread before the first use
        for (; i + 3 * T < chunks; i += 4 * T) {
            const v4u a = __builtin_nontemporal_load(src + i);
            const v4u b = __builtin_nontemporal_load(src + i + T);
            const v4u c = __builtin_nontemporal_load(src + i + 2 * T);
            const v4u d = __builtin_nontemporal_load(src + i + 3 * T);
            x ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
        }
        for (; i < chunks; i += T) {
            const v4u a = __builtin_nontemporal_load(src + i);
            x ^= a.x ^ a.y ^ a.z ^ a.w;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x ^= __shfl_xor(x, off);
    if ((threadIdx.x & 63) == 0) s_x[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned v = 0;
        for (int w = 0; w < (int)(blockDim.x >> 6); ++w) v ^= s_x[w];
        sink[blockIdx.x] = v;
    }
}

// Each wave keeps 8 independent 32x32 int32 accumulators and issues
// `iters` rounds of 8 MFMAs on operands held in registers: one operand pair
// of small values (mostly zero bytes) for every MFMA, or (RND) eight pairs of
// hashed, full-range bytes, a different pair for each MFMA of a round, as the
// fragments of a GEMM on real data are (the datapath's switching, and with it
// the power the chip draws, depends on the operand bits).
__device__ __forceinline__ int probe_hash(unsigned x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return (int)x;
}
template <bool RND>
__global__ __launch_bounds__(256) void mfma_probe_kernel(int iters, int* __restrict__ sink) {
    v16i acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0;
    const int t = threadIdx.x;
    v4i a[8], b[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const unsigned seed = (blockIdx.x * 256u + t) * 64u + 8u * j;
        a[j] = RND ? v4i{probe_hash(seed), probe_hash(seed + 1), probe_hash(seed + 2), probe_hash(seed + 3)}
                   : v4i{t, t + 1, t + 2, t + 3};
        b[j] = RND ? v4i{probe_hash(seed + 4), probe_hash(seed + 5), probe_hash(seed + 6), probe_hash(seed + 7)}
                   : v4i{t ^ 5, t ^ 6, t ^ 7, t ^ 9};
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[j], b[j], acc[j], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[j][r];
    sink[(size_t)blockIdx.x * blockDim.x + t] = s;
}

// LDS read bandwidth: every wave of the block streams conflict-free 16-byte
// reads (lane l of a wave reads chunk l of a 1 KB row; 8 reads in flight)
// out of a 64 KB buffer, `iters` rounds of 8 rows per wave. Wave 0 of each
// block records the shader-clock cycles (s_memtime) and the 100 MHz real-time
// ticks (s_memrealtime) the loop took, so bytes per clock per CU follow.
__global__ __launch_bounds__(512) void lds_probe_kernel(int iters, unsigned* __restrict__ sink,
                                                        unsigned long long* __restrict__ clocks) {
    extern __shared__ v4u lds_buf[];  // 4096 chunks of 16 bytes
    for (int i = threadIdx.x; i < 4096; i += blockDim.x) lds_buf[i] = v4u{(unsigned)i, (unsigned)i + 1, 7u, 9u};
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const unsigned long long c0 = __builtin_amdgcn_s_memtime();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    v4u x = {0u, 0u, 0u, 0u};
    int row = wave * 8;
    for (int it = 0; it < iters; ++it) {
        v4u v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = lds_buf[((row + j) & 63) * 64 + lane];
#pragma unroll
        for (int j = 0; j < 8; ++j) x ^= v[j];
        row += 64;
    }
    const unsigned long long c1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    unsigned y = x.x ^ x.y ^ x.z ^ x.w;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) y ^= __shfl_xor(y, off);
    if (lane == 0) sink[(size_t)blockIdx.x * (blockDim.x >> 6) + wave] = y;
    if (threadIdx.x == 0) {
        clocks[2 * blockIdx.x] = c1 - c0;
        clocks[2 * blockIdx.x + 1] = r1 - r0;
    }
}

// Global -> LDS (or register) load rate: wave w of block b starts at chunk
// (b * waves + w) * 613 of the region and walks it chunk by chunk, wrapping
// at its end. The LDS path keeps DEPTH DMA loads in flight (each wave its
// own DEPTH-slot ring of 1-KB slots, slot i % DEPTH); the register path
// issues DEPTH loads, then folds them into an xor that is stored.
template <int DEPTH, bool TO_LDS>
__global__ __launch_bounds__(512) void load_probe_kernel(const uint8_t* __restrict__ src, size_t span_chunks,
                                                         int iters, unsigned* __restrict__ sink,
                                                         unsigned long long* __restrict__ clocks) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_ring[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    size_t c = ((size_t)blockIdx.x * waves + wave) * 613 % span_chunks;
    uint8_t* ring = lds_ring + (size_t)wave * DEPTH * 1024;
    v4u x = {0u, 0u, 0u, 0u};
    const unsigned long long c0 = __builtin_amdgcn_s_memtime();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    if constexpr (TO_LDS) {
        for (int i = 0; i < iters; ++i) {
            __builtin_amdgcn_global_load_lds(src + c * 1024 + lane * 16,
                                             (__attribute__((address_space(3))) void*)(ring + (i % DEPTH) * 1024), 16,
                                             0, 0);
            c = (c + 1 == span_chunks) ? 0 : c + 1;
            // (vmcnt: bits 3:0 and 15:14; expcnt and lgkmcnt at their maxima)
            __builtin_amdgcn_s_waitcnt(((DEPTH - 1) & 15) | (((DEPTH - 1) >> 4) << 14) | (7 << 4) | (15 << 8));
        }
        __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
        __syncthreads();
        x = *reinterpret_cast<const v4u*>(ring + lane * 16);
    } else {
        for (int i = 0; i < iters; i += DEPTH) {
            v4u r[DEPTH];
#pragma unroll
            for (int j = 0; j < DEPTH; ++j) {
                r[j] = *reinterpret_cast<const v4u*>(src + c * 1024 + lane * 16);
                c = (c + 1 == span_chunks) ? 0 : c + 1;
            }
#pragma unroll
            for (int j = 0; j < DEPTH; ++j) x ^= r[j];
        }
    }
    const unsigned long long c1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    unsigned y = x.x ^ x.y ^ x.z ^ x.w;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) y ^= __shfl_xor(y, off);
    if (lane == 0) sink[(size_t)blockIdx.x * waves + wave] = y;
    if (threadIdx.x == 0) {
        clocks[2 * blockIdx.x] = c1 - c0;
        clocks[2 * blockIdx.x + 1] = r1 - r0;
    }
}

// Where the waves of a block run: wave w of block b stores the hardware id
// register (HW_REG_HW_ID: bits 3:0 wave slot, 5:4 SIMD, 11:8 CU, 15:13 shader
// engine) at out[b * waves + w].
__global__ void wave_place_kernel(unsigned* __restrict__ out) {
    const unsigned id = __builtin_amdgcn_s_getreg((31 << 11) | (0 << 6) | 4);
    if ((threadIdx.x & 63) == 0) out[blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)] = id;
}

}  // namespace hm

using namespace hm;

extern "C" {

int rk_npu_hip_stream_probe(const void* src, uint64_t bytes, int blocks, int threads, int read, uint32_t* sink,
                            void* stream) {
    if (blocks < 1 || blocks > (1 << 20) || threads < 64 || threads > 512 || threads % 64 != 0 ||
        !sink || (read && (!src || (reinterpret_cast<uintptr_t>(src) & 15) != 0)))
        return RK_NPU_ERR_PARAM;
    hipLaunchKernelGGL(stream_probe_kernel, dim3(blocks), dim3(threads), 0, static_cast<hipStream_t>(stream),
                       static_cast<const v4u*>(src), (size_t)(read ? bytes / 16 : 0), read, sink);
    return hipGetLastError() == hipSuccess ? RK_NPU_OK : RK_NPU_ERR_DEVICE;
}

int rk_npu_hip_mfma_probe(int blocks, int iters, int32_t* sink, void* stream) {
    if (blocks < 1 || blocks > (1 << 20) || iters < 1 || !sink) return RK_NPU_ERR_PARAM;
    hipLaunchKernelGGL(mfma_probe_kernel<false>, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), iters,
                       sink);
    return hipGetLastError() == hipSuccess ? RK_NPU_OK : RK_NPU_ERR_DEVICE;
}

int rk_npu_hip_mfma_rand_probe(int blocks, int iters, int32_t* sink, void* stream) {
    if (blocks < 1 || blocks > (1 << 20) || iters < 1 || !sink) return RK_NPU_ERR_PARAM;
    hipLaunchKernelGGL(mfma_probe_kernel<true>, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), iters,
                       sink);
    return hipGetLastError() == hipSuccess ? RK_NPU_OK : RK_NPU_ERR_DEVICE;
}

int rk_npu_hip_lds_probe(int blocks, int threads, int iters, uint32_t* sink, uint64_t* clocks, void* stream) {
    if (blocks < 1 || blocks > (1 << 20) || threads < 64 || threads > 512 || threads % 64 != 0 || iters < 1 ||
        !sink || !clocks)
        return RK_NPU_ERR_PARAM;
    hipLaunchKernelGGL(lds_probe_kernel, dim3(blocks), dim3(threads), 65536, static_cast<hipStream_t>(stream), iters,
                       sink, reinterpret_cast<unsigned long long*>(clocks));
    return hipGetLastError() == hipSuccess ? RK_NPU_OK : RK_NPU_ERR_DEVICE;
}

int rk_npu_hip_load_probe(int blocks, int threads, int depth, int to_lds, const void* src, uint64_t span, int iters,
                          uint32_t* sink, uint64_t* clocks, void* stream) {
    if (blocks < 1 || blocks > (1 << 20) || threads < 64 || threads > 512 || threads % 64 != 0 || iters < 1 ||
        (depth != 4 && depth != 8 && depth != 16) || iters % depth != 0 || !src || span < 1024 || !sink || !clocks ||
        (reinterpret_cast<uintptr_t>(src) & 15) != 0)
        return RK_NPU_ERR_PARAM;
    const size_t lds = to_lds ? (size_t)(threads / 64) * depth * 1024 : 0;
    if (lds > 160 * 1024) return RK_NPU_ERR_PARAM;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t* p = static_cast<const uint8_t*>(src);
    const size_t chunks = span / 1024;
    unsigned long long* ck = reinterpret_cast<unsigned long long*>(clocks);
#define HM_LOAD_PROBE(D, L) \
    hipLaunchKernelGGL((load_probe_kernel<D, L>), dim3(blocks), dim3(threads), lds, s, p, chunks, iters, sink, ck)
    if (to_lds) {
        if (depth == 4) HM_LOAD_PROBE(4, true);
        else if (depth == 8) HM_LOAD_PROBE(8, true);
        else HM_LOAD_PROBE(16, true);
    } else {
        if (depth == 4) HM_LOAD_PROBE(4, false);
        else if (depth == 8) HM_LOAD_PROBE(8, false);
        else HM_LOAD_PROBE(16, false);
    }
#undef HM_LOAD_PROBE
    return hipGetLastError() == hipSuccess ? RK_NPU_OK : RK_NPU_ERR_DEVICE;
}

int rk_npu_hip_wave_place_probe(int blocks, int threads, uint32_t* out, void* stream) {
    if (blocks < 1 || blocks > (1 << 16) || threads < 64 || threads > 1024 || threads % 64 != 0 || !out)
        return RK_NPU_ERR_PARAM;
    hipLaunchKernelGGL(wave_place_kernel, dim3(blocks), dim3(threads), 0, static_cast<hipStream_t>(stream), out);
    return hipGetLastError() == hipSuccess ? RK_NPU_OK : RK_NPU_ERR_DEVICE;
}

}  // extern "C"

// Internal runtime of the hip_matmul library: context, allocation domains,
// device weights and workspaces behind the opaque rk_npu_* handles.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <mutex>

#include "../../include/rk_npu_hip.h"
#include "../../include/rk_npu_moe_w8.h"
#include "../../include/rk_npu_quant_matmul.h"
#include "../../include/rk_npu_w4a8.h"
#include "../../include/rk_npu_w4a8_tune.h"

struct rk_npu_ctx {
    int device;
};

struct rk_npu_iommu_domain {
    rk_npu_ctx* ctx;
    uint32_t id;
    std::atomic<uint64_t> live{0}, peak{0}, creates{0}, destroys{0};
    std::mutex reclaim_mu;
    void (*reclaim)(void*) = nullptr;
    void* cookie = nullptr;
};

namespace hm {

struct Domain : rk_npu_iommu_domain {};

constexpr uint32_t MAGIC_W4 = 0x57344841u;  // weights, 4-bit
constexpr uint32_t MAGIC_W8 = 0x57384841u;  // weights, 8-bit
constexpr uint32_t MAGIC_WS4 = 0x53344841u;
constexpr uint32_t MAGIC_WS8 = 0x53384841u;

inline int round_up(int v, int m) { return (v + m - 1) / m * m; }
inline size_t round_up_z(size_t v, size_t m) { return (v + m - 1) / m * m; }

// Device allocation through a domain: accounting, injected failures for
// tests, and one retry after the domain's reclaim callback.
void* domain_alloc(Domain* d, size_t bytes);
void domain_free(Domain* d, void* p, size_t bytes);

// Geometry shared by weights and workspaces.
struct Geometry {
    int bits;
    int K, N;
    int K_pad;  // multiple of 64
    int N_pad;  // multiple of 256
    int half;   // N/2 when N % 64 == 0 (gate/up interleaved packing), else 0
};
Geometry make_geometry(int bits, int K, int N);
size_t weight_bytes(const Geometry& g);

struct Weights {
    uint32_t magic;
    Geometry g;
    Domain* domain;
    uint8_t* packed;
    float* colscale;
    size_t bytes;
    uint64_t fingerprint;
};

// Pinned host staging of host-buffer calls: coherent (fine-grained) pinned
// memory of `bytes` data bytes, then 256 bytes holding a completion word that
// a kernel sets to a call's sequence number; dev / done_dev are the device
// addresses of both. Allocated on first use and grown on demand (up to
// 8 MiB); stage_reserve returns nullptr for larger requests or when the
// allocation fails, and the caller then copies pageable memory directly.
struct HostStage {
    void* host = nullptr;
    void* dev = nullptr;
    size_t bytes = 0;
    unsigned* done = nullptr;
    unsigned* done_dev = nullptr;
    unsigned seq = 0;
    hipStream_t last = nullptr;  // the stream of the last transfer through the stage
};
// The stage's data (at least `bytes`), growing it after the stream of its
// last transfer has finished with the old one. A stage is only used on its
// owner's stream; stage_release expects that stream to be idle.
void* stage_reserve(HostStage& st, size_t bytes);
void stage_release(HostStage& st);

struct Workspace {
    uint32_t magic;
    Geometry g;
    int M;        // rows per call (the caller's bucket) / max rows for device calls
    int M_alloc;  // multiple of 256
    Domain* domain;
    hipStream_t stream;
    std::atomic<bool> busy;
    size_t bytes;
    // device buffers
    float* a_f32;     // [M][K]   host-call input staging
    int8_t* codes;    // [K_pad/16][M_alloc][16]
    float* rowscale;  // [M_alloc]
    int* rowsum;      // [M_alloc]
    unsigned* rowmax; // [M_alloc]  max|middle| of a fused SwiGLU output
    float* c_f32;     // [M][N]   output staging / fused middle
    float* partmax;   // [8][N_pad/8] per-block max|middle| of a GEMV SwiGLU
    int* split_part;        // split-K int32 partials [pieces][tiles][tile ints]
    size_t split_part_ints; // partial ints available
    unsigned long long* kacc;  // split-K GEMV column slots [N_pad] + row code-sum slot, kept zero between calls
    unsigned* sync;            // one-launch FFN synchronisation words (FfnSync), kept zero between calls
    bool fused_pending;        // a one-launch FFN ran since its error word was last read (host side)
    HostStage hs;  // pinned host staging of the host-buffer calls (allocated on first use)
};

size_t workspace_bytes(const Geometry& g, int M);
Workspace* workspace_create(Domain* d, int bits, int M, int K, int N);
void workspace_destroy(Workspace* ws);
// The workspace's pinned host stage of at least `bytes` (stage_reserve).
float* host_stage(Workspace* ws, size_t bytes);

Weights* weights_create(Domain* d, int bits, int K, int N, const int8_t* codes, const float* scales,
                        bool device_codes);
void weights_destroy(Weights* w);
Weights* weights_create_ckpt(Domain* d, int bits, int K, const rk_npu_hip_checkpoint_part* parts, int count);

struct Plan {
    int kind;  // 0 GEMV, 1 GEMM
    int bm, bn;
    int mr;
    int ksplit;  // GEMM: K pieces per tile
    int grid;
    int variant;
    int tiles;   // GEMM: output tiles
};
Plan plan_linear(int rows, const Geometry& g);

// Row maxima as partials: the max of row r is max_i p[r * count + i].
struct RowMax {
    const float* p;
    int count;
};

// Enqueue helpers (no synchronization).
// Where a quantization writes its codes, row scales and code sums when not
// into the workspace's own buffers (codes [K_pad/16][M_alloc][16]).
struct QuantOut {
    int8_t* codes;
    float* rowscale;
    int* rowsum;
    int M_alloc;
};
// Quantizes `rows` rows of x (rows_dev: a device-side count <= rows). With
// row_map, output row r quantizes input row row_map[r] / map_div (the MoE
// slot order: slot r holds its assignment's token).
int enqueue_quant(Workspace* ws, const void* x, int x_type, long lda, int rows, int rule, RowMax in_max,
                  unsigned* rowmax_clear, hipStream_t s, const int* rows_dev = nullptr, const int* row_map = nullptr,
                  int map_div = 1, const QuantOut* out = nullptr);
// A full dynamic-int8 linear from activations x: the GEMV quantizes inside
// its blocks; the GEMM path quantizes with a separate kernel first. With a
// SwiGLU+max epilogue, *out_max tells where the middle's row maxima are.
// A MoE combine that a one-row plain GEMV can run in its epilogue: the output
// becomes sum_rank fma(contrib[rank][col], routes[rank], .) + the GEMV's
// value (moe_combine_kernel's arithmetic, slot = assignment), in f32.
// *combined tells whether the launch did it (else the caller combines).
struct GemvCombine {
    const float* contrib;
    const float* routes;
    int top, h;
    bool* combined;
};
int enqueue_linear(Workspace* ws, const Weights* w, const void* x, int x_type, long lda, int rows, int rule,
                   RowMax in_max, void* c, int c_type, long ldc, int epi, RowMax* out_max, hipStream_t s,
                   const GemvCombine* comb = nullptr);
// gate_up (SwiGLU + row max) -> requant of the middle (same rule) -> down
// (with comb: the down launch may also run the MoE combine).
int enqueue_ffn(Workspace* gws, const Weights* gw, Workspace* dws, const Weights* dw, const void* A, int a_type,
                void* C, int c_type, int rows, int rule, hipStream_t s, const GemvCombine* comb = nullptr);

// RK_NPU_ERR_DEVICE (and cleared) when a one-launch FFN on this down
// workspace gave up waiting for its gate_up blocks since the last check.
int ffn_take_error(Workspace* dws);

int device_of(Domain* d);
// Wait for a host-buffer call's stream (block in hipStreamSynchronize, or
// poll hipStreamQuery with HM_HOST_SPIN=1).
hipError_t host_wait(hipStream_t s);
// Host-buffer transfers through a stage's data `p` (from stage_reserve, sized
// for the call; nullptr: pageable copies). A call is small (stage_small)
// when its input and output fit the kernel path: its inputs are fetched by
// one kernel launch and its output published by a copy kernel and the
// completion word, which the CPU polls; otherwise copies and a wait on the
// stream. Both ends of a call take the same `small`.
struct HostSeg {
    const void* src;   // caller's host memory
    void* dst;         // device memory (16-byte aligned, extending to a whole 16-byte piece)
    size_t bytes;
    size_t stage_off;  // 256-byte aligned offset of this segment in the stage
};
bool stage_small(const HostStage& st, const void* p, size_t in_bytes, size_t out_bytes);
// HM_HOST_FLAG: host-buffer calls may take the kernel path at all.
bool host_kernels_enabled();
bool stage_upload(HostStage& st, bool small, void* p, const HostSeg* segs, int n, hipStream_t s);
// Returns once C holds `bytes` of the device output `src` (bytes may be 0:
// then it returns once the work enqueued before it has finished).
bool stage_download(HostStage& st, bool small, void* p, void* C, const void* src, size_t bytes, hipStream_t s);
struct BusyGuard {
    std::atomic<bool>* flag;
    bool ok;
    explicit BusyGuard(std::atomic<bool>& f) : flag(&f) {
        bool expected = false;
        ok = f.compare_exchange_strong(expected, true);
    }
    ~BusyGuard() {
        if (ok) flag->store(false);
    }
};

double now_us();

// Launch profiling (rk_npu_hip_profile_*): returns a slot index to pass to
// prof_end, or -1 when profiling is off or the event pool is exhausted.
int prof_begin(hipStream_t s, int kind, int bits, int epi, int rows, int K, int N, const char* name);
void prof_end(int slot, hipStream_t s);

}  // namespace hm

// The public opaque types are thin tags over the internal structures.
struct rk_npu_f32i8f32_weights : hm::Weights {};
struct rk_npu_w4a8_weights : hm::Weights {};
struct rk_npu_matmul_workspace : hm::Workspace {};
struct rk_npu_w4a8_workspace : hm::Workspace {};

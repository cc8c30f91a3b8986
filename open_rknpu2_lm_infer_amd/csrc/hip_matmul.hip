// hip_matmul: MI355X-native quantized linear library behind the reference's
// rk_npu_* C ABI (context, domains, W8A8 and W4A8 linears, fused SwiGLU and
// fused FFN). MoE entry points live in moe.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <cstdio>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <tuple>
#include <vector>

#include "kernels.hpp"
#include "launch.hpp"
#include "runtime.hpp"

namespace hm {

static std::atomic<int> g_fail_allocs{0};

double now_us() {
    return std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

int device_of(Domain* d) { return d->ctx->device; }

// --- launch profiling -----------------------------------------------------------

struct ProfRecord {
    int kind, bits, epi, rows, K, N;
    std::string name;
};
static std::mutex g_prof_mu;
static std::atomic<bool> g_prof_on{false};
static std::vector<hipEvent_t> g_prof_events;
static std::vector<ProfRecord> g_prof_records;

int prof_begin(hipStream_t s, int kind, int bits, int epi, int rows, int K, int N, const char* name) {
    if (!g_prof_on.load()) return -1;
    std::lock_guard<std::mutex> lock(g_prof_mu);
    const size_t slot = g_prof_records.size();
    if (2 * slot + 1 >= g_prof_events.size()) return -1;
    g_prof_records.push_back(ProfRecord{kind, bits, epi, rows, K, N, name});
    (void)hipEventRecord(g_prof_events[2 * slot], s);
    return (int)slot;
}

void prof_end(int slot, hipStream_t s) {
    if (slot < 0) return;
    (void)hipEventRecord(g_prof_events[2 * slot + 1], s);
}

static bool try_alloc(void** p, size_t bytes) {
    int pending = g_fail_allocs.load();
    while (pending > 0) {
        if (g_fail_allocs.compare_exchange_weak(pending, pending - 1)) return false;
    }
    return hipMalloc(p, bytes) == hipSuccess;
}

void* domain_alloc(Domain* d, size_t bytes) {
    void* p = nullptr;
    if (bytes == 0) bytes = 256;
    if (!try_alloc(&p, bytes)) {
        (void)hipGetLastError();
        void (*cb)(void*) = nullptr;
        void* cookie = nullptr;
        {
            std::lock_guard<std::mutex> lock(d->reclaim_mu);
            cb = d->reclaim;
            cookie = d->cookie;
        }
        if (cb) cb(cookie);
        if (!try_alloc(&p, bytes)) {
            (void)hipGetLastError();
            return nullptr;
        }
    }
    uint64_t live = d->live.fetch_add(bytes) + bytes;
    uint64_t peak = d->peak.load();
    while (live > peak && !d->peak.compare_exchange_weak(peak, live)) {
    }
    d->creates.fetch_add(1);
    return p;
}

void domain_free(Domain* d, void* p, size_t bytes) {
    if (!p) return;
    if (bytes == 0) bytes = 256;
    (void)hipFree(p);
    d->live.fetch_sub(bytes);
    d->destroys.fetch_add(1);
}

Geometry make_geometry(int bits, int K, int N) {
    Geometry g;
    g.bits = bits;
    g.K = K;
    g.N = N;
    g.K_pad = round_up(K, 64);
    g.N_pad = round_up(N, 256);
    g.half = (N % 64 == 0) ? N / 2 : 0;
    return g;
}

size_t weight_bytes(const Geometry& g) {
    size_t payload = (size_t)g.K_pad * g.N_pad / (g.bits == 8 ? 1 : 2);
    return payload + (size_t)g.N_pad * sizeof(float);
}

// --- weights ----------------------------------------------------------------

static uint64_t mix64(uint64_t h, uint64_t v) {
    h ^= v + 0x9e3779b97f4a7c15ull + (h << 6) + (h >> 2);
    h *= 0xbf58476d1ce4e5b9ull;
    return h ^ (h >> 31);
}

Weights* weights_create(Domain* d, int bits, int K, int N, const int8_t* codes, const float* scales,
                        bool device_codes) {
    if (!d || !codes || !scales || (bits != 4 && bits != 8) || K <= 0 || N <= 0) return nullptr;
    if ((size_t)K * (size_t)N > (size_t)1 << 40) return nullptr;
    Geometry g = make_geometry(bits, K, N);
    const size_t n_codes = (size_t)K * N;
    uint64_t fp = mix64(mix64(mix64(0x5eedull, (uint64_t)bits), (uint64_t)K), (uint64_t)N);
    if (!device_codes) {
        for (int n = 0; n < N; ++n) {
            if (!(scales[n] > 0.0f)) return nullptr;  // src/model/checkpoint.rs:486-489
        }
        if (bits == 4) {
            for (size_t i = 0; i < n_codes; ++i)
                if (codes[i] < -8 || codes[i] > 7) return nullptr;
        }
        for (int n = 0; n < N; ++n) {
            uint32_t b;
            std::memcpy(&b, scales + n, 4);
            fp = mix64(fp, b);
        }
        const size_t stride = std::max<size_t>(1, n_codes / 65536);
        for (size_t i = 0; i < n_codes; i += stride) fp = mix64(fp, (uint8_t)codes[i] + (i << 8));
    }
    if (hipSetDevice(device_of(d)) != hipSuccess) return nullptr;
    Weights* w = (bits == 8) ? static_cast<Weights*>(new (std::nothrow) rk_npu_f32i8f32_weights())
                             : static_cast<Weights*>(new (std::nothrow) rk_npu_w4a8_weights());
    if (!w) return nullptr;
    w->magic = bits == 8 ? MAGIC_W8 : MAGIC_W4;
    w->g = g;
    w->domain = d;
    w->fingerprint = fp;
    w->bytes = weight_bytes(g);
    const size_t payload = w->bytes - (size_t)g.N_pad * sizeof(float);
    w->packed = static_cast<uint8_t*>(domain_alloc(d, payload));
    w->colscale = static_cast<float*>(domain_alloc(d, (size_t)g.N_pad * sizeof(float)));
    int8_t* raw = nullptr;
    float* dscales = nullptr;
    unsigned* bad = nullptr;
    bool ok = w->packed && w->colscale;
    if (ok && !device_codes) {
        raw = static_cast<int8_t*>(domain_alloc(d, n_codes));
        dscales = static_cast<float*>(domain_alloc(d, (size_t)N * sizeof(float)));
        ok = raw && dscales && hipMemcpy(raw, codes, n_codes, hipMemcpyHostToDevice) == hipSuccess &&
             hipMemcpy(dscales, scales, (size_t)N * 4, hipMemcpyHostToDevice) == hipSuccess;
    }
    if (ok) bad = static_cast<unsigned*>(domain_alloc(d, 256));
    ok = ok && bad && hipMemset(bad, 0, 4) == hipSuccess;
    if (ok) {
        PackParams P;
        P.codes = device_codes ? codes : raw;
        P.scales = device_codes ? scales : dscales;
        P.K = K;
        P.N = N;
        P.K_pad = g.K_pad;
        P.N_pad = g.N_pad;
        P.half = g.half;
        P.out = w->packed;
        P.colscale = w->colscale;
        P.bad = bad;
        const size_t entries = (size_t)(g.K_pad / (bits == 8 ? 16 : 32)) * g.N_pad;
        const unsigned blocks = (unsigned)((entries + 255) / 256);
        if (bits == 8)
            hipLaunchKernelGGL(pack_w8_kernel, dim3(blocks), dim3(256), 0, 0, P);
        else
            hipLaunchKernelGGL(pack_w4_kernel, dim3(blocks), dim3(256), 0, 0, P);
        ok = hipGetLastError() == hipSuccess && hipDeviceSynchronize() == hipSuccess;
        unsigned flag = 0;
        ok = ok && hipMemcpy(&flag, bad, 4, hipMemcpyDeviceToHost) == hipSuccess;
        if (ok && device_codes) {
            if (flag) ok = false;
            // scales must be positive: checked from the packed copy
            float* hs = static_cast<float*>(std::malloc((size_t)g.N_pad * 4));
            ok = ok && hs && hipMemcpy(hs, w->colscale, (size_t)g.N_pad * 4, hipMemcpyDeviceToHost) == hipSuccess;
            if (ok) {
                int valid = 0;
                for (int p = 0; p < g.N_pad; ++p) {
                    if (hs[p] > 0.0f) ++valid;
                    uint32_t b;
                    std::memcpy(&b, hs + p, 4);
                    w->fingerprint = mix64(w->fingerprint, b);
                }
                ok = valid == N;
            }
            std::free(hs);
        }
    }
    domain_free(d, raw, n_codes);
    domain_free(d, dscales, (size_t)N * sizeof(float));
    domain_free(d, bad, 256);
    if (!ok) {
        weights_destroy(w);
        return nullptr;
    }
    return w;
}

// Weights straight from checkpoint storage on the device (parts fused along
// N in order), packed by one kernel; scales checked positive on the packed copy.
Weights* weights_create_ckpt(Domain* d, int bits, int K, const rk_npu_hip_checkpoint_part* parts, int count) {
    if (!d || !parts || count < 1 || count > CKPT_MAX_PARTS || (bits != 4 && bits != 8) || K <= 0) return nullptr;
    CkptParams P{};
    long N = 0;
    for (int i = 0; i < count; ++i) {
        const rk_npu_hip_checkpoint_part& q = parts[i];
        const bool fmt_ok = q.format == RK_NPU_HIP_PACK_QUANTIZED || (q.format == RK_NPU_HIP_INT_QUANTIZED && bits == 8);
        if (!q.data || !q.scales || q.n <= 0 || !fmt_ok) return nullptr;
        P.part[i].data = q.data;
        P.part[i].scales = q.scales;
        P.part[i].start = (int)N;
        P.part[i].n = q.n;
        P.part[i].format = q.format == RK_NPU_HIP_INT_QUANTIZED ? 1 : 0;
        P.part[i].words = (K + 32 / bits - 1) / (32 / bits);
        N += q.n;
    }
    if (N > INT32_MAX || (size_t)K * (size_t)N > (size_t)1 << 40) return nullptr;
    if (hipSetDevice(device_of(d)) != hipSuccess) return nullptr;
    const Geometry g = make_geometry(bits, K, (int)N);
    Weights* w = (bits == 8) ? static_cast<Weights*>(new (std::nothrow) rk_npu_f32i8f32_weights())
                             : static_cast<Weights*>(new (std::nothrow) rk_npu_w4a8_weights());
    if (!w) return nullptr;
    w->magic = bits == 8 ? MAGIC_W8 : MAGIC_W4;
    w->g = g;
    w->domain = d;
    w->fingerprint = mix64(mix64(mix64(0x5eedull, (uint64_t)bits), (uint64_t)K), (uint64_t)N);
    w->bytes = weight_bytes(g);
    const size_t payload = w->bytes - (size_t)g.N_pad * sizeof(float);
    w->packed = static_cast<uint8_t*>(domain_alloc(d, payload));
    w->colscale = static_cast<float*>(domain_alloc(d, (size_t)g.N_pad * sizeof(float)));
    bool ok = w->packed && w->colscale;
    if (ok) {
        P.count = count;
        P.bits = bits;
        P.K = K;
        P.N = (int)N;
        P.K_pad = g.K_pad;
        P.N_pad = g.N_pad;
        P.half = g.half;
        P.out = w->packed;
        P.colscale = w->colscale;
        const size_t entries = (size_t)(g.K_pad / (bits == 8 ? 16 : 32)) * g.N_pad;
        hipLaunchKernelGGL(pack_ckpt_kernel, dim3((unsigned)((entries + 255) / 256)), dim3(256), 0, 0, P);
        ok = hipGetLastError() == hipSuccess && hipDeviceSynchronize() == hipSuccess;
    }
    if (ok) {
        std::vector<float> hs((size_t)g.N_pad);
        ok = hipMemcpy(hs.data(), w->colscale, (size_t)g.N_pad * 4, hipMemcpyDeviceToHost) == hipSuccess;
        int valid = 0;
        for (int p = 0; ok && p < g.N_pad; ++p) {
            if (hs[p] > 0.0f) ++valid;  // src/model/checkpoint.rs:486-489
            uint32_t b;
            std::memcpy(&b, &hs[p], 4);
            w->fingerprint = mix64(w->fingerprint, b);
        }
        ok = ok && valid == N;
    }
    if (!ok) {
        weights_destroy(w);
        return nullptr;
    }
    return w;
}

void weights_destroy(Weights* w) {
    if (!w) return;
    (void)hipSetDevice(device_of(w->domain));
    const size_t payload = w->bytes - (size_t)w->g.N_pad * sizeof(float);
    domain_free(w->domain, w->packed, payload);
    domain_free(w->domain, w->colscale, (size_t)w->g.N_pad * sizeof(float));
    if (w->magic == MAGIC_W8)
        delete static_cast<rk_npu_f32i8f32_weights*>(w);
    else
        delete static_cast<rk_npu_w4a8_weights*>(w);
}

// --- launch plans -------------------------------------------------------------

// (GemmVariant: launch.hpp)
static const int kBM[] = {256, 256, 128, 64, 32, 192};
static const int kBN[] = {256, 128, 128, 128, 128, 256};

// Plan switches for tests and measurements. Each starts from its environment
// variable, read once when the library first plans a launch; afterwards only
// rk_npu_hip_set_switch changes it, so no launch reads the environment.
enum SwitchId { SW_GEMM_VARIANT, SW_SPLITS, SW_FORCE_GEMM, SW_GEMV_QW, SW_GEMV_SPLITS, SW_FFN_FUSED, SW_FFN_SPIN,
                SW_GEMV_PREQ, SW_HOST_SPIN, SW_GEMV_COMBINE, SW_HOST_FLAG, SW_HOST_POLL, SW_COUNT };
struct SwitchDef {
    const char* name;
    int fallback;
};
static const SwitchDef kSwitches[SW_COUNT] = {
    {"HM_GEMM_VARIANT", -1}, {"HM_SPLITS", 0},         {"HM_FORCE_GEMM", 0}, {"HM_GEMV_QW", -1},
    {"HM_GEMV_SPLITS", 0},   {"HM_FFN_FUSED", 0},      {"HM_FFN_SPIN", 1 << 16}, {"HM_GEMV_PREQ", -1},
    {"HM_HOST_SPIN", 0},     {"HM_GEMV_COMBINE", 1},   {"HM_HOST_FLAG", 1},       {"HM_HOST_POLL", 2000}};

static std::atomic<int>* switch_table() {
    static std::atomic<int> table[SW_COUNT];
    static std::once_flag once;
    std::call_once(once, [] {
        for (int i = 0; i < SW_COUNT; ++i) {
            const char* v = std::getenv(kSwitches[i].name);
            table[i].store(v ? std::atoi(v) : kSwitches[i].fallback);
        }
    });
    return table;
}

static int switch_value(SwitchId id) { return switch_table()[id].load(std::memory_order_relaxed); }

// Activation codes of the whole K live in the GEMV's LDS.
constexpr int GEMV_MAX_LDS = 60 * 1024;

// GEMM plan for a given variant (-1: chosen by shape). Measured on the
// Qwen3-4B projection shapes: up to M = 1024 the 4-wave 64x128 tile (wave
// tile 32x64) leads, since more, smaller tiles keep every CU busy (M = 512:
// 36 us vs 47 us for 128x128 and 110 us for 256x256 on the 9728x2560 down
// projection); up to M = 2048 the 4-wave 128x128 tile (the 256x256 tile
// leaves CUs idle on N = 2560). Above 2048 rows the 128x128 tile (two blocks
// per CU, one's epilogue under the other's main loop) still leads on most
// shapes (M = 4096: qkv 2560x6144 104 -> 97 us, gate_up 2560x19456 + SwiGLU
// 247 -> 233 us, o 4096x2560 75 -> 74 us; M = 3072: every projection); the
// 8-wave 256x256 tile wins where its higher reuse is not paid for by idle
// CUs: very wide outputs (lm_head 2560x151936 at M = 4096: 2045 -> 1864 us)
// and long K once the 128x128 tiles overflow one round of two per CU
// (9728x2560 down at M = 4096: 176 -> 165 us; at M = 3072, 480 tiles fit a
// round and 128x128 wins, 148 -> 120 us). Rows <= 32 take the 32x128 tile.
// Split-K (two launches: partials, then sum + epilogue) when the tiles leave
// CUs idle and K is long: measured on 9728x2560 it takes M=512 from 45 to
// 38 us (3 pieces) and M=64 from 38 to 22 us (6 pieces); with K <= 4096 or
// as many tiles as CUs the partial traffic costs more than it saves.
// HM_SPLITS forces a piece count (experiments).
int device_cus() {
    static std::atomic<int> cached{0};
    int c = cached.load();
    if (c > 0) return c;
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        n = 256;  // MI355X
    (void)hipGetLastError();
    cached.store(n);
    return n;
}

static Plan plan_gemm(int rows, const Geometry& g, int variant) {
    Plan p{};
    p.kind = 1;
    int v = variant;
    if (v < 0) {
        const int forced = switch_value(SW_GEMM_VARIANT);
        if (forced >= 0 && forced <= 5)
            v = forced;
        else
            v = rows <= 32 ? V32x128 : rows <= 1024 ? V64x128 : V128x128;
        if (v == V128x128 && rows > 2048 && forced < 0) {
            const int cus = device_cus();
            const long long t256 = (long long)((rows + 255) / 256) * (g.N_pad / 256);
            const long long t128 = (long long)((rows + 127) / 128) * (g.N_pad / 128);
            // 256x256 for very wide outputs (lm_head), and for K >= 4096 once the
            // 128x128 tiles overflow two per CU: at M=4096 the 256x256 tile runs
            // o 4096x2560 in 68 us against 73 and down 9728x2560 in 158 against
            // 172 (bench.py --tile-sweep), although its 160 tiles leave CUs idle.
            if (t256 >= 8LL * cus || (g.K_pad >= 4096 && t128 > 2LL * cus)) v = V256x256;
            // 192x256 where it takes fewer rows per CU: M=4096 o 4096x2560 and
            // down 9728x2560 run 220 tiles of 192 rows in one round instead of
            // 160 tiles of 256 rows, which left 96 CUs idle.
            if (v == V256x256) {
                const long long t192 = (long long)((rows + 191) / 192) * (g.N_pad / 256);
                if ((t192 + cus - 1) / cus * 192 < (t256 + cus - 1) / cus * 256) v = V192x256;
            }
        }
    }
    const int KT = g.K_pad / 64;
    const int cus = device_cus();
    int f = 1;
    // Long K over more than 256 rows with too few 64x128 tiles for the CUs:
    // the 128x128 tile split into as many K pieces as one round of blocks
    // holds (9728x2560 down at M = 512: 80 tiles x 3 pieces 37.4 us against
    // 64x128 x 3 pieces 41.1 us, bench.py --tile-sweep).
    const long long t64 = (long long)((rows + 63) / 64) * (g.N_pad / 128);
    if (variant < 0 && switch_value(SW_GEMM_VARIANT) < 0 && v == V64x128 && rows > 256 && KT >= 128 && t64 < cus) {
        const int t128 = ((rows + 127) / 128) * (g.N_pad / 128);
        const int f128 = std::min(std::min(cus / t128, KT / 24), 8);
        if (f128 >= 2) {
            v = V128x128;
            f = f128;
        }
    }
    p.variant = v;
    p.bm = kBM[v];
    p.bn = kBN[v];
    p.tiles = ((rows + p.bm - 1) / p.bm) * (g.N_pad / p.bn);
    if (f == 1 && (v == V64x128 || v == V128x128) && p.tiles < cus && KT >= 128)
        f = std::max(1, std::min(std::min((3 * cus / 2 + p.tiles - 1) / p.tiles, KT / 24), 8));
    const int forced_f = switch_value(SW_SPLITS);
    p.ksplit = forced_f > 0 ? std::min(forced_f, KT) : f;
    p.grid = p.tiles * p.ksplit;
    return p;
}

Plan plan_linear(int rows, const Geometry& g) {
    const int mr = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8;
    // (2 to 8 rows take their GEMV dot products on the matrix cores, which
    // needs K_pad % 128 == 0 for W8 and % 256 for W4; other K take the GEMM)
    if (rows <= 8 && g.K_pad * mr <= GEMV_MAX_LDS && switch_value(SW_FORCE_GEMM) == 0 &&
        (mr == 1 || g.K_pad % (g.bits == 8 ? 128 : 256) == 0)) {
        Plan p{};
        p.kind = 0;
        p.mr = mr;
        p.ksplit = 1;
        p.grid = g.N_pad / 8;  // one 8-column tile per block (SwiGLU: a tile pair)
        p.tiles = p.grid;
        p.bm = p.mr;
        p.bn = 8;
        return p;
    }
    return plan_gemm(rows, g, -1);
}

// --- workspaces -------------------------------------------------------------

struct WsLayout {
    size_t a, codes, rows, c, part, split_part, kacc, sync, total;
    size_t split_part_ints;
};

static Plan plan_gemm(int rows, const Geometry& g, int variant);

// Split-K partials cover the plan of `M` rows.
static size_t split_need(const Geometry& g, int M) {
    const Plan p = plan_linear(M, g);
    return (p.kind == 1 && p.ksplit > 1) ? (size_t)p.tiles * p.ksplit * p.bm * p.bn : 0;
}

static WsLayout ws_layout(const Geometry& g, int M) {
    WsLayout L;
    const int M_alloc = round_up(M, 256);
    L.a = round_up_z((size_t)M * g.K * 4, 256);
    L.codes = (size_t)(g.K_pad / 16) * M_alloc * 16;
    L.rows = round_up_z((size_t)M_alloc * 4, 256);
    L.c = round_up_z((size_t)M * g.N * 4, 256);
    L.part = round_up_z((size_t)8 * (g.N_pad / 8) * 4, 256);
    L.split_part_ints = split_need(g, M);
    L.split_part = round_up_z(L.split_part_ints * 4, 256);
    L.kacc = round_up_z(((size_t)g.N_pad + 8) * 8, 256);
    L.sync = round_up_z((size_t)FFN_SYNC_WORDS * 4, 256);
    L.total = L.a + L.codes + 3 * L.rows + L.c + L.part + L.split_part + L.kacc + L.sync;
    return L;
}

size_t workspace_bytes(const Geometry& g, int M) { return ws_layout(g, M).total; }

Workspace* workspace_create(Domain* d, int bits, int M, int K, int N) {
    if (!d || (bits != 4 && bits != 8) || M <= 0 || M > 65536 || K <= 0 || N <= 0) return nullptr;
    if (hipSetDevice(device_of(d)) != hipSuccess) return nullptr;
    Workspace* ws = (bits == 8) ? static_cast<Workspace*>(new (std::nothrow) rk_npu_matmul_workspace())
                                : static_cast<Workspace*>(new (std::nothrow) rk_npu_w4a8_workspace());
    if (!ws) return nullptr;
    ws->magic = bits == 8 ? MAGIC_WS8 : MAGIC_WS4;
    ws->g = make_geometry(bits, K, N);
    ws->M = M;
    ws->M_alloc = round_up(M, 256);
    ws->domain = d;
    ws->busy.store(false);
    ws->stream = nullptr;
    ws->hs = HostStage{};
    ws->fused_pending = false;
    const WsLayout L = ws_layout(ws->g, M);
    ws->bytes = L.total;
    uint8_t* base = static_cast<uint8_t*>(domain_alloc(d, L.total));
    if (!base) {
        delete ws;
        return nullptr;
    }
    size_t off = 0;
    ws->a_f32 = reinterpret_cast<float*>(base + off);
    off += L.a;
    ws->codes = reinterpret_cast<int8_t*>(base + off);
    off += L.codes;
    ws->rowscale = reinterpret_cast<float*>(base + off);
    off += L.rows;
    ws->rowsum = reinterpret_cast<int*>(base + off);
    off += L.rows;
    ws->rowmax = reinterpret_cast<unsigned*>(base + off);
    off += L.rows;
    ws->c_f32 = reinterpret_cast<float*>(base + off);
    off += L.c;
    ws->partmax = reinterpret_cast<float*>(base + off);
    off += L.part;
    ws->split_part = reinterpret_cast<int*>(base + off);
    ws->split_part_ints = L.split_part_ints;
    off += L.split_part;
    ws->kacc = reinterpret_cast<unsigned long long*>(base + off);
    off += L.kacc;
    ws->sync = reinterpret_cast<unsigned*>(base + off);
    // Zero everything once (padding rows of the code planes stay zero).
    bool ok = hipMemset(base, 0, L.total) == hipSuccess &&
              hipStreamCreateWithFlags(&ws->stream, hipStreamNonBlocking) == hipSuccess &&
              hipDeviceSynchronize() == hipSuccess;
    if (!ok) {
        workspace_destroy(ws);
        return nullptr;
    }
    return ws;
}

void workspace_destroy(Workspace* ws) {
    if (!ws) return;
    (void)hipSetDevice(device_of(ws->domain));
    if (ws->stream) {
        (void)hipStreamSynchronize(ws->stream);
        (void)hipStreamDestroy(ws->stream);
    }
    domain_free(ws->domain, ws->a_f32, ws->bytes);
    stage_release(ws->hs);
    if (ws->magic == MAGIC_WS8)
        delete static_cast<rk_npu_matmul_workspace*>(ws);
    else
        delete static_cast<rk_npu_w4a8_workspace*>(ws);
}

// --- enqueue ------------------------------------------------------------------

int enqueue_quant(Workspace* ws, const void* x, int x_type, long lda, int rows, int rule, RowMax in_max,
                  unsigned* rowmax_clear, hipStream_t s, const int* rows_dev, const int* row_map, int map_div,
                  const QuantOut* out) {
    QuantParams P;
    P.x = x;
    P.x_type = x_type;
    P.lda = lda;
    P.rows = rows;
    P.K = ws->g.K;
    P.K_pad = ws->g.K_pad;
    P.M_alloc = ws->M_alloc;
    const size_t esz = x_type == DT_F32 ? 4 : 2;
    P.vec = (ws->g.K % 16 == 0) && ((lda * esz) % 16 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0);
    P.codes = ws->codes;
    P.rowscale = ws->rowscale;
    P.rowsum = ws->rowsum;
    P.part_in = in_max.p;
    P.part_count = in_max.count;
    P.rowmax_clear = rowmax_clear;
    P.rows_dev = rows_dev;
    P.row_map = row_map;
    P.map_div = map_div;
    if (out) {
        P.codes = out->codes;
        P.rowscale = out->rowscale;
        P.rowsum = out->rowsum;
        P.M_alloc = out->M_alloc;
    }
    // Measured on the Qwen3-4B activation shapes (M = 128 ... 4096): with
    // aligned rows the row-tiled kernel (4 rows per block, one wave per row,
    // code planes written as 64-byte runs) is fastest, e.g. 31 us instead of
    // 51 us for the 4096 x 9728 f32 middle and 13 us instead of 20 us for
    // 4096 x 4096 f16 rows. Up to 256 rows a block per row has the shortest
    // critical path. Rows with no precomputed max must fit in registers
    // (16 * 64 * 8 elements); others, and unaligned rows, take the per-row
    // kernel: one wave per row (4 rows per block) when short, one block per
    // row when long.
    const int KG = P.K_pad / 16;
    const int ni = (KG + 63) / 64;
    const bool tiled = P.vec && rows > 256 && (in_max.p != nullptr || ni <= 8);
    const bool wave_rows = !(rows <= 256 && KG >= 64) && KG <= 64 * QUANT_CHUNKS;
    const int slot = prof_begin(s, 2, 8, rule, rows, ws->g.K, 0, rule == QUANT_DENSE ? "quant_rows<dense>" : "quant_rows<moe>");
    if (tiled) {
        const dim3 grid((rows + 3) / 4), block(256);
#define HM_QT(T_, R_)                                                                                           \
    do {                                                                                                        \
        if (in_max.p)                                                                                           \
            hipLaunchKernelGGL((quant_tile_kernel<T_, R_, 4, 4, true>), grid, block, 0, s, P);                  \
        else if (ni <= 1)                                                                                       \
            hipLaunchKernelGGL((quant_tile_kernel<T_, R_, 4, 1, false>), grid, block, 0, s, P);                 \
        else if (ni <= 2)                                                                                       \
            hipLaunchKernelGGL((quant_tile_kernel<T_, R_, 4, 2, false>), grid, block, 0, s, P);                 \
        else if (ni <= 4)                                                                                       \
            hipLaunchKernelGGL((quant_tile_kernel<T_, R_, 4, 4, false>), grid, block, 0, s, P);                 \
        else                                                                                                    \
            hipLaunchKernelGGL((quant_tile_kernel<T_, R_, 4, 8, false>), grid, block, 0, s, P);                 \
    } while (0)
        if (x_type == DT_F32) {
            if (rule == QUANT_DENSE)
                HM_QT(float, QUANT_DENSE);
            else
                HM_QT(float, QUANT_MOE);
        } else {
            if (rule == QUANT_DENSE)
                HM_QT(__half, QUANT_DENSE);
            else
                HM_QT(__half, QUANT_MOE);
        }
#undef HM_QT
        prof_end(slot, s);
        return hipGetLastError() == hipSuccess ? RK_NPU_OK : RK_NPU_ERR_DEVICE;
    }
    const dim3 grid(wave_rows ? (rows + 3) / 4 : rows), block(256);
#define HM_QUANT_LAUNCH(T_, R_)                                                                \
    do {                                                                                       \
        if (wave_rows)                                                                         \
            hipLaunchKernelGGL((quant_rows_kernel<T_, R_, 64>), grid, block, 0, s, P);         \
        else                                                                                   \
            hipLaunchKernelGGL((quant_rows_kernel<T_, R_, 256>), grid, block, 0, s, P);        \
    } while (0)
    if (x_type == DT_F32) {
        if (rule == QUANT_DENSE)
            HM_QUANT_LAUNCH(float, QUANT_DENSE);
        else
            HM_QUANT_LAUNCH(float, QUANT_MOE);
    } else {
        if (rule == QUANT_DENSE)
            HM_QUANT_LAUNCH(__half, QUANT_DENSE);
        else
            HM_QUANT_LAUNCH(__half, QUANT_MOE);
    }
#undef HM_QUANT_LAUNCH
    prof_end(slot, s);
    return hipGetLastError() == hipSuccess ? RK_NPU_OK : RK_NPU_ERR_DEVICE;
}

int enqueue_linear(Workspace* ws, const Weights* w, const void* x, int x_type, long lda, int rows, int rule,
                   RowMax in_max, void* c, int c_type, long ldc, int epi, RowMax* out_max, hipStream_t s,
                   const GemvCombine* comb) {
    const Geometry& g = w->g;
    if (comb && comb->combined) *comb->combined = false;
    const Plan pv = plan_linear(rows, g);
    if (pv.kind == 0) {
        GemvParams V{};
        V.x = x;
        V.lda = lda;
        V.rule = rule;
        const size_t esz = x_type == DT_F32 ? 4 : 2;
        V.vec = (g.K % 16 == 0) && ((lda * esz) % 16 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0);
        V.part_in = in_max.p;
        V.part_count = in_max.count;
        V.part_out = ws->partmax;
        V.b = w->packed;
        V.colscale = w->colscale;
        V.c = c;
        V.ldc = ldc;
        V.c_type = c_type;
        V.M = rows;
        V.K = g.K;
        V.N = g.N;
        V.K_pad = g.K_pad;
        V.N_pad = g.N_pad;
        V.half = g.half;
        V.diag_codes = ws->codes;
        V.diag_scale = ws->rowscale;
        V.diag_rowsum = ws->rowsum;
        V.M_alloc = ws->M_alloc;
        V.ksplit = 1;
        V.kacc = ws->kacc;
        const int grid = epi == EPI_PLAIN ? g.N_pad / 8 : g.N_pad / 16;
        const size_t lds = (size_t)g.K_pad * pv.mr;
        // Rows the kernel cannot quantize from registers (unaligned or ragged
        // rows, or more than GEMV_XMAX chunks per thread) are quantized first;
        // so are 4 or more rows, where every block re-quantizing all rows costs
        // more than one extra launch (M=4 decode set, 36 layers in a graph:
        // 1.57 ms per step with the launch, 1.68 ms with HM_GEMV_PREQ=0, which
        // quantizes 4 rows in the blocks wherever they fit: qkv 8.4 -> 9.5 us,
        // gate_up 14.6 -> 16.7 us).
        const bool preq_rows = pv.mr > 4 || (pv.mr == 4 && switch_value(SW_GEMV_PREQ) != 0);
        const bool preq = preq_rows || !V.vec || (g.K_pad / 16) * pv.mr > 256 * GEMV_XMAX;
        // One or two rows that fit the quantization wave of the block are
        // quantized by that wave beside a long weight stream (5 to 8 rounds
        // per group: gate/up 2560x19456 W4 M=1 7.5 -> 6.7 us). Shorter streams
        // arrive before the wave's serial chain ends (qkv 4.3 -> 4.9 us, o
        // 4096x2560 3.9 -> 5.4 us with it), so their blocks quantize as a whole.
        const int w_chunks = (g.bits == 8 ? g.K_pad / 16 : g.K_pad / 32) * 8 * (epi == EPI_PLAIN ? 1 : 2);
        const int w_rounds = (w_chunks + 255) / 256;
        const int x_chunks = (g.K_pad / 16) * pv.mr;
        const int qb = x_type == DT_F32 ? gemv_qb<float>() : gemv_qb<__half>();
        // HM_GEMV_QW: 0 never, 1 whenever the rows fit (tests, experiments).
        const int qw_env = switch_value(SW_GEMV_QW);
        const bool qw_fits = !preq && pv.mr <= 2 && x_chunks <= 64 * qb && w_rounds <= 8;
        int qwn = 0;
        if (qw_fits && (qw_env == 1 || (qw_env < 0 && w_rounds >= 5))) qwn = 1;
        // One row with precomputed maxima (the down projection after the
        // SwiGLU GEMV) whose groups stream more than 8 rounds splits K so that
        // about 1280 blocks run (5 per CU) and each quantizes only its piece
        // of the row: the 320 blocks of the 9728x2560 down projection each
        // loaded and quantized all 38.9 KB of the f32 row before their first
        // dot product (7.45 -> 7.1 us; decode step +3.4% at 4 pieces, 6 and 8
        // pieces slower). Short groups lose to the pieces' extra partial-max
        // loads and atomic tail (MoE shared down 2048x2048). Pieces are whole
        // 64-k units, at least 8 of them; HM_GEMV_SPLITS forces a count.
        const int units = g.K_pad / 64;
        int ksplit = 1;
        const int forced_splits = switch_value(SW_GEMV_SPLITS);
        if (!preq && qwn == 0 && pv.mr == 1 && epi == EPI_PLAIN && in_max.p && ws->kacc &&
            (w_rounds > 8 || forced_splits > 0)) {
            ksplit = forced_splits > 0 ? forced_splits : (1280 + grid / 2) / grid;
            ksplit = std::max(1, std::min(std::min(ksplit, 8), units / 8));
        }
        const int piece_units = (units + ksplit - 1) / ksplit;
        const int piece_rounds = ((g.bits == 8 ? 4 : 2) * piece_units * 8 + 255) / 256;
        if (ksplit > 1 && piece_rounds > 8) ksplit = 1;
        if (preq) {
            int rc = enqueue_quant(ws, x, x_type, lda, rows, rule, in_max, nullptr, s);
            if (rc != RK_NPU_OK) return rc;
        }
        char name[64];
        std::snprintf(name, sizeof(name), "gemv<mr=%d,w%d,epi=%d>", pv.mr, g.bits, epi);
        const int slot = prof_begin(s, 0, g.bits, epi, rows, g.K, g.N, name);
        const bool combine = comb && switch_value(SW_GEMV_COMBINE) != 0 && rows == 1 && epi == EPI_PLAIN && !preq &&
                             qwn == 0 && ksplit == 1 &&
                             x_type == DT_F32 && c_type == DT_F32 && comb->top >= 1 && comb->top <= GEMV_COMB_TOP &&
                             w_rounds <= 8 && comb->h == g.N;
        if (combine) {
            V.comb_contrib = comb->contrib;
            V.comb_routes = comb->routes;
            V.comb_top = comb->top;
            V.comb_h = comb->h;
            launch_gemv_combine_any(g.bits, V, grid, w_rounds, lds, s);
            if (comb->combined) *comb->combined = true;
        } else if (ksplit > 1) {
            V.ksplit = ksplit;
            const size_t piece_lds = (size_t)64 * piece_units;
            launch_gemv_split_any(x_type, g.bits, V, grid * ksplit, piece_rounds, piece_lds, s);
        } else {
            launch_gemv_any(x_type, g.bits, epi, pv.mr, V, grid, lds, s, preq, qwn);
        }
        prof_end(slot, s);
        if (out_max) *out_max = RowMax{ws->partmax, grid};
    } else {
        int rc = enqueue_quant(ws, x, x_type, lda, rows, rule, in_max, epi != EPI_PLAIN ? ws->rowmax : nullptr, s);
        if (rc != RK_NPU_OK) return rc;
        const size_t c_esz = c_type == DT_F32 ? 4 : 2;
        const bool staged = (reinterpret_cast<uintptr_t>(c) & 15) == 0 && ((size_t)ldc * c_esz) % 16 == 0;
        Plan p = staged ? plan_linear(rows, g) : plan_gemm(rows, g, V128x128);
        // Split-K: staged 64x128 / 128x128 plans only, partials sized for the
        // workspace's own row count; otherwise the launch runs unsplit (same
        // result: the integer sums are exact).
        if (p.ksplit > 1 && (!staged || (p.variant != V64x128 && p.variant != V128x128) ||
                             (size_t)p.tiles * p.ksplit * p.bm * p.bn > ws->split_part_ints)) {
            p.ksplit = 1;
            p.grid = p.tiles;
        }
        GemmParams G;
        G.a = ws->codes;
        G.b = w->packed;
        G.rowscale = ws->rowscale;
        G.rowsum = ws->rowsum;
        G.colscale = w->colscale;
        G.c = c;
        G.ldc = ldc;
        G.c_type = c_type;
        G.M = rows;
        G.N = g.N;
        G.K_pad = g.K_pad;
        G.M_alloc = ws->M_alloc;
        G.N_pad = g.N_pad;
        G.half = g.half;
        G.rowmax = ws->rowmax;
        G.tiles_m = (rows + p.bm - 1) / p.bm;
        G.tiles_n = g.N_pad / p.bn;
        G.splits = p.ksplit;
        G.split_part = ws->split_part;
        char name[64];
        std::snprintf(name, sizeof(name), "gemm<%dx%d,w%d,epi=%d,k/%d>", p.bm, p.bn, g.bits, epi, p.ksplit);
        const int slot = prof_begin(s, 1, g.bits, epi, rows, g.K, g.N, name);
        launch_gemm_any(g.bits, epi, p.variant, staged, G, p.tiles, s);
        prof_end(slot, s);
        if (out_max) *out_max = RowMax{reinterpret_cast<const float*>(ws->rowmax), 1};
    }
    return hipGetLastError() == hipSuccess ? RK_NPU_OK : RK_NPU_ERR_DEVICE;
}

// --- the FFN of one row in one launch (ffn_m1_kernel, opt-in: HM_FFN_FUSED=1) ------
// Eligible: one row, a W4 SwiGLU gate_up whose tile pairs take 5 to 8 rounds of
// the block's 192 weight threads (K in 1600..3072; 2560x19456: 7) with a
// quantization wave, 16-byte aligned activations, and a down projection split
// into K pieces of at most 48 (W4) / 40 (W8) units of 64 (3 / 5 rounds of 256
// threads). Measured on the Qwen3-4B decode FFN (2560 -> 2x9728 -> 2560, W4,
// 36 distinct layers in a graph, one MI355X): 16.5 us per call against 14.3 us
// for the gate_up and split-K down launches, so it is not the default. Block
// timestamps of one call: every block starts within 1.1 us; the gate/up work
// publishes at 6.2 us (p50) but the last producer only at 8.5 us (the early
// finishers' down-weight loads compete with it); the arrival chain and the
// flag reach the down pieces at 11.0 us (p50); quantizing the middle slice
// (its loads, the barriers) ends at 13.2 us, the dots at 13.8, the split-K
// sums at 14.3 us: each step is a memory round trip of ~0.5 us under the
// full weight stream, and together they cost more than the second launch.
struct FfnFusedPlan {
    int rwg, rwd, ksplit, piece_units, producers, consumers;
};

static bool plan_ffn_fused(const Weights* gw, const Weights* dw, const void* A, int a_type, int rows,
                           FfnFusedPlan& fp) {
    if (rows != 1 || switch_value(SW_FFN_FUSED) == 0) return false;
    const Geometry& G = gw->g;
    const Geometry& Dg = dw->g;
    if (G.bits != 4 || !G.half || (a_type != DT_F32 && a_type != DT_F16)) return false;
    if (plan_linear(1, G).kind != 0 || plan_linear(1, Dg).kind != 0) return false;
    const size_t esz = a_type == DT_F32 ? 4 : 2;
    if (G.K % 16 != 0 || ((size_t)G.K * esz) % 16 != 0 || (reinterpret_cast<uintptr_t>(A) & 15) != 0) return false;
    // rounds of the block's weight threads over a gate/up tile pair
    const int w_rounds = ((G.K_pad / 32) * 8 * 2 + FFN_WEIGHT_THREADS - 1) / FFN_WEIGHT_THREADS;
    const int qb = a_type == DT_F32 ? gemv_qb<float>() : gemv_qb<__half>();
    if (w_rounds < 5 || w_rounds > 8 || G.K_pad / 16 > 64 * qb) return false;
    fp.rwg = w_rounds <= 6 ? 6 : (w_rounds <= 7 ? 7 : 8);
    // down: pieces of whole 64-k units, about 1280 blocks as the split-K GEMV
    const int units = Dg.K_pad / 64;
    const int max_units = Dg.bits == 4 ? 48 : 40;  // 3 / 5 rounds of 256 threads per piece
    const int groups = Dg.N_pad / 8;
    int ksplit = std::max(1, std::min((1280 + groups / 2) / groups, 8));
    const int forced = switch_value(SW_GEMV_SPLITS);
    if (forced > 0) ksplit = forced;
    ksplit = std::max(ksplit, (units + max_units - 1) / max_units);
    ksplit = std::min(ksplit, units);
    fp.piece_units = (units + ksplit - 1) / ksplit;
    if (fp.piece_units > max_units) return false;
    fp.ksplit = ksplit;
    fp.rwd = Dg.bits == 4 ? 3 : 5;
    fp.producers = G.N_pad / 16;
    fp.consumers = groups * ksplit;
    return true;
}

static GemvParams gemv_params(Workspace* ws, const Weights* w, const void* x, long lda, int rows, int rule, void* c,
                              int c_type, long ldc) {
    const Geometry& g = w->g;
    GemvParams V{};
    V.x = x;
    V.lda = lda;
    V.rule = rule;
    V.vec = 1;
    V.b = w->packed;
    V.colscale = w->colscale;
    V.c = c;
    V.ldc = ldc;
    V.c_type = c_type;
    V.M = rows;
    V.K = g.K;
    V.N = g.N;
    V.K_pad = g.K_pad;
    V.N_pad = g.N_pad;
    V.half = g.half;
    V.part_out = ws->partmax;
    V.diag_codes = ws->codes;
    V.diag_scale = ws->rowscale;
    V.diag_rowsum = ws->rowsum;
    V.M_alloc = ws->M_alloc;
    V.ksplit = 1;
    V.kacc = ws->kacc;
    return V;
}

// Enqueues the one-launch FFN; false (nothing enqueued) when the launch could
// not be resident as a whole on this GPU.
static bool enqueue_ffn_fused(Workspace* gws, const Weights* gw, Workspace* dws, const Weights* dw, const void* A,
                              int a_type, void* C, int c_type, int rule, const FfnFusedPlan& fp, hipStream_t s) {
    const int F = gw->g.N / 2;
    GemvParams Pg = gemv_params(gws, gw, A, gw->g.K, 1, rule, gws->c_f32, DT_F32, F);
    GemvParams Pd = gemv_params(dws, dw, gws->c_f32, F, 1, rule, C, c_type, dw->g.N);
    Pd.ksplit = fp.ksplit;
    for (GemvParams* P : {&Pg, &Pd}) {
        P->sync = dws->sync;
        P->producers = fp.producers;
        P->consumers = fp.consumers;
        P->spin_limit = switch_value(SW_FFN_SPIN);
    }
    const int grid = std::max(fp.producers, fp.consumers);
    const size_t lds = (size_t)gw->g.K_pad + (size_t)64 * fp.piece_units;
    char name[64];
    std::snprintf(name, sizeof(name), "ffn_m1<w4,w%d,k/%d>", dw->g.bits, fp.ksplit);
    const int slot = prof_begin(s, 0, dw->g.bits, EPI_SWIGLU_MAX, 1, gw->g.K, dw->g.N, name);
    bool launched;
    launched = launch_ffn_fused_any(a_type, dw->g.bits, fp.rwg, Pg, Pd, grid, lds, s);
    prof_end(slot, s);
    if (launched) dws->fused_pending = true;
    return launched;
}

// The down workspace's one-launch FFN error word: nonzero when a consumer of
// an earlier call gave up waiting for its producers (its output is then not
// valid). Reading clears it. The caller has synchronized the stream. The word
// is read only when a one-launch FFN ran since the last read, so the
// two-launch path (the default) adds no copy to the call.
int ffn_take_error(Workspace* dws) {
    if (!dws->sync || !dws->fused_pending) return RK_NPU_OK;
    dws->fused_pending = false;
    unsigned err = 0;
    unsigned* word = dws->sync + (4 * FFN_SLOTS + 2) * FFN_LINE;
    if (hipMemcpy(&err, word, 4, hipMemcpyDeviceToHost) != hipSuccess) return RK_NPU_ERR_DEVICE;
    if (!err) return RK_NPU_OK;
    const unsigned zero = 0;
    (void)hipMemcpy(word, &zero, 4, hipMemcpyHostToDevice);
    return RK_NPU_ERR_DEVICE;
}

int enqueue_ffn(Workspace* gws, const Weights* gw, Workspace* dws, const Weights* dw, const void* A, int a_type,
                void* C, int c_type, int rows, int rule, hipStream_t s, const GemvCombine* comb) {
    if (comb && comb->combined) *comb->combined = false;
    FfnFusedPlan fp;
    if (plan_ffn_fused(gw, dw, A, a_type, rows, fp) &&
        enqueue_ffn_fused(gws, gw, dws, dw, A, a_type, C, c_type, rule, fp, s))
        return hipGetLastError() == hipSuccess ? RK_NPU_OK : RK_NPU_ERR_DEVICE;
    const int F = gw->g.N / 2;
    RowMax mid_max{nullptr, 0};
    int rc = enqueue_linear(gws, gw, A, a_type, gw->g.K, rows, rule, RowMax{nullptr, 0}, gws->c_f32, DT_F32, F,
                            EPI_SWIGLU_MAX, &mid_max, s);
    if (rc == RK_NPU_OK)
        rc = enqueue_linear(dws, dw, gws->c_f32, DT_F32, F, rows, rule, mid_max, C, c_type, dw->g.N, EPI_PLAIN,
                            nullptr, s, comb);
    return rc;
}

// --- allocation-free linear (rk_npu_hip_linear_run_static) ----------------------
// The buffers a linear call needs besides its inputs and outputs (activation
// codes, row scales, code sums and maxima, GEMV partial maxima, split-K
// partials and slots) in one file-scope device array instead of a workspace.
// Each GPU holds its own copy until the process ends; in host code the name
// `scratch` is only a stand-in, so host code uses the device address that
// hipGetSymbolAddress returns for the current GPU, kept per device.
constexpr size_t STATIC_SCRATCH_BYTES = (size_t)RK_NPU_HIP_STATIC_SCRATCH_BYTES;
constexpr int STATIC_MAX_ROWS = RK_NPU_HIP_STATIC_MAX_ROWS;
static __device__ __attribute__((aligned(256))) uint8_t scratch[STATIC_SCRATCH_BYTES];

struct ScratchTable {
    std::mutex mu;
    std::vector<uint8_t*> ptr;  // by device ordinal
};
static ScratchTable& scratch_table() {
    static ScratchTable t;
    return t;
}

// Once per device, with that device current (rk_npu_open): look up this
// GPU's copy of the array and zero it once. Nothing in it needs to start at
// zero for a call: the buffers a call reads (codes, scales, maxima, split
// partials) are written by that call's own launches first, and the view holds
// no split-K GEMV slots (see scratch_workspace).
static int scratch_init(int dev) {
    ScratchTable& t = scratch_table();
    std::lock_guard<std::mutex> lock(t.mu);
    if (dev < 0) return RK_NPU_ERR_PARAM;
    if ((size_t)dev < t.ptr.size() && t.ptr[dev]) return RK_NPU_OK;
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
        (void)hipGetLastError();
        return RK_NPU_ERR_DEVICE;
    }
    if (hipMemset(p, 0, STATIC_SCRATCH_BYTES) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        (void)hipGetLastError();
        return RK_NPU_ERR_DEVICE;
    }
    if (t.ptr.size() <= (size_t)dev) t.ptr.resize((size_t)dev + 1, nullptr);
    t.ptr[dev] = static_cast<uint8_t*>(p);
    return RK_NPU_OK;
}

static uint8_t* scratch_of(int dev) {
    ScratchTable& t = scratch_table();
    std::lock_guard<std::mutex> lock(t.mu);
    return (dev >= 0 && (size_t)dev < t.ptr.size()) ? t.ptr[dev] : nullptr;
}

// A workspace view of the scratch array for `rows` rows of w's shape (no
// allocation: every buffer is a slice of the array); false when the rows or
// the shape's buffers exceed the array.
static bool scratch_workspace(uint8_t* base, const Weights* w, int rows, Workspace& ws) {
    if (rows < 1 || rows > STATIC_MAX_ROWS) return false;
    const Geometry& g = w->g;
    ws.magic = g.bits == 8 ? MAGIC_WS8 : MAGIC_WS4;
    ws.g = g;
    ws.M = rows;
    ws.M_alloc = round_up(rows, 256);
    ws.domain = w->domain;
    ws.stream = nullptr;
    ws.busy.store(false);
    ws.hs = HostStage{};
    ws.fused_pending = false;
    ws.a_f32 = nullptr;
    ws.c_f32 = nullptr;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        uint8_t* p = base + off;
        off += round_up_z(bytes, 256);
        return p;
    };
    ws.codes = reinterpret_cast<int8_t*>(take((size_t)(g.K_pad / 16) * ws.M_alloc * 16));
    ws.rowscale = reinterpret_cast<float*>(take((size_t)ws.M_alloc * 4));
    ws.rowsum = reinterpret_cast<int*>(take((size_t)ws.M_alloc * 4));
    ws.rowmax = reinterpret_cast<unsigned*>(take((size_t)ws.M_alloc * 4));
    ws.partmax = reinterpret_cast<float*>(take((size_t)g.N_pad * 4));
    // No split-K GEMV slots: that plan needs precomputed row maxima, which
    // this entry never takes, and the planner requires the slots.
    ws.kacc = nullptr;
    ws.sync = nullptr;  // (a linear call has no one-launch FFN)
    if (off > STATIC_SCRATCH_BYTES) return false;
    // the rest holds split-K partials; plans whose partials do not fit run unsplit
    ws.split_part = reinterpret_cast<int*>(base + off);
    ws.split_part_ints = (STATIC_SCRATCH_BYTES - off) / 4;
    ws.bytes = STATIC_SCRATCH_BYTES;
    return true;
}

// Pinned staging for the host-buffer calls. Copies between pageable caller
// memory and the device go through the runtime's own staging, which costs
// tens of microseconds per call at decode sizes (a few KB); the workspace
// instead keeps one pinned buffer, allocated on the first host call, that the
// caller's A is copied into and C out of by the CPU. Transfers above the cap
// (and a failed pinned allocation) keep the direct pageable copies.
constexpr size_t HOST_STAGE_CAP = 8u << 20;

// The stage is coherent (fine-grained) pinned memory, so the copy kernel's
// stores and its completion word reach host memory without a cache flush.
void* stage_reserve(HostStage& st, size_t bytes) {
    if (bytes == 0 || bytes > HOST_STAGE_CAP) return nullptr;
    if (st.bytes < bytes) {
        if (st.host) {
            if (st.last) (void)hipStreamSynchronize(st.last);  // (a previous call's copy kernel may still be ending)
            (void)hipHostFree(st.host);
        }
        st = HostStage{};
        const size_t want = std::min(HOST_STAGE_CAP, std::max(bytes, (size_t)64 << 10));
        void* dev = nullptr;
        void* host = nullptr;
        if (hipHostMalloc(&host, want + 256, hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess ||
            hipHostGetDevicePointer(&dev, host, 0) != hipSuccess) {
            if (host) (void)hipHostFree(host);
            (void)hipGetLastError();
            return nullptr;
        }
        st.host = host;
        st.dev = dev;
        st.bytes = want;
        st.done = reinterpret_cast<unsigned*>(static_cast<uint8_t*>(host) + want);
        st.done_dev = reinterpret_cast<unsigned*>(static_cast<uint8_t*>(dev) + want);
        __atomic_store_n(st.done, 0u, __ATOMIC_RELEASE);
    }
    return st.host;
}

void stage_release(HostStage& st) {
    if (st.host) (void)hipHostFree(st.host);
    st = HostStage{};
}

float* host_stage(Workspace* ws, size_t bytes) { return static_cast<float*>(stage_reserve(ws->hs, bytes)); }

// Host-buffer transfers. A small call (input and output each at most
// HOST_SMALL bytes, and a stage) stays on the compute queue from start to
// end: one launch fetches the inputs from the stage into device memory,
// the work runs, one block copies C into the stage and then sets the
// stage's completion word to the call's sequence number, and the CPU polls
// that word instead of waiting for the runtime to report the stream done.
// Measured on the box (M=1, C++ driver, us per rk_npu_w4a8_run_f32): qkv
// 2560x6144 26.2 -> 22.6, o 4096x2560 20.1 -> 21.2, down 9728x2560 27.8 ->
// 24.1 against copies and hipStreamSynchronize; with the copies kept for
// the upload only the download side changes and down takes 35.8 (the next
// call's copy engine then waits on the compute queue's completion). The
// poll gives way to hipStreamSynchronize after HM_HOST_POLL microseconds
// (2000; tests set 0 to take that way every time), which also reports a
// failed stream. Larger calls copy through the stage (or pageable
// memory) and wait on the stream (HM_HOST_SPIN). HM_HOST_FLAG=0 makes every
// call take the copies.
constexpr size_t HOST_SMALL = 64u << 10;

// Segments of a fetch: up to three (source in the stage, device destination,
// 16-byte pieces); every source and destination is 16-byte aligned and
// extends to a whole piece.
struct HostFetch {
    const v4u* src[3];
    v4u* dst[3];
    int pieces[3];
    int n;
};

__global__ __launch_bounds__(256) void host_fetch_kernel(HostFetch F) {
#pragma unroll
    for (int k = 0; k < 3; ++k)
        if (k < F.n)
            for (int i = blockIdx.x * 256 + threadIdx.x; i < F.pieces[k]; i += gridDim.x * 256) F.dst[k][i] = F.src[k][i];
}

__global__ __launch_bounds__(1024) void host_publish_kernel(const v4u* __restrict__ src, v4u* __restrict__ dst,
                                                            int pieces, unsigned* done, unsigned seq) {
    for (int i = threadIdx.x; i < pieces; i += blockDim.x) dst[i] = src[i];
    __threadfence_system();  // (this thread's stores reach the host before the word)
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(done, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

bool host_kernels_enabled() { return switch_value(SW_HOST_FLAG) != 0; }

bool stage_small(const HostStage& st, const void* p, size_t in_bytes, size_t out_bytes) {
    return p && st.done && in_bytes <= HOST_SMALL && out_bytes <= HOST_SMALL && switch_value(SW_HOST_FLAG) != 0;
}

bool stage_upload(HostStage& stg, bool small, void* st, const HostSeg* segs, int n, hipStream_t s) {
    if (n < 1 || n > 3) return false;
    if (st) stg.last = s;
    if (!st) {
        for (int k = 0; k < n; ++k)
            if (hipMemcpyAsync(segs[k].dst, segs[k].src, segs[k].bytes, hipMemcpyHostToDevice, s) != hipSuccess)
                return false;
        return true;
    }
    HostFetch F;
    F.n = n;
    int most = 0;
    for (int k = 0; k < n; ++k) {
        uint8_t* at = static_cast<uint8_t*>(st) + segs[k].stage_off;
        std::memcpy(at, segs[k].src, segs[k].bytes);
        if (!small && hipMemcpyAsync(segs[k].dst, at, segs[k].bytes, hipMemcpyHostToDevice, s) != hipSuccess)
            return false;
        F.src[k] = reinterpret_cast<const v4u*>(static_cast<uint8_t*>(stg.dev) + segs[k].stage_off);
        F.dst[k] = static_cast<v4u*>(segs[k].dst);
        F.pieces[k] = (int)((segs[k].bytes + 15) / 16);
        most = std::max(most, F.pieces[k]);
    }
    if (!small) return true;
    hipLaunchKernelGGL(host_fetch_kernel, dim3(std::max(1, std::min(64, (most + 255) / 256))), dim3(256), 0, s, F);
    return hipGetLastError() == hipSuccess;
}

// The end of a host-buffer call: wait until everything enqueued on its stream
// has finished. HM_HOST_SPIN=0 (default): block in hipStreamSynchronize;
// 1: poll hipStreamQuery. Polling measured slower (M=1 decode set of four
// host calls per layer: 131 us blocking, 157-159 us polling).
hipError_t host_wait(hipStream_t s) {
    if (switch_value(SW_HOST_SPIN) != 0) {
        for (;;) {
            const hipError_t e = hipStreamQuery(s);
            if (e != hipErrorNotReady) return e;
            __builtin_ia32_pause();
        }
    }
    return hipStreamSynchronize(s);
}

bool stage_download(HostStage& stg, bool small, void* st, void* C, const void* src, size_t bytes, hipStream_t s) {
    if (st) stg.last = s;
    if (!small) {
        if (bytes == 0) return host_wait(s) == hipSuccess;
        if (!st)
            return hipMemcpyAsync(C, src, bytes, hipMemcpyDeviceToHost, s) == hipSuccess && host_wait(s) == hipSuccess;
        if (hipMemcpyAsync(st, src, bytes, hipMemcpyDeviceToHost, s) != hipSuccess || host_wait(s) != hipSuccess)
            return false;
        std::memcpy(C, st, bytes);
        return true;
    }
    const unsigned seq = ++stg.seq == 0 ? ++stg.seq : stg.seq;  // (0 is the word's initial value)
    const int pieces = (int)((bytes + 15) / 16);
    hipLaunchKernelGGL(host_publish_kernel, dim3(1), dim3(1024), 0, s, static_cast<const v4u*>(src),
                       static_cast<v4u*>(stg.dev), pieces, stg.done_dev, seq);
    if (hipGetLastError() != hipSuccess) {
        (void)hipStreamSynchronize(s);
        return false;
    }
    const double t0 = now_us(), limit = (double)switch_value(SW_HOST_POLL);
    for (unsigned n = 1; __atomic_load_n(stg.done, __ATOMIC_ACQUIRE) != seq; ++n) {
        if ((n & 255) == 0 && now_us() - t0 >= limit) {
            if (hipStreamSynchronize(s) != hipSuccess || __atomic_load_n(stg.done, __ATOMIC_ACQUIRE) != seq)
                return false;
            break;
        }
        __builtin_ia32_pause();
    }
    if (bytes) std::memcpy(C, st, bytes);
    return true;
}

}  // namespace hm

using namespace hm;

// ============================================================================
// C ABI
// ============================================================================
extern "C" {

const char* rk_npu_strerror(int rc) {
    switch (rc) {
        case RK_NPU_OK:
            return "success";
        case RK_NPU_ERR_PARAM:
            return "invalid argument";
        case RK_NPU_ERR_NOMEM:
            return "out of device memory";
        case RK_NPU_ERR_DEVICE:
            return "HIP device error";
        case RK_NPU_ERR_CACHE_MISS:
            return "tuning cache miss";
        case RK_NPU_ERR_BUSY:
            return "workspace busy";
        case RK_NPU_ERR_UNSUPPORTED:
            return "unsupported operation";
        case RK_NPU_ERR_FORMAT:
            return "invalid expert record";
        default:
            return "unknown error";
    }
}

rk_npu_ctx* rk_npu_open(const char* device) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        return nullptr;
    }
    int dev = 0;
    if (device && *device) {
        char* end = nullptr;
        long v = std::strtol(device, &end, 10);
        if (*end != '\0' || v < 0 || v >= count) return nullptr;
        dev = (int)v;
    } else if (hipGetDevice(&dev) != hipSuccess) {
        return nullptr;
    }
    if (hipSetDevice(dev) != hipSuccess) return nullptr;
    // (a failure leaves rk_npu_hip_linear_run_static returning RK_NPU_ERR_DEVICE
    // on this device; the context itself stays usable)
    (void)scratch_init(dev);
    rk_npu_ctx* ctx = new (std::nothrow) rk_npu_ctx();
    if (ctx) ctx->device = dev;
    return ctx;
}

void rk_npu_close(rk_npu_ctx* ctx) { delete ctx; }

rk_npu_iommu_domain* rk_npu_iommu_domain_create(rk_npu_ctx* ctx, uint32_t id) {
    if (!ctx || id >= RK_NPU_IOMMU_DOMAIN_COUNT) return nullptr;
    Domain* d = new (std::nothrow) Domain();
    if (!d) return nullptr;
    d->ctx = ctx;
    d->id = id;
    return d;
}

void rk_npu_iommu_domain_free(rk_npu_iommu_domain* domain) { delete static_cast<Domain*>(domain); }

void rk_npu_iommu_domain_set_reclaim(rk_npu_iommu_domain* domain, void (*reclaim)(void*), void* cookie) {
    if (!domain) return;
    std::lock_guard<std::mutex> lock(domain->reclaim_mu);
    domain->reclaim = reclaim;
    domain->cookie = cookie;
}

int rk_npu_iommu_domain_memory_stats(const rk_npu_iommu_domain* domain, rk_npu_domain_memory_stats* stats) {
    if (!domain || !stats) return RK_NPU_ERR_PARAM;
    stats->live_bytes = domain->live.load();
    stats->peak_bytes = domain->peak.load();
    stats->creates = domain->creates.load();
    stats->destroys = domain->destroys.load();
    return RK_NPU_OK;
}

// ---- W8 ---------------------------------------------------------------------

rk_npu_f32i8f32_weights* rk_npu_f32i8f32_weights_create(rk_npu_iommu_domain* domain,
                                                        const rk_npu_matmul_weight_config* config,
                                                        const int8_t* codes, const float* scales) {
    if (!config) return nullptr;
    return static_cast<rk_npu_f32i8f32_weights*>(
        weights_create(static_cast<Domain*>(domain), 8, config->K, config->N, codes, scales, false));
}

rk_npu_f32i8f32_weights* rk_npu_f32i8f32_weights_create_compress(rk_npu_iommu_domain* domain,
                                                                 const rk_npu_matmul_weight_config* config,
                                                                 const int8_t* codes, const float* scales) {
    return rk_npu_f32i8f32_weights_create(domain, config, codes, scales);
}

void rk_npu_f32i8f32_weights_free(rk_npu_f32i8f32_weights* weights) { weights_destroy(weights); }

int rk_npu_f32i8f32_weights_memory_query(const rk_npu_matmul_weight_config* config,
                                         rk_npu_matmul_weight_requirements* requirements) {
    if (!config || !requirements || config->K <= 0 || config->N <= 0) return RK_NPU_ERR_PARAM;
    requirements->bytes = weight_bytes(make_geometry(8, config->K, config->N));
    return RK_NPU_OK;
}

uint64_t rk_npu_f32i8f32_weights_compressed_layout_generation(const rk_npu_f32i8f32_weights*) { return 0; }

// Legality table of the caller's W8 K partition (src/npu.rs:1568-1595):
// a tile must be a positive multiple of 32 no larger than min(K, 4096), and a
// multiple of 512 unless the call has at most 4 rows.
int rk_npu_matmul_k_partition_query(int rows, int K, int k_tile) {
    if (rows <= 0 || K <= 0 || k_tile <= 0) return RK_NPU_ERR_PARAM;
    if (k_tile > K || k_tile > 4096 || k_tile % 32 != 0) return RK_NPU_ERR_PARAM;
    if (k_tile % 512 != 0 && rows > 4) return RK_NPU_ERR_PARAM;
    return RK_NPU_OK;
}

void rk_npu_matmul_autotune_config_init(rk_npu_matmul_autotune_config* config, int M, int N, int K) {
    if (!config) return;
    std::memset(config, 0, sizeof(*config));
    config->M = M;
    config->N = N;
    config->K = K;
    config->required_k_tile = K;
    config->allowed_npu_core_mask = 1;
    config->warmup = 1;
    config->loops = 3;
    config->repeats = 3;
}

int rk_npu_matmul_autotune_cache_load(rk_npu_ctx*, const char*, rk_npu_matmul_op_kind,
                                      const rk_npu_matmul_autotune_config* config, rk_npu_matmul_strategy*,
                                      rk_npu_matmul_strategy*) {
    return config ? RK_NPU_ERR_CACHE_MISS : RK_NPU_ERR_PARAM;
}

static void fill_w8_strategy(const rk_npu_matmul_autotune_config* c, rk_npu_matmul_strategy* s) {
    std::memset(s, 0, sizeof(*s));
    s->op_kind = RK_NPU_MATMUL_F32I8F32_DYNAMIC;
    s->M = c->M;
    s->N = c->N;
    s->K = c->K;
    s->k_tile = c->required_k_tile > 0 ? c->required_k_tile : c->K;
    const Plan p = plan_linear(c->M, make_geometry(8, c->K, c->N));
    s->n_tile = p.bn;
    s->a_layout = RK_NPU_MATMUL_A_LAYOUT_NORMAL;
    s->c_layout = RK_NPU_MATMUL_C_LAYOUT_NATIVE;
    s->wave_count = 1;
    s->n_groups = (round_up(c->N, 256) + p.bn - 1) / p.bn;
    s->npu_core_mask = c->allowed_npu_core_mask;
    s->cpu_core_mask = c->allowed_cpu_core_mask;
    s->cpu_threads = 1;
    s->total_us = 1.0;
}

int rk_npu_matmul_autotune_cached(rk_npu_ctx* ctx, const rk_npu_matmul_autotune_config* config,
                                  rk_npu_matmul_op_kind op, const char*, int, rk_npu_matmul_strategy* fastest,
                                  rk_npu_matmul_strategy* stable, int* hit) {
    if (!ctx || !config || !fastest || op != RK_NPU_MATMUL_F32I8F32_DYNAMIC || config->M <= 0 ||
        config->N <= 0 || config->K <= 0)
        return RK_NPU_ERR_PARAM;
    fill_w8_strategy(config, fastest);
    if (stable) *stable = *fastest;
    if (hit) *hit = 0;
    return RK_NPU_OK;
}

int rk_npu_matmul_workspace_memory_query(const rk_npu_matmul_strategy* strategy,
                                         rk_npu_matmul_workspace_requirements* requirements) {
    if (!strategy || !requirements || strategy->M <= 0 || strategy->K <= 0 || strategy->N <= 0)
        return RK_NPU_ERR_PARAM;
    requirements->bytes = workspace_bytes(make_geometry(8, strategy->K, strategy->N), strategy->M);
    return RK_NPU_OK;
}

rk_npu_matmul_workspace* rk_npu_matmul_workspace_create(rk_npu_iommu_domain* domain,
                                                        const rk_npu_matmul_strategy* strategy) {
    if (!strategy) return nullptr;
    return static_cast<rk_npu_matmul_workspace*>(
        workspace_create(static_cast<Domain*>(domain), 8, strategy->M, strategy->K, strategy->N));
}

void rk_npu_matmul_workspace_free(rk_npu_matmul_workspace* workspace) { workspace_destroy(workspace); }

// Host-buffer call: upload A, quantize, multiply, download C, synchronize.
static int run_host(Workspace* ws, const Weights* w, const float* A, float* C, int epi,
                    rk_npu_w4a8_timings* timings) {
    const double t0 = now_us();
    if (!ws || !w || !A || !C) return RK_NPU_ERR_PARAM;
    if (ws->g.K != w->g.K || ws->g.N != w->g.N || ws->g.bits != w->g.bits) return RK_NPU_ERR_PARAM;
    if (epi != EPI_PLAIN && !w->g.half) return RK_NPU_ERR_UNSUPPORTED;  // SwiGLU needs N % 64 == 0
    BusyGuard guard(ws->busy);
    if (!guard.ok) return RK_NPU_ERR_BUSY;
    if (hipSetDevice(device_of(ws->domain)) != hipSuccess) return RK_NPU_ERR_DEVICE;
    const int M = ws->M, K = w->g.K, N = w->g.N;
    const int width = epi == EPI_PLAIN ? N : N / 2;
    float* st = host_stage(ws, std::max((size_t)M * K * 4, (size_t)M * width * 4));
    const bool small = stage_small(ws->hs, st, (size_t)M * K * 4, (size_t)M * width * 4);
    const HostSeg seg{A, ws->a_f32, (size_t)M * K * 4, 0};
    if (!stage_upload(ws->hs, small, st, &seg, 1, ws->stream)) {
        (void)hipStreamSynchronize(ws->stream);
        return RK_NPU_ERR_DEVICE;
    }
    const double t1 = now_us();
    int rc = enqueue_linear(ws, w, ws->a_f32, DT_F32, K, M, QUANT_DENSE, RowMax{nullptr, 0}, ws->c_f32, DT_F32,
                            width, epi, nullptr, ws->stream);
    if (rc != RK_NPU_OK) {
        (void)hipStreamSynchronize(ws->stream);
        return rc;
    }
    if (timings && hipStreamSynchronize(ws->stream) != hipSuccess) return RK_NPU_ERR_DEVICE;
    const double t2 = now_us();
    if (!stage_download(ws->hs, small, st, C, ws->c_f32, (size_t)M * width * 4, ws->stream)) return RK_NPU_ERR_DEVICE;
    if (timings) {
        const double t3 = now_us();
        timings->upload_us = t1 - t0;
        timings->device_us = t2 - t1;
        timings->download_us = t3 - t2;
        timings->total_us = t3 - t0;
    }
    return RK_NPU_OK;
}

static Workspace* as_ws(void* p, int bits) {
    Workspace* ws = static_cast<Workspace*>(p);
    if (!ws || ws->magic != (bits == 8 ? MAGIC_WS8 : MAGIC_WS4)) return nullptr;
    return ws;
}
static const Weights* as_w(const void* p, int bits) {
    const Weights* w = static_cast<const Weights*>(p);
    if (!w || w->magic != (bits == 8 ? MAGIC_W8 : MAGIC_W4)) return nullptr;
    return w;
}

int rk_npu_f32i8f32_run_dynamic(rk_npu_matmul_workspace* workspace, const rk_npu_f32i8f32_weights* weights,
                                const float* A, float* C) {
    return run_host(as_ws(workspace, 8), as_w(weights, 8), A, C, EPI_PLAIN, nullptr);
}

// ---- W4 ---------------------------------------------------------------------

rk_npu_w4a8_weights* rk_npu_w4a8_weights_create(rk_npu_iommu_domain* domain, const rk_npu_i4_weight_config* config,
                                                const int8_t* codes, const float* scales) {
    if (!config) return nullptr;
    return static_cast<rk_npu_w4a8_weights*>(
        weights_create(static_cast<Domain*>(domain), 4, config->K, config->N, codes, scales, false));
}

void rk_npu_w4a8_weights_free(rk_npu_w4a8_weights* weights) { weights_destroy(weights); }

int rk_npu_w4a8_weights_query(const rk_npu_w4a8_weights* weights, rk_npu_w4a8_weight_info* info) {
    if (!weights || !info || weights->magic != MAGIC_W4) return RK_NPU_ERR_PARAM;
    info->bound_relaxed = 0;
    info->multiplier = 1.0f;
    info->config.K = weights->g.K;
    info->config.N = weights->g.N;
    info->config.k_tile = weights->g.K;
    return RK_NPU_OK;
}

int rk_npu_i4_weights_memory_query(const rk_npu_i4_weight_config* config, uint64_t* bytes) {
    if (!config || !bytes || config->K <= 0 || config->N <= 0) return RK_NPU_ERR_PARAM;
    *bytes = weight_bytes(make_geometry(4, config->K, config->N));
    return RK_NPU_OK;
}

void rk_npu_w4a8_config_init(rk_npu_w4a8_config* config, int M, int N, int K) {
    if (!config) return;
    std::memset(config, 0, sizeof(*config));
    config->M = M;
    config->N = N;
    config->K = K;
    config->k_tile = K;
    config->m_tile = std::min(M, 64);
    config->n_tile = std::min(round_up(N, 64), 1024);
    config->npu_core_mask = 1;
    config->cpu_threads = 1;
    config->pipeline = RK_NPU_W4A8_PIPELINED;
}

void rk_npu_w4a8_options_init(rk_npu_w4a8_options* options) {
    if (options) options->reduce_backend = RK_NPU_W4A8_REDUCE_DEVICE;
}

int rk_npu_w4a8_memory_query_ex(const rk_npu_w4a8_config* config, const rk_npu_w4a8_options*,
                                rk_npu_w4a8_memory_info_ex* info) {
    if (!config || !info || config->M <= 0 || config->K <= 0 || config->N <= 0) return RK_NPU_ERR_PARAM;
    info->workspace_bytes = workspace_bytes(make_geometry(4, config->K, config->N), config->M);
    return RK_NPU_OK;
}

rk_npu_w4a8_workspace* rk_npu_w4a8_workspace_create_ex(rk_npu_iommu_domain* domain, const rk_npu_w4a8_config* config,
                                                       const rk_npu_w4a8_options*) {
    if (!config) return nullptr;
    return static_cast<rk_npu_w4a8_workspace*>(
        workspace_create(static_cast<Domain*>(domain), 4, config->M, config->K, config->N));
}

void rk_npu_w4a8_workspace_free(rk_npu_w4a8_workspace* workspace) { workspace_destroy(workspace); }

int rk_npu_w4a8_run_f32(rk_npu_w4a8_workspace* workspace, const rk_npu_w4a8_weights* weights, const float* A,
                        float* C, rk_npu_w4a8_timings* timings) {
    return run_host(as_ws(workspace, 4), as_w(weights, 4), A, C, EPI_PLAIN, timings);
}

int rk_npu_w4a8_run_swiglu_f32(rk_npu_w4a8_workspace* workspace, const rk_npu_w4a8_weights* weights,
                               const float* A, float* C, rk_npu_w4a8_timings* timings) {
    // The SwiGLU+max epilogue also records the middle's row maxima in the
    // workspace; the outputs are identical to the plain SwiGLU epilogue.
    return run_host(as_ws(workspace, 4), as_w(weights, 4), A, C, EPI_SWIGLU_MAX, timings);
}

static int check_ffn(Workspace* gws, const Weights* gw, Workspace* dws, const Weights* dw, int rows) {
    if (!gws || !gw || !dws || !dw) return RK_NPU_ERR_PARAM;
    if (gws->g.K != gw->g.K || gws->g.N != gw->g.N || dws->g.K != dw->g.K || dws->g.N != dw->g.N)
        return RK_NPU_ERR_PARAM;
    if (!gw->g.half || dw->g.K != gw->g.N / 2 || dw->g.N != gw->g.K) return RK_NPU_ERR_PARAM;
    if (rows < 1 || rows > gws->M || rows > dws->M) return RK_NPU_ERR_PARAM;
    return RK_NPU_OK;
}

int rk_npu_w4a8_run_ffn_f32(rk_npu_w4a8_workspace* gate_up_workspace, const rk_npu_w4a8_weights* gate_up,
                            void* down_workspace, const void* down, int down_bits, const float* A, float* C,
                            rk_npu_w4a8_timings* timings) {
    const double t0 = now_us();
    Workspace* gws = as_ws(gate_up_workspace, 4);
    const Weights* gw = as_w(gate_up, 4);
    Workspace* dws = as_ws(down_workspace, down_bits);
    const Weights* dw = as_w(down, down_bits);
    if (!A || !C || (down_bits != 4 && down_bits != 8)) return RK_NPU_ERR_PARAM;
    int rc = check_ffn(gws, gw, dws, dw, gws ? gws->M : 0);
    if (rc != RK_NPU_OK) return rc;
    if (gws->M != dws->M) return RK_NPU_ERR_PARAM;
    BusyGuard g1(gws->busy);
    if (!g1.ok) return RK_NPU_ERR_BUSY;
    BusyGuard g2(dws->busy);
    if (!g2.ok) return RK_NPU_ERR_BUSY;
    if (hipSetDevice(device_of(gws->domain)) != hipSuccess) return RK_NPU_ERR_DEVICE;
    const int M = gws->M, H = gw->g.K;
    hipStream_t s = gws->stream;
    // A in and C out through the gate_up workspace's stage (both M x H f32),
    // on that workspace's stream, which runs the whole call
    float* st = host_stage(gws, (size_t)M * H * 4);
    const bool small = stage_small(gws->hs, st, (size_t)M * H * 4, (size_t)M * H * 4);
    const HostSeg seg{A, gws->a_f32, (size_t)M * H * 4, 0};
    if (!stage_upload(gws->hs, small, st, &seg, 1, s)) {
        (void)hipStreamSynchronize(s);
        return RK_NPU_ERR_DEVICE;
    }
    const double t1 = now_us();
    rc = enqueue_ffn(gws, gw, dws, dw, gws->a_f32, DT_F32, dws->c_f32, DT_F32, M, QUANT_DENSE, s);
    if (rc != RK_NPU_OK) {
        (void)hipStreamSynchronize(s);
        return rc;
    }
    if (timings && hipStreamSynchronize(s) != hipSuccess) return RK_NPU_ERR_DEVICE;
    const double t2 = now_us();
    if (!stage_download(gws->hs, small, st, C, dws->c_f32, (size_t)M * H * 4, s)) return RK_NPU_ERR_DEVICE;
    rc = ffn_take_error(dws);
    if (rc != RK_NPU_OK) return rc;
    if (timings) {
        const double t3 = now_us();
        timings->upload_us = t1 - t0;
        timings->device_us = t2 - t1;
        timings->download_us = t3 - t2;
        timings->total_us = t3 - t0;
    }
    return RK_NPU_OK;
}

// ---- tuning (W4) ------------------------------------------------------------

struct rk_npu_w4a8_tuning_profile {
    uint64_t fingerprint;
};

rk_npu_w4a8_tuning_profile* rk_npu_w4a8_tuning_profile_from_weights(const rk_npu_w4a8_weights* weights) {
    if (!weights || weights->magic != MAGIC_W4) return nullptr;
    rk_npu_w4a8_tuning_profile* p = new (std::nothrow) rk_npu_w4a8_tuning_profile();
    if (p) p->fingerprint = weights->fingerprint;
    return p;
}

void rk_npu_w4a8_tuning_profile_free(rk_npu_w4a8_tuning_profile* profile) { delete profile; }

uint64_t rk_npu_w4a8_tuning_profile_fingerprint(const rk_npu_w4a8_tuning_profile* profile) {
    return profile ? profile->fingerprint : 0;
}

void rk_npu_w4a8_autotune_config_init(rk_npu_w4a8_autotune_config* config, int M, int N, int K) {
    if (!config) return;
    std::memset(config, 0, sizeof(*config));
    config->M = M;
    config->N = N;
    config->K = K;
    config->required_k_tile = 0;
    config->k_tile_multiplier = 1.0;
    config->allowed_npu_core_mask = 1;
    config->warmup = 1;
    config->loops = 3;
    config->repeats = 3;
}

int rk_npu_w4a8_autotune_cache_load_profile_ex(rk_npu_ctx*, const rk_npu_w4a8_autotune_config* config,
                                               const rk_npu_w4a8_tuning_profile*, const char*,
                                               rk_npu_w4a8_strategy_ex*, rk_npu_w4a8_strategy_ex*) {
    return config ? RK_NPU_ERR_CACHE_MISS : RK_NPU_ERR_PARAM;
}

static void fill_w4_strategy(const rk_npu_w4a8_autotune_config* c, rk_npu_w4a8_strategy_ex* s) {
    std::memset(s, 0, sizeof(*s));
    rk_npu_w4a8_config_init(&s->base.config, c->M, c->N, c->K);
    if (c->required_k_tile > 0) s->base.config.k_tile = c->required_k_tile;
    const Plan p = plan_linear(c->M, make_geometry(4, c->K, c->N));
    s->base.config.m_tile = p.bm;
    s->base.config.n_tile = p.bn;
    s->base.config.npu_core_mask = c->allowed_npu_core_mask;
    s->base.cpu_core_mask = c->allowed_cpu_core_mask;
    s->base.total_us = 1.0;
    rk_npu_w4a8_options_init(&s->execution);
}

int rk_npu_w4a8_autotune_cached_ex(rk_npu_ctx* ctx, const rk_npu_w4a8_autotune_config* config, const int8_t*,
                                   const float*, const char*, int, rk_npu_w4a8_strategy_ex* fastest,
                                   rk_npu_w4a8_strategy_ex* stable, int* hit) {
    if (!ctx || !config || !fastest || config->M <= 0 || config->N <= 0 || config->K <= 0) return RK_NPU_ERR_PARAM;
    fill_w4_strategy(config, fastest);
    if (stable) *stable = *fastest;
    if (hit) *hit = 0;
    return RK_NPU_OK;
}

int rk_npu_w4a8_autotune_ex(rk_npu_ctx* ctx, const rk_npu_w4a8_autotune_config* config, const int8_t* codes,
                            const float* scales, rk_npu_w4a8_strategy_ex* fastest, rk_npu_w4a8_strategy_ex* stable) {
    int hit = 0;
    return rk_npu_w4a8_autotune_cached_ex(ctx, config, codes, scales, nullptr, 0, fastest, stable, &hit);
}

// ---- device-resident extensions -------------------------------------------------

int rk_npu_hip_linear_run(void* workspace, const void* weights, int bits, const void* A, int a_type, void* C,
                          int c_type, int rows, int epilogue, void* stream) {
    Workspace* ws = as_ws(workspace, bits);
    const Weights* w = as_w(weights, bits);
    if (!ws || !w || !A || !C) return RK_NPU_ERR_PARAM;
    if ((a_type != DT_F32 && a_type != DT_F16) || (c_type != DT_F32 && c_type != DT_F16)) return RK_NPU_ERR_PARAM;
    if (ws->g.K != w->g.K || ws->g.N != w->g.N || rows < 1 || rows > ws->M) return RK_NPU_ERR_PARAM;
    if (epilogue != RK_NPU_HIP_PLAIN && epilogue != RK_NPU_HIP_SWIGLU) return RK_NPU_ERR_PARAM;
    const int epi = epilogue == RK_NPU_HIP_SWIGLU ? EPI_SWIGLU_MAX : EPI_PLAIN;
    if (epi != EPI_PLAIN && !w->g.half) return RK_NPU_ERR_UNSUPPORTED;  // SwiGLU needs N % 64 == 0
    BusyGuard guard(ws->busy);
    if (!guard.ok) return RK_NPU_ERR_BUSY;
    if (hipSetDevice(device_of(ws->domain)) != hipSuccess) return RK_NPU_ERR_DEVICE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int width = epi == EPI_PLAIN ? w->g.N : w->g.N / 2;
    return enqueue_linear(ws, w, A, a_type, w->g.K, rows, QUANT_DENSE, RowMax{nullptr, 0}, C, c_type, width, epi,
                          nullptr, s);
}

int rk_npu_hip_linear_run_static(const void* weights, int bits, const void* A, int a_type, void* C, int c_type,
                                 int rows, int epilogue, void* stream) {
    const Weights* w = as_w(weights, bits);
    if (!w || !A || !C) return RK_NPU_ERR_PARAM;
    if ((a_type != DT_F32 && a_type != DT_F16) || (c_type != DT_F32 && c_type != DT_F16)) return RK_NPU_ERR_PARAM;
    if (epilogue != RK_NPU_HIP_PLAIN && epilogue != RK_NPU_HIP_SWIGLU) return RK_NPU_ERR_PARAM;
    const int epi = epilogue == RK_NPU_HIP_SWIGLU ? EPI_SWIGLU_MAX : EPI_PLAIN;
    if (epi != EPI_PLAIN && !w->g.half) return RK_NPU_ERR_UNSUPPORTED;  // SwiGLU needs N % 64 == 0
    const int dev = device_of(w->domain);
    uint8_t* base = scratch_of(dev);
    if (!base) return RK_NPU_ERR_DEVICE;
    Workspace ws;
    if (!scratch_workspace(base, w, rows, ws)) return RK_NPU_ERR_PARAM;  // rows or shape beyond the array
    if (hipSetDevice(dev) != hipSuccess) return RK_NPU_ERR_DEVICE;
    const int width = epi == EPI_PLAIN ? w->g.N : w->g.N / 2;
    return enqueue_linear(&ws, w, A, a_type, w->g.K, rows, QUANT_DENSE, RowMax{nullptr, 0}, C, c_type, width, epi,
                          nullptr, static_cast<hipStream_t>(stream));
}

int rk_npu_hip_ffn_run(void* gate_up_workspace, const void* gate_up, int gu_bits, void* down_workspace,
                       const void* down, int dn_bits, const void* A, int a_type, void* C, int c_type, int rows,
                       void* stream) {
    Workspace* gws = as_ws(gate_up_workspace, gu_bits);
    const Weights* gw = as_w(gate_up, gu_bits);
    Workspace* dws = as_ws(down_workspace, dn_bits);
    const Weights* dw = as_w(down, dn_bits);
    if (!A || !C || (a_type != DT_F32 && a_type != DT_F16) || (c_type != DT_F32 && c_type != DT_F16))
        return RK_NPU_ERR_PARAM;
    int rc = check_ffn(gws, gw, dws, dw, rows);
    if (rc != RK_NPU_OK) return rc;
    BusyGuard g1(gws->busy);
    if (!g1.ok) return RK_NPU_ERR_BUSY;
    BusyGuard g2(dws->busy);
    if (!g2.ok) return RK_NPU_ERR_BUSY;
    if (hipSetDevice(device_of(gws->domain)) != hipSuccess) return RK_NPU_ERR_DEVICE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    return enqueue_ffn(gws, gw, dws, dw, A, a_type, C, c_type, rows, QUANT_DENSE, s);
}

int rk_npu_hip_ffn_status(void* down_workspace, int dn_bits) {
    Workspace* dws = as_ws(down_workspace, dn_bits);
    if (!dws) return RK_NPU_ERR_PARAM;
    if (hipSetDevice(device_of(dws->domain)) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
        return RK_NPU_ERR_DEVICE;
    return ffn_take_error(dws);
}

rk_npu_f32i8f32_weights* rk_npu_hip_f32i8f32_weights_create_device(rk_npu_iommu_domain* domain,
                                                                   const rk_npu_matmul_weight_config* config,
                                                                   const int8_t* codes, const float* scales) {
    if (!config) return nullptr;
    return static_cast<rk_npu_f32i8f32_weights*>(
        weights_create(static_cast<Domain*>(domain), 8, config->K, config->N, codes, scales, true));
}

rk_npu_w4a8_weights* rk_npu_hip_w4a8_weights_create_device(rk_npu_iommu_domain* domain,
                                                           const rk_npu_i4_weight_config* config, const int8_t* codes,
                                                           const float* scales) {
    if (!config) return nullptr;
    return static_cast<rk_npu_w4a8_weights*>(
        weights_create(static_cast<Domain*>(domain), 4, config->K, config->N, codes, scales, true));
}

void* rk_npu_hip_weights_create_checkpoint(rk_npu_iommu_domain* domain, int bits, int k,
                                           const rk_npu_hip_checkpoint_part* parts, int count) {
    Weights* w = weights_create_ckpt(static_cast<Domain*>(domain), bits, k, parts, count);
    if (!w) return nullptr;
    if (bits == 8) return static_cast<rk_npu_f32i8f32_weights*>(w);
    return static_cast<rk_npu_w4a8_weights*>(w);
}

int rk_npu_hip_workspace_codes(void* workspace, int bits, int rows, int8_t* codes, float* scales,
                               int32_t* rowsums) {
    Workspace* ws = as_ws(workspace, bits);
    if (!ws || rows < 1 || rows > ws->M) return RK_NPU_ERR_PARAM;
    if (hipSetDevice(device_of(ws->domain)) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
        return RK_NPU_ERR_DEVICE;
    const int K = ws->g.K, KG = ws->g.K_pad / 16;
    if (codes) {
        const size_t plane = (size_t)ws->M_alloc * 16;
        uint8_t* tmp = static_cast<uint8_t*>(std::malloc(plane * KG));
        if (!tmp) return RK_NPU_ERR_NOMEM;
        if (hipMemcpy(tmp, ws->codes, plane * KG, hipMemcpyDeviceToHost) != hipSuccess) {
            std::free(tmp);
            return RK_NPU_ERR_DEVICE;
        }
        for (int r = 0; r < rows; ++r)
            for (int k = 0; k < K; ++k)
                codes[(size_t)r * K + k] = (int8_t)tmp[(size_t)(k / 16) * plane + (size_t)r * 16 + k % 16];
        std::free(tmp);
    }
    if (scales && hipMemcpy(scales, ws->rowscale, (size_t)rows * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return RK_NPU_ERR_DEVICE;
    if (rowsums && hipMemcpy(rowsums, ws->rowsum, (size_t)rows * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return RK_NPU_ERR_DEVICE;
    return RK_NPU_OK;
}

int rk_npu_hip_profile_begin(int max_launches) {
    if (max_launches < 1 || max_launches > (1 << 20)) return RK_NPU_ERR_PARAM;
    std::lock_guard<std::mutex> lock(g_prof_mu);
    for (hipEvent_t e : g_prof_events) (void)hipEventDestroy(e);
    g_prof_events.assign(2 * (size_t)max_launches, nullptr);
    for (hipEvent_t& e : g_prof_events)
        if (hipEventCreate(&e) != hipSuccess) {
            g_prof_events.clear();
            return RK_NPU_ERR_DEVICE;
        }
    g_prof_records.clear();
    g_prof_on.store(true);
    return RK_NPU_OK;
}

int rk_npu_hip_profile_end(void) {
    g_prof_on.store(false);
    return RK_NPU_OK;
}

int rk_npu_hip_profile_read(rk_npu_hip_kernel_stat* stats, int capacity, int* count) {
    if (!count || (capacity > 0 && !stats)) return RK_NPU_ERR_PARAM;
    std::lock_guard<std::mutex> lock(g_prof_mu);
    if (hipDeviceSynchronize() != hipSuccess) return RK_NPU_ERR_DEVICE;
    std::map<std::tuple<int, int, int, int, int, int>, rk_npu_hip_kernel_stat> agg;
    for (size_t i = 0; i < g_prof_records.size(); ++i) {
        const ProfRecord& r = g_prof_records[i];
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, g_prof_events[2 * i], g_prof_events[2 * i + 1]) != hipSuccess)
            return RK_NPU_ERR_DEVICE;
        auto key = std::make_tuple(r.kind, r.bits, r.epi, r.rows, r.K, r.N);
        auto it = agg.find(key);
        if (it == agg.end()) {
            rk_npu_hip_kernel_stat st{};
            st.kind = r.kind;
            st.bits = r.bits;
            st.epilogue = r.epi;
            st.rows = r.rows;
            st.K = r.K;
            st.N = r.N;
            std::snprintf(st.name, sizeof(st.name), "%s", r.name.c_str());
            it = agg.emplace(key, st).first;
        }
        it->second.launches += 1;
        it->second.total_ms += ms;
    }
    int n = 0;
    for (auto& kv : agg) {
        if (n < capacity) stats[n] = kv.second;
        ++n;
    }
    *count = n;
    return RK_NPU_OK;
}

int rk_npu_hip_inject_alloc_failures(int count) { return g_fail_allocs.exchange(count < 0 ? 0 : count); }

int rk_npu_hip_set_switch(const char* name, int value, int* previous) {
    if (!name) return RK_NPU_ERR_PARAM;
    for (int i = 0; i < SW_COUNT; ++i) {
        if (std::strcmp(name, kSwitches[i].name) != 0) continue;
        const int was = switch_table()[i].exchange(value);
        if (previous) *previous = was;
        return RK_NPU_OK;
    }
    return RK_NPU_ERR_PARAM;
}

int rk_npu_hip_linear_plan(int rows, int K, int N, int bits, rk_npu_hip_plan* plan) {
    if (!plan || rows < 1 || K < 1 || N < 1 || (bits != 4 && bits != 8)) return RK_NPU_ERR_PARAM;
    const Plan p = plan_linear(rows, make_geometry(bits, K, N));
    plan->kind = p.kind;
    plan->block_m = p.bm;
    plan->block_n = p.bn;
    plan->k_splits = p.ksplit;
    plan->grid = p.grid;
    return RK_NPU_OK;
}

}  // extern "C"

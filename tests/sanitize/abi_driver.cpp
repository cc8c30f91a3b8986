// Host-code sanitizer run of libhip_matmul's C ABI (AddressSanitizer and
// UndefinedBehaviorSanitizer on the host side only; the GPU code is the
// product's). Built by tests/sanitize/Makefile from the library's own sources
// plus the oracle (the checker), run on a GPU by tests/test_sanitizers.py.
//
// It drives the C ABI the way the reference's Rust backend does (src/npu.rs:
// open, domains, weights, workspaces, host-buffer runs, frees) and checks
// every result bit-exact against the oracle: W4 and W8 linear at several row
// buckets, SwiGLU, the fused FFN, the device-pointer and allocation-free entry
// points, two lanes sharing weights on two threads, a workspace contended by
// two threads (RK_NPU_ERR_BUSY, never a wrong result), the MoE bank with
// repeated experts and zero routes, error returns, and the domain's live
// device bytes back at their starting value after every free.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/rk_npu_hip.h"
#include "../../include/rk_npu_moe_w8.h"
#include "../../include/rk_npu_quant_matmul.h"
#include "../../include/rk_npu_w4a8.h"
#include "../../oracle/rk_oracle.h"

static int failures = 0;
#define CHECK(cond, ...)                      \
    do {                                      \
        if (!(cond)) {                        \
            std::fprintf(stderr, __VA_ARGS__); \
            std::fputc('\n', stderr);         \
            ++failures;                       \
        }                                     \
    } while (0)

static uint64_t rng = 0xA5A5F00Dull;
static uint32_t next_u32() {
    rng = rng * 6364136223846793005ull + 1442695040888963407ull;
    return (uint32_t)(rng >> 33);
}
static float next_f() { return ((float)(next_u32() & 0xFFFFFF) / 16777216.0f) * 2.0f - 1.0f; }

struct Mat {
    int bits, k, n;
    std::vector<int8_t> codes;
    std::vector<float> scales;
};
static Mat make_mat(int bits, int k, int n) {
    Mat m{bits, k, n, std::vector<int8_t>((size_t)k * n), std::vector<float>(n)};
    for (auto& c : m.codes) c = bits == 4 ? (int8_t)((int)(next_u32() % 16) - 8) : (int8_t)((int)(next_u32() % 255) - 127);
    for (auto& s : m.scales) s = 0.001f + 0.009f * (next_f() * 0.5f + 0.5f);
    return m;
}
static std::vector<float> make_x(int rows, int k) {
    std::vector<float> x((size_t)rows * k);
    for (auto& v : x) v = next_f() * 3.0f;
    if (rows > 1)
        for (int i = 0; i < k; ++i) x[i] = 0.0f;  // a zero row
    return x;
}
static std::vector<float> oracle_linear(const Mat& m, const std::vector<float>& x, int rows) {
    std::vector<float> y((size_t)rows * m.n);
    orc_linear(m.codes.data(), m.scales.data(), m.k, m.n, x.data(), rows, y.data(), nullptr, nullptr, nullptr);
    return y;
}
static bool same(const std::vector<float>& a, const std::vector<float>& b) {
    return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(float)) == 0;
}

// A weight set of either width, created through the reference's entry points.
struct W {
    int bits;
    void* p;
};
static W create_weights(rk_npu_iommu_domain* d, const Mat& m) {
    if (m.bits == 4) {
        rk_npu_i4_weight_config c{m.k, m.n, 0};
        return {4, rk_npu_w4a8_weights_create(d, &c, m.codes.data(), m.scales.data())};
    }
    rk_npu_matmul_weight_config c{m.k, m.n, m.k};
    return {8, rk_npu_f32i8f32_weights_create(d, &c, m.codes.data(), m.scales.data())};
}
static void free_weights(W w) {
    if (w.bits == 4)
        rk_npu_w4a8_weights_free(static_cast<rk_npu_w4a8_weights*>(w.p));
    else
        rk_npu_f32i8f32_weights_free(static_cast<rk_npu_f32i8f32_weights*>(w.p));
}
static void* create_ws(rk_npu_iommu_domain* d, int bits, int rows, int k, int n) {
    if (bits == 4) {
        rk_npu_w4a8_config c;
        rk_npu_w4a8_options o;
        rk_npu_w4a8_config_init(&c, rows, n, k);
        rk_npu_w4a8_options_init(&o);
        return rk_npu_w4a8_workspace_create_ex(d, &c, &o);
    }
    rk_npu_matmul_strategy s;
    std::memset(&s, 0, sizeof(s));
    s.op_kind = RK_NPU_MATMUL_F32I8F32_DYNAMIC;
    s.M = rows, s.N = n, s.K = k, s.k_tile = k;
    return rk_npu_matmul_workspace_create(d, &s);
}
static void free_ws(int bits, void* ws) {
    if (bits == 4)
        rk_npu_w4a8_workspace_free(static_cast<rk_npu_w4a8_workspace*>(ws));
    else
        rk_npu_matmul_workspace_free(static_cast<rk_npu_matmul_workspace*>(ws));
}
static int run_host(int bits, void* ws, W w, const float* a, float* c) {
    if (bits == 4)
        return rk_npu_w4a8_run_f32(static_cast<rk_npu_w4a8_workspace*>(ws), static_cast<rk_npu_w4a8_weights*>(w.p),
                                   a, c, nullptr);
    return rk_npu_f32i8f32_run_dynamic(static_cast<rk_npu_matmul_workspace*>(ws),
                                       static_cast<rk_npu_f32i8f32_weights*>(w.p), a, c);
}
static uint64_t live_bytes(rk_npu_iommu_domain* d) {
    rk_npu_domain_memory_stats st;
    return rk_npu_iommu_domain_memory_stats(d, &st) == RK_NPU_OK ? st.live_bytes : ~0ull;
}

static void linear_host(rk_npu_iommu_domain* d) {
    for (int bits : {4, 8})
        for (auto kn : {std::pair<int, int>{640, 768}, {2560, 6144}}) {
            const Mat m = make_mat(bits, kn.first, kn.second);
            W w = create_weights(d, m);
            CHECK(w.p, "weights create W%d %dx%d", bits, m.k, m.n);
            if (!w.p) continue;
            for (int rows : {1, 4, 64, 256}) {
                void* ws = create_ws(d, bits, rows, m.k, m.n);
                CHECK(ws, "workspace W%d rows %d", bits, rows);
                if (!ws) continue;
                const auto x = make_x(rows, m.k);
                std::vector<float> y((size_t)rows * m.n, -1.0f);
                CHECK(run_host(bits, ws, w, x.data(), y.data()) == RK_NPU_OK, "run W%d rows %d", bits, rows);
                CHECK(same(y, oracle_linear(m, x, rows)), "W%d %dx%d rows %d differs from the oracle", bits, m.k, m.n,
                      rows);
                free_ws(bits, ws);
            }
            free_weights(w);
        }
}

static void swiglu_and_ffn(rk_npu_iommu_domain* d) {
    const int h = 640, f = 1024, rows = 4;
    const Mat gu = make_mat(4, h, 2 * f), dn = make_mat(8, f, h);
    W wg = create_weights(d, gu), wd = create_weights(d, dn);
    void* gws = create_ws(d, 4, rows, h, 2 * f);
    void* dws = create_ws(d, 8, rows, f, h);
    CHECK(wg.p && wd.p && gws && dws, "ffn objects");
    if (!(wg.p && wd.p && gws && dws)) return;
    const auto x = make_x(rows, h);
    std::vector<float> mid((size_t)rows * f), ref_mid((size_t)rows * f);
    CHECK(rk_npu_w4a8_run_swiglu_f32(static_cast<rk_npu_w4a8_workspace*>(gws), static_cast<rk_npu_w4a8_weights*>(wg.p),
                                     x.data(), mid.data(), nullptr) == RK_NPU_OK,
          "swiglu run");
    orc_linear_swiglu(gu.codes.data(), gu.scales.data(), h, 2 * f, x.data(), rows, ref_mid.data());
    CHECK(same(mid, ref_mid), "swiglu differs from the oracle");
    std::vector<float> y((size_t)rows * h), ref((size_t)rows * h);
    CHECK(rk_npu_w4a8_run_ffn_f32(static_cast<rk_npu_w4a8_workspace*>(gws), static_cast<rk_npu_w4a8_weights*>(wg.p),
                                  dws, wd.p, 8, x.data(), y.data(), nullptr) == RK_NPU_OK,
          "ffn run");
    orc_ffn(gu.codes.data(), gu.scales.data(), dn.codes.data(), dn.scales.data(), h, f, x.data(), rows, ref.data(),
            nullptr);
    CHECK(same(y, ref), "ffn differs from the oracle");
    free_ws(4, gws);
    free_ws(8, dws);
    free_weights(wg);
    free_weights(wd);
}

static void device_entries(rk_npu_iommu_domain* d) {
    const Mat m = make_mat(4, 2560, 1536);
    W w = create_weights(d, m);
    const int rows = 8;
    void* ws = create_ws(d, 4, rows, m.k, m.n);
    CHECK(w.p && ws, "device-entry objects");
    if (!(w.p && ws)) return;
    float *da = nullptr, *dc = nullptr;
    CHECK(hipMalloc(&da, sizeof(float) * rows * m.k) == hipSuccess && hipMalloc(&dc, sizeof(float) * rows * m.n) == hipSuccess,
          "hipMalloc");
    for (int r : {rows, 3}) {  // the static entry twice, the second call smaller
        const auto x = make_x(r, m.k);
        const auto ref = oracle_linear(m, x, r);
        CHECK(hipMemcpy(da, x.data(), sizeof(float) * r * m.k, hipMemcpyHostToDevice) == hipSuccess, "upload");
        std::vector<float> y((size_t)r * m.n);
        CHECK(rk_npu_hip_linear_run(ws, w.p, 4, da, RK_NPU_HIP_F32, dc, RK_NPU_HIP_F32, r, RK_NPU_HIP_PLAIN, nullptr) ==
                  RK_NPU_OK,
              "device run");
        CHECK(hipMemcpy(y.data(), dc, sizeof(float) * r * m.n, hipMemcpyDeviceToHost) == hipSuccess, "download");
        CHECK(same(y, ref), "device entry rows %d differs from the oracle", r);
        CHECK(rk_npu_hip_linear_run_static(w.p, 4, da, RK_NPU_HIP_F32, dc, RK_NPU_HIP_F32, r, RK_NPU_HIP_PLAIN,
                                           nullptr) == RK_NPU_OK,
              "static run");
        CHECK(hipMemcpy(y.data(), dc, sizeof(float) * r * m.n, hipMemcpyDeviceToHost) == hipSuccess, "download");
        CHECK(same(y, ref), "static entry rows %d differs from the oracle", r);
    }
    CHECK(rk_npu_hip_linear_run_static(w.p, 4, da, RK_NPU_HIP_F32, dc, RK_NPU_HIP_F32, RK_NPU_HIP_STATIC_MAX_ROWS + 1,
                                       RK_NPU_HIP_PLAIN, nullptr) == RK_NPU_ERR_PARAM,
          "static entry accepted too many rows");
    (void)hipFree(da);
    (void)hipFree(dc);
    free_ws(4, ws);
    free_weights(w);
}

static void lanes_and_busy(rk_npu_iommu_domain* d) {
    const Mat m = make_mat(8, 2560, 2048);
    W w = create_weights(d, m);
    const int rows = 4;
    void* ws[2] = {create_ws(d, 8, rows, m.k, m.n), create_ws(d, 8, rows, m.k, m.n)};
    CHECK(w.p && ws[0] && ws[1], "lane objects");
    if (!(w.p && ws[0] && ws[1])) return;
    const auto x = make_x(rows, m.k);
    const auto ref = oracle_linear(m, x, rows);
    std::atomic<int> wrong{0}, busy{0}, ok{0};
    auto lane = [&](void* own) {
        std::vector<float> y((size_t)rows * m.n);
        for (int i = 0; i < 20; ++i) {
            const int rc = run_host(8, own, w, x.data(), y.data());
            if (rc == RK_NPU_ERR_BUSY) {
                ++busy;
                continue;
            }
            if (rc != RK_NPU_OK || !same(y, ref)) ++wrong;
            else ++ok;
        }
    };
    {  // two lanes, own workspaces, shared weights
        std::thread a(lane, ws[0]), b(lane, ws[1]);
        a.join(), b.join();
        CHECK(wrong == 0 && busy == 0 && ok == 40, "lanes: %d wrong, %d busy", wrong.load(), busy.load());
    }
    wrong = busy = ok = 0;
    {  // two threads on one workspace: each call either runs correctly or is refused
        std::thread a(lane, ws[0]), b(lane, ws[0]);
        a.join(), b.join();
        CHECK(wrong == 0 && ok + busy == 40, "shared workspace: %d wrong", wrong.load());
    }
    free_ws(8, ws[0]);
    free_ws(8, ws[1]);
    free_weights(w);
}

static void moe(rk_npu_iommu_domain* d) {
    const int h = 256, inter = 96, experts = 6, top = 2, rows = 5;
    std::vector<Mat> gu, dn;
    std::vector<rk_npu_moe_w8_expert> ex(experts);
    for (int e = 0; e < experts; ++e) {
        gu.push_back(make_mat(4, h, 2 * inter));
        dn.push_back(make_mat(8, inter, h));
    }
    for (int e = 0; e < experts; ++e)
        ex[e] = {gu[e].codes.data(), gu[e].scales.data(), dn[e].codes.data(), dn[e].scales.data()};
    rk_npu_moe_w8_config cfg;
    rk_npu_moe_w8_config_init(&cfg, h, inter, experts, 0, top, 8);
    rk_npu_moe_w8_weights* bank = rk_npu_moe_w4w8_weights_create(d, &cfg.weights, ex.data());
    rk_npu_moe_w8_workspace* ws = rk_npu_moe_w4w8_workspace_create(d, &cfg);
    CHECK(bank && ws, "moe objects");
    if (!(bank && ws)) return;
    const auto x = make_x(rows, h);
    // repeated expert in a row, a zero route, a negative route, all routes of a row skipped
    const int32_t ids[rows * top] = {0, 5, 3, 3, 1, 2, 4, 0, 2, 1};
    const float routes[rows * top] = {0.6f, 0.4f, 0.5f, 0.5f, 1.0f, 0.0f, -0.5f, 0.25f, 0.0f, -1.0f};
    std::vector<float> y((size_t)rows * h), ref((size_t)rows * h);
    CHECK(rk_npu_moe_w8_run_f32(ws, bank, rows, x.data(), ids, routes, y.data(), nullptr) == RK_NPU_OK, "moe run");
    std::vector<const int8_t*> gc(experts), dc(experts);
    std::vector<const float*> gs(experts), ds(experts);
    for (int e = 0; e < experts; ++e)
        gc[e] = gu[e].codes.data(), gs[e] = gu[e].scales.data(), dc[e] = dn[e].codes.data(), ds[e] = dn[e].scales.data();
    orc_moe(gc.data(), gs.data(), dc.data(), ds.data(), experts, h, inter, nullptr, nullptr, nullptr, nullptr, 0, x.data(),
            rows, ids, routes, top, ref.data());
    CHECK(same(y, ref), "moe differs from the oracle");
    const int32_t bad[rows * top] = {0, 1, 2, 3, 4, 5, 6, 0, 1, 2};  // expert 6 does not exist
    CHECK(rk_npu_moe_w8_run_f32(ws, bank, rows, x.data(), bad, routes, y.data(), nullptr) == RK_NPU_ERR_PARAM,
          "moe accepted an out-of-range expert id");
    rk_npu_moe_w8_workspace_free(ws);
    rk_npu_moe_w8_weights_free(bank);
}

int main() {
    rk_npu_ctx* ctx = rk_npu_open(nullptr);
    CHECK(ctx, "rk_npu_open");
    if (!ctx) {
        std::fflush(stderr);
        std::_Exit(1);
    }
    rk_npu_iommu_domain* d = rk_npu_iommu_domain_create(ctx, 0);
    CHECK(d, "domain create");
    if (!d) return 1;
    const uint64_t base = live_bytes(d);
    CHECK(rk_npu_w4a8_run_f32(nullptr, nullptr, nullptr, nullptr, nullptr) == RK_NPU_ERR_PARAM, "NULL run accepted");
    CHECK(rk_npu_f32i8f32_run_dynamic(nullptr, nullptr, nullptr, nullptr) == RK_NPU_ERR_PARAM, "NULL run accepted");
    const std::pair<const char*, void (*)(rk_npu_iommu_domain*)> sections[] = {
        {"linear host calls", linear_host}, {"swiglu and ffn", swiglu_and_ffn}, {"device entries", device_entries},
        {"lanes and busy", lanes_and_busy}, {"moe", moe}};
    for (const auto& sec : sections) {
        const int before = failures;
        sec.second(d);
        std::printf("%s: %d failed checks\n", sec.first, failures - before);
        std::fflush(stdout);
    }
    CHECK(live_bytes(d) == base, "domain live bytes %llu after every free, %llu at the start",
          (unsigned long long)live_bytes(d), (unsigned long long)base);
    rk_npu_iommu_domain_free(d);
    rk_npu_close(ctx);
    std::printf("abi sanitizer run: %d failed checks\n", failures);
    std::fflush(stdout);
    std::fflush(stderr);
    // Leave without the process's static destructors: the HIP runtime's own
    // teardown at exit trips a check inside the sanitizer runtime's hooks on
    // device allocations, after everything above has been freed and checked.
    std::_Exit(failures == 0 ? 0 : 1);
}

// hip_matmul MoE: expert banks, workspaces, the grouped routed FFN and the
// expert-record (blob) import/export/swap entry points of rk_npu_moe_w8.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

#include "moe_kernels.hpp"
#include "runtime.hpp"

namespace hm {

constexpr uint32_t MAGIC_MOE_W = 0x574d4841u;
constexpr uint32_t MAGIC_MOE_WS = 0x534d4841u;
constexpr uint32_t BLOB_MAGIC = 0x31584d48u;  // "HMX1"
constexpr int MOE_BM = 64, MOE_BN = 128;

// One routed expert in device memory: [gate_up payload | gate_up scales |
// down payload | down scales], each region 256-byte aligned.
struct ExpertLayout {
    size_t gu, gus, dn, dns, total;
};

static ExpertLayout expert_layout(const Geometry& ggu, const Geometry& gdn) {
    ExpertLayout L;
    L.gu = round_up_z(weight_bytes(ggu) - (size_t)ggu.N_pad * 4, 256);
    L.gus = round_up_z((size_t)ggu.N_pad * 4, 256);
    L.dn = round_up_z(weight_bytes(gdn) - (size_t)gdn.N_pad * 4, 256);
    L.dns = round_up_z((size_t)gdn.N_pad * 4, 256);
    L.total = L.gu + L.gus + L.dn + L.dns;
    return L;
}

struct MoeBank {
    uint32_t magic;
    int h, inter, experts, shared;
    int gu_bits, dn_bits;
    Geometry ggu, gdn;
    ExpertLayout L;
    Domain* domain;
    std::vector<uint8_t*> expert;  // owning, one allocation per routed expert
    const uint8_t** d_gu;          // device tables
    const float** d_gus;
    const uint8_t** d_dn;
    const float** d_dns;
    Weights* shared_gu;
    Weights* shared_dn;
    size_t bytes;
};

struct MoeWork {
    uint32_t magic;
    int h, inter, experts, shared, top, max_rows;
    Domain* domain;
    hipStream_t stream;
    std::atomic<bool> busy;
    Workspace* xws;   // token rows: input staging, quantized input, shared middle
    Workspace* mws;   // slots: middle f32, requantized middle, contributions
    Workspace* sgws;  // shared expert gate_up (nullable)
    Workspace* sdws;  // shared expert down (nullable)
    int* ids;
    float* routes;
    int* pos;
    int* perm;
    int4* tiles;
    int* counts;
    unsigned* error;
    float* out;
    int8_t* gcodes;   // token codes quantized in slot order [h_pad/16][g_alloc][16]
    float* gscale;    // [g_alloc]
    int* gsum;        // [g_alloc]
    int g_alloc;
    float* gpart;     // per-block row maxima of the slot GEMV's middle [slots][gu groups]
    int gu_groups;
    unsigned* host_error;  // pinned
    size_t bytes;
};

}  // namespace hm

struct rk_npu_moe_w8_weights : hm::MoeBank {};
struct rk_npu_moe_w8_workspace : hm::MoeWork {};

namespace hm {

static bool upload_tables(MoeBank* b) {
    std::vector<const uint8_t*> gu(b->experts), dn(b->experts);
    std::vector<const float*> gus(b->experts), dns(b->experts);
    for (int e = 0; e < b->experts; ++e) {
        uint8_t* base = b->expert[e];
        gu[e] = base;
        gus[e] = reinterpret_cast<const float*>(base + b->L.gu);
        dn[e] = base + b->L.gu + b->L.gus;
        dns[e] = reinterpret_cast<const float*>(base + b->L.gu + b->L.gus + b->L.dn);
    }
    const size_t n = sizeof(void*) * b->experts;
    return hipMemcpy(b->d_gu, gu.data(), n, hipMemcpyHostToDevice) == hipSuccess &&
           hipMemcpy(b->d_gus, gus.data(), n, hipMemcpyHostToDevice) == hipSuccess &&
           hipMemcpy(b->d_dn, dn.data(), n, hipMemcpyHostToDevice) == hipSuccess &&
           hipMemcpy(b->d_dns, dns.data(), n, hipMemcpyHostToDevice) == hipSuccess;
}

static void bank_destroy(MoeBank* b) {
    if (!b) return;
    (void)hipSetDevice(device_of(b->domain));
    for (uint8_t* p : b->expert) domain_free(b->domain, p, b->L.total);
    domain_free(b->domain, (void*)b->d_gu, sizeof(void*) * b->experts * 4);
    weights_destroy(b->shared_gu);
    weights_destroy(b->shared_dn);
    delete static_cast<rk_npu_moe_w8_weights*>(b);
}

// Packs one expert matrix (host codes) into a region of an expert allocation
// through a temporary Weights object of the same geometry.
static bool pack_into(Domain* d, int bits, int K, int N, const int8_t* codes, const float* scales, uint8_t* dst,
                      float* dst_scales) {
    Weights* w = weights_create(d, bits, K, N, codes, scales, false);
    if (!w) return false;
    const size_t payload = w->bytes - (size_t)w->g.N_pad * 4;
    bool ok = hipMemcpy(dst, w->packed, payload, hipMemcpyDeviceToDevice) == hipSuccess &&
              hipMemcpy(dst_scales, w->colscale, (size_t)w->g.N_pad * 4, hipMemcpyDeviceToDevice) == hipSuccess;
    weights_destroy(w);
    return ok;
}

static MoeBank* bank_create(Domain* d, const rk_npu_moe_w8_weight_config* cfg, const rk_npu_moe_w8_expert* experts,
                            int gu_bits, int dn_bits, bool with_routed, bool want_shared,
                            const rk_npu_moe_w8_expert* shared_expert) {
    if (!d || !cfg) return nullptr;
    const int h = cfg->hidden, inter = cfg->intermediate, E = cfg->routed_experts;
    if (h <= 0 || inter <= 0 || inter % 32 != 0 || E <= 0 || E > MOE_MAX_EXPERTS) return nullptr;
    if ((cfg->shared_expert != 0) != want_shared) return nullptr;
    if (with_routed && !experts) return nullptr;
    if (want_shared && !shared_expert) return nullptr;
    if (hipSetDevice(device_of(d)) != hipSuccess) return nullptr;
    MoeBank* b = new (std::nothrow) rk_npu_moe_w8_weights();
    if (!b) return nullptr;
    b->magic = MAGIC_MOE_W;
    b->h = h;
    b->inter = inter;
    b->experts = E;
    b->shared = want_shared ? 1 : 0;
    b->gu_bits = gu_bits;
    b->dn_bits = dn_bits;
    b->ggu = make_geometry(gu_bits, h, 2 * inter);
    b->gdn = make_geometry(dn_bits, inter, h);
    b->L = expert_layout(b->ggu, b->gdn);
    b->domain = d;
    b->d_gu = nullptr;
    b->shared_gu = b->shared_dn = nullptr;
    b->bytes = 0;
    bool ok = true;
    void* tables = domain_alloc(d, sizeof(void*) * E * 4);
    if (!tables) ok = false;
    if (ok) {
        b->d_gu = static_cast<const uint8_t**>(tables);
        b->d_gus = reinterpret_cast<const float**>(b->d_gu + E);
        b->d_dn = reinterpret_cast<const uint8_t**>(b->d_gu + 2 * E);
        b->d_dns = reinterpret_cast<const float**>(b->d_gu + 3 * E);
    }
    for (int e = 0; ok && e < E; ++e) {
        uint8_t* p = static_cast<uint8_t*>(domain_alloc(d, b->L.total));
        if (!p) {
            ok = false;
            break;
        }
        b->expert.push_back(p);
        if (hipMemset(p, 0, b->L.total) != hipSuccess) ok = false;
        if (ok && with_routed) {
            const rk_npu_moe_w8_expert& x = experts[e];
            ok = pack_into(d, gu_bits, h, 2 * inter, x.gate_up, x.gate_up_scales, p,
                           reinterpret_cast<float*>(p + b->L.gu)) &&
                 pack_into(d, dn_bits, inter, h, x.down, x.down_scales, p + b->L.gu + b->L.gus,
                           reinterpret_cast<float*>(p + b->L.gu + b->L.gus + b->L.dn));
        }
    }
    if (ok && want_shared) {
        const rk_npu_moe_w8_expert& s = *shared_expert;
        b->shared_gu = weights_create(d, 8, h, 2 * inter, s.gate_up, s.gate_up_scales, false);
        b->shared_dn = weights_create(d, 8, inter, h, s.down, s.down_scales, false);
        ok = b->shared_gu && b->shared_dn;
    }
    ok = ok && upload_tables(b);
    if (!ok) {
        bank_destroy(b);
        return nullptr;
    }
    b->bytes = b->L.total * E + (b->shared_gu ? b->shared_gu->bytes + b->shared_dn->bytes : 0);
    return b;
}

static MoeWork* work_create(Domain* d, const rk_npu_moe_w8_config* cfg) {
    if (!d || !cfg) return nullptr;
    const rk_npu_moe_w8_weight_config& w = cfg->weights;
    if (w.hidden <= 0 || w.intermediate <= 0 || w.intermediate % 32 != 0 || w.routed_experts <= 0 ||
        w.routed_experts > MOE_MAX_EXPERTS || cfg->top < 1 || cfg->top > 8 || cfg->top > w.routed_experts ||
        cfg->max_rows < 1 || cfg->max_rows > 8192)
        return nullptr;
    if (hipSetDevice(device_of(d)) != hipSuccess) return nullptr;
    MoeWork* ws = new (std::nothrow) rk_npu_moe_w8_workspace();
    if (!ws) return nullptr;
    ws->magic = MAGIC_MOE_WS;
    ws->h = w.hidden;
    ws->inter = w.intermediate;
    ws->experts = w.routed_experts;
    ws->shared = w.shared_expert ? 1 : 0;
    ws->top = cfg->top;
    ws->max_rows = cfg->max_rows;
    ws->domain = d;
    ws->busy.store(false);
    ws->stream = nullptr;
    ws->xws = ws->mws = ws->sgws = ws->sdws = nullptr;
    ws->ids = nullptr;
    ws->host_error = nullptr;
    const int A = cfg->max_rows * cfg->top;
    ws->xws = workspace_create(d, 8, cfg->max_rows, w.hidden, 2 * w.intermediate);
    ws->mws = workspace_create(d, 8, A, w.intermediate, w.hidden);
    if (ws->shared) {
        ws->sgws = workspace_create(d, 8, cfg->max_rows, w.hidden, 2 * w.intermediate);
        ws->sdws = workspace_create(d, 8, cfg->max_rows, w.intermediate, w.hidden);
    }
    // ids | routes | pos | perm | tiles | counts | error | out | slot-order codes | scales | sums
    const size_t sz_a = round_up_z((size_t)A * 4, 256);
    const size_t sz_tiles = round_up_z((size_t)A * 16, 256);
    const size_t sz_out = round_up_z((size_t)cfg->max_rows * w.hidden * 4, 256);
    ws->g_alloc = round_up(A, 256);
    const size_t sz_g = (size_t)round_up(w.hidden, 64) * ws->g_alloc, sz_gs = (size_t)ws->g_alloc * 4;
    ws->gu_groups = round_up(2 * w.intermediate, 256) / 16;
    const size_t sz_gp = round_up_z((size_t)A * ws->gu_groups * 4, 256);
    const size_t total = 4 * sz_a + sz_tiles + 256 + 256 + sz_out + sz_g + 2 * sz_gs + sz_gp;
    uint8_t* base = static_cast<uint8_t*>(domain_alloc(d, total));
    bool ok = ws->xws && ws->mws && (!ws->shared || (ws->sgws && ws->sdws)) && base;
    if (base) {
        size_t off = 0;
        ws->ids = reinterpret_cast<int*>(base + off);
        off += sz_a;
        ws->routes = reinterpret_cast<float*>(base + off);
        off += sz_a;
        ws->pos = reinterpret_cast<int*>(base + off);
        off += sz_a;
        ws->perm = reinterpret_cast<int*>(base + off);
        off += sz_a;
        ws->tiles = reinterpret_cast<int4*>(base + off);
        off += sz_tiles;
        ws->counts = reinterpret_cast<int*>(base + off);
        off += 256;
        ws->error = reinterpret_cast<unsigned*>(base + off);
        off += 256;
        ws->out = reinterpret_cast<float*>(base + off);
        off += sz_out;
        ws->gcodes = reinterpret_cast<int8_t*>(base + off);
        off += sz_g;
        ws->gscale = reinterpret_cast<float*>(base + off);
        off += sz_gs;
        ws->gsum = reinterpret_cast<int*>(base + off);
        off += sz_gs;
        ws->gpart = reinterpret_cast<float*>(base + off);
        ok = ok && hipMemset(base, 0, total) == hipSuccess;
    }
    ws->bytes = total + (ws->xws ? ws->xws->bytes : 0) + (ws->mws ? ws->mws->bytes : 0) +
                (ws->sgws ? ws->sgws->bytes : 0) + (ws->sdws ? ws->sdws->bytes : 0);
    ok = ok && hipHostMalloc(reinterpret_cast<void**>(&ws->host_error), 4, hipHostMallocDefault) == hipSuccess;
    ok = ok && hipStreamCreateWithFlags(&ws->stream, hipStreamNonBlocking) == hipSuccess;
    ok = ok && hipDeviceSynchronize() == hipSuccess;
    if (!ok) {
        if (base) domain_free(d, base, total);
        ws->ids = nullptr;
        workspace_destroy(ws->xws);
        workspace_destroy(ws->mws);
        workspace_destroy(ws->sgws);
        workspace_destroy(ws->sdws);
        if (ws->host_error) (void)hipHostFree(ws->host_error);
        if (ws->stream) (void)hipStreamDestroy(ws->stream);
        delete static_cast<rk_npu_moe_w8_workspace*>(ws);
        return nullptr;
    }
    return ws;
}

static size_t work_table_bytes(const MoeWork* ws) {
    const int A = ws->max_rows * ws->top;
    return 4 * round_up_z((size_t)A * 4, 256) + round_up_z((size_t)A * 16, 256) + 512 +
           round_up_z((size_t)ws->max_rows * ws->h * 4, 256) + (size_t)round_up(ws->h, 64) * ws->g_alloc +
           2 * (size_t)ws->g_alloc * 4 + round_up_z((size_t)A * ws->gu_groups * 4, 256);
}

static void work_destroy(MoeWork* ws) {
    if (!ws) return;
    (void)hipSetDevice(device_of(ws->domain));
    if (ws->stream) {
        (void)hipStreamSynchronize(ws->stream);
        (void)hipStreamDestroy(ws->stream);
    }
    if (ws->ids) domain_free(ws->domain, ws->ids, work_table_bytes(ws));
    workspace_destroy(ws->xws);
    workspace_destroy(ws->mws);
    workspace_destroy(ws->sgws);
    workspace_destroy(ws->sdws);
    if (ws->host_error) (void)hipHostFree(ws->host_error);
    delete static_cast<rk_npu_moe_w8_workspace*>(ws);
}

template <int BITS, int EPI>
static void launch_moe_gemm(const MoeGemmParams& G, int grid, hipStream_t s, int rows) {
    const int slot = prof_begin(s, 3, BITS, EPI, rows, G.K_pad, G.N, EPI == EPI_PLAIN ? "moe_gemm<down>" : "moe_gemm<gate_up>");
    const size_t esz = G.c_type == DT_F32 ? 4 : 2;
    if ((reinterpret_cast<uintptr_t>(G.c) & 15) == 0 && ((size_t)G.ldc * esz) % 16 == 0)
        hipLaunchKernelGGL((moe_gemm_kernel<MOE_BM, MOE_BN, 2, 2, BITS, EPI, true>), dim3(grid), dim3(256), 0, s, G);
    else
        hipLaunchKernelGGL((moe_gemm_kernel<MOE_BM, MOE_BN, 2, 2, BITS, EPI, false>), dim3(grid), dim3(256), 0, s, G);
    prof_end(slot, s);
}

// One GEMV block row per routed slot (decode-sized batches): the slot's
// expert weights streamed like a dense M=1 GEMV. Register windows as in the
// dense launch.
template <typename T, int BITS, int EPI, bool PREQ>
static void launch_slot_gemv(const GemvParams& V, int slots, hipStream_t s) {
    const int planes = BITS == 8 ? V.K_pad / 16 : V.K_pad / 32;
    const int rounds = (planes * 8 * (EPI == EPI_PLAIN ? 1 : 2) + 255) / 256;
    const dim3 grid(EPI == EPI_PLAIN ? V.N_pad / 8 : V.N_pad / 16, slots);
    const size_t lds = V.K_pad;
    if (rounds <= 2)
        hipLaunchKernelGGL((gemv_kernel<T, 1, BITS, EPI, 2, 1, PREQ, 1, 256, true>), grid, dim3(256), lds, s, V);
    else if (rounds <= 3)
        hipLaunchKernelGGL((gemv_kernel<T, 1, BITS, EPI, 3, 1, PREQ, 1, 256, true>), grid, dim3(256), lds, s, V);
    else if (rounds <= 4)
        hipLaunchKernelGGL((gemv_kernel<T, 1, BITS, EPI, 4, 1, PREQ, 1, 256, true>), grid, dim3(256), lds, s, V);
    else if (rounds <= 6)
        hipLaunchKernelGGL((gemv_kernel<T, 1, BITS, EPI, 6, 1, PREQ, 1, 256, true>), grid, dim3(256), lds, s, V);
    else if (rounds <= 8)
        hipLaunchKernelGGL((gemv_kernel<T, 1, BITS, EPI, 8, 1, PREQ, 1, 256, true>), grid, dim3(256), lds, s, V);
    else
        hipLaunchKernelGGL((gemv_kernel<T, 1, BITS, EPI, 8, 2, PREQ, 1, 256, true>), grid, dim3(256), lds, s, V);
}

// Enqueues the whole routed FFN (plus shared expert) for `rows` token rows
// whose input, ids and routes already sit in device memory.
static int enqueue_moe(MoeWork* ws, const MoeBank* b, int rows, const float* input, const int* ids,
                       const float* routes, float* out, hipStream_t s) {
    const int A = rows * ws->top;
    // Decode-sized batches (at most 64 slots): one GEMV block row per
    // assignment (slot = assignment, no routing launch: the blocks of a
    // skipped route return at once, those of an out-of-range expert id flag
    // the error word); gate/up on the tokens' quantized rows -> SwiGLU middle
    // [slot][inter] and per-block row maxima -> down quantizes each middle
    // row itself from them. (T=1: 43 -> 26 us with the slot GEMVs.)
    const bool slot_gemv = A <= 64 && (ws->inter % 16) == 0 && b->ggu.half != 0 &&
                           (ws->mws->g.K_pad / 16) <= 256 * GEMV_XMAX;
    // On the slot path the gate/up blocks quantize their token's row
    // themselves when it is 16-byte aligned and fits their registers (no
    // quantization launch); otherwise the rows are quantized first.
    const bool slot_quant = slot_gemv && (ws->h % 16) == 0 && (reinterpret_cast<uintptr_t>(input) & 15) == 0 &&
                            (b->ggu.K_pad / 16) <= 256 * GEMV_XMAX;
    // Many slots: after routing, the tokens' rows are quantized straight into
    // slot order (slot s holds token perm[s] / top), so the grouped GEMM's A
    // loads are contiguous rows; one launch for what was a token quantization
    // and a gather of its codes (measured at 4096 slots: gate/up 69 -> 57 us
    // with contiguous rows). Few slots: the tokens are quantized once and the
    // GEMM gathers rows itself.
    const bool slot_order = !slot_gemv && A >= 256;
    int rc = RK_NPU_OK;
    if (!slot_quant && !slot_order) {
        rc = enqueue_quant(ws->xws, input, DT_F32, ws->h, rows, QUANT_MOE, RowMax{nullptr, 0}, nullptr, s);
        if (rc != RK_NPU_OK) return rc;
    }
    if (!slot_gemv) {
    RouteParams R;
    R.ids = ids;
    R.routes = routes;
    R.rows = rows;
    R.top = ws->top;
    R.experts = ws->experts;
    R.pos = ws->pos;
    R.perm = ws->perm;
    R.tiles = ws->tiles;
    R.counts = ws->counts;
    R.rowmax_mid = ws->mws->rowmax;
    R.rowmax_count = A;
    R.error = ws->error;
    hipLaunchKernelGGL(moe_route_kernel<MOE_BM>, dim3(1), dim3(1024), 0, s, R);
    }

    if (slot_gemv) {
        GemvParams V{};
        V.rule = QUANT_MOE;
        V.vec = 1;
        V.M = 1;
        V.b_tab = b->d_gu;
        V.s_tab = b->d_gus;
        V.perm = nullptr;
        V.ids = ids;
        V.routes = routes;
        V.experts = ws->experts;
        V.error = ws->error;
        V.top = ws->top;
        if (slot_quant) {
            V.x = input;  // the token's f32 row, quantized in every block
            V.lda = ws->h;
            V.x_by_token = 1;
        } else {
            V.x = ws->xws->codes;  // unused (rows quantized beforehand)
            V.diag_codes = ws->xws->codes;
            V.diag_scale = ws->xws->rowscale;
            V.diag_rowsum = ws->xws->rowsum;
        }
        V.M_alloc = ws->xws->M_alloc;
        V.c = ws->mws->a_f32;  // middle [slot][inter]
        V.ldc = ws->inter;
        V.c_type = DT_F32;
        V.part_out = ws->gpart;
        V.K = b->ggu.K;
        V.N = b->ggu.N;
        V.K_pad = b->ggu.K_pad;
        V.N_pad = b->ggu.N_pad;
        V.half = b->ggu.half;
        if (slot_quant)
            launch_slot_gemv<float, 4, EPI_SWIGLU_MAX, false>(V, A, s);
        else
            launch_slot_gemv<float, 4, EPI_SWIGLU_MAX, true>(V, A, s);

        GemvParams D{};
        D.rule = QUANT_MOE;
        D.vec = 1;
        D.M = 1;
        D.b_tab = b->d_dn;
        D.s_tab = b->d_dns;
        D.perm = nullptr;
        D.ids = ids;
        D.routes = routes;
        D.experts = ws->experts;
        D.error = ws->error;
        D.top = ws->top;
        D.x = ws->mws->a_f32;
        D.lda = ws->inter;
        D.part_in = ws->gpart;
        D.part_count = b->ggu.N_pad / 16;
        D.c = ws->mws->c_f32;  // contributions [slot][h]
        D.ldc = ws->h;
        D.c_type = DT_F32;
        D.K = b->gdn.K;
        D.N = b->gdn.N;
        D.K_pad = b->gdn.K_pad;
        D.N_pad = b->gdn.N_pad;
        D.half = b->gdn.half;
        D.M_alloc = ws->mws->M_alloc;
        if (b->dn_bits == 8)
            launch_slot_gemv<float, 8, EPI_PLAIN, false>(D, A, s);
        else
            launch_slot_gemv<float, 4, EPI_PLAIN, false>(D, A, s);
        if (hipGetLastError() != hipSuccess) return RK_NPU_ERR_DEVICE;
    }

    // Upper bound of the m-tile count: every tile holds >= 1 slot, and at most
    // one partial tile per expert.
    const int max_tiles = std::min(A, (A + std::min(A, ws->experts) * (MOE_BM - 1)) / MOE_BM);

    if (slot_order) {
        const QuantOut q{ws->gcodes, ws->gscale, ws->gsum, ws->g_alloc};
        rc = enqueue_quant(ws->xws, input, DT_F32, ws->h, A, QUANT_MOE, RowMax{nullptr, 0}, nullptr, s, ws->counts,
                           ws->perm, ws->top, &q);
        if (rc != RK_NPU_OK) return rc;
    }

    if (!slot_gemv) {
    MoeGemmParams G;
    G.a = slot_order ? ws->gcodes : ws->xws->codes;
    G.a_alloc = slot_order ? ws->g_alloc : ws->xws->M_alloc;
    G.perm = slot_order ? nullptr : ws->perm;
    G.top = ws->top;
    G.rowscale = slot_order ? ws->gscale : ws->xws->rowscale;
    G.rowsum = slot_order ? ws->gsum : ws->xws->rowsum;
    G.b_tab = b->d_gu;
    G.s_tab = b->d_gus;
    G.tiles = ws->tiles;
    G.counts = ws->counts;
    G.c = ws->mws->a_f32;  // middle [slot][inter]
    G.ldc = ws->inter;
    G.c_type = DT_F32;
    G.rowmax = ws->mws->rowmax;
    G.N = b->ggu.N;
    G.K_pad = b->ggu.K_pad;
    G.N_pad = b->ggu.N_pad;
    G.half = b->ggu.half;
    G.tiles_n = b->ggu.N_pad / MOE_BN;
    launch_moe_gemm<4, EPI_SWIGLU_MAX>(G, round_up(max_tiles, 8) * G.tiles_n, s, A);

    rc = enqueue_quant(ws->mws, ws->mws->a_f32, DT_F32, ws->inter, A, QUANT_MOE,
                       RowMax{reinterpret_cast<const float*>(ws->mws->rowmax), 1}, nullptr, s, ws->counts);
    if (rc != RK_NPU_OK) return rc;

    G.a = ws->mws->codes;
    G.a_alloc = ws->mws->M_alloc;
    G.perm = nullptr;
    G.rowscale = ws->mws->rowscale;
    G.rowsum = ws->mws->rowsum;
    G.b_tab = b->d_dn;
    G.s_tab = b->d_dns;
    G.c = ws->mws->c_f32;  // contributions [slot][h]
    G.ldc = ws->h;
    G.rowmax = nullptr;
    G.N = b->gdn.N;
    G.K_pad = b->gdn.K_pad;
    G.N_pad = b->gdn.N_pad;
    G.half = b->gdn.half;
    G.tiles_n = b->gdn.N_pad / MOE_BN;
    if (b->dn_bits == 8)
        launch_moe_gemm<8, EPI_PLAIN>(G, round_up(max_tiles, 8) * G.tiles_n, s, A);
    else
        launch_moe_gemm<4, EPI_PLAIN>(G, round_up(max_tiles, 8) * G.tiles_n, s, A);
    if (hipGetLastError() != hipSuccess) return RK_NPU_ERR_DEVICE;
    }

    const float* shared = nullptr;
    if (b->shared && slot_gemv && rows == 1) {
        // One token: the shared expert's down GEMV can run the combine in its
        // epilogue and write `out` itself; when it does not, `out` holds the
        // shared expert's output and the combine runs in place.
        bool combined = false;
        const GemvCombine comb{ws->mws->c_f32, routes, ws->top, ws->h, &combined};
        rc = enqueue_ffn(ws->sgws, b->shared_gu, ws->sdws, b->shared_dn, input, DT_F32, out, DT_F32, rows, QUANT_MOE,
                         s, &comb);
        if (rc != RK_NPU_OK) return rc;
        if (combined) return hipGetLastError() == hipSuccess ? RK_NPU_OK : RK_NPU_ERR_DEVICE;
        shared = out;
    } else if (b->shared) {
        // The shared expert is an ordinary fused FFN with the MoE rounding rule.
        rc = enqueue_ffn(ws->sgws, b->shared_gu, ws->sdws, b->shared_dn, input, DT_F32, ws->sdws->c_f32, DT_F32,
                         rows, QUANT_MOE, s);
        if (rc != RK_NPU_OK) return rc;
        shared = ws->sdws->c_f32;
    }
    CombineParams Cb;
    Cb.contrib = ws->mws->c_f32;
    Cb.pos = slot_gemv ? nullptr : ws->pos;
    Cb.routes = routes;
    Cb.shared = shared;
    Cb.rows = rows;
    Cb.top = ws->top;
    Cb.h = ws->h;
    Cb.out = out;
    const bool vec4 = ws->h % 4 == 0 && ((reinterpret_cast<uintptr_t>(Cb.contrib) | reinterpret_cast<uintptr_t>(out) |
                                           reinterpret_cast<uintptr_t>(shared)) & 15) == 0;
    if (vec4)
        hipLaunchKernelGGL(moe_combine_kernel<4>, dim3((ws->h / 4 + 255) / 256, rows), dim3(256), 0, s, Cb);
    else
        hipLaunchKernelGGL(moe_combine_kernel<1>, dim3((ws->h + 255) / 256, rows), dim3(256), 0, s, Cb);
    return hipGetLastError() == hipSuccess ? RK_NPU_OK : RK_NPU_ERR_DEVICE;
}

static bool compatible(const MoeWork* ws, const MoeBank* b) {
    return ws && b && ws->magic == MAGIC_MOE_WS && b->magic == MAGIC_MOE_W && ws->h == b->h &&
           ws->inter == b->inter && ws->experts == b->experts && ws->shared == b->shared;
}

struct BlobHeader {
    uint32_t magic, version;
    int32_t hidden, intermediate, gu_bits, dn_bits;
    uint64_t payload;
};

}  // namespace hm

using namespace hm;

extern "C" {

void rk_npu_moe_w8_config_init(rk_npu_moe_w8_config* config, int hidden, int intermediate, int routed_experts,
                               int shared_expert, int top, int max_rows) {
    if (!config) return;
    std::memset(config, 0, sizeof(*config));
    config->weights.hidden = hidden;
    config->weights.intermediate = intermediate;
    config->weights.routed_experts = routed_experts;
    config->weights.shared_expert = shared_expert ? 1 : 0;
    config->top = top;
    config->max_rows = max_rows;
    config->npu_cores = 1;
    config->cpu_threads = 1;
}

rk_npu_moe_w8_weights* rk_npu_moe_quant_weights_create(rk_npu_iommu_domain* domain,
                                                       const rk_npu_moe_w8_weight_config* config,
                                                       const rk_npu_moe_w8_expert* experts) {
    return static_cast<rk_npu_moe_w8_weights*>(
        bank_create(static_cast<Domain*>(domain), config, experts, 4, 4, true, false, nullptr));
}

rk_npu_moe_w8_weights* rk_npu_moe_quant_weights_create_full_k(rk_npu_iommu_domain* domain,
                                                              const rk_npu_moe_w8_weight_config* config,
                                                              const rk_npu_moe_w8_expert* experts) {
    return rk_npu_moe_quant_weights_create(domain, config, experts);
}

rk_npu_moe_w8_weights* rk_npu_moe_w4_weights_create(rk_npu_iommu_domain* domain,
                                                    const rk_npu_moe_w8_weight_config* config,
                                                    const rk_npu_moe_w8_expert* experts) {
    if (!config || !experts || !config->shared_expert) return nullptr;
    return static_cast<rk_npu_moe_w8_weights*>(bank_create(static_cast<Domain*>(domain), config, experts, 4, 4, true,
                                                           true, experts + config->routed_experts));
}

rk_npu_moe_w8_weights* rk_npu_moe_w4w8_weights_create(rk_npu_iommu_domain* domain,
                                                      const rk_npu_moe_w8_weight_config* config,
                                                      const rk_npu_moe_w8_expert* experts) {
    if (!config || !experts) return nullptr;
    const bool shared = config->shared_expert != 0;
    return static_cast<rk_npu_moe_w8_weights*>(bank_create(static_cast<Domain*>(domain), config, experts, 4, 8, true,
                                                           shared, shared ? experts + config->routed_experts : nullptr));
}

rk_npu_moe_w8_weights* rk_npu_moe_quant_slots_create(rk_npu_iommu_domain* domain,
                                                     const rk_npu_moe_w8_weight_config* config) {
    return static_cast<rk_npu_moe_w8_weights*>(
        bank_create(static_cast<Domain*>(domain), config, nullptr, 4, 4, false, false, nullptr));
}

rk_npu_moe_w8_weights* rk_npu_moe_w4_slots_create(rk_npu_iommu_domain* domain,
                                                  const rk_npu_moe_w8_weight_config* config,
                                                  const rk_npu_moe_w8_expert* shared) {
    return static_cast<rk_npu_moe_w8_weights*>(
        bank_create(static_cast<Domain*>(domain), config, nullptr, 4, 4, false, true, shared));
}

void rk_npu_moe_w8_weights_free(rk_npu_moe_w8_weights* weights) {
    if (weights && weights->magic == MAGIC_MOE_W) bank_destroy(weights);
}

uint64_t rk_npu_moe_w8_weights_device_bytes(const rk_npu_moe_w8_weights* weights) {
    return (weights && weights->magic == MAGIC_MOE_W) ? weights->bytes : 0;
}

rk_npu_moe_w8_workspace* rk_npu_moe_quant_workspace_create(rk_npu_iommu_domain* domain,
                                                           const rk_npu_moe_w8_config* config) {
    if (!config || config->weights.shared_expert) return nullptr;
    return static_cast<rk_npu_moe_w8_workspace*>(work_create(static_cast<Domain*>(domain), config));
}

rk_npu_moe_w8_workspace* rk_npu_moe_w4_workspace_create(rk_npu_iommu_domain* domain,
                                                        const rk_npu_moe_w8_config* config) {
    if (!config || !config->weights.shared_expert) return nullptr;
    return static_cast<rk_npu_moe_w8_workspace*>(work_create(static_cast<Domain*>(domain), config));
}

rk_npu_moe_w8_workspace* rk_npu_moe_w4w8_workspace_create(rk_npu_iommu_domain* domain,
                                                          const rk_npu_moe_w8_config* config) {
    return static_cast<rk_npu_moe_w8_workspace*>(work_create(static_cast<Domain*>(domain), config));
}

void rk_npu_moe_w8_workspace_free(rk_npu_moe_w8_workspace* workspace) {
    if (workspace && workspace->magic == MAGIC_MOE_WS) work_destroy(workspace);
}

uint64_t rk_npu_moe_w8_workspace_device_bytes(const rk_npu_moe_w8_workspace* workspace) {
    return (workspace && workspace->magic == MAGIC_MOE_WS) ? workspace->bytes : 0;
}

int rk_npu_moe_w8_run_f32(rk_npu_moe_w8_workspace* workspace, const rk_npu_moe_w8_weights* weights, int rows,
                          const float* input, const int32_t* ids, const float* routes, float* output,
                          rk_npu_moe_w8_timings* timings) {
    const double t0 = now_us();
    if (!compatible(workspace, weights) || !input || !ids || !routes || !output) return RK_NPU_ERR_PARAM;
    MoeWork* ws = workspace;
    if (rows < 1 || rows > ws->max_rows) return RK_NPU_ERR_PARAM;
    const int A = rows * ws->top;
    for (int a = 0; a < A; ++a)
        if (ids[a] < 0 || ids[a] >= ws->experts) return RK_NPU_ERR_PARAM;
    BusyGuard guard(ws->busy);
    if (!guard.ok) return RK_NPU_ERR_BUSY;
    if (hipSetDevice(device_of(ws->domain)) != hipSuccess) return RK_NPU_ERR_DEVICE;
    hipStream_t s = ws->stream;
    float* x = ws->xws->a_f32;
    // Inputs (rows, ids, routes) and later the output pass through the input
    // workspace's pinned stage when they fit it (each input at a 256-byte
    // aligned offset), else straight from pageable memory.
    const size_t xb = (size_t)rows * ws->h * 4, ab = (size_t)A * 4;
    const size_t off_ids = round_up_z(xb, 256), off_routes = off_ids + round_up_z(ab, 256);
    void* st = host_stage(ws->xws, std::max(off_routes + round_up_z(ab, 16), xb));
    const bool small = stage_small(ws->xws->hs, st, off_routes + ab, xb);
    const HostSeg segs[3] = {{input, x, xb, 0}, {ids, ws->ids, ab, off_ids}, {routes, ws->routes, ab, off_routes}};
    if (!stage_upload(ws->xws->hs, small, st, segs, 3, s)) {
        (void)hipStreamSynchronize(s);
        return RK_NPU_ERR_DEVICE;
    }
    const double t1 = now_us();
    int rc = enqueue_moe(ws, weights, rows, x, ws->ids, ws->routes, ws->out, s);
    if (rc != RK_NPU_OK) {
        (void)hipStreamSynchronize(s);
        return rc;
    }
    if (timings && hipStreamSynchronize(s) != hipSuccess) return RK_NPU_ERR_DEVICE;
    const double t2 = now_us();
    if (!stage_download(ws->xws->hs, small, st, output, ws->out, xb, s)) return RK_NPU_ERR_DEVICE;
    if (timings) {
        std::memset(timings, 0, sizeof(*timings));
        const double t3 = now_us();
        timings->input_us = t1 - t0;
        timings->gate_us = t2 - t1;
        timings->combine_us = t3 - t2;
        timings->total_us = t3 - t0;
        timings->gemm_tasks = 2;
    }
    return RK_NPU_OK;
}

int rk_npu_hip_moe_run(rk_npu_moe_w8_workspace* workspace, const rk_npu_moe_w8_weights* weights, int rows,
                       const float* input, const int32_t* ids, const float* routes, float* output, void* stream) {
    if (!compatible(workspace, weights) || !input || !ids || !routes || !output) return RK_NPU_ERR_PARAM;
    MoeWork* ws = workspace;
    if (rows < 1 || rows > ws->max_rows) return RK_NPU_ERR_PARAM;
    BusyGuard guard(ws->busy);
    if (!guard.ok) return RK_NPU_ERR_BUSY;
    if (hipSetDevice(device_of(ws->domain)) != hipSuccess) return RK_NPU_ERR_DEVICE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    return enqueue_moe(ws, weights, rows, input, ids, routes, output, s);
}

int rk_npu_hip_moe_status(rk_npu_moe_w8_workspace* workspace) {
    if (!workspace || workspace->magic != MAGIC_MOE_WS) return RK_NPU_ERR_PARAM;
    MoeWork* ws = workspace;
    if (hipSetDevice(device_of(ws->domain)) != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(ws->host_error, ws->error, 4, hipMemcpyDeviceToHost) != hipSuccess)
        return RK_NPU_ERR_DEVICE;
    const unsigned flag = *ws->host_error;
    if (flag && hipMemset(ws->error, 0, 4) != hipSuccess) return RK_NPU_ERR_DEVICE;
    return flag ? RK_NPU_ERR_PARAM : RK_NPU_OK;
}

// ---- expert records ------------------------------------------------------------

uint64_t rk_npu_moe_quant_expert_blob_bytes(const rk_npu_moe_w8_weights* weights) {
    if (!weights || weights->magic != MAGIC_MOE_W) return 0;
    return sizeof(BlobHeader) + weights->L.total;
}

int rk_npu_moe_quant_export_expert(const rk_npu_moe_w8_weights* weights, int expert, void* data, uint64_t bytes) {
    if (!weights || weights->magic != MAGIC_MOE_W || !data) return RK_NPU_ERR_PARAM;
    if (expert < 0 || expert >= weights->experts) return RK_NPU_ERR_PARAM;
    if (bytes != rk_npu_moe_quant_expert_blob_bytes(weights)) return RK_NPU_ERR_PARAM;
    BlobHeader hdr{BLOB_MAGIC, RK_NPU_MOE_QUANT_BLOB_VERSION, weights->h, weights->inter, weights->gu_bits,
                   weights->dn_bits, weights->L.total};
    std::memcpy(data, &hdr, sizeof(hdr));
    if (hipSetDevice(device_of(weights->domain)) != hipSuccess) return RK_NPU_ERR_DEVICE;
    if (hipMemcpy(static_cast<uint8_t*>(data) + sizeof(hdr), weights->expert[expert], weights->L.total,
                  hipMemcpyDeviceToHost) != hipSuccess)
        return RK_NPU_ERR_DEVICE;
    return RK_NPU_OK;
}

int rk_npu_moe_quant_import_expert_timed(rk_npu_moe_w8_weights* weights, int slot, const void* data, uint64_t bytes,
                                         rk_npu_moe_import_timings* timings) {
    const double t0 = now_us();
    if (!weights || weights->magic != MAGIC_MOE_W || !data) return RK_NPU_ERR_PARAM;
    if (slot < 0 || slot >= weights->experts) return RK_NPU_ERR_PARAM;
    if (bytes != rk_npu_moe_quant_expert_blob_bytes(weights)) return RK_NPU_ERR_FORMAT;
    BlobHeader hdr;
    std::memcpy(&hdr, data, sizeof(hdr));
    if (hdr.magic != BLOB_MAGIC || hdr.version != RK_NPU_MOE_QUANT_BLOB_VERSION || hdr.hidden != weights->h ||
        hdr.intermediate != weights->inter || hdr.gu_bits != weights->gu_bits || hdr.dn_bits != weights->dn_bits ||
        hdr.payload != weights->L.total)
        return RK_NPU_ERR_FORMAT;
    const double t1 = now_us();
    if (hipSetDevice(device_of(weights->domain)) != hipSuccess) return RK_NPU_ERR_DEVICE;
    if (hipMemcpy(weights->expert[slot], static_cast<const uint8_t*>(data) + sizeof(hdr), weights->L.total,
                  hipMemcpyHostToDevice) != hipSuccess)
        return RK_NPU_ERR_DEVICE;
    if (timings) {
        const double t2 = now_us();
        timings->validate_us = t1 - t0;
        timings->copy_us = t2 - t1;
        timings->gate_sync_us = 0.0;
        timings->down_sync_us = 0.0;
        timings->total_us = t2 - t0;
    }
    return RK_NPU_OK;
}

int rk_npu_moe_quant_import_expert(rk_npu_moe_w8_weights* weights, int slot, const void* data, uint64_t bytes) {
    return rk_npu_moe_quant_import_expert_timed(weights, slot, data, bytes, nullptr);
}

int rk_npu_moe_quant_swap_slots(rk_npu_moe_w8_weights* weights, int slot, rk_npu_moe_w8_weights* bank, int staged) {
    if (!weights || !bank || weights->magic != MAGIC_MOE_W || bank->magic != MAGIC_MOE_W) return RK_NPU_ERR_PARAM;
    if (slot < 0 || slot >= weights->experts || staged < 0 || staged >= bank->experts) return RK_NPU_ERR_PARAM;
    if (weights->h != bank->h || weights->inter != bank->inter || weights->gu_bits != bank->gu_bits ||
        weights->dn_bits != bank->dn_bits || weights->domain != bank->domain)
        return RK_NPU_ERR_PARAM;
    if (hipSetDevice(device_of(weights->domain)) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
        return RK_NPU_ERR_DEVICE;
    std::swap(weights->expert[slot], bank->expert[staged]);
    if (!upload_tables(weights) || !upload_tables(bank)) return RK_NPU_ERR_DEVICE;
    return RK_NPU_OK;
}

}  // extern "C"

// The one-launch FFN of one row (ffn_m1_kernel, opt-in: HM_FFN_FUSED=1):
// its launch variants, instantiated here so they compile beside the other
// launch units.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <utility>

#include "kernels.hpp"
#include "launch.hpp"

namespace hm {

// Blocks of the one-launch FFN kernel `fn` that fit the GPU at once with
// `lds` bytes of dynamic shared memory (0 if unknown), cached per kernel.
static long ffn_capacity(const void* fn, size_t lds) {
    static std::mutex mu;
    static std::map<std::pair<const void*, size_t>, long> cache;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find({fn, lds});
    if (it != cache.end()) return it->second;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, FFN_THREADS, lds) != hipSuccess) {
        (void)hipGetLastError();
        per_cu = 0;
    }
    const long cap = (long)per_cu * device_cus();
    cache[{fn, lds}] = cap;
    return cap;
}

template <typename TX, int RWG, int BD>
static bool launch_ffn_fused(const GemvParams& Pg, const GemvParams& Pd, int grid, size_t lds, hipStream_t s) {
    constexpr int RWD = BD == 4 ? 3 : 5;
    const void* fn = reinterpret_cast<const void*>(&ffn_m1_kernel<TX, 4, RWG, BD, RWD>);
    if (ffn_capacity(fn, lds) < grid) return false;  // must be resident as a whole
    hipLaunchKernelGGL((ffn_m1_kernel<TX, 4, RWG, BD, RWD>), dim3(grid), dim3(FFN_THREADS), lds, s, Pg, Pd);
    return true;
}

template <typename TX, int BD>
static bool launch_ffn_fused_rw(int rwg, const GemvParams& Pg, const GemvParams& Pd, int grid, size_t lds,
                                hipStream_t s) {
    if (rwg == 6) return launch_ffn_fused<TX, 6, BD>(Pg, Pd, grid, lds, s);
    if (rwg == 7) return launch_ffn_fused<TX, 7, BD>(Pg, Pd, grid, lds, s);
    return launch_ffn_fused<TX, 8, BD>(Pg, Pd, grid, lds, s);
}

bool launch_ffn_fused_any(int a_type, int dn_bits, int rwg, const GemvParams& Pg, const GemvParams& Pd, int grid,
                          size_t lds, hipStream_t s) {
    if (a_type == DT_F32)
        return dn_bits == 4 ? launch_ffn_fused_rw<float, 4>(rwg, Pg, Pd, grid, lds, s)
                            : launch_ffn_fused_rw<float, 8>(rwg, Pg, Pd, grid, lds, s);
    return dn_bits == 4 ? launch_ffn_fused_rw<__half, 4>(rwg, Pg, Pd, grid, lds, s)
                        : launch_ffn_fused_rw<__half, 8>(rwg, Pg, Pd, grid, lds, s);
}

}  // namespace hm

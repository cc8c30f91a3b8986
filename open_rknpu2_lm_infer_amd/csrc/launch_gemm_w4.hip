// GEMM launches of W4 weights (every tile variant, both epilogues).
#include "launch.hpp"
#include "launch_impl.hpp"

namespace hm {

void launch_gemm_w4(int epi, int v, bool staged, const GemmParams& G, int tiles, hipStream_t s) {
    if (epi == EPI_PLAIN)
        launch_gemm<4, EPI_PLAIN>(v, staged, G, tiles, s);
    else
        launch_gemm<4, EPI_SWIGLU_MAX>(v, staged, G, tiles, s);
}

}  // namespace hm

// GEMV launches of __half activation rows against W8 weights (every row
// count, register window and quantization placement, both epilogues; split-K
// pieces).
#include "launch.hpp"
#include "launch_impl.hpp"

namespace hm {

void launch_gemv_f16_w8(int epi, int mr, const GemvParams& V, int grid, size_t lds, hipStream_t s, bool preq,
                          int qwn) {
    launch_gemv_epi<__half, 8>(epi, mr, V, grid, lds, s, preq, qwn);
}

void launch_gemv_split_f16_w8(const GemvParams& V, int grid, int rounds, size_t lds, hipStream_t s) {
    launch_gemv_split<__half, 8>(V, grid, rounds, lds, s);
}

}  // namespace hm

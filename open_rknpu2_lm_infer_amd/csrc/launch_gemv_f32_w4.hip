// GEMV launches of float activation rows against W4 weights (every row
// count, register window and quantization placement, both epilogues; split-K
// pieces; the one-row GEMV with the MoE combine).
#include "launch.hpp"
#include "launch_impl.hpp"

namespace hm {

void launch_gemv_f32_w4(int epi, int mr, const GemvParams& V, int grid, size_t lds, hipStream_t s, bool preq,
                          int qwn) {
    launch_gemv_epi<float, 4>(epi, mr, V, grid, lds, s, preq, qwn);
}

void launch_gemv_split_f32_w4(const GemvParams& V, int grid, int rounds, size_t lds, hipStream_t s) {
    launch_gemv_split<float, 4>(V, grid, rounds, lds, s);
}

void launch_gemv_combine_w4(const GemvParams& V, int groups, int rounds, size_t lds, hipStream_t s) {
    launch_gemv_combine<4>(V, groups, rounds, lds, s);
}

}  // namespace hm

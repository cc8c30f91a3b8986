// FP32 SwiGLU of 16 values, the CPU side of this library's SwiGLU arithmetic.
//
// The reference's CPU kernels include this header from the operator library's
// source directory (native/cpu_kernels/swiglu.cpp:1, include path
// "${RK_NPU_MATMUL_ROOT}/src" at native/cpu_kernels/CMakeLists.txt:14) and, on
// aarch64, call apply16<false>(gate, up, out) for each 16 values of a row
// (native/cpu_kernels/swiglu.cpp:13-21); other architectures use their own
// loop with std::exp and only need the header to compile.
//
// The arithmetic is the one the GPU kernels of this library run in their
// SwiGLU epilogues, value for value, so the CPU fallback of
// src/model/cpu.rs:269-294 produces the same bits as the fused GPU path:
//   out = (g / (1 + exp(t))) * u,  t = clamp(-g, -80, 80),
//   out = +-0 * u for g < -80 (the sign of g: the "signed zero" tail),
// with exp written from Cody and Waite's additive range reduction
// (x = n ln2 + r, ln2 split into a 12-bit head and a tail so n ln2 is exact)
// and the degree-7 Taylor polynomial of exp(r) on |r| <= ln2/2, evaluated by
// Horner's rule with fused multiply-adds, scaled by 2^n built in the exponent
// field (|n| <= 116, so 2^n is a normal float). Saturating the argument at 80
// keeps 2^n in range; no branch depends on the polynomial.
//
// Template argument: true makes the call also return max |out| over the 16
// outputs (what a caller quantizing the middle row needs); false returns 0.
// Portable C++17 (no intrinsics); compilers vectorize the 16-wide loops.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>

namespace rknpu2_matmul_open {
namespace detail {
namespace swiglu_fp32 {

inline float exp_cw(float x) {
    const float log2e = 0x1.715476p+0f;
    const float ln2_hi = 0x1.62ep-1f;
    const float ln2_lo = 0x1.0bfbe8p-15f;
    const float kf = std::rint(x * log2e);
    float r = std::fma(kf, -ln2_hi, x);
    r = std::fma(kf, -ln2_lo, r);
    float p = 0x1.a01a02p-13f;  // 1/7!
    p = std::fma(p, r, 0x1.6c16c2p-10f);  // 1/6!
    p = std::fma(p, r, 0x1.111112p-7f);   // 1/5!
    p = std::fma(p, r, 0x1.555556p-5f);   // 1/4!
    p = std::fma(p, r, 0x1.555556p-3f);   // 1/3!
    p = std::fma(p, r, 0x1.0p-1f);        // 1/2!
    p = std::fma(p, r, 1.0f);
    p = std::fma(p, r, 1.0f);
    const int32_t bits = (static_cast<int32_t>(kf) + 127) << 23;
    float scale;
    std::memcpy(&scale, &bits, sizeof(scale));
    return p * scale;
}

inline float swiglu1(float g, float u) {
    const float t = std::fmin(std::fmax(-g, -80.0f), 80.0f);
    const float e = exp_cw(t);
    float silu = g / (1.0f + e);
    if (g < -80.0f) silu = std::copysign(0.0f, g);
    return silu * u;
}

template <bool TrackMax>
inline float apply16(const float* gate, const float* up, float* out) {
    float mx = 0.0f;
    for (int i = 0; i < 16; ++i) {
        const float o = swiglu1(gate[i], up[i]);
        out[i] = o;
        if (TrackMax) mx = std::fmax(mx, std::fabs(o));
    }
    return mx;
}

}  // namespace swiglu_fp32
}  // namespace detail
}  // namespace rknpu2_matmul_open

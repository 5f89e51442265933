// devmath.hpp - device-side activation helpers shared by the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace vdk {

// Exact (erf) GELU, x * Phi(x) = 0.5 x (1 + erf(x / sqrt 2)): HF nn.GELU() /
// ggml_gelu_erf, the activation of the wav2vec2 convs and feed-forward layers
// (reference src/analyze_w2v2.cpp:126-128, :421, :457).
//
// erf from Abramowitz & Stegun, Handbook of Mathematical Functions, formula
// 7.1.26: for a >= 0, erf(a) = 1 - q(a) with q(a) = (a1 t + a2 t^2 + a3 t^3 +
// a4 t^4 + a5 t^5) exp(-a^2), t = 1 / (1 + p a), |error| <= 1.5e-7.  So
// 1 + erf(x / sqrt 2) is 2 - q for x >= 0 and q itself for x < 0 (no
// cancellation on the negative side).  One reciprocal, one exp2 and five
// FMAs: the GELU epilogue of wav2vec2-large's ff1 at 64 x 149 frames (39 M
// values) added 31 us to the GEMM with the library erff, 15 us with this.
// The error (|GELU error| <= 4.3e-7, relative <= 1.7e-4 where |GELU| > 1e-3)
// is below the f16 rounding of the stored activations.
__device__ __forceinline__ float gelu_erf(float x) {
    const float a = fabsf(x) * 0.70710678118654752f;
    const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * a);
    const float poly =
        t * (0.254829592f + t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
    const float q = poly * __builtin_amdgcn_exp2f(-a * a * 1.44269504088896341f);
    return 0.5f * x * (x >= 0.0f ? 2.0f - q : q);
}

}  // namespace vdk

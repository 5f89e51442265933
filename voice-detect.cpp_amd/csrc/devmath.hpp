// devmath.hpp - device-side activation helpers shared by the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace vdk {

// Exact (erf) GELU, x * Phi(x) = 0.5 x (1 + erf(x / sqrt 2)): HF nn.GELU() /
// ggml_gelu_erf, the activation of the wav2vec2 convs and feed-forward layers
// (reference src/analyze_w2v2.cpp:126-128, :421, :457).
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

}  // namespace vdk

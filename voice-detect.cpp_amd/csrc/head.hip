// head.hip - statistics pooling, embedding FC and L2 normalisation on gfx950.
//
// These are bandwidth-bound reductions: TSTP reads the last feature map once
// (coalesced over channels, one thread per (clip, freq row, channel)); the FC is
// one wavefront per output element with a shuffle reduction; L2 is one
// wavefront per clip.  Sums are accumulated in f64 like the reference's ggml
// reductions and host L2 (src/encoder_resnet.cpp:140-183).
#include <cmath>

#include "common.hpp"
#include "vdk.h"

namespace vdk {
namespace {

__device__ __forceinline__ double wave_sum_d(double v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// TSTP (src/encoder_resnet.cpp:140-157): mean over time, var * N/(N-1), sqrt(var + eps).
__global__ __launch_bounds__(256) void tstp_kernel(const half_t* __restrict__ x, int H, int W, int C, float eps,
                                                   float* __restrict__ pooled) {
#pragma clang fp contract(off)
    const int h = blockIdx.x, b = blockIdx.y;
    const size_t CH = (size_t)C * H;
    float* out = pooled + (size_t)b * 2 * CH;
    const half_t* row = x + ((size_t)b * H + h) * W * C;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
        double s = 0.0;
        for (int t = 0; t < W; ++t) s += (double)(float)row[(size_t)t * C + c];
        const float mean = (float)(s / W);
        double s2 = 0.0;
        for (int t = 0; t < W; ++t) {
            const float d = (float)row[(size_t)t * C + c] - mean;
            s2 += (double)(d * d);
        }
        float var = (float)(s2 / W);
        if (W > 1) var = var * ((float)W / (float)(W - 1));
        out[(size_t)c * H + h] = mean;
        out[CH + (size_t)c * H + h] = sqrtf(var + eps);
    }
}

// y[b][o] = sum_i w[o][i] x[b][i] + bias[o] - mean_vec[o]; one wavefront per (b, o).
__global__ __launch_bounds__(256) void linear_kernel(const float* __restrict__ x, int B, int in_dim,
                                                     const float* __restrict__ w, const float* __restrict__ bias,
                                                     const float* __restrict__ mv, int out_dim,
                                                     float* __restrict__ y) {
    const long gw = ((long)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (gw >= (long)B * out_dim) return;   // uniform per wavefront
    const int b = (int)(gw / out_dim), o = (int)(gw - (long)b * out_dim);
    const float* wr = w + (size_t)o * in_dim;
    const float* xr = x + (size_t)b * in_dim;
    double s = 0.0;
    for (int i = lane; i < in_dim; i += 64) s += (double)wr[i] * (double)xr[i];
    s = wave_sum_d(s);
    if (lane == 0) {
        float v = (float)s;
        if (bias) v += bias[o];
        if (mv) v -= mv[o];
        y[(size_t)b * out_dim + o] = v;
    }
}

// In-place L2 normalisation, one wavefront per clip (src/encoder_resnet.cpp:177-183).
__global__ __launch_bounds__(64) void l2norm_kernel(float* __restrict__ x, int dim) {
    float* v = x + (size_t)blockIdx.x * dim;
    double s = 0.0;
    for (int i = threadIdx.x; i < dim; i += 64) s += (double)v[i] * (double)v[i];
    s = wave_sum_d(s);
    const double norm = sqrt(s);
    if (norm > 0.0)
        for (int i = threadIdx.x; i < dim; i += 64) v[i] = (float)((double)v[i] / norm);
}

}  // namespace
}  // namespace vdk

using namespace vdk;

extern "C" int vdk_tstp(const void* d_x, int batch, int H, int W, int C, float eps, float* d_pooled,
                        void* stream) {
    return guarded([&] {
        require(d_x && d_pooled, "tstp: NULL device pointer");
        require(batch > 0 && H > 0 && W > 0 && C > 0, "tstp: empty input");
        hipLaunchKernelGGL(tstp_kernel, dim3(H, batch), dim3(256), 0, static_cast<hipStream_t>(stream),
                           static_cast<const half_t*>(d_x), H, W, C, eps, d_pooled);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_linear(const float* d_x, int batch, int in_dim, const float* d_w, const float* d_bias,
                          const float* d_mean_vec, int out_dim, float* d_y, void* stream) {
    return guarded([&] {
        require(d_x && d_w && d_y, "linear: NULL device pointer");
        require(batch > 0 && in_dim > 0 && out_dim > 0, "linear: empty shape");
        const long waves = (long)batch * out_dim;
        hipLaunchKernelGGL(linear_kernel, dim3(cdiv(waves, 4)), dim3(256), 0, static_cast<hipStream_t>(stream),
                           d_x, batch, in_dim, d_w, d_bias, d_mean_vec, out_dim, d_y);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_l2norm(float* d_x, int batch, int dim, void* stream) {
    return guarded([&] {
        require(d_x, "l2norm: NULL device pointer");
        require(batch > 0 && dim > 0, "l2norm: empty shape");
        hipLaunchKernelGGL(l2norm_kernel, dim3(batch), dim3(64), 0, static_cast<hipStream_t>(stream), d_x, dim);
        VDK_HIP(hipGetLastError());
    });
}

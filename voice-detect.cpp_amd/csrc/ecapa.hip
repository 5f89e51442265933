// ecapa.hip - the non-GEMM pieces of the ECAPA-TDNN encoder on gfx950.
//
// The convolutions of src/encoder.cpp run on the implicit-GEMM kernels
// (vdk_conv2d_ex, time as the W axis, H = 1).  What remains is bandwidth-bound
// and lives here:
//  * feats_tmajor: FBank [B][n_mels][T] f32 -> time-major f16 [B][T+2p][Cpad]
//    with SpeechBrain's reflect padding (src/encoder.cpp:32-52) and zero
//    channels up to Cpad;
//  * reflect_pad_add: the Res2Net group input x_j (+ y_{j-1}), reflect padded
//    for the dilated k=3 conv (src/encoder.cpp:174-200);
//  * channel_mean / se_gate_residual: SE squeeze and x * sigmoid(s) + residual
//    (src/encoder.cpp:207-244);
//  * asp_stats / asp_pool: attentive statistics pooling with global context
//    (src/encoder.cpp:262-295): global mean/std (clamp 1e-12), softmax over
//    time per channel, weighted mean/std.
// Sums are accumulated in f64.
#include <cmath>

#include "common.hpp"
#include "vdk.h"

namespace vdk {
namespace {

// Reflect without repeating the edge sample; indices past a 1-sample clip clamp.
__device__ __forceinline__ int reflect_idx(int j, int pad, int T) {
    int t;
    if (j < pad) t = pad - j;
    else if (j < pad + T) t = j - pad;
    else t = (T - 2) - (j - pad - T);
    return t < 0 ? 0 : (t > T - 1 ? T - 1 : t);
}

__global__ __launch_bounds__(256) void feats_tmajor_kernel(const float* __restrict__ f, int B, int C, int T,
                                                           int pad, int Cpad, half_t* __restrict__ out) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    const int Tp = T + 2 * pad;
    if (i >= (long)B * Tp * Cpad) return;
    const int c = (int)(i % Cpad);
    const long r = i / Cpad;
    const int j = (int)(r % Tp), b = (int)(r / Tp);
    const float v = c < C ? f[((size_t)b * C + c) * T + reflect_idx(j, pad, T)] : 0.0f;
    out[i] = (half_t)v;
}

__global__ __launch_bounds__(256) void reflect_pad_add_kernel(const half_t* __restrict__ a, int as,
                                                              const half_t* __restrict__ bsrc, int bs, int B,
                                                              int T, int G, int pad, half_t* __restrict__ out) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;   // one 8-channel chunk
    const int G8 = G / 8, Tp = T + 2 * pad;
    if (i >= (long)B * Tp * G8) return;
    const int c = (int)(i % G8) * 8;
    const long r = i / G8;
    const int j = (int)(r % Tp), b = (int)(r / Tp);
    const size_t src = (size_t)b * T + reflect_idx(j, pad, T);
    half8 v = *reinterpret_cast<const half8*>(a + src * as + c);
    if (bsrc) {
        const half8 w = *reinterpret_cast<const half8*>(bsrc + src * bs + c);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (half_t)((float)v[e] + (float)w[e]);
    }
    *reinterpret_cast<half8*>(out + ((size_t)b * Tp + j) * G + c) = v;
}

// Per-channel mean over time: 64 channels x 16 time partitions per
// workgroup, f64 partition sums combined in a fixed order.
__global__ __launch_bounds__(1024) void channel_mean_kernel(const half_t* __restrict__ x, int xs, int T, int C,
                                                            float* __restrict__ out) {
    __shared__ double sp[16][64];
    const int tx = threadIdx.x & 63, tp = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + tx, b = blockIdx.y;
    double s = 0.0;
    if (c < C) {
        const half_t* p = x + (size_t)b * T * xs + c;
        for (int t = tp; t < T; t += 16) s += (double)(float)p[(size_t)t * xs];
    }
    sp[tp][tx] = s;
    __syncthreads();
    if (tp == 0 && c < C) {
        double S = 0.0;
#pragma unroll
        for (int i = 0; i < 16; ++i) S += sp[i][tx];
        out[(size_t)b * C + c] = (float)(S / T);
    }
}

__global__ __launch_bounds__(256) void se_gate_residual_kernel(const half_t* __restrict__ x, int xs,
                                                               const float* __restrict__ gate,
                                                               const half_t* __restrict__ res, int rs, int B, int T,
                                                               int C, half_t* __restrict__ y, int ys) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;   // one 8-channel chunk
    const int C8 = C / 8;
    if (i >= (long)B * T * C8) return;
    const int c = (int)(i % C8) * 8;
    const long r = i / C8;                                  // b * T + t
    const int b = (int)(r / T);
    const half8 xv = *reinterpret_cast<const half8*>(x + r * xs + c);
    const half8 rv = *reinterpret_cast<const half8*>(res + r * rs + c);
    half8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float g = 1.0f / (1.0f + expf(-gate[(size_t)b * C + c + e]));
        o[e] = (half_t)((float)xv[e] * g + (float)rv[e]);
    }
    *reinterpret_cast<half8*>(y + r * ys + c) = o;
}

// Global statistics over time per (clip, channel): out[b] = [mean ; sqrt(clamp(var, eps))].
// Per-channel mean and std over time (biased, clamped at eps): 64 channels x
// 16 time partitions per workgroup, two passes of f64 partition sums
// combined in a fixed order.
__global__ __launch_bounds__(1024) void asp_stats_kernel(const half_t* __restrict__ x, int xs, int T, int C,
                                                         float eps, float* __restrict__ out) {
    __shared__ double sp[16][64];
    const int tx = threadIdx.x & 63, tp = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + tx, b = blockIdx.y;
    const bool on = c < C;
    const half_t* p = x + (size_t)b * T * xs + (on ? c : 0);
    double s = 0.0;
    if (on)
        for (int t = tp; t < T; t += 16) s += (double)(float)p[(size_t)t * xs];
    sp[tp][tx] = s;
    __syncthreads();
    double S = 0.0;
#pragma unroll
    for (int i = 0; i < 16; ++i) S += sp[i][tx];
    const float m = (float)(S / T);
    double s2 = 0.0;
    if (on)
        for (int t = tp; t < T; t += 16) {
            const float d = (float)p[(size_t)t * xs] - m;
            s2 += (double)(d * d);
        }
    __syncthreads();   // every thread has read sp
    sp[tp][tx] = s2;
    __syncthreads();
    if (tp == 0 && on) {
        double S2 = 0.0;
#pragma unroll
        for (int i = 0; i < 16; ++i) S2 += sp[i][tx];
        float v = (float)(S2 / T);
        if (v < eps) v = eps;
        out[(size_t)b * 2 * C + c] = m;
        out[(size_t)b * 2 * C + C + c] = sqrtf(v);
    }
}

// Softmax over time of the attention logits, then attention-weighted mean / std.
// A workgroup covers 64 channels of one clip with 16 time partitions per
// channel: max, then the f64 sums of e = exp(l - max) and e*x, then of
// e*(x - mu)^2, each partitioned over time and combined in a fixed order.
__global__ __launch_bounds__(1024) void asp_pool_kernel(const float* __restrict__ logits, int ls,
                                                        const half_t* __restrict__ x, int xs, int T, int C, float eps,
                                                        float* __restrict__ out) {
    __shared__ float smax[16][64];
    __shared__ double sz[16][64], smu[16][64];
    const int tx = threadIdx.x & 63, tp = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + tx, b = blockIdx.y;
    const bool on = c < C;
    const float* l = logits + (size_t)b * T * ls + (on ? c : 0);
    const half_t* p = x + (size_t)b * T * xs + (on ? c : 0);
    float m = -INFINITY;
    if (on)
        for (int t = tp; t < T; t += 16) m = fmaxf(m, l[(size_t)t * ls]);
    smax[tp][tx] = m;
    __syncthreads();
    float mx = smax[0][tx];
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, smax[i][tx]);
    double z = 0.0, mu = 0.0;
    if (on)
        for (int t = tp; t < T; t += 16) {
            const double e = (double)expf(l[(size_t)t * ls] - mx);
            z += e;
            mu += e * (double)(float)p[(size_t)t * xs];
        }
    sz[tp][tx] = z;
    smu[tp][tx] = mu;
    __syncthreads();
    double Z = 0.0, MU = 0.0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        Z += sz[i][tx];
        MU += smu[i][tx];
    }
    const float muf = (float)(MU / Z);
    double var = 0.0;
    if (on)
        for (int t = tp; t < T; t += 16) {
            const double e = (double)expf(l[(size_t)t * ls] - mx);
            const float d = (float)p[(size_t)t * xs] - muf;
            var += e * (double)(d * d);
        }
    __syncthreads();   // every thread has read sz / smu
    sz[tp][tx] = var;
    __syncthreads();
    if (tp == 0 && on) {
        double V = 0.0;
#pragma unroll
        for (int i = 0; i < 16; ++i) V += sz[i][tx];
        float v = (float)(V / Z);
        if (v < eps) v = eps;
        out[(size_t)b * 2 * C + c] = muf;
        out[(size_t)b * 2 * C + C + c] = sqrtf(v);
    }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace vdk

using namespace vdk;

extern "C" int vdk_feats_tmajor(const float* d_feats, int batch, int n_mels, int T, int pad, int c_pad, void* d_out,
                                void* stream) {
    return guarded([&] {
        require(d_feats && d_out, "feats_tmajor: NULL device pointer");
        require(batch > 0 && n_mels > 0 && T > 0 && pad >= 0 && c_pad >= n_mels, "feats_tmajor: bad shape");
        const long n = (long)batch * (T + 2 * pad) * c_pad;
        hipLaunchKernelGGL(feats_tmajor_kernel, dim3(cdiv(n, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                           d_feats, batch, n_mels, T, pad, c_pad, static_cast<half_t*>(d_out));
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_reflect_pad_add(const void* d_a, int a_stride, const void* d_b, int b_stride, int batch, int T,
                                   int G, int pad, void* d_out, void* stream) {
    return guarded([&] {
        require(d_a && d_out, "reflect_pad_add: NULL device pointer");
        require(batch > 0 && T > 0 && G > 0 && G % 8 == 0 && pad >= 0 && a_stride >= G && (!d_b || b_stride >= G),
                "reflect_pad_add: bad shape");
        require(a_stride % 8 == 0 && (!d_b || b_stride % 8 == 0) && al16(d_a) && (!d_b || al16(d_b)) && al16(d_out),
                "reflect_pad_add: strides/pointers must be 8-channel aligned");
        const long n = (long)batch * (T + 2 * pad) * (G / 8);
        hipLaunchKernelGGL(reflect_pad_add_kernel, dim3(cdiv(n, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                           static_cast<const half_t*>(d_a), a_stride, static_cast<const half_t*>(d_b), b_stride, batch,
                           T, G, pad, static_cast<half_t*>(d_out));
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_channel_mean(const void* d_x, int x_stride, int batch, int T, int C, float* d_out, void* stream) {
    return guarded([&] {
        require(d_x && d_out, "channel_mean: NULL device pointer");
        require(batch > 0 && T > 0 && C > 0 && x_stride >= C, "channel_mean: bad shape");
        hipLaunchKernelGGL(channel_mean_kernel, dim3(cdiv(C, 64), batch), dim3(1024), 0,
                           static_cast<hipStream_t>(stream), static_cast<const half_t*>(d_x), x_stride, T, C, d_out);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_se_gate_residual(const void* d_x, int x_stride, const float* d_gate, const void* d_res,
                                    int res_stride, int batch, int T, int C, void* d_y, int y_stride, void* stream) {
    return guarded([&] {
        require(d_x && d_gate && d_res && d_y, "se_gate_residual: NULL device pointer");
        require(batch > 0 && T > 0 && C > 0 && C % 8 == 0 && x_stride >= C && res_stride >= C && y_stride >= C,
                "se_gate_residual: bad shape");
        require(x_stride % 8 == 0 && res_stride % 8 == 0 && y_stride % 8 == 0 && al16(d_x) && al16(d_res) &&
                    al16(d_y), "se_gate_residual: strides/pointers must be 8-channel aligned");
        const long n = (long)batch * T * (C / 8);
        hipLaunchKernelGGL(se_gate_residual_kernel, dim3(cdiv(n, 256)), dim3(256), 0,
                           static_cast<hipStream_t>(stream), static_cast<const half_t*>(d_x), x_stride, d_gate,
                           static_cast<const half_t*>(d_res), res_stride, batch, T, C, static_cast<half_t*>(d_y),
                           y_stride);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_asp_stats(const void* d_x, int x_stride, int batch, int T, int C, float eps, float* d_out,
                             void* stream) {
    return guarded([&] {
        require(d_x && d_out, "asp_stats: NULL device pointer");
        require(batch > 0 && T > 0 && C > 0 && x_stride >= C, "asp_stats: bad shape");
        hipLaunchKernelGGL(asp_stats_kernel, dim3(cdiv(C, 64), batch), dim3(1024), 0,
                           static_cast<hipStream_t>(stream), static_cast<const half_t*>(d_x), x_stride, T, C, eps,
                           d_out);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_asp_pool(const float* d_logits, int l_stride, const void* d_x, int x_stride, int batch, int T,
                            int C, float eps, float* d_out, void* stream) {
    return guarded([&] {
        require(d_logits && d_x && d_out, "asp_pool: NULL device pointer");
        require(batch > 0 && T > 0 && C > 0 && x_stride >= C && l_stride >= C, "asp_pool: bad shape");
        hipLaunchKernelGGL(asp_pool_kernel, dim3(cdiv(C, 64), batch), dim3(1024), 0,
                           static_cast<hipStream_t>(stream), d_logits, l_stride, static_cast<const half_t*>(d_x),
                           x_stride, T, C, eps, d_out);
        VDK_HIP(hipGetLastError());
    });
}

// campplus.hip - the non-GEMM pieces of the CAM++ D-TDNN backbone on gfx950.
//
// The convolutions of src/encoder_campplus.cpp (FCM 2D convs, the strided
// TDNN, every dense layer's 1x1 / dilated linear_local, the transits) run on
// the implicit-GEMM kernels over time-major [B][T'][C] maps.  What remains:
//  * bn_act: the standalone BatchNorm -> ReLU in front of each dense layer's
//    linear1 and each transit (src/encoder_campplus.cpp:110-134, 254-255, 286);
//  * segment_sums + cam_context: the context-aware mask.  The context
//    c.mean(T') + seg100(c) is constant over a 100-frame segment, so the mask
//    m = sigmoid(W2 relu(W1 ctx + b1) + b2) is computed once per (clip,
//    segment) (src/encoder_campplus.cpp:159-182, 260-268) and applied in the
//    linear_local conv epilogue as a per-segment gate.
// Sums are accumulated in f64.
#include <cmath>

#include "common.hpp"
#include "vdk.h"

namespace vdk {
namespace {

__global__ __launch_bounds__(256) void bn_act_kernel(const half_t* __restrict__ x, int xs, long rows, int C,
                                                     const float* __restrict__ scale,
                                                     const float* __restrict__ shift, int act,
                                                     half_t* __restrict__ y, int ys) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;   // one 8-channel chunk
    const int C8 = C / 8;
    if (i >= rows * C8) return;
    const int c = (int)(i % C8) * 8;
    const long r = i / C8;
    const half8 v = *reinterpret_cast<const half8*>(x + r * xs + c);
    const float4v s0 = *reinterpret_cast<const float4v*>(scale + c), s1 = *reinterpret_cast<const float4v*>(scale + c + 4);
    const float4v h0 = *reinterpret_cast<const float4v*>(shift + c), h1 = *reinterpret_cast<const float4v*>(shift + c + 4);
    const float sc[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
    const float sh[8] = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
    half8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        float f = (float)v[e] * sc[e] + sh[e];
        if (act == VDK_ACT_RELU) f = fmaxf(f, 0.0f);
        o[e] = (half_t)f;
    }
    *reinterpret_cast<half8*>(y + r * ys + c) = o;
}

// Workgroup (b, s, 64-channel group): 16 waves split the frames of segment s
// (frame t to wave t mod 16, a handful of loads each, all in flight at once);
// the 16 partial sums are added in a fixed order.
constexpr int kSegParts = 16;
__global__ __launch_bounds__(64 * kSegParts) void segment_sums_kernel(const half_t* __restrict__ x, int xs, int T,
                                                                      int C, int seg, float* __restrict__ out) {
    __shared__ double part[kSegParts][64];
    const int b = blockIdx.x, s = blockIdx.y, c0 = blockIdx.z * 64;
    const int nseg = gridDim.y;
    const int lane_c = threadIdx.x & 63, lane_t = threadIdx.x >> 6;
    const int c = c0 + lane_c;
    const int t0 = s * seg, t1 = min(T, t0 + seg);
    double acc = 0.0;
    if (c < C) {
        const half_t* p = x + (size_t)b * T * xs + c;
#pragma unroll 8
        for (int t = t0 + lane_t; t < t1; t += kSegParts) acc += (double)(float)p[(size_t)t * xs];
    }
    part[lane_t][lane_c] = acc;
    __syncthreads();
    if (lane_t == 0 && c < C) {
        double v = 0.0;
#pragma unroll
        for (int q = 0; q < kSegParts; ++q) v += part[q][lane_c];
        out[((size_t)b * nseg + s) * C + c] = (float)v;
    }
}

// Dot product of a weight row with an LDS vector, split over 4 lanes: lane q
// takes the q-th contiguous quarter (16-byte loads, all issued together when
// n % 16 == 0), else every 4th element; lane 0 adds the 4 partial sums in a
// fixed order.
__device__ __forceinline__ double dot4(const float* __restrict__ wr, const float* v, int n, int q) {
    double a = 0.0;
    if ((n & 15) == 0) {
        const int len = n >> 2;
        const float4v* w4 = reinterpret_cast<const float4v*>(wr + q * len);
        const float4v* v4 = reinterpret_cast<const float4v*>(v + q * len);
#pragma unroll 8
        for (int i = 0; i < (len >> 2); ++i) {
            const float4v wv = w4[i], xv = v4[i];
#pragma unroll
            for (int e = 0; e < 4; ++e) a += (double)wv[e] * (double)xv[e];
        }
    } else {
#pragma unroll 4
        for (int c = q; c < n; c += 4) a += (double)wr[c] * (double)v[c];
    }
    const double a1 = __shfl_down(a, 1, 4), a2 = __shfl_down(a, 2, 4), a3 = __shfl_down(a, 3, 4);
    return (a + a1) + (a2 + a3);
}

// One workgroup per (clip, segment): ctx = mean_T' + sum_seg / seg_len, then
// h = relu(W1 ctx + b1), gate = sigmoid(W2 h + b2).
__global__ __launch_bounds__(256) void cam_context_kernel(const float* __restrict__ sums, int nseg, int T, int C,
                                                          int seg, const float* __restrict__ w1,
                                                          const float* __restrict__ b1, int H1,
                                                          const float* __restrict__ w2,
                                                          const float* __restrict__ b2, int G,
                                                          float* __restrict__ gate) {
    extern __shared__ float sm[];
    float* ctx = sm;          // [C]
    float* hid = sm + ((C + 3) & ~3);   // [H1], 16-byte aligned
    const int b = blockIdx.x, s = blockIdx.y;
    const float* sb = sums + (size_t)b * nseg * C;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
        double tot = 0.0;
        for (int q = 0; q < nseg; ++q) tot += (double)sb[(size_t)q * C + c];
        ctx[c] = (float)(tot / T) + (float)((double)sb[(size_t)s * C + c] / seg);
    }
    __syncthreads();
    // each output's dot product split over 4 lanes (dot4)
    const int q = threadIdx.x & 3;
    for (int o = threadIdx.x >> 2; o < H1; o += blockDim.x >> 2) {
        const double a = dot4(w1 + (size_t)o * C, ctx, C, q);
        if (q == 0) hid[o] = fmaxf((float)a + (b1 ? b1[o] : 0.0f), 0.0f);
    }
    __syncthreads();
    for (int o = threadIdx.x >> 2; o < G; o += blockDim.x >> 2) {
        const double a = dot4(w2 + (size_t)o * H1, hid, H1, q);
        if (q == 0) gate[((size_t)b * nseg + s) * G + o] = 1.0f / (1.0f + expf(-((float)a + (b2 ? b2[o] : 0.0f))));
    }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace vdk

using namespace vdk;

extern "C" int vdk_bn_act(const void* d_x, int x_stride, long rows, int C, const float* d_scale,
                          const float* d_shift, int act, void* d_y, int y_stride, void* stream) {
    return guarded([&] {
        require(d_x && d_scale && d_shift && d_y, "bn_act: NULL device pointer");
        require(rows > 0 && C > 0 && C % 8 == 0 && x_stride >= C && y_stride >= C && x_stride % 8 == 0 &&
                    y_stride % 8 == 0, "bn_act: bad shape");
        require(act == VDK_ACT_NONE || act == VDK_ACT_RELU, "bn_act: unknown activation");
        require(al16(d_x) && al16(d_y) && al16(d_scale) && al16(d_shift), "bn_act: pointers must be 16-byte aligned");
        const long n = rows * (C / 8);
        hipLaunchKernelGGL(bn_act_kernel, dim3(cdiv(n, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                           static_cast<const half_t*>(d_x), x_stride, rows, C, d_scale, d_shift, act,
                           static_cast<half_t*>(d_y), y_stride);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_segment_sums(const void* d_x, int x_stride, int batch, int T, int C, int seg, float* d_out,
                                void* stream) {
    return guarded([&] {
        require(d_x && d_out, "segment_sums: NULL device pointer");
        require(batch > 0 && T > 0 && C > 0 && seg > 0 && x_stride >= C, "segment_sums: bad shape");
        const int nseg = (T + seg - 1) / seg;
        hipLaunchKernelGGL(segment_sums_kernel, dim3(batch, nseg, cdiv(C, 64)), dim3(64 * kSegParts), 0,
                           static_cast<hipStream_t>(stream), static_cast<const half_t*>(d_x), x_stride, T, C, seg,
                           d_out);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_cam_context(const float* d_sums, int batch, int T, int C, int seg, const float* d_w1,
                               const float* d_b1, int H1, const float* d_w2, const float* d_b2, int G,
                               float* d_gate, void* stream) {
    return guarded([&] {
        require(d_sums && d_w1 && d_w2 && d_gate, "cam_context: NULL device pointer");
        require(batch > 0 && T > 0 && C > 0 && seg > 0 && H1 > 0 && G > 0 && C + H1 <= 16384,
                "cam_context: bad shape");
        require(al16(d_w1) && al16(d_w2), "cam_context: weights must be 16-byte aligned");
        const int nseg = (T + seg - 1) / seg;
        hipLaunchKernelGGL(cam_context_kernel, dim3(batch, nseg), dim3(256), sizeof(float) * (((C + 3) & ~3) + H1),
                           static_cast<hipStream_t>(stream), d_sums, nseg, T, C, seg, d_w1, d_b1, H1, d_w2, d_b2,
                           G, d_gate);
        VDK_HIP(hipGetLastError());
    });
}

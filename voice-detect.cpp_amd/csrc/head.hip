// head.hip - statistics pooling, embedding FC and L2 normalisation on gfx950.
//
// These are bandwidth-bound reductions: TSTP reads the last feature map twice
// (16-byte loads of 8 channels, 256 channels x 8 time partitions per
// workgroup); the FC is a split-K tiled dot product with a fixed-order
// reduction, which for the embedding also does the L2 normalisation (one
// workgroup per clip).  Sums are accumulated in f64 like the reference's ggml
// reductions and host L2 (src/encoder_resnet.cpp:140-183).
#include <cmath>
#include <mutex>
#include <string>

#include "common.hpp"
#include "vdk.h"

namespace vdk {
namespace {

__device__ __forceinline__ double wave_sum_d(double v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// TSTP (src/encoder_resnet.cpp:140-157): mean over time, var * N/(N-1), sqrt(var + eps).
// x [B][H][W][xs] f16; split (x_lo > 0): value = x + x[.. + x_lo].
__device__ __forceinline__ float tstp_val(const half_t* p, int x_lo) {
    return x_lo ? (float)p[0] + (float)p[x_lo] : (float)p[0];
}

// A workgroup covers 64 channels of one (clip, freq row): thread (p, c)
// = (tid / 64, tid % 64) sums time steps p, p + 4, ... of channel c in f64,
// and the four partial sums are added in a fixed order (so the result does
// not depend on scheduling); the same for the squared deviations from the
// f32 mean.
__global__ __launch_bounds__(256) void tstp_kernel(const half_t* __restrict__ x, int xs, int x_lo, int H, int W,
                                                   int C, float eps, float* __restrict__ pooled) {
#pragma clang fp contract(off)
    __shared__ double part[4][64];
    const int tx = threadIdx.x & 63, tp = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + tx, h = blockIdx.y, b = blockIdx.z;
    const bool ok = c < C;
    const size_t CH = (size_t)C * H;
    const half_t* row = x + ((size_t)b * H + h) * W * xs + (ok ? c : 0);
    double s = 0.0;
    if (ok) {
#pragma unroll 4
        for (int t = tp; t < W; t += 4) s += (double)tstp_val(row + (size_t)t * xs, x_lo);
    }
    part[tp][tx] = s;
    __syncthreads();
    const float mean = (float)(((part[0][tx] + part[1][tx]) + (part[2][tx] + part[3][tx])) / W);
    __syncthreads();
    double s2 = 0.0;
    if (ok) {
#pragma unroll 4
        for (int t = tp; t < W; t += 4) {
            const float d = tstp_val(row + (size_t)t * xs, x_lo) - mean;
            s2 += (double)(d * d);
        }
    }
    part[tp][tx] = s2;
    __syncthreads();
    if (tp == 0 && ok) {
        float var = (float)(((part[0][tx] + part[1][tx]) + (part[2][tx] + part[3][tx])) / W);
        if (W > 1) var = var * ((float)W / (float)(W - 1));
        float* out = pooled + (size_t)b * 2 * CH;
        out[(size_t)c * H + h] = mean;
        out[CH + (size_t)c * H + h] = sqrtf(var + eps);
    }
}

// TSTP over 8-channel vectors: a workgroup covers 64 channels of one (clip,
// freq row); thread (p, g) = (tid / 8, tid % 8) loads channels 8 g .. 8 g + 7
// (one 16-byte vector, two for split inputs) at time steps p, p + 32, ...
// and keeps their f64 partial sums.  One thread per channel then adds the 32
// partitions in a fixed order (so the result does not depend on scheduling)
// and publishes the f32 mean through LDS; the squared deviations from it go
// the same way.  A wave's load covers 8 time steps x 128 bytes, and the
// loops per thread are short (CAM++'s 499 frames: 16 steps), so many loads
// are in flight.
__global__ __launch_bounds__(256) void tstp64_kernel(const half_t* __restrict__ x, int xs, int x_lo, int H, int W,
                                                     int C, float eps, float* __restrict__ pooled) {
#pragma clang fp contract(off)
    constexpr int NP = 32;
    __shared__ double part[NP][65];
    __shared__ float smean[64];
    const int tid = threadIdx.x, g = tid & 7, tp = tid >> 3;
    const int c0 = blockIdx.x * 64 + g * 8, h = blockIdx.y, b = blockIdx.z;
    const bool ok = c0 < C;
    const size_t CH = (size_t)C * H;
    const half_t* row = x + ((size_t)b * H + h) * W * xs + (ok ? c0 : 0);
    auto load8 = [&](int t, float* v) {
        const half8 hv = *reinterpret_cast<const half8*>(row + (size_t)t * xs);
        if (x_lo) {
            const half8 lv = *reinterpret_cast<const half8*>(row + (size_t)t * xs + x_lo);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (float)hv[e] + (float)lv[e];
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (float)hv[e];
        }
    };
    double s[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) s[e] = 0.0;
    if (ok)
#pragma unroll 4
        for (int t = tp; t < W; t += NP) {
            float v[8];
            load8(t, v);
#pragma unroll
            for (int e = 0; e < 8; ++e) s[e] += (double)v[e];
        }
#pragma unroll
    for (int e = 0; e < 8; ++e) part[tp][g * 8 + e] = s[e];
    __syncthreads();
    if (tid < 64) {
        double m = 0.0;
#pragma unroll 8
        for (int q = 0; q < NP; ++q) m += part[q][tid];
        smean[tid] = (float)(m / W);
    }
    __syncthreads();
    float mean[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        mean[e] = smean[g * 8 + e];
        s[e] = 0.0;
    }
    if (ok)
#pragma unroll 4
        for (int t = tp; t < W; t += NP) {
            float v[8];
            load8(t, v);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float d = v[e] - mean[e];
                s[e] += (double)(d * d);
            }
        }
#pragma unroll
    for (int e = 0; e < 8; ++e) part[tp][g * 8 + e] = s[e];
    __syncthreads();
    const int c = blockIdx.x * 64 + tid;
    if (tid < 64 && c < C) {
        double q2 = 0.0;
#pragma unroll 8
        for (int q = 0; q < NP; ++q) q2 += part[q][tid];
        float var = (float)(q2 / W);
        if (W > 1) var = var * ((float)W / (float)(W - 1));
        float* out = pooled + (size_t)b * 2 * CH;
        out[(size_t)c * H + h] = smean[tid];
        out[CH + (size_t)c * H + h] = sqrtf(var + eps);
    }
}

// FC, split over the input dimension: workgroup (o-tile, b-tile, split s)
// computes a (16 RB) x (16 RB) block of partial dot products over its slice
// of the input, RB x RB per thread from k-major LDS tiles (RB = 4: one
// 16-byte read of 4 batch rows and one of 4 outputs per 16 FMAs; RB = 1 for
// small products, where 64-wide tiles would leave too few workgroups); every
// output accumulates its slice in k order, so the result does not depend on
// the tiling.  linear_reduce_kernel adds the slices in a fixed order (bitwise
// reproducible) with bias and mean_vec.
constexpr int kLinK = 64, kLinSlice = 128;

template <int RB>
__global__ __launch_bounds__(256) void linear_partial_kernel(const float* __restrict__ x, int B, int in_dim,
                                                             const float* __restrict__ w, int out_dim, int slice,
                                                             int vec4, float* __restrict__ part) {
    constexpr int TILE = 16 * RB, NQ = TILE * (kLinK / 4) / 256;   // 4-k groups per thread per operand
    __shared__ __attribute__((aligned(16))) float sx[kLinK][TILE + 4];   // [k][batch row]
    __shared__ __attribute__((aligned(16))) float sw[kLinK][TILE + 4];   // [k][output]
    const int o0 = blockIdx.x * TILE, b0 = blockIdx.y * TILE, s = blockIdx.z;
    const int k_begin = s * slice, k_end = min(in_dim, k_begin + slice);
    const int tid = threadIdx.x;
    const int tb = tid >> 4, to = tid & 15;   // batch rows b0 + RB tb .., outputs o0 + RB to ..
    float acc[RB][RB];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int j = 0; j < RB; ++j) acc[i][j] = 0.0f;
    for (int k0 = k_begin; k0 < k_end; k0 += kLinK) {
        // TILE rows x 64 k of each operand in groups of 4 consecutive k
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int e = tid + q * 256, r = e >> 4, c = (e & 15) * 4, k = k0 + c;
            float xv[4] = {0.0f, 0.0f, 0.0f, 0.0f}, wv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            const float* xp = x + (size_t)(b0 + r) * in_dim + k;
            const float* wp = w + (size_t)(o0 + r) * in_dim + k;
            const bool xr = b0 + r < B, wr = o0 + r < out_dim;
            if (vec4 && k + 3 < k_end) {
                if (xr) { const float4v v = *reinterpret_cast<const float4v*>(xp); xv[0] = v[0]; xv[1] = v[1]; xv[2] = v[2]; xv[3] = v[3]; }
                if (wr) { const float4v v = *reinterpret_cast<const float4v*>(wp); wv[0] = v[0]; wv[1] = v[1]; wv[2] = v[2]; wv[3] = v[3]; }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (xr && k + i < k_end) xv[i] = xp[i];
                    if (wr && k + i < k_end) wv[i] = wp[i];
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sx[c + i][r] = xv[i];
                sw[c + i][r] = wv[i];
            }
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < kLinK; ++kk) {
            if constexpr (RB == 4) {
                const float4v xb = *reinterpret_cast<const float4v*>(&sx[kk][tb * 4]);
                const float4v wo = *reinterpret_cast<const float4v*>(&sw[kk][to * 4]);
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] += xb[i] * wo[j];
            } else {
                acc[0][0] += sx[kk][tb] * sw[kk][to];
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < RB; ++i) {
        const int b = b0 + tb * RB + i;
        if (b >= B) continue;
#pragma unroll
        for (int j = 0; j < RB; ++j) {
            const int o = o0 + to * RB + j;
            if (o < out_dim) part[((size_t)s * B + b) * out_dim + o] = acc[i][j];
        }
    }
}

__global__ __launch_bounds__(256) void linear_reduce_kernel(const float* __restrict__ part, int nsplit, int B,
                                                            int out_dim, const float* __restrict__ bias,
                                                            const float* __restrict__ mv, int act,
                                                            float* __restrict__ y) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)B * out_dim) return;
    const int o = (int)(i % out_dim);
    const size_t stride = (size_t)B * out_dim;
    // fixed summation order, 16 loads in flight per step
    double s = 0.0;
    int k = 0;
    for (; k + 16 <= nsplit; k += 16) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = part[(size_t)(k + j) * stride + i];
#pragma unroll
        for (int j = 0; j < 16; ++j) s += (double)v[j];
    }
    for (; k < nsplit; ++k) s += (double)part[(size_t)k * stride + i];
    float r = (float)s;
    if (bias) r += bias[o];
    if (mv) r -= mv[o];
    if (act == VDK_ACT_RELU) r = fmaxf(r, 0.0f);
    else if (act == VDK_ACT_SIGMOID) r = 1.0f / (1.0f + expf(-r));
    else if (act == VDK_ACT_TANH) r = tanhf(r);
    y[i] = r;
}

// The reduce of the embedding FC with the L2 normalisation: one workgroup per
// clip row, the pre-norm row to `pre`, then y = row / ||row|| (f64 norm; a
// zero row copied unchanged) as l2norm_kernel computes it.
__global__ __launch_bounds__(256) void linear_reduce_l2_kernel(const float* __restrict__ part, int nsplit, int B,
                                                               int out_dim, const float* __restrict__ bias,
                                                               const float* __restrict__ mv,
                                                               float* __restrict__ pre, float* __restrict__ y) {
    __shared__ double red[4];
    const int b = blockIdx.x;
    const size_t stride = (size_t)B * out_dim;
    double sq = 0.0;
    for (int o = threadIdx.x; o < out_dim; o += 256) {
        const size_t i = (size_t)b * out_dim + o;
        double s = 0.0;
        int k = 0;
        for (; k + 16 <= nsplit; k += 16) {   // 16 loads in flight, the sums in order
            float v[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = part[(size_t)(k + j) * stride + i];
#pragma unroll
            for (int j = 0; j < 16; ++j) s += (double)v[j];
        }
        for (; k < nsplit; ++k) s += (double)part[(size_t)k * stride + i];
        float r = (float)s;
        if (bias) r += bias[o];
        if (mv) r -= mv[o];
        pre[i] = r;
        sq += (double)r * (double)r;
    }
    sq = wave_sum_d(sq);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
    __syncthreads();
    const double norm = sqrt((red[0] + red[1]) + (red[2] + red[3]));
    for (int o = threadIdx.x; o < out_dim; o += 256) {
        const size_t i = (size_t)b * out_dim + o;
        const float v = pre[i];   // this thread's own write above
        y[i] = norm > 0.0 ? (float)((double)v / norm) : v;
    }
}

int linear_splits(int in_dim) {
    const int want = (in_dim + kLinSlice - 1) / kLinSlice;   // ~128 inputs per slice
    return want < 1 ? 1 : (want > 64 ? 64 : want);
}

// In-place L2 normalisation, one wavefront per clip (src/encoder_resnet.cpp:177-183).
// y = x / ||x|| per row (y may be x); a zero row is copied unchanged.
__global__ __launch_bounds__(64) void l2norm_kernel(const float* x, int dim, float* y) {
    const float* v = x + (size_t)blockIdx.x * dim;
    float* o = y + (size_t)blockIdx.x * dim;
    double s = 0.0;
    for (int i = threadIdx.x; i < dim; i += 64) s += (double)v[i] * (double)v[i];
    s = wave_sum_d(s);
    const double norm = sqrt(s);
    for (int i = threadIdx.x; i < dim; i += 64) o[i] = norm > 0.0 ? (float)((double)v[i] / norm) : v[i];
}

}  // namespace
}  // namespace vdk

namespace vdk {
namespace {
// One vector store of v: a dispatch that counter-collection runs can find by
// name, bracketing a labelled launch (Model::set_profiling_markers).
__global__ __launch_bounds__(64) void profile_marker_kernel(int* p, int v) {
    if (threadIdx.x == 0) p[0] = v;
}
}  // namespace

void launch_profile_marker(int* p, int v, hipStream_t s) {
    hipLaunchKernelGGL(profile_marker_kernel, dim3(1), dim3(64), 0, s, p, v);
}
}  // namespace vdk

using namespace vdk;

extern "C" int vdk_tstp_ex(const void* d_x, int x_stride, int x_lo, int batch, int H, int W, int C, float eps,
                           float* d_pooled, void* stream) {
    return guarded([&] {
        require(d_x && d_pooled, "tstp: NULL device pointer");
        require(batch > 0 && H > 0 && W > 0 && C > 0, "tstp: empty input");
        const int xs = x_stride ? x_stride : C;
        require(xs >= C && (x_lo == 0 || (x_lo >= C && x_lo + C <= xs)), "tstp: bad pixel stride / lo offset");
        const bool vec = C % 8 == 0 && xs % 8 == 0 && x_lo % 8 == 0 && (reinterpret_cast<uintptr_t>(d_x) & 15) == 0;
        if (vec)
            hipLaunchKernelGGL(tstp64_kernel, dim3(cdiv(C, 64), H, batch), dim3(256), 0,
                               static_cast<hipStream_t>(stream), static_cast<const half_t*>(d_x), xs, x_lo, H, W, C,
                               eps, d_pooled);
        else
            hipLaunchKernelGGL(tstp_kernel, dim3(cdiv(C, 64), H, batch), dim3(256), 0,
                               static_cast<hipStream_t>(stream), static_cast<const half_t*>(d_x), xs, x_lo, H, W, C,
                               eps, d_pooled);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_tstp(const void* d_x, int batch, int H, int W, int C, float eps, float* d_pooled,
                        void* stream) {
    return vdk_tstp_ex(d_x, 0, 0, batch, H, W, C, eps, d_pooled, stream);
}

extern "C" size_t vdk_linear_workspace_size(int batch, int in_dim, int out_dim) {
    if (batch <= 0 || in_dim <= 0 || out_dim <= 0) return 0;
    return sizeof(float) * (size_t)linear_splits(in_dim) * batch * out_dim;
}

namespace vdk {
namespace {

void linear_check(const float* d_x, int batch, int in_dim, const float* d_w, int out_dim, int act, float* d_y) {
    require(d_x && d_w && d_y, "linear: NULL device pointer");
    require(batch > 0 && in_dim > 0 && out_dim > 0, "linear: empty shape");
    require(act == VDK_ACT_NONE || act == VDK_ACT_RELU || act == VDK_ACT_SIGMOID || act == VDK_ACT_TANH,
            "linear: unknown activation");
}

// The two launches of the split-K FC; `part` holds nsplit x batch x out_dim
// floats, every one of which the partial kernel writes before the reduce
// reads it (nothing needs clearing between calls).
void linear_launch(const float* d_x, int batch, int in_dim, const float* d_w, const float* d_bias,
                   const float* d_mean_vec, int out_dim, int act, float* d_y, float* part, hipStream_t s,
                   float* d_l2 = nullptr) {
    const int ns = linear_splits(in_dim);
    const int slice = ((in_dim + ns - 1) / ns + kLinK - 1) / kLinK * kLinK;
    const int nsplit = (in_dim + slice - 1) / slice;
    const int vec4 = in_dim % 4 == 0 && (reinterpret_cast<uintptr_t>(d_x) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(d_w) & 15) == 0;
    if ((long)cdiv(out_dim, 64) * cdiv(batch, 64) * nsplit >= 64)
        hipLaunchKernelGGL(linear_partial_kernel<4>, dim3(cdiv(out_dim, 64), cdiv(batch, 64), nsplit), dim3(256),
                           0, s, d_x, batch, in_dim, d_w, out_dim, slice, vec4, part);
    else
        hipLaunchKernelGGL(linear_partial_kernel<1>, dim3(cdiv(out_dim, 16), cdiv(batch, 16), nsplit), dim3(256),
                           0, s, d_x, batch, in_dim, d_w, out_dim, slice, vec4, part);
    VDK_HIP(hipGetLastError());
    if (d_l2)
        hipLaunchKernelGGL(linear_reduce_l2_kernel, dim3(batch), dim3(256), 0, s, part, nsplit, batch, out_dim,
                           d_bias, d_mean_vec, d_y, d_l2);
    else
        hipLaunchKernelGGL(linear_reduce_kernel, dim3(cdiv((long)batch * out_dim, 256)), dim3(256), 0, s, part,
                           nsplit, batch, out_dim, d_bias, d_mean_vec, act, d_y);
    VDK_HIP(hipGetLastError());
}

}  // namespace
}  // namespace vdk

extern "C" int vdk_linear_ex(const float* d_x, int batch, int in_dim, const float* d_w, const float* d_bias,
                             const float* d_mean_vec, int out_dim, int act, float* d_y, void* d_work,
                             size_t work_bytes, void* stream) {
    return guarded([&] {
        linear_check(d_x, batch, in_dim, d_w, out_dim, act, d_y);
        require(d_work != nullptr, "linear: NULL device pointer");
        require(work_bytes >= vdk_linear_workspace_size(batch, in_dim, out_dim),
                "linear: workspace smaller than vdk_linear_workspace_size()");
        linear_launch(d_x, batch, in_dim, d_w, d_bias, d_mean_vec, out_dim, act, d_y, static_cast<float*>(d_work),
                      static_cast<hipStream_t>(stream));
    });
}

// Split-K partials of vdk_linear_ex_noalloc: a fixed device array, one copy
// per GPU, held until the process ends.  Host code never passes `scratch`
// itself to a kernel (on the host it names a stand-in, not device memory):
// its device address is looked up once per device with that device current
// and kept in g_scratch_dev.
static __device__ __align__(256) float scratch[VDK_LINEAR_SCRATCH_BYTES / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_dev[kMaxDevices] = {};

float* scratch_on_current_device() {
    int dev = -1;
    VDK_HIP(hipGetDevice(&dev));
    require(dev >= 0 && dev < kMaxDevices, "linear_noalloc: device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        VDK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        require(p != nullptr, "linear_noalloc: no device address for the scratch array");
        g_scratch_dev[dev] = static_cast<float*>(p);
    }
    return g_scratch_dev[dev];
}
}  // namespace

extern "C" int vdk_linear_ex_noalloc(const float* d_x, int batch, int in_dim, const float* d_w,
                                     const float* d_bias, const float* d_mean_vec, int out_dim, int act,
                                     float* d_y, void* stream) {
    return guarded([&] {
        linear_check(d_x, batch, in_dim, d_w, out_dim, act, d_y);
        const size_t need = vdk_linear_workspace_size(batch, in_dim, out_dim);
        require(need <= VDK_LINEAR_SCRATCH_BYTES,
                "linear_noalloc: batch * out_dim * splits needs " + std::to_string(need) +
                    " bytes of scratch, above the fixed " + std::to_string((size_t)VDK_LINEAR_SCRATCH_BYTES) +
                    " (use vdk_linear_ex with a workspace)");
        linear_launch(d_x, batch, in_dim, d_w, d_bias, d_mean_vec, out_dim, act, d_y, scratch_on_current_device(),
                      static_cast<hipStream_t>(stream));
    });
}

extern "C" int vdk_linear(const float* d_x, int batch, int in_dim, const float* d_w, const float* d_bias,
                          const float* d_mean_vec, int out_dim, float* d_y, void* d_work, size_t work_bytes,
                          void* stream) {
    return vdk_linear_ex(d_x, batch, in_dim, d_w, d_bias, d_mean_vec, out_dim, 0, d_y, d_work, work_bytes, stream);
}

extern "C" int vdk_linear_l2_ex(const float* d_x, int batch, int in_dim, const float* d_w, const float* d_bias,
                                const float* d_mean_vec, int out_dim, float* d_pre, float* d_y, void* d_work,
                                size_t work_bytes, void* stream) {
    return guarded([&] {
        linear_check(d_x, batch, in_dim, d_w, out_dim, VDK_ACT_NONE, d_pre);
        require(d_y != nullptr && d_work != nullptr, "linear_l2: NULL device pointer");
        require(work_bytes >= vdk_linear_workspace_size(batch, in_dim, out_dim),
                "linear_l2: workspace smaller than vdk_linear_workspace_size()");
        const uintptr_t pa = reinterpret_cast<uintptr_t>(d_pre), ya = reinterpret_cast<uintptr_t>(d_y);
        const size_t bytes = sizeof(float) * (size_t)batch * out_dim;
        require(pa + bytes <= ya || ya + bytes <= pa, "linear_l2: pre and y overlap");
        linear_launch(d_x, batch, in_dim, d_w, d_bias, d_mean_vec, out_dim, VDK_ACT_NONE, d_pre,
                      static_cast<float*>(d_work), static_cast<hipStream_t>(stream), d_y);
    });
}

extern "C" int vdk_l2norm(float* d_x, int batch, int dim, void* stream) {
    return vdk_l2norm_to(d_x, batch, dim, d_x, stream);
}

extern "C" int vdk_l2norm_to(const float* d_x, int batch, int dim, float* d_y, void* stream) {
    return guarded([&] {
        require(d_x && d_y, "l2norm: NULL device pointer");
        require(batch > 0 && dim > 0, "l2norm: empty shape");
        const uintptr_t xa = reinterpret_cast<uintptr_t>(d_x), ya = reinterpret_cast<uintptr_t>(d_y);
        const size_t bytes = sizeof(float) * (size_t)batch * dim;
        require(xa == ya || xa + bytes <= ya || ya + bytes <= xa, "l2norm: x and y overlap without being equal");
        hipLaunchKernelGGL(l2norm_kernel, dim3(batch), dim3(64), 0, static_cast<hipStream_t>(stream), d_x, dim, d_y);
        VDK_HIP(hipGetLastError());
    });
}

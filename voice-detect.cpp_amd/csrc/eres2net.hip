// eres2net.hip - the attentional feature fusion combine of ERes2Net on gfx950.
//
// AFF (src/encoder_eres2net.cpp:91-101): z = local_att(cat(x, ds)) runs as two
// 1x1 convs (SiLU, then tanh in the second conv's epilogue); this kernel forms
//   y = (x + ds) + t * (x - ds),   t = tanh(z)
// over NHWC f16 maps given as rows of channel slices, optionally split-f16
// (value = hi + lo, lo a fixed number of elements after hi).
#include "common.hpp"
#include "vdk.h"

namespace vdk {
namespace {

// 8 values at p (+ lo half at p + lo when split) as f32
__device__ __forceinline__ void load8(const half_t* p, int lo, int split, float* v) {
    const half8 h = *reinterpret_cast<const half8*>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (float)h[e];
    if (split) {
        const half8 l = *reinterpret_cast<const half8*>(p + lo);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] += (float)l[e];
    }
}

__global__ __launch_bounds__(256) void aff_combine_kernel(const half_t* __restrict__ t, int ts, int t_lo,
                                                          const half_t* __restrict__ x, int xs, int x_lo,
                                                          const half_t* __restrict__ ds, int dss, int ds_lo,
                                                          long rows, int C, int split, half_t* __restrict__ y,
                                                          int ys, int y_lo) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;   // one 8-channel chunk
    const int C8 = C / 8;
    if (i >= rows * C8) return;
    const int c = (int)(i % C8) * 8;
    const long r = i / C8;
    float tv[8], xv[8], dv[8];
    load8(t + r * ts + c, t_lo, split, tv);
    load8(x + r * xs + c, x_lo, split, xv);
    load8(ds + r * dss + c, ds_lo, split, dv);
    half8 o, ol;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float v = (xv[e] + dv[e]) + tv[e] * (xv[e] - dv[e]);
        o[e] = (half_t)v;
        ol[e] = (half_t)(v - (float)o[e]);
    }
    *reinterpret_cast<half8*>(y + r * ys + c) = o;
    if (split) *reinterpret_cast<half8*>(y + r * ys + y_lo + c) = ol;
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace vdk

using namespace vdk;

extern "C" int vdk_aff_combine(const void* d_t, int t_stride, int t_lo, const void* d_x, int x_stride, int x_lo,
                               const void* d_ds, int ds_stride, int ds_lo, long rows, int C, int split, void* d_y,
                               int y_stride, int y_lo, void* stream) {
    return guarded([&] {
        require(d_t && d_x && d_ds && d_y, "aff_combine: NULL device pointer");
        require(rows > 0 && C > 0 && C % 8 == 0 && t_stride >= C && x_stride >= C && ds_stride >= C &&
                    y_stride >= C, "aff_combine: bad shape");
        require(t_stride % 8 == 0 && x_stride % 8 == 0 && ds_stride % 8 == 0 && y_stride % 8 == 0 && al16(d_t) &&
                    al16(d_x) && al16(d_ds) && al16(d_y), "aff_combine: strides/pointers must be 8-channel aligned");
        require(!split || (t_lo >= C && x_lo >= C && ds_lo >= C && y_lo >= C && t_lo % 8 == 0 && x_lo % 8 == 0 &&
                           ds_lo % 8 == 0 && y_lo % 8 == 0), "aff_combine: split lo offsets must follow the channels");
        const long n = rows * (C / 8);
        hipLaunchKernelGGL(aff_combine_kernel, dim3(cdiv(n, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                           static_cast<const half_t*>(d_t), t_stride, t_lo, static_cast<const half_t*>(d_x), x_stride,
                           x_lo, static_cast<const half_t*>(d_ds), ds_stride, ds_lo, rows, C, split ? 1 : 0,
                           static_cast<half_t*>(d_y), y_stride, y_lo);
        VDK_HIP(hipGetLastError());
    });
}

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

// One dense layer's CAM layer in one launch (src/encoder_campplus.cpp:159-182,
// 260-268): workgroup (clip b, segment s) of 256 threads
//  0. DMAs the segment's input frames (with dil frames of halo each side,
//     zeros outside the clip) and the linear_local weights into LDS (rows
//     padded by 16 bytes), in flight during steps 1-2;
//  1. sums x [b][.][C] over all T frames and over segment s (f64; thread
//     (frame lane, 8-channel chunk), the frame lanes combined in a fixed order),
//     ctx = sum_all / T + sum_seg / seg;
//  2. gate = sigmoid(w2 relu(w1 ctx + b1) + b2) (f64 dot products, dot4);
//  3. y = (linear_local(x) + bias) * gate for the segment's frames: the k = 3
//     conv with dilation dil and zero padding as one 32 x 32 MFMA block per
//     wave and 32 frames (K = 3 * C in tap-major, channel-minor order, the
//     implicit-GEMM kernels' order), operands from LDS.
// The segment's G = 32 outputs go to y [b][t][y_stride] f16.
constexpr int kLocalOC = 32;

struct CamLocalLds {
    int xrow, wrow, nrow, xins, wins, part_bytes, x_off, w_off, ctx_off, total;
};
__host__ __device__ inline CamLocalLds cam_local_lds(int C, int seg, int dil, int H1) {
    CamLocalLds L;
    L.xrow = C * 2 + 16;                         // frame row: C f16 + 16 bytes
    L.wrow = 3 * C * 2 + 16;                     // weight row (output channel): 3*C f16 + 16 bytes
    L.nrow = seg + 2 * dil;
    L.xins = (L.nrow * (L.xrow / 16) + 63) / 64;   // DMA instructions (64 slots of 16 bytes each)
    L.wins = (kLocalOC * (L.wrow / 16) + 63) / 64;
    L.part_bytes = 8 * 2 * (256 / (C / 8)) * C;
    L.x_off = 0;
    L.w_off = L.xins * 1024;                       // the f64 partial sums follow the weights
    L.ctx_off = L.w_off + L.wins * 1024 + L.part_bytes;
    L.total = L.ctx_off + 4 * (((C + 3) & ~3) + ((H1 + 3) & ~3) + 32);
    return L;
}

// CT > 0: the channel count fixed at compile time (the K loop of step 3
// unrolls, so its LDS reads run ahead of the MFMAs); 0: C at run time.
template <int CT>
__global__ __launch_bounds__(256) void cam_local_kernel(const half_t* __restrict__ x, int xs, int T, int Cr, int seg,
                                                        int dil, const float* __restrict__ w1,
                                                        const float* __restrict__ b1, int H1,
                                                        const float* __restrict__ w2, const float* __restrict__ b2,
                                                        const half_t* __restrict__ wl, const float* __restrict__ bl,
                                                        half_t* __restrict__ y, int ys,
                                                        const double* __restrict__ segsum,
                                                        double* __restrict__ zero_next) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    const int C = CT > 0 ? CT : Cr;
    const CamLocalLds Lo = cam_local_lds(C, seg, dil, H1);
    uint8_t* const sx = smem + Lo.x_off;
    uint8_t* const sw = smem + Lo.w_off;
    double* part = reinterpret_cast<double*>(smem + Lo.w_off + Lo.wins * 1024);   // [2][256 / C8][C]
    const int C8 = C >> 3, NFL = 256 / C8;
    float* ctx = reinterpret_cast<float*>(smem + Lo.ctx_off);   // [C]
    float* hid = ctx + ((C + 3) & ~3);                          // [H1]
    float* gate = hid + ((H1 + 3) & ~3);                        // [32]
    const int b = blockIdx.x, s = blockIdx.y, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int t0 = s * seg, t1 = min(T, t0 + seg);
    const half_t* xb = x + (size_t)b * T * xs;
    {   // 0. the segment's frames t0 - dil .. t1 + dil and the weights into LDS
        const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)xb, 0, (int)(((size_t)(T - 1) * xs + C) * 2), 0x00020000);
        const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)wl, 0, (int)((size_t)kLocalOC * 3 * C * 2), 0x00020000);
        const int xspr = Lo.xrow / 16, wspr = Lo.wrow / 16;
        for (int ins = wave; ins < Lo.xins; ins += 4) {
            const int sl = ins * 64 + lane, r = sl / xspr, ch = sl - r * xspr;
            const int tf = t0 - dil + r;
            const uint32_t off = (r < Lo.nrow && ch < C / 8 && tf >= 0 && tf < T)
                                     ? (uint32_t)(((size_t)tf * xs + ch * 8) * 2) : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(sx + ins * 1024), 16, off, 0, 0, 0);
        }
        for (int ins = wave; ins < Lo.wins; ins += 4) {
            const int sl = ins * 64 + lane, r = sl / wspr, ch = sl - r * wspr;
            const uint32_t off = (r < kLocalOC && ch < 3 * C / 8) ? (uint32_t)((r * 3 * C + ch * 8) * 2) : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void*)(sw + ins * 1024), 16, off, 0, 0, 0);
        }
    }
    if (segsum) {   // 1. the segment sums came with the input: ctx from them
        const int nseg = (T + seg - 1) / seg;
        const double* sb = segsum + (size_t)b * nseg * C;
        for (int c = tid; c < C; c += 256) {
            double a = 0.0;
            for (int q = 0; q < nseg; ++q) a += sb[(size_t)q * C + c];
            ctx[c] = (float)(a / T) + (float)(sb[(size_t)s * C + c] / seg);
            if (zero_next) zero_next[((size_t)b * nseg + s) * C + c] = 0.0;
        }
    } else {   // 1. sums
        const int cc = tid % C8, fl = tid / C8;
        double tot[8], sg[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) tot[e] = sg[e] = 0.0;
        if (fl < NFL) {
            // kSumU frames per trip, their loads issued together
            constexpr int kSumU = 16;
            for (int t = fl; t < T; t += NFL * kSumU) {
                half8 v[kSumU];
#pragma unroll
                for (int u = 0; u < kSumU; ++u) {
                    const int tu = t + u * NFL;
                    if (tu < T) {
                        v[u] = *reinterpret_cast<const half8*>(xb + (size_t)tu * xs + cc * 8);
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; ++e) v[u][e] = (half_t)0.0f;
                    }
                }
#pragma unroll
                for (int u = 0; u < kSumU; ++u) {
                    const int tu = t + u * NFL;
                    const bool in = tu >= t0 && tu < t1;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const double f = (double)(float)v[u][e];
                        tot[e] += f;
                        if (in) sg[e] += f;
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                part[(size_t)fl * C + cc * 8 + e] = tot[e];
                part[(size_t)(NFL + fl) * C + cc * 8 + e] = sg[e];
            }
        }
        __syncthreads();
        for (int c = tid; c < C; c += 256) {
            double a = 0.0, g = 0.0;
            for (int q = 0; q < NFL; ++q) {
                a += part[(size_t)q * C + c];
                g += part[(size_t)(NFL + q) * C + c];
            }
            ctx[c] = (float)(a / T) + (float)(g / seg);
        }
    }
    __syncthreads();
    {   // 2. the mask MLP
        const int q = tid & 3;
        for (int o = tid >> 2; o < H1; o += 64) {
            const double a = dot4(w1 + (size_t)o * C, ctx, C, q);
            if (q == 0) hid[o] = fmaxf((float)a + (b1 ? b1[o] : 0.0f), 0.0f);
        }
        __syncthreads();
        for (int o = tid >> 2; o < kLocalOC; o += 64) {
            const double a = dot4(w2 + (size_t)o * H1, hid, H1, q);
            if (q == 0) gate[o] = 1.0f / (1.0f + expf(-((float)a + (b2 ? b2[o] : 0.0f))));
        }
    }
    __builtin_amdgcn_s_waitcnt(0);   // this wave's share of step 0 has landed
    __syncthreads();

    // 3. the gated conv: wave w covers frames t0 + 32 w .. + 31 of the segment;
    // LDS row of frame t, tap k: (t - t0) + k * dil
    const int j = lane & 31, kg = lane >> 5;
    const int nks = 3 * C / 16;
    for (int tb = t0 + wave * 32; tb < t1; tb += 4 * 32) {
        const int t = tb + j;
        const int rb = t - t0 < seg ? t - t0 : 0;   // lanes past the segment: any row, result dropped
        float16v acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
        if constexpr (CT > 0) {
            constexpr int NKS = 3 * CT / 16;
            const uint8_t* const wrow = sw + j * Lo.wrow + kg * 16;
            const uint8_t* const xrow = sx + rb * Lo.xrow + kg * 16;
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const int tap = (ks * 16) / CT, ic = ks * 16 - tap * CT;
                const half8 af = *reinterpret_cast<const half8*>(wrow + ks * 32);
                const half8 bf = *reinterpret_cast<const half8*>(xrow + tap * dil * Lo.xrow + ic * 2);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc, 0, 0, 0);
            }
        } else {
            for (int ks = 0; ks < nks; ++ks) {
                const int k = ks * 16 + kg * 8, tap = k / C, ic = k - tap * C;
                const half8 af = *reinterpret_cast<const half8*>(sw + j * Lo.wrow + k * 2);
                const half8 bf = *reinterpret_cast<const half8*>(sx + (rb + tap * dil) * Lo.xrow + ic * 2);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc, 0, 0, 0);
            }
        }
        if (t < t1) {
            half_t* yr = y + ((size_t)b * T + t) * ys;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int oc = g * 8 + kg * 4;
                half4 h;
#pragma unroll
                for (int e = 0; e < 4; ++e) h[e] = (half_t)((acc[g * 4 + e] + (bl ? bl[oc + e] : 0.0f)) * gate[oc + e]);
                *reinterpret_cast<half4*>(yr + oc) = h;
            }
        }
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

extern "C" int vdk_cam_local(const void* d_x, int x_stride, int batch, int T, int C, int seg, int dil,
                             const float* d_w1, const float* d_b1, int H1, const float* d_w2, const float* d_b2,
                             const void* d_wl, const float* d_bl, void* d_y, int y_stride, const double* d_segsum,
                             double* d_zero_next, void* stream) {
    return guarded([&] {
        require(d_x && d_w1 && d_w2 && d_wl && d_y, "cam_local: NULL device pointer");
        require(batch > 0 && T > 0 && seg > 0 && dil > 0 && H1 > 0, "cam_local: bad shape");
        require(C % 16 == 0 && C >= 16 && C <= 256 && 256 % (C / 8) == 0,
                "cam_local: C must be a multiple of 16 that divides into 256 / 8-channel lanes (16..256)");
        require(x_stride >= C && x_stride % 8 == 0 && y_stride >= kLocalOC && y_stride % 4 == 0,
                "cam_local: bad strides");
        require(al16(d_x) && al16(d_wl) && al16(d_w1) && al16(d_w2) &&
                    (reinterpret_cast<uintptr_t>(d_y) & 7) == 0,
                "cam_local: x / weights must be 16-byte and y 8-byte aligned");
        const int nseg = (T + seg - 1) / seg;
        const size_t smem = (size_t)cam_local_lds(C, seg, dil, H1).total;
        require(smem <= 160 * 1024, "cam_local: the segment tile and context buffers exceed the workgroup's LDS");
        require(!d_zero_next || d_segsum, "cam_local: zero_next goes with segsum");
        auto kern = C == 128 ? cam_local_kernel<128> : cam_local_kernel<0>;
        if (smem > 64 * 1024)
            VDK_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
        hipLaunchKernelGGL(kern, dim3(batch, nseg), dim3(256), smem, static_cast<hipStream_t>(stream),
                           static_cast<const half_t*>(d_x), x_stride, T, C, seg, dil, d_w1, d_b1, H1, d_w2, d_b2,
                           static_cast<const half_t*>(d_wl), d_bl, static_cast<half_t*>(d_y), y_stride, d_segsum,
                           d_zero_next);
        VDK_HIP(hipGetLastError());
    });
}

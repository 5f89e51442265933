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
__host__ __device__ inline CamLocalLds cam_local_lds(int C, int seg, int dil, int H1, bool sums_given = false) {
    CamLocalLds L;
    L.xrow = C * 2 + 16;                         // frame row: C f16 + 16 bytes
    L.wrow = 3 * C * 2 + 16;                     // weight row (output channel): 3*C f16 + 16 bytes
    L.nrow = seg + 2 * dil;
    L.xins = (L.nrow * (L.xrow / 16) + 63) / 64;   // DMA instructions (64 slots of 16 bytes each)
    L.wins = (kLocalOC * (L.wrow / 16) + 63) / 64;
    L.part_bytes = sums_given ? 0 : 8 * 2 * (256 / (C / 8)) * C;   // only for sums taken from x itself
    L.x_off = 0;
    L.w_off = L.xins * 1024;                       // the f64 partial sums follow the weights
    L.ctx_off = L.w_off + L.wins * 1024 + L.part_bytes;
    L.total = L.ctx_off + 4 * (((C + 3) & ~3) + ((H1 + 3) & ~3) + 32);
    return L;
}

// CT > 0: the channel count fixed at compile time (the K loop of step 3
// unrolls, so its LDS reads run ahead of the MFMAs); 0: C at run time.
// Workgroup (clip b, segment s) of 256 threads; smem: cam_local_lds(...).total bytes.
template <int CT>
__device__ __forceinline__ void cam_local_segment(uint8_t* smem, int b, int s, const half_t* __restrict__ x, int xs,
                                                  int T, int Cr, int seg, int dil, const float* __restrict__ w1,
                                                  const float* __restrict__ b1, int H1, const float* __restrict__ w2,
                                                  const float* __restrict__ b2, const half_t* __restrict__ wl,
                                                  const float* __restrict__ bl, half_t* __restrict__ y, int ys,
                                                  const double* __restrict__ segsum,
                                                  double* __restrict__ zero_next) {
    const int C = CT > 0 ? CT : Cr;
    const CamLocalLds Lo = cam_local_lds(C, seg, dil, H1, segsum != nullptr);
    uint8_t* const sx = smem + Lo.x_off;
    uint8_t* const sw = smem + Lo.w_off;
    double* part = reinterpret_cast<double*>(smem + Lo.w_off + Lo.wins * 1024);   // [2][256 / C8][C]
    const int C8 = C >> 3, NFL = 256 / C8;
    float* ctx = reinterpret_cast<float*>(smem + Lo.ctx_off);   // [C]
    float* hid = ctx + ((C + 3) & ~3);                          // [H1]
    float* gate = hid + ((H1 + 3) & ~3);                        // [32]
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int t0 = s * seg, t1 = min(T, t0 + seg);
    const half_t* xb = x + (size_t)b * T * xs;
    // the mask MLP's weights (128 inputs, 64 hidden units: thread tid holds
    // quarter tid % 4 of hidden row tid / 4 and, below 128, of mask row
    // tid / 4), loaded now so their latency overlaps steps 0-1
    constexpr bool kPre = CT == 128;
    const bool pre = kPre && H1 == 64;
    const int q4 = tid & 3, o4 = tid >> 2;
    float4v w1r[kPre ? 8 : 1], w2r[kPre ? 4 : 1];
    float b1o = 0.0f, b2o = 0.0f;
    if constexpr (kPre) {
        if (pre) {
            const float4v* p1 = reinterpret_cast<const float4v*>(w1 + (size_t)o4 * 128 + q4 * 32);
#pragma unroll
            for (int i = 0; i < 8; ++i) w1r[i] = p1[i];
            const float4v* p2 = reinterpret_cast<const float4v*>(w2 + (size_t)(o4 < kLocalOC ? o4 : 0) * 64 + q4 * 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) w2r[i] = p2[i];
            b1o = b1 ? b1[o4] : 0.0f;
            b2o = b2 && o4 < kLocalOC ? b2[o4] : 0.0f;
        }
    }
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
    if (pre) {   // 2. the mask MLP from the preloaded rows (dot4's order: quarters, then (a0 + a1) + (a2 + a3))
        if constexpr (kPre) {
            double a = 0.0;
            const float4v* v4 = reinterpret_cast<const float4v*>(ctx + q4 * 32);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4v wv = w1r[i], xv = v4[i];
#pragma unroll
                for (int e = 0; e < 4; ++e) a += (double)wv[e] * (double)xv[e];
            }
            double a1 = __shfl_down(a, 1, 4), a2 = __shfl_down(a, 2, 4), a3 = __shfl_down(a, 3, 4);
            a = (a + a1) + (a2 + a3);
            if (q4 == 0) hid[o4] = fmaxf((float)a + b1o, 0.0f);
            __syncthreads();
            if (o4 < kLocalOC) {
                a = 0.0;
                const float4v* h4 = reinterpret_cast<const float4v*>(hid + q4 * 16);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float4v wv = w2r[i], xv = h4[i];
#pragma unroll
                    for (int e = 0; e < 4; ++e) a += (double)wv[e] * (double)xv[e];
                }
                a1 = __shfl_down(a, 1, 4);
                a2 = __shfl_down(a, 2, 4);
                a3 = __shfl_down(a, 3, 4);
                a = (a + a1) + (a2 + a3);
                if (q4 == 0) gate[o4] = 1.0f / (1.0f + expf(-((float)a + b2o)));
            }
        }
    } else {   // 2. the mask MLP
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
    cam_local_segment<CT>(smem, blockIdx.x, blockIdx.y, x, xs, T, Cr, seg, dil, w1, b1, H1, w2, b2, wl, bl, y, ys,
                          segsum, zero_next);
}

// ---------------------------------------------------------------------------
// The next dense layer's linear1 over one segment's frames, run by the CAM
// launch right after it has written the segment's 32 new channels
// (cam_dense_kernel): hn = relu(W relu(D * scale + shift) + bias), a 1x1 conv
// of the block buffer's first cin channels to 128, with the implicit-GEMM
// kernels' MFMA shape (32 x 32 x 16 f16, A = weight rows, B = frames), K
// order (channels in sequence from 0) and arithmetic (the input prologue
// rounded to f16 as the operand, bias then ReLU, f16 store), so hn equals the
// conv launch's output bit for bit; the segment's f64 sums of the stored
// values are exact, so they equal the conv epilogue's atomics, and go to the
// segment's own row of the next layer's sums (a plain store: this workgroup
// is the only one that computes the segment).  Wave w takes frames
// t0 + 32 w .. + 31 against all 128 outputs (4 blocks of 32); 32-channel
// chunks of both operands DMA'd into a 4-stage ring.  A workgroup computes
// one half of the 128 outputs (oh): two workgroups per (clip, segment).
// ---------------------------------------------------------------------------
namespace l1 {
constexpr int OUT = 128;                                   // linear1's outputs
constexpr int M = 64, N = 128, KC = 32, NST = 4, CPR = KC / 8, RB = KC * 2;   // per workgroup: half the outputs
constexpr int NINS = (M + N) * CPR / 64, IPW = NINS / 4;   // DMA instructions per chunk / wave
constexpr int STAGE = NINS * 1024;
constexpr int PRO = 1024;                                  // the prologue's scale | shift, up to 1024 channels
constexpr int TS = M + 4;                                  // staged f32 row [frame][output]
constexpr int RING_OFF = 2 * PRO * 4;
constexpr int STAGING = N * TS * 4;
constexpr int LDS = RING_OFF + (NST * STAGE > STAGING ? NST * STAGE : STAGING);
static_assert(NINS % 4 == 0 && IPW * (NST - 2) <= 16, "whole DMA instructions per wave, vmcnt range");
}  // namespace l1

// 16-byte chunk c of LDS row r (32-channel rows of 64 bytes) sits at slot
// c ^ ((r / 4) % 4): the 16 rows of an MFMA operand read hit 16 distinct
// 16-byte bank groups.
__device__ __forceinline__ int swz32(int r, int c) { return c ^ ((r >> 2) & 3); }

__device__ __forceinline__ void linear1_segment(uint8_t* smem, int b, int T, int t0, int t1, int oh,
                                                const half_t* __restrict__ D, int ds, int cin,
                                                const half_t* __restrict__ w, const float* __restrict__ bias,
                                                const float* __restrict__ sc, const float* __restrict__ sh,
                                                half_t* __restrict__ hn, double* __restrict__ seg_row) {
    using namespace l1;
    w += (size_t)oh * M * cin;   // this half's weight rows, biases, outputs and sums
    bias += oh * M;
    hn += oh * M;
    seg_row += oh * M;
    float* const s_in = reinterpret_cast<float*>(smem);
    uint8_t* const ring = smem + RING_OFF;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int nk = (cin + KC - 1) / KC;   // the last chunk may hold 32 channels (the rest read as zeros, skipped)
    for (int c = tid; c < cin; c += 256) {
        s_in[c] = sc[c];
        s_in[PRO + c] = sh[c];
    }
    // DMA slots of this lane: row r < M: weight row r; else frame t0 + r - M
    const int4v wr = dma_rsrc(w, (uint32_t)(M * cin * 2));
    const int4v xr = dma_rsrc(D, (uint32_t)((((size_t)(b + 1) * T - 1) * ds + cin) * 2));
    int off[IPW], cj[IPW];   // cj: the slot's first channel within a chunk
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
        const int ins = wave + 4 * j;
        const int p = ins * 64 + lane, r = p / CPR, c = swz32(r, p - r * CPR);
        cj[j] = c * 8;
        if (r < M) {
            off[j] = (r * cin + c * 8) * 2;
        } else {
            const int t = t0 + r - M;
            off[j] = t < t1 ? (int)((((size_t)b * T + t) * ds + c * 8) * 2) : -1;
        }
    }
    auto issue = [&](int k) {
        uint8_t* const dst = ring + (k % NST) * STAGE;
#pragma unroll
        for (int j = 0; j < IPW; ++j) {
            const int ins = wave + 4 * j;
            const uint32_t o = off[j] < 0 || k * KC + cj[j] >= cin ? kOOB : (uint32_t)(off[j] + k * KC * 2);
            dma16(dst + ins * 1024, ins * 64 / CPR < M ? wr : xr, o);   // wave-uniform operand choice
        }
    };
    for (int k = 0; k < NST - 1 && k < nk; ++k) issue(k);
    constexpr int MB = M / 32;   // 32-output blocks per wave
    float16v acc[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
    const int brow = M + wave * 32 + lrow;
#pragma unroll 1
    for (int k = 0; k < nk; ++k) {
        const int younger = nk - 1 - k < NST - 2 ? nk - 1 - k : NST - 2;
        wait_vmcnt_le(younger * IPW);
        lds_barrier();   // chunk k has landed for every wave; chunk k-1's stage is free (and s_in is written)
        if (k + NST - 1 < nk) issue(k + NST - 1);
        const uint8_t* const sa = ring + (k % NST) * STAGE;
#pragma unroll
        for (int kk = 0; kk < KC / 16; ++kk) {
            if (k * KC + kk * 16 >= cin) break;   // wave-uniform: past the input channels
            const int c = kk * 2 + lhalf;
            half8 bf = *reinterpret_cast<const half8*>(sa + brow * RB + swz32(brow, c) * 16);
            const int ch = k * KC + c * 8;
            const float4v sc0 = *reinterpret_cast<const float4v*>(s_in + ch);
            const float4v sc1 = *reinterpret_cast<const float4v*>(s_in + ch + 4);
            const float4v sh0 = *reinterpret_cast<const float4v*>(s_in + PRO + ch);
            const float4v sh1 = *reinterpret_cast<const float4v*>(s_in + PRO + ch + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                bf[e] = (half_t)fmaxf((float)bf[e] * sc0[e] + sh0[e], 0.0f);
                bf[e + 4] = (half_t)fmaxf((float)bf[e + 4] * sc1[e] + sh1[e], 0.0f);
            }
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const int ar = i * 32 + lrow;
                const half8 af = *reinterpret_cast<const half8*>(sa + ar * RB + swz32(ar, c) * 16);
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc[i], 0, 0, 0);
            }
        }
    }
    __syncthreads();   // the ring is free: stage the f32 results as [frame][output]
    float* const sT = reinterpret_cast<float*>(ring);
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int r = i * 32 + g * 8 + lhalf * 4;
            *reinterpret_cast<float4v*>(sT + (wave * 32 + lrow) * TS + r) =
                float4v{acc[i][g * 4], acc[i][g * 4 + 1], acc[i][g * 4 + 2], acc[i][g * 4 + 3]};
        }
    __syncthreads();
    // bias, ReLU, f16 out (8 threads per frame, 8 outputs each) and the
    // segment's sums of the stored values per output
    constexpr int TPF = M / 8;   // threads per frame
    const int cc = tid % TPF, nfr = t1 - t0;
    double sum[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) sum[e] = 0.0;
    const float4v bb0 = *reinterpret_cast<const float4v*>(bias + cc * 8);
    const float4v bb1 = *reinterpret_cast<const float4v*>(bias + cc * 8 + 4);
    const float bv[8] = {bb0[0], bb0[1], bb0[2], bb0[3], bb1[0], bb1[1], bb1[2], bb1[3]};
    for (int fr = tid / TPF; fr < nfr; fr += 256 / TPF) {
        const float4v u0 = *reinterpret_cast<const float4v*>(sT + fr * TS + cc * 8);
        const float4v u1 = *reinterpret_cast<const float4v*>(sT + fr * TS + cc * 8 + 4);
        const float u[8] = {u0[0], u0[1], u0[2], u0[3], u1[0], u1[1], u1[2], u1[3]};
        half8 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = u[e];
            v += bv[e];
            v = fmaxf(v, 0.0f);
            h[e] = (half_t)v;
            sum[e] += (double)(float)h[e];
        }
        *reinterpret_cast<half8*>(hn + ((size_t)b * T + t0 + fr) * OUT + cc * 8) = h;
    }
    // threads of one output chunk: the lanes cc + TPF j of each wave, then the 4 waves
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int m = TPF; m < 64; m <<= 1) sum[e] += __shfl_xor(sum[e], m);
    __syncthreads();   // the staging area is read
    double* const ws = reinterpret_cast<double*>(ring);   // [4 waves][M]
    if (lane < TPF) {
#pragma unroll
        for (int e = 0; e < 8; ++e) ws[wave * M + cc * 8 + e] = sum[e];
    }
    __syncthreads();
    if (tid < M) seg_row[tid] = ((ws[tid] + ws[M + tid]) + (ws[2 * M + tid] + ws[3 * M + tid]));
}

// One dense layer's CAM (cam_local_segment) and the next layer's linear1
// over the same segment in one launch (workgroup = (clip, segment)): the
// next layer's input at a frame is the block buffer's older channels plus
// the 32 this workgroup has just written, so no other workgroup's output is
// needed.  The CAM reads linear1's previous output h (with a dil-frame halo
// from the neighbouring segments) while linear1 writes the next one, hn: two
// buffers.  seg_next gets each segment's sums of hn; nothing needs clearing.
__global__ __launch_bounds__(256) void cam_dense_kernel(const half_t* __restrict__ h, int T, int seg, int dil,
                                                        const float* __restrict__ w1, const float* __restrict__ b1,
                                                        int H1, const float* __restrict__ w2,
                                                        const float* __restrict__ b2, const half_t* __restrict__ wl,
                                                        const float* __restrict__ bl, half_t* __restrict__ D, int ds,
                                                        int cin_cur, const double* __restrict__ segsum,
                                                        const half_t* __restrict__ wn, const float* __restrict__ bn,
                                                        const float* __restrict__ scn, const float* __restrict__ shn,
                                                        half_t* __restrict__ hn, double* __restrict__ seg_next) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    const int b = blockIdx.x, s = blockIdx.y, oh = blockIdx.z, nseg = gridDim.y;
    // both halves of a segment run the CAM (the same bits: the second write of
    // each value stores what the first did)
    cam_local_segment<128>(smem, b, s, h, 128, T, 128, seg, dil, w1, b1, H1, w2, b2, wl, bl, D + cin_cur, ds, segsum,
                           nullptr);
    __syncthreads();   // the segment's new channels are in memory (and visible to this workgroup)
    const int t0 = s * seg, t1 = min(T, t0 + seg);
    linear1_segment(smem, b, T, t0, t1, oh, D, ds, cin_cur + kLocalOC, wn, bn, scn, shn, hn,
                    seg_next + ((size_t)b * nseg + s) * l1::OUT);
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
        const size_t smem = (size_t)cam_local_lds(C, seg, dil, H1, d_segsum != nullptr).total;
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

extern "C" int vdk_cam_dense(const void* d_h, int batch, int T, int seg, int dil, const float* d_w1,
                             const float* d_b1, int H1, const float* d_w2, const float* d_b2, const void* d_wl,
                             const float* d_bl, void* d_dense, int dense_stride, int cin, const double* d_segsum,
                             const void* d_wn, const float* d_bn, const float* d_scale_n, const float* d_shift_n,
                             void* d_hn, double* d_seg_next, void* stream) {
    return guarded([&] {
        require(d_h && d_w1 && d_w2 && d_wl && d_dense && d_segsum && d_wn && d_bn && d_scale_n && d_shift_n && d_hn &&
                    d_seg_next, "cam_dense: NULL device pointer");
        require(batch > 0 && T > 0 && seg > 0 && seg <= l1::N && dil > 0 && H1 > 0, "cam_dense: bad shape");
        const int cn = cin + kLocalOC;
        require(cin % 32 == 0 && cin >= 32 && cn <= l1::PRO && cn <= dense_stride && dense_stride % 8 == 0,
                "cam_dense: channel counts must be multiples of 32 within the block buffer (next input <= 1024)");
        require(al16(d_h) && al16(d_wl) && al16(d_w1) && al16(d_w2) && al16(d_dense) && al16(d_wn) && al16(d_bn) &&
                    al16(d_scale_n) && al16(d_shift_n) && al16(d_hn),
                "cam_dense: pointers must be 16-byte aligned");
        require(d_hn != d_h, "cam_dense: hn must be a different buffer from h (other segments read its halo)");
        require((long)batch * T * dense_stride * 2 < (1L << 31), "cam_dense: map too large for one launch");
        const int nseg = (T + seg - 1) / seg;
        const size_t a = (size_t)cam_local_lds(128, seg, dil, H1, true).total;
        const size_t smem = a > (size_t)l1::LDS ? a : (size_t)l1::LDS;
        require(smem <= 160 * 1024, "cam_dense: LDS");
        VDK_HIP(hipFuncSetAttribute((const void*)cam_dense_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)smem));
        hipLaunchKernelGGL(cam_dense_kernel, dim3(batch, nseg, 2), dim3(256), smem, static_cast<hipStream_t>(stream),
                           static_cast<const half_t*>(d_h), T, seg, dil, d_w1, d_b1, H1, d_w2, d_b2,
                           static_cast<const half_t*>(d_wl), d_bl, static_cast<half_t*>(d_dense), dense_stride, cin,
                           d_segsum, static_cast<const half_t*>(d_wn), d_bn, d_scale_n, d_shift_n,
                           static_cast<half_t*>(d_hn), d_seg_next);
        VDK_HIP(hipGetLastError());
    });
}

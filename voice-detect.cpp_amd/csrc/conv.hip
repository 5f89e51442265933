// conv.hip - speaker-encoder 2D convolutions on gfx950.
//
// conv_igemm_kernel: implicit GEMM on f16 MFMA (v_mfma_f32_32x32x16_f16) with
// f32 accumulation.  GEMM view: M = output channels, N = output pixels
// (flattened over batch, rows and columns), K = KH*KW*IC ordered tap-major,
// channel-minor so that 8 consecutive K values are 8 contiguous NHWC channels
// (one 16-byte load).  Per K chunk (one tap, KC channels) the workgroup stages
// its weight tile [BM][KC] and its im2col pixel tile [BN][KC] in LDS with
// coalesced 16-byte loads (rows padded by 16 bytes so the MFMA operand reads
// are bank-conflict free), then every wave runs (WM/32)x(WN/32) MFMA tiles.
// The epilogue fuses bias, the residual add and ReLU, and stores f16 NHWC.
//
// Follows the reference conv contract (src/directconv.hpp:22-51: zero padding,
// 3x3 or 1x1, stride 1 or 2, bias(+ReLU) fused, residual add+ReLU fused); the
// reference's f32 direct accumulation is replaced by f16 products with f32 sums.
//
// stem_conv3x3_kernel: the IC=1 stem (K = 9 is too short for MFMA); one
// thread per output pixel computes all OC channels in f32 from f32 features.
#include "common.hpp"
#include "vdk.h"

namespace vdk {
namespace {

struct ConvArgs {
    const half_t* x;
    const half_t* w;
    const float* bias;
    const half_t* res;
    half_t* y;
    int H, W, IC, Ho, Wo, OC, KH, KW, stride, pad, relu;
    int npix;  // B * Ho * Wo
};

// Spread consecutive workgroup ids over the 8 XCDs in contiguous ranges so that
// neighbouring pixel tiles (which share input rows) run under the same L2.
__device__ __forceinline__ int xcd_swizzle(int bid, int nb) {
    const int per = nb >> 3;
    if (bid >= (per << 3)) return bid;
    return (bid & 7) * per + (bid >> 3);
}

template <int BM, int BN, int WM, int WN, int KC>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void conv_igemm_kernel(ConvArgs a) {
    constexpr int NWM = BM / WM, NWN = BN / WN, NT = NWM * NWN * 64;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int LDK = KC + 8;           // +16 bytes per LDS row
    constexpr int CPR = KC / 8;           // 16-byte chunks per row
    constexpr int XCH = (BN * CPR + NT - 1) / NT;
    static_assert(WM % 32 == 0 && WN % 32 == 0 && KC % 16 == 0, "tile shape");
    __shared__ __attribute__((aligned(16))) half_t sW[BM * LDK];
    __shared__ __attribute__((aligned(16))) half_t sX[BN * LDK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % NWM, wn = wave / NWM;
    const int p0 = xcd_swizzle(blockIdx.x, gridDim.x) * BN;
    const int oc0 = blockIdx.y * BM;
    const int HoWo = a.Ho * a.Wo;
    const int KHW = a.KH * a.KW;

    // Each thread loads the same pixel rows for every K chunk: decode them once.
    int x_img[XCH], x_ih[XCH], x_iw[XCH], x_lds[XCH], x_c[XCH];
    bool x_on[XCH];
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
        const int q = tid + i * NT;
        const int r = q / CPR, c8 = q - r * CPR;
        const int P = p0 + r;
        x_on[i] = q < BN * CPR && P < a.npix;
        const int Pc = x_on[i] ? P : 0;
        const int b = Pc / HoWo, rem = Pc - b * HoWo;
        const int oh = rem / a.Wo, ow = rem - oh * a.Wo;
        x_img[i] = b * a.H;
        x_ih[i] = oh * a.stride - a.pad;
        x_iw[i] = ow * a.stride - a.pad;
        x_lds[i] = r * LDK + c8 * 8;
        x_c[i] = c8 * 8;
    }

    float16v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const half8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int tap = 0; tap < KHW; ++tap) {
        const int kh = tap / a.KW, kw = tap - kh * a.KW;
        for (int c0 = 0; c0 < a.IC; c0 += KC) {
            for (int q = tid; q < BM * CPR; q += NT) {
                const int r = q / CPR, c8 = q - r * CPR;
                const half8 v = *reinterpret_cast<const half8*>(
                    a.w + ((size_t)(oc0 + r) * KHW + tap) * a.IC + c0 + c8 * 8);
                *reinterpret_cast<half8*>(sW + r * LDK + c8 * 8) = v;
            }
#pragma unroll
            for (int i = 0; i < XCH; ++i) {
                if (tid + i * NT < BN * CPR) {
                    const int ih = x_ih[i] + kh, iw = x_iw[i] + kw;
                    half8 v = zero8;
                    if (x_on[i] && ih >= 0 && ih < a.H && iw >= 0 && iw < a.W)
                        v = *reinterpret_cast<const half8*>(
                            a.x + ((size_t)(x_img[i] + ih) * a.W + iw) * a.IC + c0 + x_c[i]);
                    *reinterpret_cast<half8*>(sX + x_lds[i]) = v;
                }
            }
            __syncthreads();
#pragma unroll
            for (int kk = 0; kk < KC / 16; ++kk) {
                half8 af[TM], bf[TN];
                const int koff = kk * 16 + (lane >> 5) * 8;
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    af[i] = *reinterpret_cast<const half8*>(sW + (wm * WM + i * 32 + (lane & 31)) * LDK + koff);
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    bf[j] = *reinterpret_cast<const half8*>(sX + (wn * WN + j * 32 + (lane & 31)) * LDK + koff);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
            __syncthreads();
        }
    }

    // Epilogue.  32x32 accumulator layout: register r of lane l holds
    // row (OC) 8*(r/4) + 4*(l/32) + r%4 and column (pixel) l%32.
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int P = p0 + wn * WN + j * 32 + (lane & 31);
        if (P >= a.npix) continue;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int oc = oc0 + wm * WM + i * 32 + g * 8 + (lane >> 5) * 4;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = acc[i][j][g * 4 + e] + (a.bias ? a.bias[oc + e] : 0.0f);
                const size_t o = (size_t)P * a.OC + oc;
                if (a.res) {
                    const half4 r = *reinterpret_cast<const half4*>(a.res + o);
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] += (float)r[e];
                }
                if (a.relu) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = v[e] > 0.0f ? v[e] : 0.0f;
                }
                half4 h;
#pragma unroll
                for (int e = 0; e < 4; ++e) h[e] = (half_t)v[e];
                *reinterpret_cast<half4*>(a.y + o) = h;
            }
        }
    }
}

template <int BM, int BN, int WM, int WN, int KC>
void launch_igemm(const ConvArgs& a, hipStream_t s) {
    constexpr int NT = (BM / WM) * (BN / WN) * 64;
    dim3 grid(cdiv(a.npix, BN), a.OC / BM);
    hipLaunchKernelGGL((conv_igemm_kernel<BM, BN, WM, WN, KC>), grid, dim3(NT), 0, s, a);
}

template <int BM, int BN, int WM, int WN>
void launch_kc(const ConvArgs& a, hipStream_t s) {
    if (a.IC % 64 == 0) launch_igemm<BM, BN, WM, WN, 64>(a, s);
    else if (a.IC % 32 == 0) launch_igemm<BM, BN, WM, WN, 32>(a, s);
    else launch_igemm<BM, BN, WM, WN, 16>(a, s);
}

template <int OC>
__global__ __launch_bounds__(256) void stem_conv3x3_kernel(const float* __restrict__ feats, int B, int H, int W,
                                                           const float* __restrict__ w,
                                                           const float* __restrict__ bias, int relu,
                                                           half_t* __restrict__ y) {
    const long P = (long)blockIdx.x * 256 + threadIdx.x;
    const long HW = (long)H * W;
    if (P >= (long)B * HW) return;
    const int b = (int)(P / HW);
    const int rem = (int)(P - (long)b * HW);
    const int h = rem / W, t = rem - h * W;
    float xv[9];
#pragma unroll
    for (int kh = 0; kh < 3; ++kh)
#pragma unroll
        for (int kw = 0; kw < 3; ++kw) {
            const int ih = h - 1 + kh, iw = t - 1 + kw;
            xv[kh * 3 + kw] = (ih >= 0 && ih < H && iw >= 0 && iw < W) ? feats[((long)b * H + ih) * W + iw] : 0.0f;
        }
    half_t* out = y + P * OC;
#pragma unroll
    for (int o8 = 0; o8 < OC / 8; ++o8) {
        half8 hv;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int oc = o8 * 8 + e;
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < 9; ++k) acc += w[oc * 9 + k] * xv[k];
            float v = acc + bias[oc];
            if (relu) v = v > 0.0f ? v : 0.0f;
            hv[e] = (half_t)v;
        }
        *reinterpret_cast<half8*>(out + o8 * 8) = hv;
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace vdk

using namespace vdk;

extern "C" int vdk_conv2d_nhwc(const void* d_x, int batch, int H, int W, int IC,
                               const void* d_w, int OC, int KH, int KW, int stride, int pad,
                               const float* d_bias, const void* d_residual, int relu,
                               void* d_y, void* stream) {
    return guarded([&] {
        require(d_x && d_w && d_y, "conv2d: NULL device pointer");
        require(batch > 0 && H > 0 && W > 0, "conv2d: empty input");
        require(IC > 0 && IC % 16 == 0, "conv2d: IC must be a positive multiple of 16");
        require(OC > 0 && OC % 32 == 0, "conv2d: OC must be a positive multiple of 32");
        require(KH >= 1 && KW >= 1 && KH <= 7 && KW <= 7, "conv2d: kernel size out of range");
        require(stride >= 1 && pad >= 0, "conv2d: invalid stride/pad");
        const int Ho = (H + 2 * pad - KH) / stride + 1, Wo = (W + 2 * pad - KW) / stride + 1;
        require(H + 2 * pad >= KH && W + 2 * pad >= KW && Ho > 0 && Wo > 0, "conv2d: output would be empty");
        require((long)batch * Ho * Wo < (1L << 31) && (long)batch * H * W < (1L << 31),
                "conv2d: too many pixels for one launch");
        require(aligned16(d_x) && aligned16(d_w) && aligned16(d_y) && (!d_residual || aligned16(d_residual)),
                "conv2d: device pointers must be 16-byte aligned");
        ConvArgs a;
        a.x = static_cast<const half_t*>(d_x);
        a.w = static_cast<const half_t*>(d_w);
        a.bias = d_bias;
        a.res = static_cast<const half_t*>(d_residual);
        a.y = static_cast<half_t*>(d_y);
        a.H = H; a.W = W; a.IC = IC; a.Ho = Ho; a.Wo = Wo; a.OC = OC;
        a.KH = KH; a.KW = KW; a.stride = stride; a.pad = pad; a.relu = relu ? 1 : 0;
        a.npix = batch * Ho * Wo;
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (OC % 128 == 0) {
            if (a.npix >= 64 * 1024) launch_kc<128, 128, 64, 64>(a, s);
            else launch_kc<128, 64, 64, 32>(a, s);
        } else if (OC % 64 == 0) {
            launch_kc<64, 128, 32, 64>(a, s);
        } else {
            launch_kc<32, 256, 32, 64>(a, s);
        }
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_stem_conv3x3(const float* d_feats, int batch, int H, int W,
                                const float* d_w, const float* d_bias, int OC, int relu,
                                void* d_y, void* stream) {
    return guarded([&] {
        require(d_feats && d_w && d_bias && d_y, "stem: NULL device pointer");
        require(batch > 0 && H > 0 && W > 0, "stem: empty input");
        require((long)batch * H * W < (1L << 31), "stem: too many pixels for one launch");
        require(aligned16(d_y), "stem: output must be 16-byte aligned");
        hipStream_t s = static_cast<hipStream_t>(stream);
        const long n = (long)batch * H * W;
        dim3 grid(cdiv(n, 256));
        half_t* y = static_cast<half_t*>(d_y);
        switch (OC) {
            case 16: hipLaunchKernelGGL(stem_conv3x3_kernel<16>, grid, dim3(256), 0, s, d_feats, batch, H, W, d_w, d_bias, relu, y); break;
            case 32: hipLaunchKernelGGL(stem_conv3x3_kernel<32>, grid, dim3(256), 0, s, d_feats, batch, H, W, d_w, d_bias, relu, y); break;
            case 64: hipLaunchKernelGGL(stem_conv3x3_kernel<64>, grid, dim3(256), 0, s, d_feats, batch, H, W, d_w, d_bias, relu, y); break;
            default: throw Error("stem: OC must be 16, 32 or 64");
        }
        VDK_HIP(hipGetLastError());
    });
}

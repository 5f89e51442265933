// w2v2.hip - wav2vec2 analyze kernels on gfx950 (reference src/analyze_w2v2.cpp).
//
// The GEMM-shaped work of the analyze path (feature-encoder convs 1..n,
// feature projection, q/k/v/out projections, feed-forward, positional conv)
// runs on the implicit-GEMM conv kernels (conv.hip) over time-major f16
// [B][T][C] maps.  This file holds the rest:
//   wave_stats_kernel      do_normalize statistics of the raw waveform
//   conv0_*_kernel         conv layer 0 (one input channel, so no GEMM) with its
//                          GroupNorm (per channel over time) or LayerNorm (per
//                          frame over channels) and the exact GELU
//   layer_norm_kernel      LayerNorm over rows, optional GELU and a weighted
//                          accumulation (the emotion head's layer sum)
//   attention_kernel       softmax(q k^T * scale) v per (clip, head) on f16
//                          MFMA, streaming 64-key blocks with an online softmax
//   time_mean_kernel       per-clip mean over time
// Reductions run in a fixed order (f64 where they feed a normalisation), so
// results do not depend on scheduling.
#include <cfloat>
#include <cmath>

#include "common.hpp"
#include "devmath.hpp"
#include "vdk.h"

namespace vdk {
namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Sum over a workgroup of NT threads, fixed order; every thread gets the total.
template <int NT>
__device__ __forceinline__ double block_sum_d(double v, double* red) {
    v = wave_sum_d(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) s += red[i];
    return s;
}

// ---- do_normalize statistics: mean and 1/sqrt(biased var + eps) per clip,
// two passes in f64 (src/analyze_w2v2.cpp:63-70).
__global__ __launch_bounds__(1024) void wave_stats_kernel(const float* __restrict__ x, int n, float eps,
                                                          float* __restrict__ stats) {
    __shared__ double red[16];
    const float* xc = x + (size_t)blockIdx.x * n;
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += 1024) s += (double)xc[i];
    const double mean = block_sum_d<1024>(s, red) / n;
    double v = 0.0;
    for (int i = threadIdx.x; i < n; i += 1024) {
        const double d = (double)xc[i] - mean;
        v += d * d;
    }
    v = block_sum_d<1024>(v, red) / n;
    if (threadIdx.x == 0) {
        stats[2 * blockIdx.x] = (float)mean;
        stats[2 * blockIdx.x + 1] = (float)(1.0 / sqrt(v + (double)eps));
    }
}

// ---- conv layer 0: y[b][t][c] = bias[c] + sum_k w[c][k] xn[b][t*S + k] ----
// xn = (x - mean) * rstd when do_normalize statistics are given.  A
// workgroup covers kFrames frames of one clip; the waveform window it needs
// is staged in LDS once.
constexpr int kFrames = 64, kMaxK = 16, kMaxS = 8;
constexpr int kWin = (kFrames - 1) * kMaxS + kMaxK;

__device__ __forceinline__ void load_window(const float* x, int n, const float* wstats, int b, int start, int len,
                                            float* sx) {
    const float* xc = x + (size_t)b * n;
    const float mean = wstats ? wstats[2 * b] : 0.0f, rstd = wstats ? wstats[2 * b + 1] : 1.0f;
    for (int i = threadIdx.x; i < len; i += blockDim.x) {
        const float v = xc[start + i];
        sx[i] = wstats ? (v - mean) * rstd : v;
    }
}

// GroupNorm statistics (num_groups == channels) without a pass over the
// conv output: y_c(t) = bias_c + w_c . u(t) with u(t) = xn[t*S .. t*S+K-1], so
//   mean_c = bias_c + w_c . m,   var_c = w_c^T (G - m m^T) w_c
// with m = mean_t u(t) and G = mean_t u(t) u(t)^T (biased, as GroupNorm).
// conv0_moments_kernel sums u_k and u_k u_k' (k <= k') over the clip's frames
// in f64, one sum per thread; conv0_finalize_kernel forms the per-channel
// affine scale = gamma / sqrt(var + eps), shift = beta - mean * scale.
__global__ __launch_bounds__(256) void conv0_moments_kernel(const float* __restrict__ x, int n,
                                                            const float* __restrict__ wstats, int K, int S, int T0,
                                                            double* __restrict__ part) {
    __shared__ float sx[kWin];
    const int b = blockIdx.y, chunk = blockIdx.x, p = threadIdx.x, t0 = chunk * kFrames;
    const int NP = K + K * (K + 1) / 2;
    const int nt = T0 - t0 < kFrames ? T0 - t0 : kFrames;
    load_window(x, n, wstats, b, t0 * S, (nt - 1) * S + K, sx);
    __syncthreads();
    if (p >= NP) return;
    int k1 = p, k2 = -1;   // p < K: the sum of u_p; then the pairs k1 <= k2 in row order
    if (p >= K) {
        int q = p - K;
        k1 = 0;
        while (q >= K - k1) { q -= K - k1; ++k1; }
        k2 = k1 + q;
    }
    double acc = 0.0;
    for (int t = 0; t < nt; ++t) {
        const float u = sx[t * S + k1];
        acc += k2 < 0 ? (double)u : (double)u * (double)sx[t * S + k2];
    }
    part[((size_t)b * gridDim.x + chunk) * NP + p] = acc;
}

// Chunk partials -> per-clip moment sums, in chunk order.
__global__ __launch_bounds__(256) void conv0_moments_reduce_kernel(const double* __restrict__ part, int nchunk,
                                                                   int NP, double* __restrict__ mom) {
    const int b = blockIdx.x, p = threadIdx.x;
    if (p >= NP) return;
    double s = 0.0;
    for (int j = 0; j < nchunk; ++j) s += part[((size_t)b * nchunk + j) * NP + p];
    mom[(size_t)b * NP + p] = s;
}

__global__ __launch_bounds__(256) void conv0_finalize_kernel(const double* __restrict__ mom,
                                                             const float* __restrict__ w,
                                                             const float* __restrict__ bias, int C, int K, int T0,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta, float eps,
                                                             float* __restrict__ scale, float* __restrict__ shift) {
    const int c = blockIdx.x * 256 + threadIdx.x, b = blockIdx.y;
    if (c >= C) return;
    const int NP = K + K * (K + 1) / 2;
    const double* mb = mom + (size_t)b * NP;
    double wc[kMaxK], m[kMaxK];
    double mean = bias ? (double)bias[c] : 0.0;
    for (int k = 0; k < K; ++k) {
        wc[k] = (double)w[c * K + k];
        m[k] = mb[k] / T0;
        mean += wc[k] * m[k];
    }
    double var = 0.0;
    int q = K;
    for (int k1 = 0; k1 < K; ++k1)
        for (int k2 = k1; k2 < K; ++k2, ++q) {
            const double cov = mb[q] / T0 - m[k1] * m[k2];
            var += (k1 == k2 ? 1.0 : 2.0) * wc[k1] * wc[k2] * cov;
        }
    var = var > 0.0 ? var : 0.0;
    const double sc = (double)gamma[c] / sqrt(var + (double)eps);
    const size_t o = (size_t)b * C + c;
    scale[o] = (float)sc;
    shift[o] = (float)((double)beta[c] - mean * sc);
}

// One wave per frame; lane l owns channels l*CPL .. l*CPL + CPL - 1 and
// holds their KT taps (zero past K) in registers.  A workgroup covers
// kApplyFrames frames of one clip: the waveform window and the weights
// (staged through LDS as [K][C] so every global read is coalesced) are loaded
// once per workgroup.  norm 0: none; 1: GroupNorm affine from scale/shift
// [B][C]; 2: LayerNorm over the frame's C channels (gamma, beta, eps).  Then
// GELU, stored f16.
constexpr int kApplyFrames = 256;
constexpr int kApplyWin = (kApplyFrames - 1) * kMaxS + kMaxK;

template <int CPL, int KT>
__global__ __launch_bounds__(256) void conv0_apply_kernel(const float* __restrict__ x, int n,
                                                          const float* __restrict__ wstats,
                                                          const float* __restrict__ w, const float* __restrict__ bias,
                                                          int K, int S, int T0, int norm,
                                                          const float* __restrict__ scale,
                                                          const float* __restrict__ shift,
                                                          const float* __restrict__ gamma,
                                                          const float* __restrict__ beta, float eps,
                                                          half_t* __restrict__ y) {
    constexpr int C = CPL * 64;
    __shared__ float sx[kApplyWin];
    __shared__ __attribute__((aligned(16))) float sw[KT * C];   // [tap][channel]
    const int b = blockIdx.y, t0 = blockIdx.x * kApplyFrames;
    const int nt = T0 - t0 < kApplyFrames ? T0 - t0 : kApplyFrames;
    const int len = (nt - 1) * S + K;
    load_window(x, n, wstats, b, t0 * S, len, sx);
    for (int i = len + threadIdx.x; i < (nt - 1) * S + KT; i += 256) sx[i] = 0.0f;   // taps K..KT-1
    for (int i = threadIdx.x; i < KT * C; i += 256) {
        const int c = i / KT, k = i - c * KT;   // coalesced read of w [C][K]
        sw[k * C + c] = k < K ? w[c * K + k] : 0.0f;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c0 = lane * CPL;
    float bc[CPL], sa[CPL], sb[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        bc[j] = bias ? bias[c0 + j] : 0.0f;
        sa[j] = 1.0f;
        sb[j] = 0.0f;
        if (norm == 1) {
            sa[j] = scale[(size_t)b * C + c0 + j];
            sb[j] = shift[(size_t)b * C + c0 + j];
        } else if (norm == 2) {
            sa[j] = gamma[c0 + j];
            sb[j] = beta[c0 + j];
        }
    }
    __syncthreads();
    float wr[CPL][KT];
#pragma unroll
    for (int k = 0; k < KT; ++k)
#pragma unroll
        for (int j = 0; j < CPL; j += 4) {
            const float4v v = *reinterpret_cast<const float4v*>(&sw[k * C + c0 + j]);
#pragma unroll
            for (int e = 0; e < 4; ++e) wr[j + e][k] = v[e];
        }
    for (int t = wave; t < nt; t += 4) {
        float u[KT];
#pragma unroll
        for (int k = 0; k < KT; ++k) u[k] = sx[t * S + k];
        float v[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            float a = bc[j];
#pragma unroll
            for (int k = 0; k < KT; ++k) a += wr[j][k] * u[k];
            v[j] = a;
        }
        if (norm == 2) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < CPL; ++j) s += v[j];
            const float mu = wave_sum(s) / C;
            float q = 0.0f;
#pragma unroll
            for (int j = 0; j < CPL; ++j) q += (v[j] - mu) * (v[j] - mu);
            const float rstd = 1.0f / sqrtf(wave_sum(q) / C + eps);
#pragma unroll
            for (int j = 0; j < CPL; ++j) v[j] = (v[j] - mu) * rstd;
        }
        half_t* yo = y + ((size_t)b * T0 + t0 + t) * C + c0;
#pragma unroll
        for (int j0 = 0; j0 < CPL; j0 += 4) {
            half4 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = (half_t)gelu_erf(v[j0 + e] * sa[j0 + e] + sb[j0 + e]);
            *reinterpret_cast<half4*>(yo + j0) = h;
        }
    }
}

template <int CPL>
void launch_conv0_apply(dim3 g, hipStream_t s, const float* x, int n, const float* wstats, const float* w,
                        const float* bias, int K, int S, int T0, int norm, const float* scale, const float* shift,
                        const float* gamma, const float* beta, float eps, half_t* y) {
    if (K == 10)
        hipLaunchKernelGGL((conv0_apply_kernel<CPL, 10>), g, dim3(256), 0, s, x, n, wstats, w, bias, K, S, T0, norm,
                           scale, shift, gamma, beta, eps, y);
    else
        hipLaunchKernelGGL((conv0_apply_kernel<CPL, kMaxK>), g, dim3(256), 0, s, x, n, wstats, w, bias, K, S, T0,
                           norm, scale, shift, gamma, beta, eps, y);
}

// ---- LayerNorm over rows of C (one wave per row, lane l owns elements
// l + 64 j) with optional GELU and acc = [acc +] acc_w * (input | output).
template <int EMAX>
__global__ __launch_bounds__(256) void layer_norm_kernel(const void* __restrict__ x, int rows, int C,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ beta, float eps, int flags,
                                                         void* __restrict__ y, float* __restrict__ acc, float acc_w) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int E = C >> 6;
    const bool xf = flags & VDK_LN_X_F32;
    const size_t base = (size_t)row * C;
    float v[EMAX];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < EMAX; ++j) {
        v[j] = 0.0f;
        if (j < E) {
            const size_t i = base + lane + 64 * j;
            v[j] = xf ? static_cast<const float*>(x)[i] : (float)static_cast<const half_t*>(x)[i];
            s += v[j];
        }
    }
    const float mu = wave_sum(s) / C;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < EMAX; ++j)
        if (j < E) q += (v[j] - mu) * (v[j] - mu);
    const float rstd = 1.0f / sqrtf(wave_sum(q) / C + eps);
#pragma unroll
    for (int j = 0; j < EMAX; ++j) {
        if (j >= E) continue;
        const int e = lane + 64 * j;
        const size_t i = base + e;
        float o = (v[j] - mu) * rstd * gamma[e] + beta[e];
        if (flags & VDK_LN_GELU) o = gelu_erf(o);
        if (acc) {
            const float src = (flags & VDK_LN_ACC_INPUT) ? v[j] : o;
            acc[i] = (flags & VDK_LN_ACC_INIT) ? acc_w * src : acc[i] + acc_w * src;
        }
        if (y) {
            if (flags & VDK_LN_Y_F32) static_cast<float*>(y)[i] = o;
            else static_cast<half_t*>(y)[i] = (half_t)o;
        }
    }
}

// Same for C = 256 * NV: lane l owns the 4-element groups l + 64 j (j < NV),
// moved as 16-byte (f32) / 8-byte (f16) vectors.
template <int NV>
__global__ __launch_bounds__(256) void layer_norm_vec_kernel(const void* __restrict__ x, int rows,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta, float eps, int flags,
                                                             void* __restrict__ y, float* __restrict__ acc,
                                                             float acc_w) {
    constexpr int C = 256 * NV;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const bool xf = flags & VDK_LN_X_F32;
    const size_t base = (size_t)row * C;
    float v[NV][4];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const size_t i = base + 4 * (lane + 64 * j);
        if (xf) {
            const float4v u = *reinterpret_cast<const float4v*>(static_cast<const float*>(x) + i);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[j][e] = u[e];
        } else {
            const half4 u = *reinterpret_cast<const half4*>(static_cast<const half_t*>(x) + i);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[j][e] = (float)u[e];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) s += v[j][e];
    }
    const float mu = wave_sum(s) / C;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) q += (v[j][e] - mu) * (v[j][e] - mu);
    const float rstd = 1.0f / sqrtf(wave_sum(q) / C + eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e0 = 4 * (lane + 64 * j);
        const size_t i = base + e0;
        const float4v gm = *reinterpret_cast<const float4v*>(gamma + e0);
        const float4v bt = *reinterpret_cast<const float4v*>(beta + e0);
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            o[e] = (v[j][e] - mu) * rstd * gm[e] + bt[e];
            if (flags & VDK_LN_GELU) o[e] = gelu_erf(o[e]);
        }
        if (acc) {
            float4v a = (flags & VDK_LN_ACC_INIT) ? float4v{0.0f, 0.0f, 0.0f, 0.0f}
                                                  : *reinterpret_cast<const float4v*>(acc + i);
#pragma unroll
            for (int e = 0; e < 4; ++e) a[e] += acc_w * ((flags & VDK_LN_ACC_INPUT) ? v[j][e] : o[e]);
            *reinterpret_cast<float4v*>(acc + i) = a;
        }
        if (y) {
            if (flags & VDK_LN_Y_F32) {
                *reinterpret_cast<float4v*>(static_cast<float*>(y) + i) = float4v{o[0], o[1], o[2], o[3]};
            } else {
                half4 h;
#pragma unroll
                for (int e = 0; e < 4; ++e) h[e] = (half_t)o[e];
                *reinterpret_cast<half4*>(static_cast<half_t*>(y) + i) = h;
            }
        }
    }
}

// ---- self-attention per (clip, head), head_dim 64 ----
// qkv [B][T][3H] f16 (q | k | v, head h at columns h*64 of each), out [B][T][H].
// A workgroup (4 waves) owns 128 queries of one (clip, head); wave w owns 32.
// Scores are computed transposed, S^T = K Q^T (32 keys x 32 queries per MFMA
// block), so each lane holds one query's column: the row max / sum need one
// exchange with lane ^ 32, and P^T is already the B operand of
// O^T += V^T P^T.  MFMA k-slot j of lane half h stands for key
// 16c + 4h + j (j < 4) or 16c + 8 + 4h + (j - 4): the keys the S^T
// accumulator gives that lane, so P^T needs no shuffle; V is staged in LDS
// transposed ([dim][key]) so the matching A operand is two 8-byte reads.
constexpr int kHD = 64, kKB = 64, kKR = kHD + 8, kVR = kKB + 8;

// NWQ waves per workgroup (32 queries each); the next key block's K and V rows
// are loaded into registers while the current block is computed.
template <int NWQ>
__global__ __launch_bounds__(64 * NWQ) void attention_kernel(const half_t* __restrict__ qkv, int T, int H,
                                                             float scale_log2, half_t* __restrict__ out) {
    constexpr int NT = 64 * NWQ;
    constexpr int NCH = kKB * kHD / 8;          // 16-byte K (and V) chunks per block
    constexpr int NLD = (NCH + NT - 1) / NT;     // per thread (the last slot partial when NT does not divide NCH)
    __shared__ __attribute__((aligned(16))) half_t sK[kKB * kKR];   // [key][dim]
    __shared__ __attribute__((aligned(16))) half_t sVs[kKB * kKR];  // [key][dim] staging of V
    __shared__ __attribute__((aligned(16))) half_t sV[kHD * kVR];   // [dim][key]
    const int b = blockIdx.z, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hl = lane >> 5, lr = lane & 31;
    const size_t rs = 3 * (size_t)H;
    const half_t* base = qkv + (size_t)b * T * rs;
    const int q0 = blockIdx.x * 32 * NWQ + wave * 32;
    const int qr = q0 + lr < T ? q0 + lr : T - 1;
    half8 qf[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
        qf[kk] = *reinterpret_cast<const half8*>(base + qr * rs + h * kHD + 16 * kk + 8 * hl);
    float16v o0, o1;
#pragma unroll
    for (int r = 0; r < 16; ++r) { o0[r] = 0.0f; o1[r] = 0.0f; }
    float m = -INFINITY, l = 0.0f;
    const half8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
    half8 kn[NLD], vn[NLD];
    // 32-bit element offsets within the clip (T * 3H stays far below 2^31)
    int koff[NLD];
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
        const int i = tid + j * NT;
        koff[j] = (i >> 3) * (int)rs + h * kHD + (i & 7) * 8 + H;
    }
    auto fetch = [&](int kb) {
#pragma unroll
        for (int j = 0; j < NLD; ++j) {
            const int i = tid + j * NT, kg = kb + (i >> 3);
            const half_t* src = base + (koff[j] + kb * (int)rs);
            const bool ok = (NCH % NT == 0 || i < NCH) && kg < T;
            kn[j] = ok ? *reinterpret_cast<const half8*>(src) : zero8;
            vn[j] = ok ? *reinterpret_cast<const half8*>(src + H) : zero8;
        }
    };
    fetch(0);
    for (int kb = 0; kb < T; kb += kKB) {
        __syncthreads();   // the previous block's operands are no longer read
#pragma unroll
        for (int j = 0; j < NLD; ++j) {
            const int i = tid + j * NT, key = i >> 3, d0 = (i & 7) * 8;
            if (NCH % NT != 0 && i >= NCH) continue;
            *reinterpret_cast<half8*>(&sK[key * kKR + d0]) = kn[j];
            *reinterpret_cast<half8*>(&sVs[key * kKR + d0]) = vn[j];
        }
        __syncthreads();
        if (kb + kKB < T) fetch(kb + kKB);
        // V transposed through the staging rows: item (dim d, keys 8g .. 8g+7)
        // gathers one dim of 8 key rows (a wave's 64 lanes read 64 dims of one
        // row) and writes them as one 16-byte chunk of the [dim][key] tile
        // (2-byte scattered writes had made most LDS cycles bank conflicts)
        for (int it = tid; it < kHD * (kKB / 8); it += NT) {
            const int d = it & (kHD - 1), g = it >> 6;
            half8 col;
#pragma unroll
            for (int e = 0; e < 8; ++e) col[e] = sVs[(8 * g + e) * kKR + d];
            *reinterpret_cast<half8*>(&sV[d * kVR + 8 * g]) = col;
        }
        __syncthreads();
        float16v s[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s[kt][r] = 0.0f;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const half8 a = *reinterpret_cast<const half8*>(&sK[(kt * 32 + lr) * kKR + 16 * kk + 8 * hl]);
                s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[kk], s[kt], 0, 0, 0);
            }
        }
        // s[kt][r]: key kb + 32 kt + 8 (r / 4) + 4 hl + r % 4 of query q0 + lr
        // (keys past T masked, in the last block only)
        float mx = -INFINITY;
        if (kb + kKB <= T) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float v = s[kt][r] * scale_log2;
                    s[kt][r] = v;
                    mx = fmaxf(mx, v);
                }
        } else {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kb + kt * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
                    const float v = key < T ? s[kt][r] * scale_log2 : -INFINITY;
                    s[kt][r] = v;
                    mx = fmaxf(mx, v);
                }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m, mx);   // finite: every block holds a key < T
        // v_exp_f32 directly: it differs from exp2f only below 2^-126, where
        // p rounds to an f16 zero and is nothing against the row sum (>= 1)
        const float alpha = __builtin_amdgcn_exp2f(m - m_new);
        float ls = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = __builtin_amdgcn_exp2f(s[kt][r] - m_new);
                s[kt][r] = p;
                ls += p;
            }
        ls += __shfl_xor(ls, 32, 64);
        l = l * alpha + ls;
        m = m_new;
#pragma unroll
        for (int r = 0; r < 16; ++r) { o0[r] *= alpha; o1[r] *= alpha; }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            half8 pb;
#pragma unroll
            for (int j = 0; j < 8; ++j) pb[j] = (half_t)s[c >> 1][8 * (c & 1) + j];
            const int kc = 16 * c + 4 * hl;
            const half4 a0l = *reinterpret_cast<const half4*>(&sV[lr * kVR + kc]);
            const half4 a0h = *reinterpret_cast<const half4*>(&sV[lr * kVR + kc + 8]);
            const half4 a1l = *reinterpret_cast<const half4*>(&sV[(lr + 32) * kVR + kc]);
            const half4 a1h = *reinterpret_cast<const half4*>(&sV[(lr + 32) * kVR + kc + 8]);
            const half8 a0 = {a0l[0], a0l[1], a0l[2], a0l[3], a0h[0], a0h[1], a0h[2], a0h[3]};
            const half8 a1 = {a1l[0], a1l[1], a1l[2], a1l[3], a1h[0], a1h[1], a1h[2], a1h[3]};
            o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, pb, o0, 0, 0, 0);
            o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, pb, o1, 0, 0, 0);
        }
    }
    if (q0 + lr >= T) return;
    const float inv = 1.0f / l;
    half_t* dst = out + ((size_t)b * T + q0 + lr) * H + h * kHD;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int d = 8 * g + 4 * hl;
        half4 v0, v1;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v0[e] = (half_t)(o0[4 * g + e] * inv);
            v1[e] = (half_t)(o1[4 * g + e] * inv);
        }
        *reinterpret_cast<half4*>(dst + d) = v0;
        *reinterpret_cast<half4*>(dst + 32 + d) = v1;
    }
}

// ---- positional conv embedding (src/analyze_w2v2.cpp:280-326) ----
// Grouped 1-D conv with a long kernel, its bias, GELU and the residual:
//   y[b][t][gC + o] = x[b][t][gC + o]
//                     + gelu(bias[gC + o] + sum_k sum_i W[g][o][k][i] x[b][t + k - pad][gC + i])
// for C = ICG channels per group.  An implicit GEMM per (clip, group) whose
// im2col rows are the same input frames shifted by one per tap, so a
// workgroup stages its frames' input halo (kPosTT + K - 1 rows of the group's
// ICG channels, zero outside the clip) in LDS once and runs every tap from it;
// the weights of tap k ([64 padded outputs][ICG]) are double-buffered through
// LDS.  MFMA 32x32x16: M = 32 frames, N = 32 outputs, K = 16 channels; each
// of the 3 waves owns 64 frames x 64 outputs (2 x 2 blocks).
constexpr int kPosTT = 192, kPosMaxK = 128;

template <int ICG>
__global__ __launch_bounds__(192) void pos_conv_kernel(const half_t* __restrict__ x, const half_t* __restrict__ w,
                                                       const float* __restrict__ bias, float* __restrict__ y, int T,
                                                       int H, int K, int pad) {
    constexpr int RS = ICG + 8;              // halo / weight row stride in halfs (16 B of padding)
    constexpr int CH = ICG / 8;              // 16-byte chunks per row
    constexpr int NWCH = 64 * CH;            // chunks per tap of weights
    constexpr int WPT = (NWCH + 191) / 192;  // weight chunks per thread
    __shared__ __attribute__((aligned(16))) half_t sx[(kPosTT + kPosMaxK - 1) * RS];
    __shared__ __attribute__((aligned(16))) half_t sw[2][64 * RS];
    const int b = blockIdx.z, g = blockIdx.y, t0 = blockIdx.x * kPosTT;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 31, hl = lane >> 5;
    const size_t cb = (size_t)g * ICG;
    const half8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
    // input halo: row r is frame t0 - pad + r
    const int rows = kPosTT + K - 1;
    for (int i = tid; i < rows * CH; i += 192) {
        const int r = i / CH, c = i - r * CH, f = t0 - pad + r;
        const half8 v = (f >= 0 && f < T) ? *reinterpret_cast<const half8*>(x + ((size_t)b * T + f) * H + cb + c * 8)
                                          : zero8;
        *reinterpret_cast<half8*>(&sx[r * RS + c * 8]) = v;
    }
    const half_t* wg = w + (size_t)g * 64 * K * ICG;
    half8 wr[WPT];
    auto fetch_w = [&](int k) {
#pragma unroll
        for (int j = 0; j < WPT; ++j) {
            const int i = tid + j * 192;
            wr[j] = zero8;
            if (i < NWCH) {
                const int o = i / CH, c = i - o * CH;
                wr[j] = *reinterpret_cast<const half8*>(wg + ((size_t)o * K + k) * ICG + c * 8);
            }
        }
    };
    auto stash_w = [&](int buf) {
#pragma unroll
        for (int j = 0; j < WPT; ++j) {
            const int i = tid + j * 192;
            if (i < NWCH) {
                const int o = i / CH, c = i - o * CH;
                *reinterpret_cast<half8*>(&sw[buf][o * RS + c * 8]) = wr[j];
            }
        }
    };
    float16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    fetch_w(0);
    stash_w(0);
    __syncthreads();
    const int f0 = wave * 64 + lr;   // this lane's A row (frame) in M block 0
    for (int k = 0; k < K; ++k) {
        const int buf = k & 1;
        if (k + 1 < K) fetch_w(k + 1);
#pragma unroll
        for (int kk = 0; kk < ICG / 16; ++kk) {
            const int c = 16 * kk + 8 * hl;
            half8 a[2], bw[2];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) a[mi] = *reinterpret_cast<const half8*>(&sx[(f0 + 32 * mi + k) * RS + c]);
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) bw[ni] = *reinterpret_cast<const half8*>(&sw[buf][(32 * ni + lr) * RS + c]);
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[mi], bw[ni], acc[mi][ni], 0, 0, 0);
        }
        if (k + 1 < K) stash_w(buf ^ 1);
        __syncthreads();
    }
    // lane holds output o = 32 ni + lr, frames 8 (r / 4) + 4 hl + r % 4 of each 32-frame block
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
        const int o = 32 * ni + lr;
        if (o >= ICG) continue;
        const float bo = bias[cb + o];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = t0 + wave * 64 + 32 * mi + 8 * (r >> 2) + 4 * hl + (r & 3);
                if (t >= T) continue;
                const size_t i = ((size_t)b * T + t) * H + cb + o;
                y[i] = (float)x[i] + gelu_erf(acc[mi][ni][r] + bo);
            }
    }
}

// ---- per-clip mean over time: out[b][c] = [out +] w * mean_t x[b][t][c] ----
// A workgroup covers 256 channels of one clip: 64 lanes x 4 channels (one
// 8- or 16-byte load per row) x 16 time partitions, f64 sums combined in a
// fixed order.  C % 4 == 0.
__global__ __launch_bounds__(1024) void time_mean_kernel(const void* __restrict__ x, int x_f32, int T, int C, float w,
                                                         int accumulate, float* __restrict__ out) {
    __shared__ double part[16][256];
    const int cg = threadIdx.x & 63, tp = threadIdx.x >> 6;
    const int c = blockIdx.x * 256 + cg * 4, b = blockIdx.y;
    double s[4] = {0.0, 0.0, 0.0, 0.0};
    if (c < C) {
#pragma unroll 4   // four rows' loads in flight; the sums keep their order
        for (int t = tp; t < T; t += 16) {
            const size_t i = ((size_t)b * T + t) * C + c;
            if (x_f32) {
                const float4v v = *reinterpret_cast<const float4v*>(static_cast<const float*>(x) + i);
#pragma unroll
                for (int e = 0; e < 4; ++e) s[e] += (double)v[e];
            } else {
                const half4 v = *reinterpret_cast<const half4*>(static_cast<const half_t*>(x) + i);
#pragma unroll
                for (int e = 0; e < 4; ++e) s[e] += (double)(float)v[e];
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) part[tp][cg * 4 + e] = s[e];
    __syncthreads();
    if (threadIdx.x < 256) {
        const int cc = blockIdx.x * 256 + threadIdx.x;
        if (cc < C) {
            double a = 0.0;
#pragma unroll
            for (int p = 0; p < 16; ++p) a += part[p][threadIdx.x];
            const float m = (float)(a / T);
            const size_t o = (size_t)b * C + cc;
            out[o] = accumulate ? out[o] + w * m : w * m;
        }
    }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int conv0_frames(int n, int K, int S) { return n < K ? 0 : (n - K) / S + 1; }

size_t conv0_work(int batch, int n, int C, int K, int S) {
    // per-chunk moment partials [B][nchunk][NP] and sums [B][NP] f64
    // (NP = K + K(K+1)/2), then scale / shift [B][C] f32
    const size_t np = (size_t)K + (size_t)K * (K + 1) / 2;
    const size_t nchunk = (size_t)(conv0_frames(n, K, S) + kFrames - 1) / kFrames;
    return (size_t)batch * (np * 8 * (nchunk + 1) + (size_t)C * 8) + 256;
}

}  // namespace
}  // namespace vdk

using namespace vdk;

extern "C" int vdk_wave_stats(const float* d_x, int batch, int n, float eps, float* d_stats, void* stream) {
    return guarded([&] {
        require(d_x && d_stats, "wave_stats: NULL device pointer");
        require(batch > 0 && n > 0, "wave_stats: empty input");
        hipLaunchKernelGGL(wave_stats_kernel, dim3(batch), dim3(1024), 0, static_cast<hipStream_t>(stream), d_x, n,
                           eps, d_stats);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" size_t vdk_w2v2_conv0_workspace_size(int batch, int n, int C, int K, int S) {
    if (batch <= 0 || C <= 0 || K <= 0 || S <= 0 || conv0_frames(n, K, S) <= 0) return 0;
    return conv0_work(batch, n, C, K, S);
}

extern "C" int vdk_w2v2_conv0(const float* d_x, int batch, int n, const float* d_stats, const float* d_w,
                              const float* d_bias, int C, int K, int S, int norm, const float* d_gamma,
                              const float* d_beta, float eps, void* d_work, size_t work_bytes, void* d_y,
                              void* stream) {
    return guarded([&] {
        require(d_x && d_w && d_y, "w2v2_conv0: NULL device pointer");
        require(batch > 0 && K >= 1 && K <= kMaxK && S >= 1 && S <= kMaxS, "w2v2_conv0: kernel 1..16, stride 1..8");
        require(C == 256 || C == 512 || C == 1024, "w2v2_conv0: channels must be 256, 512 or 1024");
        require(norm >= 0 && norm <= 2, "w2v2_conv0: norm must be 0 (none), 1 (group) or 2 (layer)");
        require(norm == 0 || (d_gamma && d_beta), "w2v2_conv0: a norm needs gamma and beta");
        const int T0 = conv0_frames(n, K, S);
        require(T0 > 0, "w2v2_conv0: clip shorter than the kernel");
        require((size_t)batch * n < (1ull << 31) && (size_t)batch * T0 * C < (1ull << 31),
                "w2v2_conv0: input too large for one launch");
        require(al16(d_y), "w2v2_conv0: output must be 16-byte aligned");
        hipStream_t s = static_cast<hipStream_t>(stream);
        const float* scale = nullptr;
        const float* shift = nullptr;
        if (norm == 1) {
            require(d_work && work_bytes >= conv0_work(batch, n, C, K, S), "w2v2_conv0: workspace too small");
            const int NP = K + K * (K + 1) / 2;
            const int nchunk = (T0 + kFrames - 1) / kFrames;
            double* part = static_cast<double*>(d_work);
            double* mom = part + (size_t)batch * nchunk * NP;
            float* sc = reinterpret_cast<float*>(mom + (size_t)batch * NP);
            float* sh = sc + (size_t)batch * C;
            hipLaunchKernelGGL(conv0_moments_kernel, dim3(nchunk, batch), dim3(256), 0, s, d_x, n, d_stats, K, S, T0,
                               part);
            VDK_HIP(hipGetLastError());
            hipLaunchKernelGGL(conv0_moments_reduce_kernel, dim3(batch), dim3(256), 0, s, part, nchunk, NP, mom);
            VDK_HIP(hipGetLastError());
            hipLaunchKernelGGL(conv0_finalize_kernel, dim3(cdiv(C, 256), batch), dim3(256), 0, s, mom, d_w, d_bias,
                               C, K, T0, d_gamma, d_beta, eps, sc, sh);
            VDK_HIP(hipGetLastError());
            scale = sc;
            shift = sh;
        }
        half_t* y = static_cast<half_t*>(d_y);
        const dim3 g(cdiv(T0, kApplyFrames), batch);
        switch (C) {
            case 256:
                launch_conv0_apply<4>(g, s, d_x, n, d_stats, d_w, d_bias, K, S, T0, norm, scale, shift, d_gamma,
                                      d_beta, eps, y);
                break;
            case 512:
                launch_conv0_apply<8>(g, s, d_x, n, d_stats, d_w, d_bias, K, S, T0, norm, scale, shift, d_gamma,
                                      d_beta, eps, y);
                break;
            default:
                launch_conv0_apply<16>(g, s, d_x, n, d_stats, d_w, d_bias, K, S, T0, norm, scale, shift, d_gamma,
                                       d_beta, eps, y);
                break;
        }
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_layer_norm(const void* d_x, int rows, int C, const float* d_gamma, const float* d_beta, float eps,
                              int flags, void* d_y, float* d_acc, float acc_w, void* stream) {
    return guarded([&] {
        require(d_x && d_gamma && d_beta && (d_y || d_acc), "layer_norm: NULL device pointer");
        require(rows > 0 && C > 0 && C % 64 == 0 && C <= 4096, "layer_norm: C must be a multiple of 64 up to 4096");
        require((flags & ~(VDK_LN_X_F32 | VDK_LN_Y_F32 | VDK_LN_GELU | VDK_LN_ACC_INPUT | VDK_LN_ACC_INIT)) == 0,
                "layer_norm: unknown flag");
        hipStream_t s = static_cast<hipStream_t>(stream);
        const dim3 g(cdiv(rows, 4));
        const bool vec = C % 256 == 0 && al16(d_x) && al16(d_gamma) && al16(d_beta) && al16(d_y) && al16(d_acc);
#define VDK_LN_VEC(NV)                                                                                              \
    case NV:                                                                                                        \
        hipLaunchKernelGGL(layer_norm_vec_kernel<NV>, g, dim3(256), 0, s, d_x, rows, d_gamma, d_beta, eps, flags, \
                           d_y, d_acc, acc_w);                                                                     \
        break;
        if (vec) {
            switch (C / 256) {
                VDK_LN_VEC(1) VDK_LN_VEC(2) VDK_LN_VEC(3) VDK_LN_VEC(4) VDK_LN_VEC(6) VDK_LN_VEC(8)
                VDK_LN_VEC(12) VDK_LN_VEC(16)
                default: goto scalar;
            }
            VDK_HIP(hipGetLastError());
            return;
        }
#undef VDK_LN_VEC
    scalar:
        if (C <= 1024)
            hipLaunchKernelGGL(layer_norm_kernel<16>, g, dim3(256), 0, s, d_x, rows, C, d_gamma, d_beta, eps, flags,
                               d_y, d_acc, acc_w);
        else
            hipLaunchKernelGGL(layer_norm_kernel<64>, g, dim3(256), 0, s, d_x, rows, C, d_gamma, d_beta, eps, flags,
                               d_y, d_acc, acc_w);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_attention(const void* d_qkv, int batch, int T, int n_heads, int head_dim, float scale,
                             void* d_out, void* stream) {
    return guarded([&] {
        require(d_qkv && d_out, "attention: NULL device pointer");
        require(batch > 0 && T > 0 && n_heads > 0, "attention: empty shape");
        require(head_dim == kHD, "attention: head_dim must be 64");
        require(al16(d_qkv) && al16(d_out), "attention: buffers must be 16-byte aligned");
        const size_t H = (size_t)n_heads * head_dim;
        require((size_t)batch * T * 3 * H < (1ull << 31), "attention: too many tokens for one launch");
        require(T <= 65535 * 64 && n_heads <= 65535 && batch <= 65535, "attention: grid too large");
        hipStream_t s = static_cast<hipStream_t>(stream);
        const half_t* q = static_cast<const half_t*>(d_qkv);
        half_t* o = static_cast<half_t*>(d_out);
        const float sl2 = scale * 1.4426950408889634f;
        // up to 160 frames (clips up to ~3.2 s): the whole clip's queries in one
        // 5-wave workgroup per (clip, head), so K and V are staged once;
        // short clips: 64 queries per workgroup (less padding past T); long
        // ones: 128, so each staged key block serves more queries
        if (T <= 160)
            hipLaunchKernelGGL(attention_kernel<5>, dim3(1, n_heads, batch), dim3(320), 0, s, q, T, (int)H, sl2, o);
        else if (T <= 512)
            hipLaunchKernelGGL(attention_kernel<2>, dim3(cdiv(T, 64), n_heads, batch), dim3(128), 0, s, q, T, (int)H,
                               sl2, o);
        else
            hipLaunchKernelGGL(attention_kernel<4>, dim3(cdiv(T, 128), n_heads, batch), dim3(256), 0, s, q, T, (int)H,
                               sl2, o);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_time_mean_acc(const void* d_x, int x_f32, int batch, int T, int C, float w, int accumulate,
                                 float* d_out, void* stream) {
    return guarded([&] {
        require(d_x && d_out, "time_mean: NULL device pointer");
        require(batch > 0 && T > 0 && C > 0 && C % 4 == 0, "time_mean: C must be a positive multiple of 4");
        require(al16(d_x), "time_mean: input must be 16-byte aligned");
        hipLaunchKernelGGL(time_mean_kernel, dim3(cdiv(C, 256), batch), dim3(1024), 0, static_cast<hipStream_t>(stream),
                           d_x, x_f32 ? 1 : 0, T, C, w, accumulate ? 1 : 0, d_out);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_time_mean(const void* d_x, int x_f32, int batch, int T, int C, float* d_out, void* stream) {
    return guarded([&] {
        require(d_x && d_out, "time_mean: NULL device pointer");
        require(batch > 0 && T > 0 && C > 0 && C % 4 == 0, "time_mean: C must be a positive multiple of 4");
        require(al16(d_x), "time_mean: input must be 16-byte aligned");
        hipLaunchKernelGGL(time_mean_kernel, dim3(cdiv(C, 256), batch), dim3(1024), 0, static_cast<hipStream_t>(stream),
                           d_x, x_f32 ? 1 : 0, T, C, 1.0f, 0, d_out);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_pos_conv(const void* d_x, int batch, int T, int H, int groups, const void* d_w, const float* d_bias,
                            int K, int pad, float* d_y, void* stream) {
    return guarded([&] {
        require(d_x && d_w && d_bias && d_y, "pos_conv: NULL device pointer");
        require(batch > 0 && T > 0 && groups > 0 && H % groups == 0, "pos_conv: groups must divide H");
        const int icg = H / groups;
        require(icg == 48 || icg == 64, "pos_conv: channels per group must be 48 or 64");
        require(K >= 1 && K <= kPosMaxK && pad >= 0 && pad < K, "pos_conv: kernel 1..128, pad < kernel");
        require(al16(d_x) && al16(d_w), "pos_conv: buffers must be 16-byte aligned");
        require((size_t)batch * T * H < (1ull << 31), "pos_conv: too many frames for one launch");
        require(batch <= 65535 && groups <= 65535, "pos_conv: grid too large");
        const dim3 grid(cdiv(T, kPosTT), groups, batch);
        hipStream_t s = static_cast<hipStream_t>(stream);
        const half_t* x = static_cast<const half_t*>(d_x);
        const half_t* w = static_cast<const half_t*>(d_w);
        if (icg == 48)
            hipLaunchKernelGGL(pos_conv_kernel<48>, grid, dim3(192), 0, s, x, w, d_bias, d_y, T, H, K, pad);
        else
            hipLaunchKernelGGL(pos_conv_kernel<64>, grid, dim3(192), 0, s, x, w, d_bias, d_y, T, H, K, pad);
        VDK_HIP(hipGetLastError());
    });
}

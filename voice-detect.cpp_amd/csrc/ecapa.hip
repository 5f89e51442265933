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
//  * channel_stats (asp_stats), asp_attn_pool / asp_pool: attentive statistics
//    pooling with global context
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

__global__ __launch_bounds__(256) void feats_tmajor_kernel(const float* __restrict__ f,
                                                           const float* __restrict__ rmean, int B, int C, int T,
                                                           int pad, int Cpad, half_t* __restrict__ out) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    const int Tp = T + 2 * pad;
    if (i >= (long)B * Tp * Cpad) return;
    const int c = (int)(i % Cpad);
    const long r = i / Cpad;
    const int j = (int)(r % Tp), b = (int)(r / Tp);
    const float v = c < C ? f[((size_t)b * C + c) * T + reflect_idx(j, pad, T)] - (rmean ? rmean[(size_t)b * C + c] : 0.0f)
                          : 0.0f;
    out[i] = (half_t)v;
}

// The same map through an LDS tile: workgroup (64-frame block, clip) reads
// the frames of every mel row along time (coalesced) and stores each frame's
// Cpad channels as 16-byte chunks.  Cpad % 8 == 0, Cpad <= kFtC.
constexpr int kFtF = 64, kFtC = 128;
__global__ __launch_bounds__(256) void feats_tmajor_tiled_kernel(const float* __restrict__ f,
                                                                 const float* __restrict__ rmean, int C, int T,
                                                                 int pad, int Cpad, half_t* __restrict__ out) {
    __shared__ float sv[kFtC][kFtF + 1];
    const int Tp = T + 2 * pad, j0 = blockIdx.x * kFtF, b = blockIdx.y, tid = threadIdx.x;
    const int nf = Tp - j0 < kFtF ? Tp - j0 : kFtF;
    for (int i = tid; i < C * kFtF; i += 256) {
        const int c = i / kFtF, jj = i - c * kFtF;
        if (jj < nf)
            sv[c][jj] = f[((size_t)b * C + c) * T + reflect_idx(j0 + jj, pad, T)] -
                        (rmean ? rmean[(size_t)b * C + c] : 0.0f);
    }
    __syncthreads();
    const int C8 = Cpad / 8;
    for (int i = tid; i < nf * C8; i += 256) {
        const int jj = i / C8, c0 = (i - jj * C8) * 8;
        half8 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = c0 + e < C ? (half_t)sv[c0 + e][jj] : (half_t)0.0f;
        *reinterpret_cast<half8*>(out + ((size_t)b * Tp + j0 + jj) * Cpad + c0) = h;
    }
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

// Per-channel sums over time of x [B][T][xs] f16 (and, MODE 1, of x^2): a
// workgroup covers 128 channels (16 lanes x 8 channels, 16-byte loads) of
// one clip in 16 time partitions; f64 partition sums combined in a fixed
// order.  MODE 0: out [B][C] = mean; MODE 1: out [B][2C] = [mean ;
// sqrt(max(var, eps))] with var = E[x^2] - mean^2 in f64 (x is f16, so the
// cancellation costs ~1e-16 of E[x^2], far below the statistic's rounding).
template <int MODE>
__global__ __launch_bounds__(256) void channel_stats_kernel(const half_t* __restrict__ x, int xs, int T, int C,
                                                            float eps, float* __restrict__ out) {
    constexpr int NP = 16, CW = 128;
    __shared__ double sp[NP][CW], sq[MODE == 1 ? NP : 1][CW];
    const int lx = threadIdx.x & 15, tp = threadIdx.x >> 4;
    const int c8 = blockIdx.x * CW + lx * 8, b = blockIdx.y;
    double s[8], q[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) { s[e] = 0.0; q[e] = 0.0; }
    if (c8 < C) {
        const half_t* p = x + (size_t)b * T * xs + c8;
#pragma unroll 4   // four rows' loads in flight; the sums keep their order
        for (int t = tp; t < T; t += NP) {
            const half8 v = *reinterpret_cast<const half8*>(p + (size_t)t * xs);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const double d = (double)(float)v[e];
                s[e] += d;
                if constexpr (MODE == 1) q[e] += d * d;
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        sp[tp][lx * 8 + e] = s[e];
        if constexpr (MODE == 1) sq[tp][lx * 8 + e] = q[e];
    }
    __syncthreads();
    const int c = blockIdx.x * CW + threadIdx.x;
    if (threadIdx.x < CW && c < C) {
        double S = 0.0, Q = 0.0;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            S += sp[i][threadIdx.x];
            if constexpr (MODE == 1) Q += sq[i][threadIdx.x];
        }
        const double mean = S / T;
        if constexpr (MODE == 0) {
            out[(size_t)b * C + c] = (float)mean;
        } else {
            float v = (float)(Q / T - mean * mean);
            if (v < eps) v = eps;
            out[(size_t)b * 2 * C + c] = (float)mean;
            out[(size_t)b * 2 * C + C + c] = sqrtf(v);
        }
    }
}

// y = x * g + res with g = sigmoid(gate) (SIG) or g = gate, the sigmoid
// already taken once per (clip, channel).
template <bool SIG>
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
    const float4v ga = *reinterpret_cast<const float4v*>(gate + (size_t)b * C + c);
    const float4v gb = *reinterpret_cast<const float4v*>(gate + (size_t)b * C + c + 4);
    half8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float gv = e < 4 ? ga[e] : gb[e - 4];
        const float g = SIG ? 1.0f / (1.0f + expf(-gv)) : gv;
        float v = (float)xv[e] * g + (float)rv[e];
        asm volatile("" : "+v"(v));   // rounded to f32, then to f16 (no one-rounding v_fma_mix*_f16)
        o[e] = (half_t)v;
    }
    *reinterpret_cast<half8*>(y + r * ys + c) = o;
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

// ---------------------------------------------------------------------------
// asp_attn_pool_kernel: the attention logits and the pooling in one launch
// (src/encoder.cpp:283-294): l[t][c] = b[c] + sum_k W[c][k] a1[t][k] (the
// 1x1 asp.conv), softmax over time per channel, then
//   mu = sum_t a_t x_t,  sd = sqrt(clamp(sum_t a_t (x_t - mu)^2, eps)).
// The logits never reach memory: a workgroup owns 64 channels of one clip
// and streams the clip's frames once, in chunks of 64 (the chunk's a1 rows,
// all ATT channels, and x rows, its 64 channels, DMA'd two chunks ahead
// into a three-stage LDS ring), computing each 32-channel x 32-frame logit
// block with MFMAs (W from registers, a1 from LDS, the bias added after the
// K sum like the conv kernels).  The chunk's f32 logits then take the
// bytes of its a1 rows, and each thread pools one channel over a quarter
// of the chunk's frames: an online softmax state (running max m and the
// sums z = sum e, s1 = sum e x, s2 = sum e x^2 with e = exp(l - m), in
// f64) rescaled once per chunk by the chunk's own max.  The four quarters
// merge in a fixed order.  Then mu = s1 / z and var = s2 / z - mu^2 (f64:
// the cancellation loses ~1e-16 mu^2, far below the f16 resolution of x).
// Rows 256 / 128 bytes wide with their 16-byte chunks XOR-swizzled by row,
// so the MFMA operand reads hit 16 distinct chunks per 16 lanes.
// ---------------------------------------------------------------------------
constexpr int kAspChunk = 64;   // frames per LDS chunk
constexpr int kAspStages = 3;

template <int ATT>
struct AspLds {
    static constexpr int A_ROW = ATT * 2, X_ROW = 128;                 // bytes per frame
    static constexpr int A_BYTES = kAspChunk * A_ROW, X_BYTES = kAspChunk * X_ROW;
    static constexpr int STAGE = A_BYTES + X_BYTES;
    static constexpr int A_INS = A_BYTES / 1024, X_INS = X_BYTES / 1024, INS = A_INS + X_INS;
    static_assert(ATT % 16 == 0 && A_BYTES % 1024 == 0 && INS % 4 == 0, "whole DMA instructions, even per wave");
};

// DMA of frames [t0, t0 + 64) of clip b: a1 rows (ATT channels) and x rows
// (the workgroup's 64 channels from c0); frames past T read as zeros.
template <int ATT>
__device__ __forceinline__ void asp_issue(uint8_t* st, int4v ar, int4v xr, int as, int xs, int b, int T, int t0, int c0,
                                          int wave, int lane) {
    using G = AspLds<ATT>;
    constexpr int ACH = ATT / 8;   // 16-byte chunks per a1 row
#pragma unroll
    for (int i = 0; i < G::INS / 4; ++i) {
        const int ins = wave + 4 * i;
        uint32_t off;
        if (ins < G::A_INS) {
            const int slot = ins * 64 + lane, row = slot / ACH, pos = slot % ACH;
            const int g = pos ^ (row & (ACH - 1) & 15);   // global chunk held at this position
            const int t = t0 + row;
            off = t < T ? (uint32_t)((((size_t)b * T + t) * as + g * 8) * 2) : kOOB;
        } else {
            const int slot = (ins - G::A_INS) * 64 + lane, row = slot / 8, pos = slot % 8;
            const int g = pos ^ (row & 7);
            const int t = t0 + row;
            off = t < T ? (uint32_t)((((size_t)b * T + t) * xs + c0 + g * 8) * 2) : kOOB;
        }
        dma16(st + ins * 1024, ins < G::A_INS ? ar : xr, off);
    }
}

// One 32-channel x 32-frame block of logits into acc: channels c0 + cb*32 +
// (8g + 4*lhalf + e) for register g*4+e, frame tb*32 + lrow of the chunk.
template <int ATT>
__device__ __forceinline__ void asp_logits(const uint8_t* st, const half8* wf, int tb, int lrow, int lhalf,
                                           float16v& acc) {
    constexpr int ACH = ATT / 8;
    const int row = tb * 32 + lrow;
    const uint8_t* const ab = st + row * (ATT * 2);
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < ATT / 16; ++kk) {
        const int g = kk * 2 + lhalf;
        const half8 bf = *reinterpret_cast<const half8*>(ab + ((g ^ (row & (ACH - 1) & 15)) * 16));
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[kk], bf, acc, 0, 0, 0);
    }
}

// x (4 channels: register group g of this lane's channel block) of frame
// row `row` of a stage's swizzled x rows.
__device__ __forceinline__ half4 asp_x4(const uint8_t* xs_lds, int row, int cb, int g, int lhalf) {
    return *reinterpret_cast<const half4*>(xs_lds + row * 128 + (((cb * 4 + g) ^ (row & 7)) * 16) + lhalf * 8);
}

// Online-softmax state: running max and the sums scaled by exp(-m).
struct AspState {
    float m;
    double z, s1, s2;
};

// Merge of two states; commutative, so both lanes of a butterfly pair get
// the same bits.
__device__ __forceinline__ void asp_merge(AspState& a, const AspState& o) {
    if (o.m == -INFINITY) return;
    if (a.m == -INFINITY) { a = o; return; }
    const float M = fmaxf(a.m, o.m);
    const double f1 = (double)__expf(a.m - M), f2 = (double)__expf(o.m - M);
    a.z = a.z * f1 + o.z * f2;
    a.s1 = a.s1 * f1 + o.s1 * f2;
    a.s2 = a.s2 * f1 + o.s2 * f2;
    a.m = M;
}

template <int ATT>
__global__ __launch_bounds__(256, 2) void asp_attn_pool_kernel(const half_t* __restrict__ a1, int as,
                                                               const half_t* __restrict__ wc,
                                                               const float* __restrict__ bc,
                                                               const half_t* __restrict__ x, int xs, int T, int C,
                                                               float eps, float* __restrict__ out) {
    using G = AspLds<ATT>;
    static_assert(G::A_BYTES >= kAspChunk * 64 * 4, "a chunk's f32 logits fit its a1 rows");
    __shared__ __attribute__((aligned(1024))) uint8_t ring[kAspStages * G::STAGE];
    __shared__ float pm[4][64];            // per frame quarter: each channel's state
    __shared__ double pz[4][64], ps1[4][64], ps2[4][64];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int cb = wave & 1, tb = wave >> 1;   // 32-channel block, 32-frame block of the chunk
    const int b = blockIdx.y, c0 = blockIdx.x * 64;
    const int4v ar = dma_rsrc(a1, (uint32_t)((size_t)gridDim.y * T * as * 2));
    const int4v xr = dma_rsrc(x, (uint32_t)((size_t)gridDim.y * T * xs * 2));
    const int nq = (T + kAspChunk - 1) / kAspChunk;

    // A fragments of this wave's 32 channels and their biases (register
    // g*4+e: channel 8g + 4*lhalf + e of the block)
    half8 wf[ATT / 16];
#pragma unroll
    for (int kk = 0; kk < ATT / 16; ++kk)
        wf[kk] = *reinterpret_cast<const half8*>(wc + (size_t)(c0 + cb * 32 + lrow) * ATT + kk * 16 + lhalf * 8);
    float bv[16];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[g * 4 + e] = bc[c0 + cb * 32 + g * 8 + lhalf * 4 + e];
    __builtin_amdgcn_s_waitcnt(0);

    // pooling: thread = channel pc of the 64, frames fq * 16 .. + 15 of each chunk
    const int pc = tid & 63, fq = tid >> 6;
    AspState S{-INFINITY, 0.0, 0.0, 0.0};
    // chunks 0 and 1 go out together; then the ring stays two chunks ahead
    asp_issue<ATT>(ring, ar, xr, as, xs, b, T, 0, c0, wave, lane);
    if (nq > 1) asp_issue<ATT>(ring + G::STAGE, ar, xr, as, xs, b, T, kAspChunk, c0, wave, lane);
    int slot = 0;
    for (int q = 0; q < nq; ++q) {
        // this wave's share of chunk q has landed (at most chunk q+1's
        // instructions are younger; loads complete in issue order)
        if (q + 1 < nq) wait_vmcnt<G::INS / 4>();
        else __builtin_amdgcn_s_waitcnt(0);
        lds_barrier();   // everyone's; chunk q-1's stage is free for chunk q+2
        uint8_t* const st = ring + slot * G::STAGE;
        if (q + 2 < nq) {
            const int s2 = slot == 0 ? 2 : slot - 1;
            asp_issue<ATT>(ring + s2 * G::STAGE, ar, xr, as, xs, b, T, (q + 2) * kAspChunk, c0, wave, lane);
        }
        float16v acc;
        asp_logits<ATT>(st, wf, tb, lrow, lhalf, acc);
        lds_barrier();   // every wave has read the chunk's a1 rows: their bytes take the logits
        {   // l = acc + bias as f32 [frame][64 channels], 16-byte columns XOR-swizzled by frame
            const int row = tb * 32 + lrow;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int c4 = cb * 8 + g * 2 + lhalf;
                const float4v l4 = {acc[g * 4] + bv[g * 4], acc[g * 4 + 1] + bv[g * 4 + 1],
                                    acc[g * 4 + 2] + bv[g * 4 + 2], acc[g * 4 + 3] + bv[g * 4 + 3]};
                *reinterpret_cast<float4v*>(st + row * 256 + ((c4 ^ (row & 15)) * 16)) = l4;
            }
        }
        lds_barrier();
        {   // this thread's 16 frames: the chunk's max first, one rescale, then the sums
            const uint8_t* const xs_lds = st + G::A_BYTES;
            float lv[16];
            float mc = -INFINITY;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = fq * 16 + i;
                lv[i] = q * kAspChunk + row < T
                            ? *reinterpret_cast<const float*>(st + row * 256 + (((pc >> 2) ^ (row & 15)) * 16) +
                                                              (pc & 3) * 4)
                            : -INFINITY;
                mc = fmaxf(mc, lv[i]);
            }
            if (mc > -INFINITY) {   // (S.m - mn is -inf on the first update: the scale is 0)
                const float mn = fmaxf(S.m, mc);
                const double sc = (double)__expf(S.m - mn);
                S.z *= sc;
                S.s1 *= sc;
                S.s2 *= sc;
                S.m = mn;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int row = fq * 16 + i;
                    if (q * kAspChunk + row < T) {
                        const half_t xh = *reinterpret_cast<const half_t*>(
                            xs_lds + row * 128 + (((pc >> 3) ^ (row & 7)) * 16) + (pc & 7) * 2);
                        const double ex = (double)__expf(lv[i] - mn), xd = (double)(float)xh, ex_x = ex * xd;
                        S.z += ex;
                        S.s1 += ex_x;
                        S.s2 += ex_x * xd;
                    }
                }
            }
        }
        slot = slot == 2 ? 0 : slot + 1;
    }
    // the four frame quarters of each channel, merged in a fixed order
    pm[fq][pc] = S.m;
    pz[fq][pc] = S.z;
    ps1[fq][pc] = S.s1;
    ps2[fq][pc] = S.s2;
    __syncthreads();
    if (tid < 64) {
        AspState R{pm[0][tid], pz[0][tid], ps1[0][tid], ps2[0][tid]};
#pragma unroll
        for (int k = 1; k < 4; ++k) asp_merge(R, AspState{pm[k][tid], pz[k][tid], ps1[k][tid], ps2[k][tid]});
        const double mu = R.s1 / R.z;
        float var = (float)(R.s2 / R.z - mu * mu);
        if (var < eps) var = eps;
        out[(size_t)b * 2 * C + c0 + tid] = (float)mu;
        out[(size_t)b * 2 * C + C + c0 + tid] = sqrtf(var);
    }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// ---------------------------------------------------------------------------
// res2_block_kernel: the scale - 1 dependent group convs of one ECAPA Res2Net
// block (src/encoder.cpp:174-200) in one launch.  A workgroup owns one clip's
// time tile [t0, t1) and walks the groups j = 1 .. L (L = scale - 1): group
// j is needed on R_j = [t0 - (L - j) D, t1 + (L - j) D) (clipped to the
// clip; D the dilation), so the tile's halo shrinks by D per group and no
// other workgroup's result is ever read.  Its input in_j (x_1, then
// f16(v_{j-1} + x_j) with v the previous group's f32 output) lives in one of
// two LDS buffers and the next one is written by the group's epilogue; the
// weights stream through LDS one tap (128 x 128 f16) at a time in a
// two-stage DMA ring; y_j = f16(v_j) leaves for its slot of the Res2Net
// buffer for the tile's own frames.  Per group the conv runs exactly like the
// one-group DMA conv (taps outer, 16-channel k-steps inner, accumulators from
// zero, bias -> ReLU -> BN scale, shift, the same reflect rule), so the
// results are the same bits as the chain of single-group launches.
// Layout of the buffer (stride S per frame): x_m in slot m + 1 (m = 0 ..
// scale - 1, slots of G = 128 channels), y_1 written to slot 0, y_j (j >= 2)
// to slot j.
// ---------------------------------------------------------------------------
constexpr int kR2G = 128;          // channels per group
constexpr int kR2Rows = 160;       // frames an input buffer holds (t1 - t0 + 2 L D <= 160)
constexpr int kR2MaxL = 7;

struct Res2Args {
    half_t* t1;                    // [B][T][S]
    int S, T, D, L, Tt, nt;
    const half_t* w[kR2MaxL];      // [G][3][G] per group
    const float* bias[kR2MaxL];
    const float* scale[kR2MaxL];
    const float* shift[kR2MaxL];
};

__device__ __forceinline__ int r2_refl(int s, int T) {
    s = s < 0 ? -s : (s >= T ? 2 * (T - 1) - s : s);
    return s < 0 ? 0 : (s >= T ? T - 1 : s);
}

// byte offset of 8-channel chunk c of LDS row r (rows of 256 bytes, chunk c
// at slot c ^ (r & 15): the 16 rows an MFMA operand read touches hit
// distinct 16-byte bank groups)
__device__ __forceinline__ int r2_off(int r, int c) { return r * 256 + ((c ^ (r & 15)) << 4); }

__global__ __launch_bounds__(512) void res2_block_kernel(Res2Args a) {
    __shared__ __attribute__((aligned(1024))) uint8_t s_in[2][kR2Rows * 256];
    __shared__ __attribute__((aligned(1024))) uint8_t s_w[2][kR2G * 256];
    __shared__ float s_ep[kR2MaxL][3][kR2G];   // bias, scale, shift
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int b = blockIdx.x / a.nt, tile = blockIdx.x - b * a.nt;
    const int T = a.T, D = a.D, L = a.L, S = a.S;
    const int t0 = tile * a.Tt, t1 = t0 + a.Tt < T ? t0 + a.Tt : T;
    auto lo = [&](int j) { const int v = t0 - (L - j) * D; return v > 0 ? v : 0; };
    auto hi = [&](int j) { const int v = t1 + (L - j) * D; return v < T ? v : T; };
    const int base = lo(0);
    half_t* const clip = a.t1 + (size_t)b * T * S;

    for (int i = tid; i < L * 3 * kR2G; i += 512) {
        const int j = i / (3 * kR2G), r = i - j * 3 * kR2G, q = r / kR2G, c = r - q * kR2G;
        const float* src = q == 0 ? a.bias[j] : (q == 1 ? a.scale[j] : a.shift[j]);
        s_ep[j][q][c] = src ? src[c] : (q == 1 ? 1.0f : 0.0f);
    }
    // weights of tap k of group j: 2048 16-byte slots, 4 DMA instructions per wave
    auto issue_w = [&](int c) {
        const int j = c / 3, k = c - j * 3;
        const int4v rs = dma_rsrc(a.w[j], (uint32_t)(kR2G * 3 * kR2G * 2));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ins = wave * 4 + i, s = ins * 64 + lane, r = s >> 4, pc = s & 15, lc = pc ^ (r & 15);
            dma16(s_w[c & 1] + ins * 1024, rs, (uint32_t)(((r * 3 + k) * kR2G + lc * 8) * 2));
        }
    };
    issue_w(0);
    // in_1 = x_1 (slot 2) on R_0
    {
        const int n = (hi(0) - base) * 16;
        for (int i = tid; i < n; i += 512) {
            const int r = i >> 4, c = i & 15;
            *reinterpret_cast<half8*>(s_in[0] + r2_off(r, c)) =
                *reinterpret_cast<const half8*>(clip + (size_t)(base + r) * S + 2 * kR2G + c * 8);
        }
    }

    const int ob = wave & 3, fb0 = wave >> 2;   // 32-channel block, first frame block (then every second)
    float16v acc[3];
    int fcol[3];        // per frame block: this lane's frame (masked columns: a valid one)
    half4 xn[3][4];     // x_{j+1} of the epilogue's (frame, 4 channels)
    int nfb = 0, lo_j = 0, hi_j = 0, nx = 0;
    for (int c = 0; c < 3 * L; ++c) {
        const int j = c / 3 + 1, k = c - (j - 1) * 3;
        const uint8_t* const in = s_in[(j - 1) & 1];
        if (k == 0) {
            lo_j = lo(j);
            hi_j = hi(j);
            nfb = (hi_j - lo_j + 31) >> 5;
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                const int fb = fb0 + 2 * i;
                const int f = lo_j + fb * 32 + lrow;
                fcol[i] = f < hi_j ? f : hi_j - 1;   // masked columns: any valid row, result dropped
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
            }
        }
        // chunk c (issued one step ago, or before the loop) has landed; after
        // the barrier every wave is past chunk c - 1, so its stage is free,
        // and the previous group's epilogue writes of `in` are complete
        if (k == 0 || nx == 0) wait_vmcnt<0>();
        else wait_vmcnt_le(nx);
        lds_barrier();
        if (c + 1 < 3 * L) issue_w(c + 1);
        nx = 0;
        if (k == 0 && j < L) {   // x_{j+1} for this group's epilogue, in flight behind the weights
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                const int fb = fb0 + 2 * i;
                if (fb >= nfb) continue;
                const int f = lo_j + fb * 32 + lrow;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int oc = ob * 32 + g * 8 + lhalf * 4;
                    xn[i][g] = f < hi_j ? *reinterpret_cast<const half4*>(clip + (size_t)f * S + (j + 2) * kR2G + oc)
                                        : half4{0, 0, 0, 0};
                    ++nx;
                }
            }
        }
        const uint8_t* const wt = s_w[c & 1];
        int rk[3];   // per frame block: the LDS input row of tap k (reflected into the clip)
#pragma unroll
        for (int i = 0; i < 3; ++i) rk[i] = r2_refl(fcol[i] + (k - 1) * D, T) - base;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const int ch = ks * 2 + lhalf;
            const half8 af = *reinterpret_cast<const half8*>(wt + r2_off(ob * 32 + lrow, ch));
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                if (fb0 + 2 * i >= nfb) continue;
                const half8 bf = *reinterpret_cast<const half8*>(in + r2_off(rk[i], ch));
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc[i], 0, 0, 0);
            }
        }
        if (k < 2) continue;
        // epilogue of group j: bias -> ReLU -> BN; y_j out for the tile's frames,
        // in_{j+1} = f16(v + x_{j+1}) into the other input buffer on R_j
        uint8_t* const out = s_in[j & 1];
        half_t* const yslot = clip + (j == 1 ? 0 : j) * kR2G;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int fb = fb0 + 2 * i;
            if (fb >= nfb) continue;
            const int f = lo_j + fb * 32 + lrow;
            if (f >= hi_j) continue;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int oc = ob * 32 + g * 8 + lhalf * 4;
                half4 yv, iv;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v = acc[i][g * 4 + e] + s_ep[j - 1][0][oc + e];
                    v = fmaxf(v, 0.0f);
                    v = v * s_ep[j - 1][1][oc + e];
                    v = v + s_ep[j - 1][2][oc + e];
                    yv[e] = (half_t)v;
                    iv[e] = (half_t)(v + (float)xn[i][g][e]);
                }
                if (f >= t0 && f < t1) *reinterpret_cast<half4*>(yslot + (size_t)f * S + oc) = yv;
                if (j < L) *reinterpret_cast<half4*>(out + r2_off(f - base, oc >> 3) + (oc & 7) * 2) = iv;
            }
        }
    }
}

}  // namespace
}  // namespace vdk

using namespace vdk;

extern "C" int vdk_feats_tmajor(const float* d_feats, const float* d_row_mean, int batch, int n_mels, int T, int pad,
                                int c_pad, void* d_out, void* stream) {
    return guarded([&] {
        require(d_feats && d_out, "feats_tmajor: NULL device pointer");
        require(batch > 0 && n_mels > 0 && T > 0 && pad >= 0 && c_pad >= n_mels, "feats_tmajor: bad shape");
        if (c_pad % 8 == 0 && c_pad <= kFtC && al16(d_out)) {
            hipLaunchKernelGGL(feats_tmajor_tiled_kernel, dim3(cdiv(T + 2 * pad, kFtF), batch), dim3(256), 0,
                               static_cast<hipStream_t>(stream), d_feats, d_row_mean, n_mels, T, pad, c_pad,
                               static_cast<half_t*>(d_out));
        } else {
            const long n = (long)batch * (T + 2 * pad) * c_pad;
            hipLaunchKernelGGL(feats_tmajor_kernel, dim3(cdiv(n, 256)), dim3(256), 0,
                               static_cast<hipStream_t>(stream), d_feats, d_row_mean, batch, n_mels, T, pad, c_pad,
                               static_cast<half_t*>(d_out));
        }
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
        require(C % 8 == 0 && x_stride % 8 == 0 && al16(d_x), "channel_mean: channels must be 8-aligned");
        hipLaunchKernelGGL(channel_stats_kernel<0>, dim3(cdiv(C, 128), batch), dim3(256), 0,
                           static_cast<hipStream_t>(stream), static_cast<const half_t*>(d_x), x_stride, T, C, 0.0f,
                           d_out);
        VDK_HIP(hipGetLastError());
    });
}

namespace vdk {
namespace {
int se_residual(const void* d_x, int x_stride, const float* d_gate, bool sig, const void* d_res, int res_stride,
                int batch, int T, int C, void* d_y, int y_stride, void* stream) {
    return guarded([&] {
        require(d_x && d_gate && d_res && d_y, "se_gate_residual: NULL device pointer");
        require(batch > 0 && T > 0 && C > 0 && C % 8 == 0 && x_stride >= C && res_stride >= C && y_stride >= C,
                "se_gate_residual: bad shape");
        require(x_stride % 8 == 0 && res_stride % 8 == 0 && y_stride % 8 == 0 && al16(d_x) && al16(d_res) &&
                    al16(d_y) && al16(d_gate), "se_gate_residual: strides/pointers must be 8-channel aligned");
        const long n = (long)batch * T * (C / 8);
        hipLaunchKernelGGL(sig ? se_gate_residual_kernel<true> : se_gate_residual_kernel<false>, dim3(cdiv(n, 256)),
                           dim3(256), 0, static_cast<hipStream_t>(stream), static_cast<const half_t*>(d_x), x_stride,
                           d_gate, static_cast<const half_t*>(d_res), res_stride, batch, T, C,
                           static_cast<half_t*>(d_y), y_stride);
        VDK_HIP(hipGetLastError());
    });
}
}  // namespace
}  // namespace vdk

extern "C" int vdk_se_gate_residual(const void* d_x, int x_stride, const float* d_gate, const void* d_res,
                                    int res_stride, int batch, int T, int C, void* d_y, int y_stride, void* stream) {
    return vdk::se_residual(d_x, x_stride, d_gate, true, d_res, res_stride, batch, T, C, d_y, y_stride, stream);
}

extern "C" int vdk_se_scale_residual(const void* d_x, int x_stride, const float* d_scale, const void* d_res,
                                     int res_stride, int batch, int T, int C, void* d_y, int y_stride, void* stream) {
    return vdk::se_residual(d_x, x_stride, d_scale, false, d_res, res_stride, batch, T, C, d_y, y_stride, stream);
}

extern "C" int vdk_res2_block(void* d_buf, int stride, int batch, int T, int G, int scale, int dil,
                              const vdk_res2_weights* wts, void* stream) {
    return guarded([&] {
        require(d_buf && wts, "res2_block: NULL pointer");
        require(G == kR2G, "res2_block: groups of 128 channels only");
        require(scale >= 2 && scale - 1 <= kR2MaxL, "res2_block: scale must be 2 .. 8");
        require(batch > 0 && T > dil && dil >= 1, "res2_block: T must exceed the dilation");
        require(stride >= (scale + 1) * G && stride % 8 == 0 && al16(d_buf), "res2_block: bad buffer stride / alignment");
        require((size_t)batch * T * stride < (1ull << 31), "res2_block: buffer too large for one launch");
        Res2Args a{};
        a.t1 = static_cast<half_t*>(d_buf);
        a.S = stride; a.T = T; a.D = dil; a.L = scale - 1;
        const int tmax = kR2Rows - 2 * a.L * dil;
        require(tmax >= 32, "res2_block: dilation too large for the LDS tile");
        a.nt = cdiv(T, tmax);
        a.Tt = cdiv(T, a.nt);
        for (int j = 0; j < a.L; ++j) {
            require(wts->w[j] && wts->bias[j] && al16(wts->w[j]), "res2_block: missing group weights");
            a.w[j] = static_cast<const half_t*>(wts->w[j]);
            a.bias[j] = wts->bias[j];
            a.scale[j] = wts->scale[j];
            a.shift[j] = wts->shift[j];
        }
        hipLaunchKernelGGL(res2_block_kernel, dim3(batch * a.nt), dim3(512), 0, static_cast<hipStream_t>(stream), a);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_asp_stats(const void* d_x, int x_stride, int batch, int T, int C, float eps, float* d_out,
                             void* stream) {
    return guarded([&] {
        require(d_x && d_out, "asp_stats: NULL device pointer");
        require(batch > 0 && T > 0 && C > 0 && x_stride >= C, "asp_stats: bad shape");
        require(C % 8 == 0 && x_stride % 8 == 0 && al16(d_x), "asp_stats: channels must be 8-aligned");
        hipLaunchKernelGGL(channel_stats_kernel<1>, dim3(cdiv(C, 128), batch), dim3(256), 0,
                           static_cast<hipStream_t>(stream), static_cast<const half_t*>(d_x), x_stride, T, C, eps,
                           d_out);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_asp_attn_pool(const void* d_a1, int a1_stride, const void* d_w, const float* d_b, int att,
                                 const void* d_x, int x_stride, int batch, int T, int C, float eps, float* d_out,
                                 void* stream) {
    return guarded([&] {
        require(d_a1 && d_w && d_b && d_x && d_out, "asp_attn_pool: NULL device pointer");
        require(batch > 0 && T > 0 && C > 0 && C % 64 == 0, "asp_attn_pool: bad shape (C % 64 == 0)");
        require(att == 128, "asp_attn_pool: only 128 attention channels have a kernel");
        require(a1_stride == att && x_stride == C, "asp_attn_pool: a1 / x must be dense");
        require(al16(d_a1) && al16(d_w) && al16(d_x), "asp_attn_pool: device pointers must be 16-byte aligned");
        require((size_t)batch * T * C * 2 < (1ull << 31), "asp_attn_pool: too many frames for one launch");
        hipLaunchKernelGGL(asp_attn_pool_kernel<128>, dim3(C / 64, batch), dim3(256), 0,
                           static_cast<hipStream_t>(stream), static_cast<const half_t*>(d_a1), a1_stride,
                           static_cast<const half_t*>(d_w), d_b, static_cast<const half_t*>(d_x), x_stride, T, C, eps,
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

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
// stem_mfma_kernel: the IC=1 stem in f32 on v_mfma_f32_32x32x2_f32 (K = the 9
// taps padded to 10); stem_conv3x3_kernel, the f32 FMA loop, serves OC = 16.
#include <algorithm>
#include <atomic>
#include <climits>
#include <cstdlib>
#include <mutex>
#include <string>
#include <type_traits>
#include <unordered_map>

#include "common.hpp"
#include "devmath.hpp"
#include "vdk.h"

namespace vdk {
namespace {

struct ConvArgs {
    const half_t* x;
    const half_t* w;
    const half_t* wc;          // optional chunk-major copy of w: [IC/16][KH*KW][OC][16] (may be NULL)
    const float* bias;
    const half_t* res;
    void* y;
    const float* post_scale;   // per-OC affine applied after the activation (may be NULL)
    const float* post_shift;
    const float* gate;         // per-(clip, time segment, OC) multiplier (may be NULL)
    int H, W, IC, Ho, Wo, OC, KH, KW;
    int sh, sw, ph, pw, dh, dw;  // stride / zero pad / dilation per axis
    int act, tanh_after, y_f32, y_tr;   // act: VDK_ACT_NONE / RELU / SIGMOID / SILU
    float clamp_hi;            // > 0: min(v, clamp_hi) after the ReLU
    int gate_seg, gate_nseg;   // output columns per gate segment, segments per clip
    int xs, ys, rs;            // elements between consecutive pixels of x / y / residual
    int bias_bs;               // elements between clips' bias vectors (0: one shared vector)
    int split;                 // split-f16 tensors: value = hi + lo, lo at +x_lo / +r_lo / +y_lo elements;
    int x_lo, r_lo, y_lo;      //   weights per tap [hi | hi | lo] (split 1) or [hi | hi] (split 2: lo = 0)
    int res_f32, res_after;    // f32 residual; residual added after the activation
    const float* in_scale;     // input prologue x' = relu(x * in_scale[c] + in_shift[c]) (may be NULL)
    const float* in_shift;
    int npix;                  // B * Ho * Wo
    int npix_in;               // B * H * W
    int reflect;               // 1-D time axis padded by reflection (DMA kernel only)
    half_t* y2;                // second output y2 = v + r2 (may be NULL)
    const half_t* r2;
    int y2s, r2s;
    const uint8_t* wq;         // 1x1 weights as q8_0 blocks [OC][IC/32] x {f16 d, 32 x int8} (register-staged kernel)
    double* segsum;            // per-(clip, segment, OC) f64 sums of the stored outputs (may be NULL)
    int seg_len, seg_n;        // output columns per segment, segments per clip
    const half_t* ax;          // AFF combine operands x, ds (may be NULL): v = (x + ds) + v * (x - ds)
    const half_t* ads;
    int axs, ax_lo, adss, ads_lo;
    int xgl = 4, ygl = 4;      // log2 of the channels per group of x / y (16 or 32)
    int xgs = 16, ygs = 16;    // elements between channel groups of x / y (= group size: contiguous)
};

// Element offset of channel c in a layout of 2^gl-channel groups gs elements
// apart (an 8-channel access with c % 8 == 0 stays inside one group).
__device__ __forceinline__ int chan_off(int c, int gl, int gs) { return (c >> gl) * gs + (c & ((1 << gl) - 1)); }

// Epilogue for 8 consecutive output channels oc..oc+7 of pixel P (P
// enumerates (clip, oh, ow) row-major), with every operand moved as 16-byte
// vectors: v = acc + bias; [* gate]; [+ residual]; [relu [min(v, clamp_hi)] |
// sigmoid | silu]; [* post_scale + post_shift]; [tanh]; store f16 / f32 /
// split-f16 at pixel P, or at (clip, ow, oh) when y_tr (time-major output of
// an NHWC map).  Bias, gate and post-affine pointers are 16-byte aligned.
__device__ __forceinline__ void add8(float* v, const float* p, bool mul = false) {
    const float4v a = *reinterpret_cast<const float4v*>(p), b = *reinterpret_cast<const float4v*>(p + 4);
    if (mul) {
#pragma unroll
        for (int e = 0; e < 4; ++e) { v[e] *= a[e]; v[e + 4] *= b[e]; }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) { v[e] += a[e]; v[e + 4] += b[e]; }
    }
}

__device__ __forceinline__ void add_residual(const ConvArgs& a, int P, int oc, float* v) {
    if (a.res_f32) {
        add8(v, reinterpret_cast<const float*>(a.res) + (size_t)P * a.rs + oc);
        return;
    }
    const half8 r = *reinterpret_cast<const half8*>(a.res + (size_t)P * a.rs + oc);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] += (float)r[e];
    if (a.split) {
        const half8 rl = *reinterpret_cast<const half8*>(a.res + (size_t)P * a.rs + a.r_lo + oc);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] += (float)rl[e];
    }
}

// 8 f16 values at p (+ the lo halves at p + lo with split) as f32
__device__ __forceinline__ void load8f(const half_t* p, int lo, int split, float* v) {
    const half8 h = *reinterpret_cast<const half8*>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (float)h[e];
    if (split) {
        const half8 l = *reinterpret_cast<const half8*>(p + lo);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] += (float)l[e];
    }
}

__device__ __forceinline__ void epi8(const ConvArgs& a, int P, int oc, float* v) {
    const int HoWo = a.Ho * a.Wo;
    if (a.bias) add8(v, a.bias + oc + (a.bias_bs ? (size_t)(P / HoWo) * a.bias_bs : 0));
    if (a.gate) {
        const int b = P / HoWo, ow = (P - b * HoWo) % a.Wo;
        add8(v, a.gate + ((size_t)b * a.gate_nseg + ow / a.gate_seg) * a.OC + oc, true);
    }
    if (a.res && !a.res_after) add_residual(a, P, oc, v);
    if (a.act == VDK_ACT_RELU) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = fmaxf(v[e], 0.0f);
        if (a.clamp_hi > 0.0f) {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = fminf(v[e], a.clamp_hi);
        }
    } else if (a.act == VDK_ACT_SIGMOID) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 1.0f / (1.0f + expf(-v[e]));
    } else if (a.act == VDK_ACT_SILU) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = v[e] / (1.0f + expf(-v[e]));
    } else if (a.act == VDK_ACT_GELU) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = gelu_erf(v[e]);
    }
    if (a.res && a.res_after) add_residual(a, P, oc, v);
    if (a.post_scale) {
        add8(v, a.post_scale + oc, true);
        add8(v, a.post_shift + oc);
    }
    if (a.tanh_after) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = tanhf(v[e]);
    }
    if (a.ax) {
        float xv[8], dv[8];
        load8f(a.ax + (size_t)P * a.axs + oc, a.ax_lo, a.split, xv);
        load8f(a.ads + (size_t)P * a.adss + oc, a.ads_lo, a.split, dv);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (xv[e] + dv[e]) + v[e] * (xv[e] - dv[e]);
    }
}

__device__ __forceinline__ void store8(const ConvArgs& a, int P, int oc, const float* v) {
    const int HoWo = a.Ho * a.Wo;
    size_t Po = (size_t)P;
    if (a.y_tr) {
        const int b = P / HoWo, rem = P - b * HoWo, oh = rem / a.Wo, ow = rem - oh * a.Wo;
        Po = ((size_t)b * a.Wo + ow) * a.Ho + oh;
    }
    const size_t o = Po * a.ys + chan_off(oc, a.ygl, a.ygs);
    if (a.y2) {   // f16 only, no split, no time-major store (conv_impl)
        const half8 r = *reinterpret_cast<const half8*>(a.r2 + (size_t)P * a.r2s + oc);
        half8 h2;
#pragma unroll
        for (int e = 0; e < 8; ++e) h2[e] = (half_t)(v[e] + (float)r[e]);
        *reinterpret_cast<half8*>(a.y2 + (size_t)P * a.y2s + oc) = h2;
    }
    if (a.y_f32) {
        float* y = static_cast<float*>(a.y) + o;
        *reinterpret_cast<float4v*>(y) = float4v{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<float4v*>(y + 4) = float4v{v[4], v[5], v[6], v[7]};
    } else {
        half8 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (half_t)v[e];
        *reinterpret_cast<half8*>(static_cast<half_t*>(a.y) + o) = h;
        if (a.split) {
            half8 l;
#pragma unroll
            for (int e = 0; e < 8; ++e) l[e] = (half_t)(v[e] - (float)h[e]);
            *reinterpret_cast<half8*>(static_cast<half_t*>(a.y) + o + a.y_lo) = l;
        }
    }
}

// The finished 32x32 MFMA blocks are staged through LDS as f32 [pixel][oc]
// (row stride TS = M + 4 floats, so consecutive pixels start 16 bytes apart
// across the 64 banks) and then every thread finishes 8 consecutive channels
// of one pixel: bias, gate, residual and the output move as coalesced
// 16-byte rows instead of the MFMA layout's 8-byte pieces 32 pixels apart.
// Accumulator layout: register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4
// and column l%32 of its 32x32 block.
__device__ __forceinline__ void stage_block(float* sT, int TS, int pix0, int row0, const float16v& acc, int lane) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int r = row0 + g * 8 + (lane >> 5) * 4;
        *reinterpret_cast<float4v*>(sT + (pix0 + (lane & 31)) * TS + r) =
            float4v{acc[g * 4], acc[g * 4 + 1], acc[g * 4 + 2], acc[g * 4 + 3]};
    }
}

// Finish NPIX staged pixels x M channels; pix(pl) maps a staged pixel to P
// (or -1 when outside the output).
__device__ __forceinline__ int seg_id(const ConvArgs& a, int P) {
    const int HoWo = a.Ho * a.Wo, b = P / HoWo;
    return b * a.seg_n + (P - b * HoWo) / a.seg_len;
}

// SEGS: part accumulates f64 sums of the stored f16 values of this thread's
// 8 channels for the segments sid0 and sid0 + 1; values of any later segment
// in the tile are added to ConvArgs::segsum directly; see stage_epilogue_impl.
template <int M, bool SEGS = false, class PixFn>
__device__ __forceinline__ void finish_staged(const ConvArgs& a, const float* sT, int npix_tile, int oc0, int tid,
                                              int nthreads, PixFn pix, double (&part)[2][8], int sid0) {
    constexpr int TS = M + 4, C8 = M / 8;
    for (int q = tid; q < npix_tile * C8; q += nthreads) {
        const int pl = q / C8, c8 = q - pl * C8;
        const int P = pix(pl), oc = oc0 + c8 * 8;
        if (P < 0 || oc >= a.OC) continue;
        const float4v u0 = *reinterpret_cast<const float4v*>(sT + pl * TS + c8 * 8);
        const float4v u1 = *reinterpret_cast<const float4v*>(sT + pl * TS + c8 * 8 + 4);
        float v[8] = {u0[0], u0[1], u0[2], u0[3], u1[0], u1[1], u1[2], u1[3]};
        epi8(a, P, oc, v);
        if constexpr (SEGS) {
            const int rel = seg_id(a, P) - sid0;
            if (rel < 2) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const double h = (double)(float)(half_t)v[e];   // the stored value
                    part[0][e] += rel == 0 ? h : 0.0;
                    part[1][e] += rel == 0 ? 0.0 : h;
                }
            } else {
                // a third or later segment in this tile (a clip's short last
                // segment, or clips shorter than the tile): straight to memory
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const double h = (double)(float)(half_t)v[e];
                    if (oc + e < a.OC && h != 0.0) atomicAdd(a.segsum + (size_t)(sid0 + rel) * a.OC + oc + e, h);
                }
            }
        }
        store8(a, P, oc, v);
    }
}

// Pixel tile and output-channel tile of an implicit-GEMM workgroup (grid:
// pixel tiles x output-channel tiles).  Consecutive ids of the logical order
// run on one XCD (xcd_swizzle), and the output-channel tiles of a pixel tile
// are consecutive in it, so the workgroups that read the same input pixels
// run at about the same time under the same L2: the input leaves HBM once,
// not once per output-channel tile.
__device__ __forceinline__ void tile_ids(int& ptile, int& otile) {
    const int lid = xcd_swizzle(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
    ptile = lid / gridDim.y;
    otile = lid - ptile * gridDim.y;
}

// Staged epilogue of an implicit-GEMM tile (BM channels x BN consecutive
// pixels): waves write their blocks in passes of PB pixel columns that fit the
// kernel's LDS buffer, then all threads finish 8-channel rows.
// Segment sums of the stored f16 outputs (ConvArgs::segsum): part 0 is the
// segment of the tile's first pixel, part 1 the next one.  Each thread keeps
// its 8 channels' sums per part (a fixed channel chunk: NT is a multiple of
// BM / 8), the threads of a chunk are summed within the wave and then across
// the waves, and each (part, channel) goes out as one f64 atomic add.  A tile
// can reach further segments (a clip's last segment may be a few frames, and
// the tile runs on into the next clip): their values go out one atomic add
// each.  Every term is an f16 (a multiple of 2^-24 below 2^16) and a segment
// holds far fewer than 2^13 of them, so all these f64 sums are exact and the
// result does not depend on the order of the additions.
template <int BM, int BN, int WN, int SMEM, int NT, int TM, int TN, bool SEGS = false>
__device__ __forceinline__ void stage_epilogue_impl(const ConvArgs& a, uint8_t* smem, const float16v (*acc)[TN],
                                                    int m_off, int n_off, int p0, int oc0, int tid, int lane) {
    constexpr int TS = BM + 4;
    constexpr int FIT = SMEM / (TS * 4);
    constexpr int PB = FIT >= BN ? BN : (FIT / WN) * WN;
    static_assert(PB >= WN, "epilogue staging holds at least one wave's pixel columns");
    static_assert(NT % (BM / 8) == 0 && SMEM >= 2 * BM * 8, "segment sums: fixed channel chunk per thread");
    float* sT = reinterpret_cast<float*>(smem);
    const int sid0 = SEGS ? seg_id(a, p0) : 0;
    double part[2][8];
#pragma unroll
    for (int e = 0; e < 8; ++e) part[0][e] = part[1][e] = 0.0;
    for (int pb = 0; pb < BN; pb += PB) {
        __syncthreads();   // every wave is done with the previous contents of smem
        if (n_off >= pb && n_off < pb + PB) {
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int i = 0; i < TM; ++i) stage_block(sT, TS, n_off - pb + j * 32, m_off + i * 32, acc[i][j], lane);
        }
        __syncthreads();
        const int np = BN - pb < PB ? BN - pb : PB;
        finish_staged<BM, SEGS>(
            a, sT, np, oc0, tid, NT,
            [&](int pl) {
                const int P = p0 + pb + pl;
                return P < a.npix ? P : -1;
            },
            part, sid0);
    }
    if constexpr (SEGS) {
        // lanes of a wave with the same channel chunk (lane % C8) first, by a
        // butterfly, then the waves through LDS, then one global add per
        // (part, channel)
        constexpr int C8 = BM / 8, NWV = NT / 64;
        static_assert(C8 <= 64 && NWV * 2 * BM * 8 <= SMEM, "per-wave segment sums fit the staging area");
#pragma unroll
        for (int pt = 0; pt < 2; ++pt)
#pragma unroll
            for (int e = 0; e < 8; ++e)
#pragma unroll
                for (int m = C8; m < 64; m <<= 1) part[pt][e] += __shfl_xor(part[pt][e], m);
        double* wsum = reinterpret_cast<double*>(smem);   // [NWV][2][BM]
        __syncthreads();   // the staged tile is consumed
        const int wave = tid >> 6;
        if (lane < C8) {
#pragma unroll
            for (int pt = 0; pt < 2; ++pt)
#pragma unroll
                for (int e = 0; e < 8; ++e) wsum[(wave * 2 + pt) * BM + lane * 8 + e] = part[pt][e];
        }
        __syncthreads();
        const int last = (p0 + BN < a.npix ? p0 + BN : a.npix) - 1;
        const int nparts = seg_id(a, last) - sid0 + 1;
        for (int i = tid; i < 2 * BM; i += NT) {
            const int pt = i / BM, c = i - pt * BM;
            double v = 0.0;
#pragma unroll
            for (int w = 0; w < NWV; ++w) v += wsum[(w * 2 + pt) * BM + c];
            if (pt < nparts && oc0 + c < a.OC && v != 0.0)
                atomicAdd(a.segsum + (size_t)(sid0 + pt) * a.OC + oc0 + c, v);
        }
    }
}


// PRO: the input prologue relu(x * in_scale + in_shift) (its scale / shift
// registers exist only in these instantiations).  Q8: 1x1 weights read as
// q8_0 blocks (34 bytes: an f16 scale d and 32 int8 quants q along IC) and
// dequantised in registers, w = f16(q * d) with the product in f32, the value
// a host-side dequantisation to f16 stores.
template <int BM, int BN, int WM, int WN, int KC, bool PRO, bool Q8 = false, bool SEG = false>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void conv_igemm_kernel(ConvArgs a) {
    constexpr int NWM = BM / WM, NWN = BN / WN, NT = NWM * NWN * 64;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int LDK = KC + 8;           // +16 bytes per LDS row: conflict-free operand reads
    constexpr int CPR = KC / 8;           // 16-byte chunks per row
    constexpr int XCH = (BN * CPR + NT - 1) / NT;
    constexpr int WCH = (BM * CPR + NT - 1) / NT;
    static_assert(WM % 32 == 0 && WN % 32 == 0 && KC % 16 == 0, "tile shape");
    // two LDS stages: chunk k is read from stage k&1 while chunk k+1 is written to the other
    constexpr int SMEM_K = 2 * (BM + BN) * LDK * 2, SMEM_E = WN * (BM + 4) * 4;   // K stages / epilogue pass
    constexpr int SMEM = SMEM_K > SMEM_E ? SMEM_K : SMEM_E;
    constexpr int PRO_MAX = 1024;         // input channels whose prologue scale / shift stage in LDS
    __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];
    __shared__ __attribute__((aligned(16))) float s_pro[PRO ? 2 * PRO_MAX : 4];   // in_scale | in_shift
    half_t (*sW)[BM * LDK] = reinterpret_cast<half_t (*)[BM * LDK]>(smem);
    half_t (*sX)[BN * LDK] = reinterpret_cast<half_t (*)[BN * LDK]>(smem + 2 * BM * LDK * 2);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % NWM, wn = wave / NWM;
    int ptile, otile;
    tile_ids(ptile, otile);
    const int p0 = ptile * BN;
    const int oc0 = otile * BM;
    const int HoWo = a.Ho * a.Wo;
    const int KHW = a.KH * a.KW;
    const int nc = a.IC / KC;
    const int nk = KHW * nc;

    // Each thread loads the same pixel rows / weight rows for every K chunk: decode once.
    int x_img[XCH], x_ih[XCH], x_iw[XCH], x_lds[XCH], x_c[XCH];
    bool x_on[XCH], x_row[XCH];
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
        const int q = tid + i * NT;
        const int r = q / CPR, c8 = q - r * CPR;
        const int P = p0 + r;
        x_row[i] = q < BN * CPR;
        x_on[i] = x_row[i] && P < a.npix;
        const int Pc = x_on[i] ? P : 0;
        const int b = Pc / HoWo, rem = Pc - b * HoWo;
        const int oh = rem / a.Wo, ow = rem - oh * a.Wo;
        x_img[i] = b * a.H;
        x_ih[i] = oh * a.sh - a.ph;
        x_iw[i] = ow * a.sw - a.pw;
        x_lds[i] = r * LDK + c8 * 8;
        x_c[i] = c8 * 8;
    }
    uint32_t w_off[WCH];   // byte offset of the slot's weight row at chunk 0 (kOOB: no such row)
    int w_lds[WCH];
    bool w_on[WCH];        // slot is part of the tile
    const int nqb = a.IC >> 5;   // Q8: blocks per weight row
#pragma unroll
    for (int i = 0; i < WCH; ++i) {
        const int q = tid + i * NT;
        const int r = q / CPR, c8 = q - r * CPR;
        w_on[i] = q < BM * CPR;
        if constexpr (Q8)   // the row's first block; the slot's channels c8*8.. are added per chunk
            w_off[i] = w_on[i] && oc0 + r < a.OC ? (uint32_t)((oc0 + r) * nqb * 34) : kOOB;
        else
            w_off[i] = w_on[i] && oc0 + r < a.OC ? (uint32_t)(((size_t)(oc0 + r) * KHW * a.IC + c8 * 8) * 2) : kOOB;
        w_lds[i] = r * LDK + c8 * 8;
    }
    // buffer loads: a masked lane reads an out-of-range offset (zero), so every
    // fetch issues the same number of loads and the waits below count exactly
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.x, 0, (int)(((size_t)(a.npix_in - 1) * a.xs + a.IC) * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t wrs =
        Q8 ? __builtin_amdgcn_make_buffer_rsrc((void*)a.wq, 0, a.OC * nqb * 34, 0x00020000)
           : __builtin_amdgcn_make_buffer_rsrc((void*)a.w, 0, (int)((size_t)a.OC * KHW * a.IC * 2), 0x00020000);

    // With the prologue (long-K 1x1 GEMMs) two register slots: chunk k+2 is
    // loaded while chunk k feeds the MFMAs and chunk k+1 waits in the other
    // slot for its turn in LDS, so two chunks of loads are in flight across
    // every barrier; the loop is unrolled by two so each slot is a fixed set
    // of registers.  Otherwise one slot (chunk k+1 in flight), which keeps
    // the register count, and so the residency, of the short-K convs.
    half8 xr[2][XCH], wr[2][WCH];
    auto fetch = [&](int k, auto slot) {
        constexpr int s = decltype(slot)::value;
        const int tap = k / nc, c0 = (k - tap * nc) * KC;
        const int kh = tap / a.KW, kw = tap - kh * a.KW;
        const uint32_t wd = (uint32_t)((tap * a.IC + c0) * 2);
#pragma unroll
        for (int i = 0; i < WCH; ++i) {
            if constexpr (Q8) {
                // channels k .. k+7 of the row (1x1: k = c0 + c8*8) sit at byte
                // 2 + k%32 of block k/32: a 2-byte aligned run, read as three
                // aligned dwords and shifted into place
                const int kq = c0 + ((tid + i * NT) % CPR) * 8;
                const uint32_t blk = w_off[i] == kOOB ? kOOB : w_off[i] + (uint32_t)((kq >> 5) * 34);
                const uint32_t qo = blk == kOOB ? kOOB : blk + 2 + (uint32_t)(kq & 31);
                const uint32_t sh = (qo & 3) * 8;
                const auto d3 = __builtin_amdgcn_raw_buffer_load_b96(wrs, qo & ~3u, 0, 0);
                const uint32_t lo = sh ? (d3[0] >> sh) | (d3[1] << (32 - sh)) : d3[0];
                const uint32_t hi = sh ? (d3[1] >> sh) | (d3[2] << (32 - sh)) : d3[1];
                const float d = (float)__builtin_bit_cast(half_t, (unsigned short)__builtin_amdgcn_raw_buffer_load_b16(
                                                                      wrs, blk, 0, 0));
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    wr[s][i][e] = (half_t)((float)(int8_t)(lo >> (8 * e)) * d);
                    wr[s][i][e + 4] = (half_t)((float)(int8_t)(hi >> (8 * e)) * d);
                }
            } else {
                const uint32_t off = w_off[i] == kOOB ? kOOB : w_off[i] + wd;
                wr[s][i] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 0));
            }
        }
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int ih = x_ih[i] + kh * a.dh, iw = x_iw[i] + kw * a.dw;
            const bool in = x_on[i] && ih >= 0 && ih < a.H && iw >= 0 && iw < a.W;
            const uint32_t off =
                in ? (uint32_t)((((size_t)(x_img[i] + ih) * a.W + iw) * a.xs + c0 + x_c[i]) * 2) : kOOB;
            xr[s][i] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
        }
    };
    // the prologue's scale / shift of chunk k's channels come from LDS (1x1
    // unpadded only, conv_impl: every fetched value is a real input)
    auto stash = [&](int st, auto slot, int k) {
        constexpr int s = decltype(slot)::value;
#pragma unroll
        for (int i = 0; i < WCH; ++i)
            if (w_on[i]) *reinterpret_cast<half8*>(&sW[st][w_lds[i]]) = wr[s][i];
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            half8 v = xr[s][i];
            if constexpr (PRO) {   // BatchNorm + ReLU of the input channels, as the f16 operand
                const int cc = k * KC + x_c[i];
                const float4v sc0 = *reinterpret_cast<const float4v*>(s_pro + cc);
                const float4v sc1 = *reinterpret_cast<const float4v*>(s_pro + cc + 4);
                const float4v sh0 = *reinterpret_cast<const float4v*>(s_pro + PRO_MAX + cc);
                const float4v sh1 = *reinterpret_cast<const float4v*>(s_pro + PRO_MAX + cc + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = (half_t)fmaxf((float)v[e] * sc0[e] + sh0[e], 0.0f);
                    v[e + 4] = (half_t)fmaxf((float)v[e + 4] * sc1[e] + sh1[e], 0.0f);
                }
            }
            if (x_row[i]) *reinterpret_cast<half8*>(&sX[st][x_lds[i]]) = v;
        }
    };

    float16v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    auto mfma_chunk = [&](int st) {
#pragma unroll
        for (int kk = 0; kk < KC / 16; ++kk) {
            half8 af[TM], bf[TN];
            const int koff = kk * 16 + (lane >> 5) * 8;
#pragma unroll
            for (int i = 0; i < TM; ++i)
                af[i] = *reinterpret_cast<const half8*>(&sW[st][(wm * WM + i * 32 + (lane & 31)) * LDK + koff]);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bf[j] = *reinterpret_cast<const half8*>(&sX[st][(wn * WN + j * 32 + (lane & 31)) * LDK + koff]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };
    if constexpr (PRO) {
        // chunk k sits in LDS stage k&1 (and arrived through register slot k&1)
        auto step = [&](int k, auto slot) {
            constexpr int s = decltype(slot)::value;
            // slot s was stashed for chunk k one step ago; past the end the last
            // chunk is fetched again (unused) to keep the load count fixed
            fetch(k + 2 < nk ? k + 2 : nk - 1, slot);
            mfma_chunk(s);
            if (k + 1 < nk) stash(s ^ 1, std::integral_constant<int, s ^ 1>(), k + 1);
            __syncthreads();
        };
        fetch(0, S0());
        fetch(nk > 1 ? 1 : 0, S1());
        for (int c = tid; c < a.IC; c += NT) {
            s_pro[c] = a.in_scale[c];
            s_pro[PRO_MAX + c] = a.in_shift[c];
        }
        __syncthreads();
        stash(0, S0(), 0);
        __syncthreads();
        for (int k = 0; k < nk; k += 2) {
            step(k, S0());
            if (k + 1 >= nk) break;
            step(k + 1, S1());
        }
    } else {
        fetch(0, S0());
        stash(0, S0(), 0);
        __syncthreads();
        for (int k = 0; k < nk; ++k) {
            const int st = k & 1;
            if (k + 1 < nk) fetch(k + 1, S0());   // global loads in flight during this chunk's MFMAs
            mfma_chunk(st);
            if (k + 1 < nk) stash(st ^ 1, S0(), k + 1);
            __syncthreads();
        }
    }

    stage_epilogue_impl<BM, BN, WN, SMEM, NT, TM, TN, SEG>(a, smem, acc, wm * WM, wn * WN, p0, oc0, tid, lane);
}

// ---------------------------------------------------------------------------
// conv_dma_kernel: the same implicit GEMM with the operand tiles moved
// HBM/L2 -> LDS by buffer_load_dwordx4 ... lds (no VGPR staging, no ds_write).
//  * Buffer loads return zero past the end of the buffer, so padding taps are
//    fetched from an out-of-range offset instead of being branched around.
//  * Tap and channel-chunk offsets are wave-uniform (SGPR soffset); each lane
//    keeps one precomputed voffset per slot it fills.
//  * LDS rows are unpadded (KC*2 bytes); the 16-byte chunk c of row r lives at
//    slot c ^ key(r), so the MFMA operand reads (32 rows, one chunk column)
//    touch distinct banks.  A DMA instruction fills 64 consecutive slots, so a
//    lane picks the global chunk that belongs in its slot.
//  * Two LDS stages; chunk k+1 is in flight while chunk k feeds the MFMAs; one
//    barrier per chunk.
//  * PRO: the input prologue relu(x * in_scale + in_shift) (1x1 convs without
//    padding) applied to each B fragment as it leaves LDS, with the scale /
//    shift vectors staged in LDS once; rounded to f16 like the register-staged
//    kernel's, so both give the same operands.
// ---------------------------------------------------------------------------


template <int KC>
__device__ __forceinline__ int swz(int r, int c) {
    // gfx950 LDS serves a ds_read_b128 16 lanes (256 bytes, 64 banks) per
    // cycle; an MFMA operand read has 16 lanes on 16 consecutive rows and one
    // chunk column, so the key makes those 16 (row, chunk) pairs hit distinct
    // 16-byte bank groups.  KC=64: 128-byte rows, key = (r/2) % 8.
    // KC=32: 64-byte rows, key = (r/4) % 4.
    if constexpr (KC == 64) return c ^ ((r >> 1) & 7);
    else return c ^ ((r >> 2) & 3);
}


template <int BM, int BN, int WM, int WN, int KC, int NST, bool PRO = false>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void conv_dma_kernel(ConvArgs a) {
    constexpr int NWM = BM / WM, NWN = BN / WN, NW = NWM * NWN;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int CPR = KC / 8;                    // 16-byte chunks per row
    constexpr int RB = KC * 2;                     // bytes per LDS row
    constexpr int ROWS = BM + BN;
    constexpr int NINS = ROWS * CPR / 64;          // DMA instructions per stage
    constexpr int IPW = (NINS + NW - 1) / NW;      // per wave; every wave issues exactly IPW
    constexpr int STAGE = IPW * NW * 1024;         // padding instructions land past the tiles
    static_assert(KC == 32 || KC == 64, "KC");
    static_assert((ROWS * CPR) % 64 == 0, "whole DMA instructions per stage");
    static_assert(BM % (64 / CPR) == 0, "weight rows fill whole DMA instructions");
    static_assert(NST >= 2 && IPW * (NST - 2) <= 60, "vmcnt range");
    constexpr int SMEM_E = WN * (BM + 4) * 4;   // one epilogue pass of a wave's pixel columns
    constexpr int SMEM = NST * STAGE > SMEM_E ? NST * STAGE : SMEM_E;
    constexpr int PRO_MAX = 1024;               // input channels with a staged prologue
    __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];
    __shared__ __attribute__((aligned(16))) float s_in[PRO ? 2 * PRO_MAX : 4];   // in_scale | in_shift

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % NWM, wn = wave / NWM;
    int ptile, otile;
    tile_ids(ptile, otile);
    const int p0 = ptile * BN;
    const int oc0 = otile * BM;
    const int HoWo = a.Ho * a.Wo;
    const int KHW = a.KH * a.KW;
    // Split-f16: per tap the K range runs over [x_hi . w_hi | x_lo . w_hi | x_hi . w_lo]
    // (split 2, weights exact in f16: the first two terms only).
    const int ICW = a.split ? (a.split == 2 ? 2 : 3) * a.IC : a.IC;
    const int nc = ICW / KC;
    const int nk = KHW * nc;

    const int xext = ((a.IC >> a.xgl) - 1) * a.xgs + (1 << a.xgl);   // elements of a pixel's channels (one plane)
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.x, 0, (int)(((size_t)(a.npix_in - 1) * a.xs + xext + (a.split ? a.x_lo : 0)) * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.w, 0, (int)((size_t)a.OC * KHW * ICW * 2), 0x00020000);

    // Per DMA slot of this lane: weight rows keep a fixed voffset (the tap /
    // chunk part is uniform); pixel rows keep the tap-0 offset and a mask of
    // the taps that fall inside the image - one bit per tap, or for a single
    // row of more than 32 taps the in-image range [lo, hi) as lo | hi << 16.
    const bool tap_range = a.KH == 1 && a.KW > 32;
    int s_off[IPW];
    uint32_t s_mask[IPW];
    bool s_is_w[IPW];
    int s_iw[IPW];   // reflect padding: the slot's tap-0 column (INT_MIN: no pixel)
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
        const int ins = wave + j * NW;
        const int p = ins * 64 + lane;
        const int r = p / CPR, slot = p - r * CPR;
        const int c = swz<KC>(r, slot);
        // one instruction covers 64/CPR whole rows and BM is a multiple of
        // that, so the weight/pixel split is per instruction (wave-uniform)
        s_is_w[j] = ins * (64 / CPR) < BM;
        s_mask[j] = 0;
        s_iw[j] = INT_MIN;
        if (ins >= NINS) {
            s_off[j] = 0;   // padding instruction: zeros into the spare slots
        } else if (s_is_w[j]) {
            s_off[j] = ((oc0 + r) * KHW * ICW + c * 8) * 2;
        } else {
            const int P = p0 + (r - BM);
            s_off[j] = 0;   // rows past the end: mask 0, every tap reads zeros
            if (P < a.npix) {
                const int b = P / HoWo, rem = P - b * HoWo;
                const int oh = rem / a.Wo, ow = rem - oh * a.Wo;
                const int ih0 = oh * a.sh - a.ph, iw0 = ow * a.sw - a.pw;
                s_off[j] = (((b * a.H + ih0) * a.W + iw0) * a.xs + chan_off(c * 8, a.xgl, a.xgs)) * 2;
                s_iw[j] = iw0;
                if (tap_range) {
                    // one row of taps: the in-image ones are kw in [lo, hi)
                    const int lo = iw0 >= 0 ? 0 : (-iw0 + a.dw - 1) / a.dw;
                    int hi = a.W - 1 - iw0 >= 0 ? (a.W - 1 - iw0) / a.dw + 1 : 0;
                    hi = hi < a.KW ? hi : a.KW;
                    s_mask[j] = lo < hi ? (uint32_t)lo | ((uint32_t)hi << 16) : 0u;
                } else {
                    for (int kh = 0; kh < a.KH; ++kh)
                        for (int kw = 0; kw < a.KW; ++kw) {
                            const int ih = ih0 + kh * a.dh, iw = iw0 + kw * a.dw;
                            if (ih >= 0 && ih < a.H && iw >= 0 && iw < a.W) s_mask[j] |= 1u << (kh * a.KW + kw);
                        }
                }
            }
        }
    }

    // Chunk cursor for the DMA side: tap (kh, kw) and logical channel offset
    // c0 in [0, ICW), advanced incrementally (no divisions in the loop).
    // f_x = byte offset of tap (kh, kw) in the input, f_xc = of the channel chunk.
    int f_tap = 0, f_kw = 0, f_c0 = 0, f_x = 0, f_xc = 0;
    const int tap_bytes = a.dw * a.xs * 2;                       // next kw
    const int row_bytes = a.dh * a.W * a.xs * 2 - a.KW * tap_bytes;   // next kh, back to kw = 0
    // This wave's DMA instructions of the cursor's chunk into stage st,
    // branch-free inside: the weight / pixel split of an instruction is fixed
    // at compile time when the weight instructions divide evenly over the
    // waves, and the tap test / reflect padding variants are chosen once per
    // chunk (a wave-uniform branch), so the loads go out back to back.
    constexpr int WI = BM * CPR / 64;   // weight instructions per stage
    auto issue_all = [&](int st, auto tap_in, auto refl) {
        const int w_soff = (f_tap * ICW + f_c0) * 2;
#pragma unroll
        for (int j = 0; j < IPW; ++j) {
            lds_void* dst = (lds_void*)(smem + st * STAGE + (wave + j * NW) * 1024);
            const bool isw = WI % NW == 0 ? j < WI / NW : s_is_w[j];
            if (isw) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, dst, 16, (uint32_t)s_off[j], w_soff, 0, 0);
            } else {
                const bool in = tap_in(s_mask[j]);
                uint32_t off = in ? (uint32_t)(s_off[j] + f_x + f_xc) : kOOB;
                if constexpr (decltype(refl)::value) {
                    // the tap's column reflected back into [0, W) (KH = 1: f_tap is the column tap)
                    const bool pix = s_iw[j] != INT_MIN;
                    const int iw0 = pix ? s_iw[j] : 0;
                    int iw = iw0 + f_tap * a.dw;
                    iw = iw < 0 ? -iw : (iw >= a.W ? 2 * (a.W - 1) - iw : iw);
                    iw = iw < 0 ? 0 : (iw >= a.W ? a.W - 1 : iw);
                    const uint32_t roff = (uint32_t)(s_off[j] + (iw - iw0) * a.xs * 2 + f_xc);
                    off = !in && pix ? roff : off;
                }
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, dst, 16, off, 0, 0, 0);
            }
        }
    };
    auto issue = [&](int st) {
        const auto bit_in = [&](uint32_t m) { return ((m >> f_tap) & 1u) != 0; };
        if (tap_range) {
            issue_all(st, [&](uint32_t m) {
                return (uint32_t)(f_tap - (int)(m & 0xFFFFu)) < (uint32_t)((int)(m >> 16) - (int)(m & 0xFFFFu));
            }, std::false_type());
        } else if (a.reflect) {
            issue_all(st, bit_in, std::true_type());
        } else {
            issue_all(st, bit_in, std::false_type());
        }
        f_c0 += KC;
        f_xc += (KC >> a.xgl) * a.xgs * 2;
        if (f_c0 == ICW) {
            f_c0 = 0;
            f_xc = 0;
            f_x += tap_bytes;
            ++f_tap;
            if (++f_kw == a.KW) {
                f_kw = 0;
                f_x += row_bytes;              // next kernel row
            }
        } else if (a.split && f_c0 == a.IC) {
            f_xc = a.x_lo * 2;                 // lo plane (with the hi weights)
        } else if (a.split && f_c0 == 2 * a.IC) {
            f_xc = 0;                          // hi plane again (with the lo weights)
        }
    };

    float16v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int lrow = lane & 31, lhalf = lane >> 5;
    // prologue: NST-1 chunks in flight
#pragma unroll
    for (int k = 0; k < NST - 1; ++k)
        if (k < nk) issue(k);
    if constexpr (PRO) {   // 1x1: chunk k covers input channels k*KC .. (conv_impl: IC <= PRO_MAX)
        for (int c = tid; c < a.IC; c += NW * 64) {
            s_in[c] = a.in_scale[c];
            s_in[PRO_MAX + c] = a.in_shift[c];
        }
        __syncthreads();
    }
    int st = 0;
    for (int k = 0; k < nk; ++k) {
        // chunk k has landed once at most (NST-2) younger chunks are outstanding
        const int younger = nk - 1 - k < NST - 2 ? nk - 1 - k : NST - 2;
        wait_vmcnt_le(younger * IPW);
        // Plain barrier + LDS acquire fence.  __syncthreads() would add a
        // release fence, which must drain every in-flight DMA stage
        // (vmcnt(0)) and collapse the ring; this wave's own chunk-k DMA is
        // already complete by the vmcnt wait above, and no ds_write precedes.
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        if (k + NST - 1 < nk) issue(st == 0 ? NST - 1 : st - 1);
        const uint8_t* sa = smem + st * STAGE;
        const uint8_t* sb = sa + BM * RB;
#pragma unroll
        for (int kk = 0; kk < KC / 16; ++kk) {
            const int c = kk * 2 + lhalf;
            half8 af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int r = wm * WM + i * 32 + lrow;
                af[i] = *reinterpret_cast<const half8*>(sa + r * RB + swz<KC>(r, c) * 16);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int r = wn * WN + j * 32 + lrow;
                bf[j] = *reinterpret_cast<const half8*>(sb + r * RB + swz<KC>(r + BM, c) * 16);
            }
            if constexpr (PRO) {   // BatchNorm + ReLU of the input channels, as the f16 operand
                const int ch = k * KC + c * 8;
                const float4v sc0 = *reinterpret_cast<const float4v*>(s_in + ch);
                const float4v sc1 = *reinterpret_cast<const float4v*>(s_in + ch + 4);
                const float4v sh0 = *reinterpret_cast<const float4v*>(s_in + PRO_MAX + ch);
                const float4v sh1 = *reinterpret_cast<const float4v*>(s_in + PRO_MAX + ch + 4);
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        bf[j][e] = (half_t)fmaxf((float)bf[j][e] * sc0[e] + sh0[e], 0.0f);
                        bf[j][e + 4] = (half_t)fmaxf((float)bf[j][e + 4] * sc1[e] + sh1[e], 0.0f);
                    }
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        st = st + 1 == NST ? 0 : st + 1;
    }

    stage_epilogue_impl<BM, BN, WN, SMEM, NW * 64, TM, TN>(a, smem, acc, wm * WM, wn * WN, p0, oc0, tid, lane);
}

template <int BM, int BN, int WM, int WN, int KC, int NST>
void launch_dma(const ConvArgs& a, hipStream_t s) {
    constexpr int NT = (BM / WM) * (BN / WN) * 64;
    dim3 grid(cdiv(a.npix, BN), cdiv(a.OC, BM));
    if (a.in_scale)
        hipLaunchKernelGGL((conv_dma_kernel<BM, BN, WM, WN, KC, NST, true>), grid, dim3(NT), 0, s, a);
    else
        hipLaunchKernelGGL((conv_dma_kernel<BM, BN, WM, WN, KC, NST>), grid, dim3(NT), 0, s, a);
}

// ---------------------------------------------------------------------------
// gemm_ws_kernel: implicit-GEMM convs (zero padding, any stride /
// dilation; the time-major GEMMs of ECAPA's TDNN / MFA layers, wav2vec2's
// linears and strided feature convs: M = output channels, N = pixels, K =
// taps x input channels) with the waves split by role, as in the band kernel: NP
// producer waves DMA each KC-channel chunk of the tile's BM weight rows and
// BN pixel rows into an NST-stage LDS ring (rows XOR-swizzled as in the
// LDS-DMA kernel), and the compute waves only read LDS and run MFMAs, each
// k-step's fragment reads issued between the previous step's MFMAs.  One
// barrier per chunk; the producers keep NST-1 chunks in flight.  The
// epilogue is the implicit-GEMM kernels' staged one (every epilogue option),
// run by all waves.
// ---------------------------------------------------------------------------
// DMA slots of one feeding wave of the GEMM kernels: instruction i of wave p
// (p + NPW * i of the chunk's NINS) fills LDS row r = q / CPR (q = 64 * ins
// + lane), 16-byte slot s with chunk swz(r, s) of weight row oc0 + r
// ([OC][KH][KW][IC]) or, past the BM weight rows, of output pixel
// p0 + r - BM.  A weight slot keeps its byte offset at tap 0 / channel 0
// (-1: past the weights, reads zeros); a pixel slot its clip's first input
// row b * H (-1: past the pixels) and the tap-0 input row / column ih0, iw0
// (with the slot's chunk in the low 4 bits), checked against the map per tap.
template <int BM, int KC, int IPW, int NPW>
struct GemmFeed {
    static constexpr int CPR = KC / 8;
    int p, lane, icw;
    int off[IPW], ih0[IPW], iw0[IPW], cof[IPW];
    __amdgpu_buffer_rsrc_t wr, xr;
    __device__ __forceinline__ GemmFeed(const ConvArgs& a, int p_, int lane_, int p0, int oc0) : p(p_), lane(lane_) {
        // split-f16 (1x1 only): K per tap runs over [x_hi . w_hi | x_lo . w_hi | x_hi . w_lo]
        icw = a.split ? (a.split == 2 ? 2 : 3) * a.IC : a.IC;
        const int xext = ((a.IC >> a.xgl) - 1) * a.xgs + (1 << a.xgl);   // a pixel's channels in one plane
        wr = __builtin_amdgcn_make_buffer_rsrc((void*)a.w, 0, (int)((size_t)a.OC * a.KH * a.KW * icw * 2),
                                               0x00020000);
        xr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)a.x, 0, (int)(((size_t)(a.npix_in - 1) * a.xs + xext + (a.split ? a.x_lo : 0)) * 2), 0x00020000);
        const int HoWo = a.Ho * a.Wo;
#pragma unroll
        for (int i = 0; i < IPW; ++i) {
            const int ins = p + NPW * i;
            const int q = ins * 64 + lane, r = q / CPR, c = swz<KC>(r, q - r * CPR);
            ih0[i] = iw0[i] = 0;
            cof[i] = chan_off(c * 8, a.xgl, a.xgs);   // the slot's 8 channels within a chunk
            if (r < BM) {
                off[i] = oc0 + r < a.OC ? ((oc0 + r) * a.KH * a.KW * icw + c * 8) * 2 : -1;
            } else {
                const int P = p0 + r - BM;
                off[i] = -1;
                if (P < a.npix) {
                    const int b = P / HoWo, rem = P - b * HoWo;
                    const int oh = rem / a.Wo, ow = rem - oh * a.Wo;
                    off[i] = b * a.H;
                    ih0[i] = oh * a.sh - a.ph;
                    iw0[i] = ow * a.sw - a.pw;
                }
            }
        }
    }
    // This wave's instructions of chunk k (tap k / ncpt, K offset (k % ncpt)
    // * KC) into the stage at dst: branch-free (selects of out-of-range
    // offsets, the weight / pixel split fixed at compile time), so the loads
    // go out back to back.  Chunks cover whole channel groups and, split,
    // lie inside one plane term.
    __device__ __forceinline__ void issue(const ConvArgs& a, uint8_t* dst, int k, int ncpt) const {
        const int tap = k / ncpt, c0 = (k - tap * ncpt) * KC;
        const int kh = tap / a.KW, kw = tap - kh * a.KW;
        const int term = a.split ? (c0 >= 2 * a.IC ? 2 : (c0 >= a.IC ? 1 : 0)) : 0;
        const int xc = (term == 1 ? a.x_lo : 0) + chan_off(c0 - term * a.IC, a.xgl, a.xgs);   // the chunk's first channel
        constexpr int WI = BM * CPR / 64;   // the weight rows' instructions (whole ones)
#pragma unroll
        for (int i = 0; i < IPW; ++i) {
            const int ins = p + NPW * i;
            // wave-uniform; known at compile time when the weight instructions
            // split evenly over the feeding waves (ins < WI iff i < WI / NPW)
            const bool wrow = WI % NPW == 0 ? i < WI / NPW : ins < WI;
            if (wrow) {
                const uint32_t o = off[i] < 0 ? kOOB : (uint32_t)(off[i] + (tap * icw + c0) * 2);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void*)(dst + ins * 1024), 16, o, 0, 0, 0);
            } else {
                const int ih = ih0[i] + kh * a.dh, iw = iw0[i] + kw * a.dw;
                const bool in = off[i] >= 0 && (unsigned)ih < (unsigned)a.H && (unsigned)iw < (unsigned)a.W;
                const uint32_t pos = (uint32_t)((((off[i] + ih) * a.W + iw) * a.xs + xc + cof[i]) * 2);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(dst + ins * 1024), 16, in ? pos : kOOB, 0, 0,
                                                         0);
            }
        }
    }
};

template <int BM, int BN, int WMG, int WNG, int KC, int NST, int NP>
struct GemmWs {
    static constexpr int NCW = WMG * WNG, NW = NCW + NP;
    static constexpr int WM = BM / WMG, WN = BN / WNG, TM = WM / 32, TN = WN / 32;
    static constexpr int CPR = KC / 8, RB = KC * 2;
    static constexpr int NINS = (BM + BN) * CPR / 64, IPP = NINS / NP;   // DMA instructions per chunk / producer
    static constexpr int STAGE = NINS * 1024;
    static_assert(KC == 32 || KC == 64, "KC");
    static_assert(NINS % NP == 0 && (BM * CPR) % 64 == 0, "whole DMA instructions, split evenly over the producers");
    static_assert(NST >= 2 && NST * STAGE <= 163840, "the ring fits the 160 KB of LDS");
    static_assert(TM >= 1 && TN >= 1, "wave tiles of whole 32 x 32 blocks");
    static_assert(IPP * (NST - 2) <= 60, "vmcnt range");
};

// PRO: the input prologue relu(x * in_scale + in_shift) of 1x1 convs (CAM++'s
// linear1), applied to the B fragments at their k-step with the scale /
// shift staged in LDS, rounded to f16 as the operand like the other kernels'
// prologues.  SEGS: the staged epilogue's segment sums of the stored outputs.
template <int BM, int BN, int WMG, int WNG, int KC, int NST, int NP, bool PRO = false, bool SEGS = false>
__global__ __launch_bounds__((WMG * WNG + NP) * 64) void gemm_ws_kernel(ConvArgs a) {
    using G = GemmWs<BM, BN, WMG, WNG, KC, NST, NP>;
    constexpr int TM = G::TM, TN = G::TN, RB = G::RB, CPR = G::CPR;
    constexpr int SMEM_E = G::WN * (BM + 4) * 4;   // one epilogue pass of a wave's pixel columns
    constexpr int SMEM = NST * G::STAGE > SMEM_E ? NST * G::STAGE : SMEM_E;
    constexpr int PRO_MAX = 1024;                  // input channels with a staged prologue
    __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];
    __shared__ __attribute__((aligned(16))) float s_in[PRO ? 2 * PRO_MAX : 4];   // in_scale | in_shift
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if constexpr (PRO) {   // 1x1: chunk k covers input channels k * KC .. (the launch checks IC <= PRO_MAX)
        for (int c = tid; c < a.IC; c += G::NW * 64) {
            s_in[c] = a.in_scale[c];
            s_in[PRO_MAX + c] = a.in_shift[c];
        }
        __syncthreads();
    }
    int ptile, otile;
    tile_ids(ptile, otile);
    const int p0 = ptile * BN, oc0 = otile * BM;
    // chunks per tap (split-f16: over the [hi | lo | hi] plane terms)
    const int ncpt = (a.split ? (a.split == 2 ? 2 : 3) * a.IC : a.IC) / KC;
    const int nk = a.KH * a.KW * ncpt; // K = taps x input channels, taps outermost

    float16v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    int m_off = 0, n_off = -1;   // producers stage nothing in the epilogue

    if (wave >= G::NCW) {
        // ---------------- producers ----------------
        GemmFeed<BM, KC, G::IPP, NP> feed(a, wave - G::NCW, lane, p0, oc0);
        auto issue = [&](int k) { feed.issue(a, smem + (k % NST) * G::STAGE, k, ncpt); };
#pragma unroll
        for (int k = 0; k < NST - 1; ++k)
            if (k < nk) issue(k);
#pragma unroll 1
        for (int k = 0; k < nk; ++k) {
            // chunk k has landed once at most min(NST-2, nk-1-k) younger chunks are in flight
            const int younger = nk - 1 - k < NST - 2 ? nk - 1 - k : NST - 2;
            wait_vmcnt_le(younger * G::IPP);
            lds_barrier();   // chunk k is visible; the compute waves are done with chunk k-1's stage
            if (k + NST - 1 < nk) issue(k + NST - 1);
        }
    } else {
        // ---------------- compute waves ----------------
        const int wm = wave % WMG, wn = wave / WMG;
        m_off = wm * G::WM;
        n_off = wn * G::WN;
        const int lrow = lane & 31, lhalf = lane >> 5;
        int aoff[TM], boff[TN];   // row bases; the swizzled chunk is added per k-step
#pragma unroll
        for (int i = 0; i < TM; ++i) aoff[i] = (m_off + i * 32 + lrow) * RB;
#pragma unroll
        for (int j = 0; j < TN; ++j) boff[j] = (BM + n_off + j * 32 + lrow) * RB;
        constexpr int KS = KC / 16;
#pragma unroll 1
        for (int k = 0; k < nk; ++k) {
            lds_barrier();   // chunk k has landed; chunk k-1's reads are done
            const uint8_t* const sa = smem + (k % NST) * G::STAGE;
            half8 af[2][TM], bf[2][TN];
            auto load = [&](int kk, int buf) {
                const int c = kk * 2 + lhalf;
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    af[buf][i] = *reinterpret_cast<const half8*>(sa + aoff[i] + swz<KC>(m_off + i * 32 + lrow, c) * 16);
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    bf[buf][j] = *reinterpret_cast<const half8*>(
                        sa + boff[j] + swz<KC>(BM + n_off + j * 32 + lrow, c) * 16);
            };
            load(0, 0);
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) {
                const int cb = kk & 1;
                if constexpr (PRO) {   // BatchNorm + ReLU of the input channels, as the f16 operand
                    const int ch = k * KC + kk * 16 + lhalf * 8;
                    const float4v sc0 = *reinterpret_cast<const float4v*>(s_in + ch);
                    const float4v sc1 = *reinterpret_cast<const float4v*>(s_in + ch + 4);
                    const float4v sh0 = *reinterpret_cast<const float4v*>(s_in + PRO_MAX + ch);
                    const float4v sh1 = *reinterpret_cast<const float4v*>(s_in + PRO_MAX + ch + 4);
#pragma unroll
                    for (int j = 0; j < TN; ++j)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            bf[cb][j][e] = (half_t)fmaxf((float)bf[cb][j][e] * sc0[e] + sh0[e], 0.0f);
                            bf[cb][j][e + 4] = (half_t)fmaxf((float)bf[cb][j][e + 4] * sc1[e] + sh1[e], 0.0f);
                        }
                }
                if (kk + 1 < KS) load(kk + 1, cb ^ 1);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cb][i], bf[cb][j], acc[i][j], 0, 0, 0);
                if (kk + 1 < KS) {
                    // one MFMA, then one fragment read, in turn
#pragma unroll
                    for (int q = 0; q < TM + TN; ++q) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
                    }
                    if constexpr (TM * TN > TM + TN)
                        __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - (TM + TN), 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    stage_epilogue_impl<BM, BN, G::WN, SMEM, G::NW * 64, TM, TN, SEGS>(a, smem, acc, m_off, n_off, p0, oc0, tid,
                                                                       lane);
}

// EXT: the tile also runs the prologue / segment-sum variants (CAM++'s linear1).
template <int BM, int BN, int WMG, int WNG, int KC, int NST, int NP, bool EXT = false>
void launch_gemm_ws(const ConvArgs& a, hipStream_t s) {
    const dim3 grid(cdiv(a.npix, BN), cdiv(a.OC, BM)), block((WMG * WNG + NP) * 64);
    if constexpr (EXT) {
        if (a.in_scale && a.segsum)
            hipLaunchKernelGGL((gemm_ws_kernel<BM, BN, WMG, WNG, KC, NST, NP, true, true>), grid, block, 0, s, a);
        else if (a.in_scale)
            hipLaunchKernelGGL((gemm_ws_kernel<BM, BN, WMG, WNG, KC, NST, NP, true, false>), grid, block, 0, s, a);
        else if (a.segsum)
            hipLaunchKernelGGL((gemm_ws_kernel<BM, BN, WMG, WNG, KC, NST, NP, false, true>), grid, block, 0, s, a);
        else
            hipLaunchKernelGGL((gemm_ws_kernel<BM, BN, WMG, WNG, KC, NST, NP>), grid, block, 0, s, a);
    } else {
        hipLaunchKernelGGL((gemm_ws_kernel<BM, BN, WMG, WNG, KC, NST, NP>), grid, block, 0, s, a);
    }
}

// ---------------------------------------------------------------------------
// conv3x3_halo_kernel: stride-1 3x3 conv for narrow layers (IC, OC <= 64).
// A workgroup owns a TH x TW output tile of one image and OCB output
// channels.  Per IC chunk it DMAs the (TH+2) x (TW+2) input halo and the
// weights of all 9 taps into LDS once, then runs 9 * KC/16 MFMA k-steps per
// barrier; each input pixel is fetched once per tile instead of once per tap.
// An MFMA column block is 32 consecutive output columns of one tile row, so
// its B operand for tap (kh, kw) is 32 consecutive halo pixels.
// ---------------------------------------------------------------------------
template <int OCB, int KC, int TH, int TW>
__global__ __launch_bounds__(256) void conv3x3_halo_kernel(ConvArgs a) {
    constexpr int NW = 4;
    constexpr int CPR = KC / 8, RB = KC * 2;
    constexpr int HW = TW + 2, HH = TH + 2, HPIX = HH * HW;
    constexpr int WROWS = 9 * OCB;                       // weight rows: (tap, oc)
    constexpr int NBLK_N = TH * TW / 32, NBLK_M = OCB / 32;
    constexpr int NBLK = NBLK_N * NBLK_M;                // 32x32 output blocks
    static_assert(NBLK % NW == 0, "blocks split evenly over 4 waves");
    constexpr int BPW = NBLK / NW;
    constexpr int W_INS = WROWS * CPR / 64;              // DMA instructions for weights
    constexpr int X_SLOTS = HPIX * CPR;
    constexpr int X_INS = (X_SLOTS + 63) / 64;
    static_assert((WROWS * CPR) % 64 == 0, "weight rows fill whole DMA instructions");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[(W_INS + X_INS) * 1024];
    uint8_t* sw = smem;
    uint8_t* sx = smem + W_INS * 1024;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tiles_w = (a.Wo + TW - 1) / TW, tiles_h = (a.Ho + TH - 1) / TH;
    const int t = xcd_swizzle(blockIdx.x, gridDim.x);
    const int b = t / (tiles_h * tiles_w);
    const int trem = t - b * tiles_h * tiles_w;
    const int oh0 = (trem / tiles_w) * TH, ow0 = (trem % tiles_w) * TW;
    const int oc0 = blockIdx.y * OCB;
    // split-f16: the chunks run over ICW = terms * IC weight columns, [hi | lo
    // (| hi)] planes of the input (each chunk inside one plane: IC % KC == 0)
    const int ICW = a.split ? (a.split == 2 ? 2 : 3) * a.IC : a.IC;
    const int nc = ICW / KC;

    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.x, 0, (int)(((size_t)(a.npix_in - 1) * a.xs + a.IC + (a.split ? a.x_lo : 0)) * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.w, 0, (int)((size_t)a.OC * 9 * ICW * 2), 0x00020000);

    float16v acc[BPW];
#pragma unroll
    for (int q = 0; q < BPW; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[q][r] = 0.0f;
    const int lrow = lane & 31, lhalf = lane >> 5;

    for (int ci = 0; ci < nc; ++ci) {
        const int c0 = ci * KC;
        const int plane = c0 / a.IC;                    // 0: hi, 1: lo, 2: hi again
        const int xc0 = c0 - plane * a.IC + (plane == 1 ? a.x_lo : 0);
        // weights: LDS row (tap*OCB + oc) holds w[oc0+oc][tap][c0 .. c0+KC)
        for (int ins = wave; ins < W_INS; ins += NW) {
            const int p = ins * 64 + lane;
            const int r = p / CPR, slot = p - r * CPR;
            const int tap = r / OCB, oc = r - tap * OCB;
            const uint32_t off = (uint32_t)((((oc0 + oc) * 9 + tap) * ICW + c0 + swz<KC>(r, slot) * 8) * 2);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_void*)(sw + ins * 1024), 16, off, 0, 0, 0);
        }
        // input halo: LDS row (hr*HW + hc) holds x[b][oh0-1+hr][ow0-1+hc][c0 .. c0+KC)
        for (int ins = wave; ins < X_INS; ins += NW) {
            const int p = ins * 64 + lane;
            const int r = p / CPR, slot = p - r * CPR;
            uint32_t off = kOOB;
            if (r < HPIX) {
                const int hr = r / HW, hc = r - hr * HW;
                const int ih = oh0 - 1 + hr, iw = ow0 - 1 + hc;
                if (ih >= 0 && ih < a.H && iw >= 0 && iw < a.W)
                    off = (uint32_t)((((b * a.H + ih) * a.W + iw) * a.xs + xc0 + swz<KC>(r, slot) * 8) * 2);
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(sx + ins * 1024), 16, off, 0, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            const int kh = tap / 3, kw = tap - kh * 3;
#pragma unroll
            for (int kk = 0; kk < KC / 16; ++kk) {
                const int c = kk * 2 + lhalf;
#pragma unroll
                for (int q = 0; q < BPW; ++q) {
                    const int blk = wave * BPW + q;
                    const int mb = blk % NBLK_M, nb = blk / NBLK_M;
                    const int orow = nb / (TW / 32), ocol = (nb % (TW / 32)) * 32 + lrow;
                    const int wr = tap * OCB + mb * 32 + lrow;
                    const int xrow = (orow + kh) * HW + ocol + kw;
                    const half8 af = *reinterpret_cast<const half8*>(sw + wr * RB + swz<KC>(wr, c) * 16);
                    const half8 bf = *reinterpret_cast<const half8*>(sx + xrow * RB + swz<KC>(xrow, c) * 16);
                    acc[q] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc[q], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    }

    // staged epilogue: the TH x TW x OCB tile as [pixel][oc] f32 in LDS
    constexpr int TS = OCB + 4;
    static_assert(TH * TW * TS * 4 <= (W_INS + X_INS) * 1024, "halo epilogue staging fits the LDS buffer");
    float* sT = reinterpret_cast<float*>(smem);
    // (the loop above ends with a barrier: every wave is done reading smem)
#pragma unroll
    for (int q = 0; q < BPW; ++q) {
        const int blk = wave * BPW + q;
        const int mb = blk % NBLK_M, nb = blk / NBLK_M;
        stage_block(sT, TS, nb * 32, mb * 32, acc[q], lane);
    }
    __syncthreads();
    double nopart[2][8];
    finish_staged<OCB>(
        a, sT, TH * TW, oc0, tid, 256,
        [&](int pl) {
            const int oh = oh0 + pl / TW, ow = ow0 + pl % TW;
            return (oh < a.Ho && ow < a.Wo) ? (b * a.Ho + oh) * a.Wo + ow : -1;
        },
        nopart, 0);
}

template <int OCB, int KC, int TH, int TW>
void launch_halo(const ConvArgs& a, hipStream_t s) {
    const int B = a.npix / (a.Ho * a.Wo);
    const int tiles = B * ((a.Ho + TH - 1) / TH) * ((a.Wo + TW - 1) / TW);
    hipLaunchKernelGGL((conv3x3_halo_kernel<OCB, KC, TH, TW>), dim3(tiles, cdiv(a.OC, OCB)), dim3(256), 0, s, a);
}

// ---------------------------------------------------------------------------
// resblock3x3_kernel: one whole stride-1 identity BasicBlock of the ResNet
// trunk (src/encoder_resnet.cpp:33-48: conv1 -> ReLU -> conv2 -> + x -> ReLU,
// with BN folded into both convs), for C = 32 channels:
//   t = f16(relu(conv1(x) + b1)),   y = f16(relu(conv2(t) + b2 + x)).
// Tiles are TH output rows x 30 output columns of one image, ordered rows
// fastest, and each persistent workgroup walks a contiguous range of them, so
// consecutive tiles share halo rows in L2.  Every wave holds both weight
// tensors' MFMA A fragments in VGPRs for the whole launch (18 + 18 fragments
// for C = 32), so LDS carries only pixels:
//   * the (TH+4) x 34 input halo, double-buffered: tile k+1's DMA is issued
//     before tile k's convs start;
//   * the (TH+2) x 32 intermediate tile, written by conv1 straight from its
//     accumulators (zero outside the image: conv2's zero padding);
//   * a 2 KB staging block per wave that turns conv2's MFMA layout into
//     16-byte channel rows for coalesced stores.
// conv2 runs over TH rows x 32 columns (the last two of each row are
// discarded); the residual comes from the halo already in LDS.  HBM sees x
// read about once and y written once; the block as two convolutions also
// writes t, reads it back and reads x a second time.  The arithmetic (f16
// products, f32 sums in tap-major, channel-minor order, f16 rounding of t,
// then + b2, + x, ReLU) is the halo conv kernel's, so y equals the two-launch
// block bit for bit.  Barriers wait for LDS traffic only; global stores drain
// in the background.
// ---------------------------------------------------------------------------

// LDS pixel rows of the fused block are C*2 bytes of channels plus 16 bytes of
// padding (80 bytes for C = 32): 16 consecutive rows then start in 16
// distinct 16-byte bank groups (5r mod 16 is a permutation), so every MFMA
// operand read (32 consecutive rows, one 16-byte chunk) is conflict-free for
// any base row, and its address is a per-lane base plus a compile-time
// immediate per (tap, k-step).
template <int C>
struct PadRow {
    static constexpr int RB = C * 2 + 16;   // bytes per LDS row
    static constexpr int SPR = C / 8 + 1;   // 16-byte slots per row (the last is padding)
};

// NR rows (row0, row0 + step, ...) of a stride-1 3x3 conv whose 32-column
// MFMA block for tap (kh, kw) is 32 consecutive pixels of LDS source row
// row + kh (SW pixels per row) from column kw; wf holds the A fragments of
// the 9 * C/16 (tap, k-step) steps in order.  The B reads run PD steps ahead
// of the MFMAs (a register ring), so with two waves per SIMD the MFMAs issue
// back to back instead of each waiting out one LDS round trip.
struct NoSide {
    __device__ __forceinline__ void operator()(int) const {}
};

// side(s) runs after step s's MFMAs are issued: work spread over the steps
// (e.g. DMA instructions) so it never stalls all waves at once.
template <int C, int NR, int SW, int PD = 4, class Side = NoSide>
__device__ __forceinline__ void conv_rows(const half8* wf, const uint8_t* src, int row0, int step, int lrow,
                                          int lhalf, float16v* acc, const Side& side = Side()) {
    constexpr int RB = PadRow<C>::RB, KS = C / 16, NS = 9 * KS, NQ = NR > 0 ? NR : 1;
    static_assert(PD >= 1 && PD < NS, "prefetch distance within the step count");
    if constexpr (NR == 0) return;
    const uint8_t* base = src + lrow * RB + lhalf * 16;
    auto load = [&](int s, half8* dst) {
        const int tap = s / KS, kk = s - tap * KS;
        const int kh = tap / 3, kw = tap - kh * 3;
#pragma unroll
        for (int q = 0; q < NR; ++q)
            dst[q] = *reinterpret_cast<const half8*>(base + ((row0 + q * step + kh) * SW + kw) * RB + kk * 32);
    };
    half8 ring[PD][NQ];
#pragma unroll
    for (int s = 0; s < PD; ++s) load(s, ring[s]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        half8 cur[NQ];
#pragma unroll
        for (int q = 0; q < NR; ++q) cur[q] = ring[s % PD][q];
        if (s + PD < NS) load(s + PD, ring[s % PD]);
        // keep the scheduler from sinking the reads back next to their MFMAs
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < NR; ++q) acc[q] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[s], cur[q], acc[q], 0, 0, 0);
        side(s);
    }
}

// Geometry of the fused block's tiles.
template <int C, int TH, int NW>
struct ResTile {
    static constexpr int RB = PadRow<C>::RB, SPR = PadRow<C>::SPR, NF = 9 * C / 16;   // NF: A fragments per conv
    static constexpr int XW = 34, XH = TH + 4, XPIX = XH * XW;       // input halo
    static constexpr int TW = 32, TH1 = TH + 2;                      // intermediate tile
    static constexpr int TPIX = TH1 * TW + 2;                        // + 2 pixels read only for discarded columns
    static constexpr int OW = TW - 2;                                // stored output columns per row
    static constexpr int X_INS = (XPIX * SPR + 63) / 64;             // DMA instructions per halo
    static constexpr int X_IPW = (X_INS + NW - 1) / NW;              // ... per wave
    static constexpr int X_BYTES = X_INS * 1024, T_BYTES = (TPIX * RB + 1023) / 1024 * 1024, S_BYTES = 32 * RB;
};

// One tile of the fused block.  The LDS regions arrive as distinct
// __restrict__ pointers: the inlined accesses then carry alias scopes, which
// lets the compiler see that conv1 / conv2 / the epilogue never touch the
// buffer the next halo is DMA'd into, so it does not make them wait for it.
// hofs / hpos: this lane's slot of each of its halo DMA instructions as a
// byte offset from the halo's origin pixel and as (row << 8 | column), with
// row 255 for padding slots.
template <int C, int TH, int NW>
__device__ __forceinline__ void resblock_tile(const uint8_t* __restrict__ sx, uint8_t* __restrict__ sxn,
                                              uint8_t* __restrict__ st, uint8_t* __restrict__ sstage,
                                              const float* __restrict__ sbias, const half8* wf1, const half8* wf2,
                                              const int* hofs, const int* hpos, __amdgpu_buffer_rsrc_t xr,
                                              bool prefetch, int nb, int noh0, int now0, int b, int oh0, int ow0,
                                              int H, int W, half_t* __restrict__ y, int wave, int lane) {
    using G = ResTile<C, TH, NW>;
    constexpr int RB = G::RB, XW = G::XW, TW = G::TW, TH1 = G::TH1, OW = G::OW, CPR = C / 8;
    constexpr int F1 = TH1 / NW, R1 = TH1 % NW, NB1 = F1 + (R1 ? 1 : 0);   // conv1 rows per wave
    constexpr int F2 = TH / NW, R2 = TH % NW, NB2 = F2 + (R2 ? 1 : 0);     // conv2 rows per wave
    const int lrow = lane & 31, lhalf = lane >> 5;

    // next tile's halo: LDS row hr * 34 + hc holds x[nb][noh0 - 2 + hr][now0 - 2 + hc][0 .. C)
    if (prefetch) {
        const int origin = ((nb * H + noh0 - 2) * W + now0 - 2) * C * 2;
#pragma unroll
        for (int i = 0; i < G::X_IPW; ++i) {
            const int ins = wave + i * NW;
            if (ins >= G::X_INS) break;
            const int ih = noh0 - 2 + (hpos[i] >> 8), iw = now0 - 2 + (hpos[i] & 255);
            const uint32_t off = ((unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W) ? (uint32_t)(origin + hofs[i])
                                                                                            : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(sxn + ins * 1024), 16, off, 0, 0, 0);
        }
    }

    // conv1: intermediate row j (image row oh0 - 1 + j, columns ow0 - 1 ..
    // ow0 + 30) is one MFMA column block; its B operand for tap (kh, kw) is
    // 32 consecutive halo pixels of halo row j + kh from column kw.  Wave w
    // owns rows w, w + NW, ...; a remainder row (waves < R1) runs as its own
    // branch-free chain.
    float16v acc1[NB1];
#pragma unroll
    for (int q = 0; q < NB1; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc1[q][r] = 0.0f;
    conv_rows<C, F1, XW>(wf1, sx, wave, NW, lrow, lhalf, acc1);
    if (R1 && wave < R1) conv_rows<C, 1, XW>(wf1, sx, wave + F1 * NW, NW, lrow, lhalf, acc1 + F1);
    // t = f16(relu(acc + b1)), zero outside the image.  Register g*4+e of a
    // lane holds channel 8g + 4*lhalf + e of intermediate column lrow.
#pragma unroll
    for (int q = 0; q < NB1; ++q) {
        const int j = wave + q * NW;
        if (j >= TH1) continue;
        const int ih = oh0 - 1 + j, iw = ow0 - 1 + lrow;
        const bool inside = ih >= 0 && ih < H && iw >= 0 && iw < W;
        uint8_t* const trow = st + (j * TW + lrow) * RB + lhalf * 8;
#pragma unroll
        for (int g = 0; g < C / 8; ++g) {
            const float4v bb = *reinterpret_cast<const float4v*>(sbias + g * 8 + lhalf * 4);
            half4 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float v = fmaxf(acc1[q][g * 4 + e] + bb[e], 0.0f);
                h[e] = inside ? (half_t)v : (half_t)0.0f;
            }
            *reinterpret_cast<half4*>(trow + g * 16) = h;
        }
    }
    lds_barrier();

    // conv2: output row i (columns ow0 .. ow0 + 31) reads intermediate rows
    // i .. i + 2, 32 consecutive pixels from column kw.
    float16v acc2[NB2];
#pragma unroll
    for (int q = 0; q < NB2; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc2[q][r] = 0.0f;
    conv_rows<C, F2, TW>(wf2, st, wave, NW, lrow, lhalf, acc2);
    if (R2 && wave < R2) conv_rows<C, 1, TW>(wf2, st, wave + F2 * NW, NW, lrow, lhalf, acc2 + F2);
    // this wave's share of the next halo must land before the next barrier;
    // waiting here, ahead of the epilogue, keeps this tile's stores out of it
    __builtin_amdgcn_s_waitcnt(0);

    // y = f16(relu(acc + b2 + x)) in the MFMA layout (residual from the
    // halo), through this wave's staging block to 16-byte channel rows
#pragma unroll
    for (int q = 0; q < NB2; ++q) {
        const int i = wave + q * NW;
        if (i >= TH) continue;
        const uint8_t* const xrow = sx + ((i + 2) * XW + lrow + 2) * RB + lhalf * 8;
        uint8_t* const srow = sstage + lrow * RB + lhalf * 8;
#pragma unroll
        for (int g = 0; g < C / 8; ++g) {
            const float4v bb = *reinterpret_cast<const float4v*>(sbias + C + g * 8 + lhalf * 4);
            const half4 r = *reinterpret_cast<const half4*>(xrow + g * 16);
            half4 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float v = acc2[q][g * 4 + e] + bb[e];
                const float o = v + (float)r[e];
                h[e] = (half_t)fmaxf(o, 0.0f);
            }
            *reinterpret_cast<half4*>(srow + g * 16) = h;
        }
        const int oh = oh0 + i;
#pragma unroll
        for (int hp = 0; hp < 32 * CPR / 64; ++hp) {
            const int pix = hp * (64 / CPR) + lane / CPR, ch = lane % CPR;
            const half8 v = *reinterpret_cast<const half8*>(sstage + pix * RB + ch * 16);
            const int ow = ow0 + pix;
            if (pix < OW && oh < H && ow < W)
                *reinterpret_cast<half8*>(y + ((size_t)(b * H + oh) * W + ow) * C + ch * 8) = v;
        }
    }
}

template <int C, int TH, int NW>
__global__ __launch_bounds__(NW * 64) void resblock3x3_kernel(const half_t* __restrict__ x,
                                                              const half_t* __restrict__ w1,
                                                              const float* __restrict__ b1,
                                                              const half_t* __restrict__ w2,
                                                              const float* __restrict__ b2, half_t* __restrict__ y,
                                                              int H, int W, int npix_in, int ntiles, int per_wg) {
    static_assert(C == 32, "both weight tensors live in VGPRs only for 32 channels");
    using G = ResTile<C, TH, NW>;
    __shared__ __attribute__((aligned(1024))) uint8_t sx0[G::X_BYTES];
    __shared__ __attribute__((aligned(1024))) uint8_t sx1[G::X_BYTES];
    __shared__ __attribute__((aligned(1024))) uint8_t st[G::T_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t sstage[NW * G::S_BYTES];
    __shared__ float sbias[2 * C];   // b1, b2: read from LDS so no global load waits behind the halo DMA

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int tiles_w = (W + G::OW - 1) / G::OW, tiles_h = (H + TH - 1) / TH;
    const int t_begin = blockIdx.x * per_wg;
    const int t_end = t_begin + per_wg < ntiles ? t_begin + per_wg : ntiles;
    if (t_begin >= t_end) return;   // the whole workgroup: no barrier is pending

    // A fragments: lane l holds w[oc = l % 32][tap][8 (kk*2 + l/32) .. + 8)
    half8 wf1[G::NF], wf2[G::NF];
#pragma unroll
    for (int tap = 0; tap < 9; ++tap)
#pragma unroll
        for (int kk = 0; kk < C / 16; ++kk) {
            const size_t off = (size_t)(lrow * 9 + tap) * C + (kk * 2 + lhalf) * 8;
            wf1[tap * (C / 16) + kk] = *reinterpret_cast<const half8*>(w1 + off);
            wf2[tap * (C / 16) + kk] = *reinterpret_cast<const half8*>(w2 + off);
        }
    if (tid < 2 * C) sbias[tid] = tid < C ? b1[tid] : b2[tid - C];
    // this lane's halo DMA slots (the same for every tile)
    int hofs[G::X_IPW], hpos[G::X_IPW];
#pragma unroll
    for (int i = 0; i < G::X_IPW; ++i) {
        const int p = (wave + i * NW) * 64 + lane;
        const int r = p / G::SPR, cc = p - r * G::SPR;
        const int hr = r / G::XW, hc = r - hr * G::XW;
        const bool data = r < G::XPIX && cc < C / 8;
        hofs[i] = (hr * W + hc) * C * 2 + cc * 16;
        hpos[i] = data ? (hr << 8 | hc) : (255 << 8);
    }

    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, npix_in * C * 2, 0x00020000);
    // tile t: rows fastest, then columns, then images
    auto coords = [&](int t, int& b, int& oh0, int& ow0) {
        const int th = t % tiles_h, r = t / tiles_h;
        const int tw = r % tiles_w;
        b = r / tiles_w;
        oh0 = th * TH;
        ow0 = tw * G::OW;
    };

    int b, oh0, ow0;
    coords(t_begin, b, oh0, ow0);
    {
        const int origin = ((b * H + oh0 - 2) * W + ow0 - 2) * C * 2;
#pragma unroll
        for (int i = 0; i < G::X_IPW; ++i) {
            const int ins = wave + i * NW;
            if (ins >= G::X_INS) break;
            const int ih = oh0 - 2 + (hpos[i] >> 8), iw = ow0 - 2 + (hpos[i] & 255);
            const uint32_t off = ((unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W) ? (uint32_t)(origin + hofs[i])
                                                                                            : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(sx0 + ins * 1024), 16, off, 0, 0, 0);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);   // weights in VGPRs and this wave's share of the first halo
#pragma unroll 1
    for (int t = t_begin; t < t_end; t += 2) {
        // Two tiles per trip so each buffer has a fixed role: tile t reads
        // sx0 while tile t+1's halo lands in sx1, and the other way round.
        // Before each tile: every wave's halo has landed (each waited for its
        // own DMA before the barrier) and the previous tile is done with the
        // intermediate buffer, its staging blocks and the halo buffer about
        // to be refilled.
        int nb, noh0, now0;
        lds_barrier();
        coords(t + 1 < t_end ? t + 1 : t, nb, noh0, now0);
        resblock_tile<C, TH, NW>(sx0, sx1, st, sstage + wave * G::S_BYTES, sbias, wf1, wf2, hofs, hpos, xr,
                                 t + 1 < t_end, nb, noh0, now0, b, oh0, ow0, H, W, y, wave, lane);
        if (t + 1 >= t_end) break;
        b = nb; oh0 = noh0; ow0 = now0;
        lds_barrier();
        coords(t + 2 < t_end ? t + 2 : t + 1, nb, noh0, now0);
        resblock_tile<C, TH, NW>(sx1, sx0, st, sstage + wave * G::S_BYTES, sbias, wf1, wf2, hofs, hpos, xr,
                                 t + 2 < t_end, nb, noh0, now0, b, oh0, ow0, H, W, y, wave, lane);
        b = nb; oh0 = noh0; ow0 = now0;
    }
}

int device_cu_count() {
    static const int n = [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        return cus;
    }();
    return n;
}

template <int TH, int NW, int WG_PER_CU>
void launch_resblock(const half_t* x, const half_t* w1, const float* b1, const half_t* w2, const float* b2, half_t* y,
                     int batch, int H, int W, hipStream_t s) {
    const int ntiles = batch * cdiv(H, TH) * cdiv(W, 30);
    const int slots = device_cu_count() * WG_PER_CU;
    const int per = cdiv(ntiles, slots);
    hipLaunchKernelGGL((resblock3x3_kernel<32, TH, NW>), dim3(cdiv(ntiles, per)), dim3(NW * 64), 0, s, x, w1, b1, w2,
                       b2, y, H, W, batch * H * W, ntiles, per);
}

// ---------------------------------------------------------------------------
// conv3x3_rw_kernel: persistent stride-1 3x3 conv (pad 1) for the narrow
// ResNet stages, IC and OC in {32, 64}, with the plain epilogue
// y = act(conv(x) + bias [+ residual]) (act: none or ReLU), dense f16 NHWC.
// The machinery of the fused block: the OC/32 MFMA row blocks are split over
// wave groups and every wave keeps the A fragments of its 32 output channels
// (9 * IC/16 fragments, 144 VGPRs at IC = 64) and their biases in registers
// for the whole launch; each workgroup walks a contiguous range of TH x 32
// output tiles (rows fastest) through an NS-stage LDS ring: a stage holds
// one tile's (TH+2) x 34 input halo and its residual tile (80/144-byte
// padded rows), and tile t+NS-1 is DMA'd while tile t computes, so NS-1
// tiles' loads are in flight per workgroup (one tile's load takes longer
// than its convolution).  The B reads run a few MFMAs ahead; results leave
// straight from the accumulators as 8-byte stores (4 channels of one pixel
// per lane, the two lane halves filling 16 contiguous bytes).  Products and
// sums are the other conv kernels' (f16 x f16, f32 accumulation in
// tap-major, channel-minor order, then + bias, + residual, act).
//
// The ring's DMA goes through dma16 (inline assembly): the compiler does not
// see it as a write to LDS, so it never makes the convolution's LDS reads
// wait for the loads in flight into the other stages; the kernel orders them
// itself with explicit vmcnt waits and the per-tile barrier.
// ---------------------------------------------------------------------------
template <int IC, int OC, int TH, int NW, int NS>
struct RwTile {
    static constexpr int RBX = PadRow<IC>::RB, SPRX = PadRow<IC>::SPR;   // halo rows
    static constexpr int RBR = PadRow<OC>::RB, SPRR = PadRow<OC>::SPR;   // residual rows
    static constexpr int XW = 34, XPIX = (TH + 2) * XW, RPIX = TH * 32;
    static constexpr int X_INS = (XPIX * SPRX + 63) / 64, R_INS = (RPIX * SPRR + 63) / 64;
    static constexpr int X_IPW = (X_INS + NW - 1) / NW, R_IPW = (R_INS + NW - 1) / NW;
    static constexpr int NWM = OC / 32, WPM = NW / NWM;                 // wave groups, waves per group
    static constexpr int F = TH / WPM, R = TH % WPM, NB = F + (R ? 1 : 0);
    static constexpr int NF = 9 * IC / 16;
    static constexpr int X_BYTES = X_INS * 1024, STAGE = X_BYTES + R_INS * 1024;
    static_assert(NS >= 2, "the tile being computed and at least the next one");
    static_assert(NS * STAGE <= 163840, "the ring fits the 160 KB of LDS");
};


// Per-workgroup constants of the register-weight kernel's tile walk.
struct RwWalk {
    const int* hofs; const int* hpos; const int* rofs; const int* rpos;
    int4v xr, rr;
    int tiles_w, tiles_h, t_end, per_tile, H, W;
};

// This wave's DMA instructions for tile t's input halo and (RES) residual
// into stage st, issued one at a time from the convolution of the tile
// before it: instruction j after step j * SP, so the issue stalls of the
// memory pipeline (every wave has a tile's worth to issue) fall between
// MFMAs instead of holding all waves at the top of the tile.
template <int IC, int OC, int TH, int NW, int NS, bool RES>
struct RwSide {
    using G = RwTile<IC, OC, TH, NW, NS>;
    static constexpr int NI = G::X_IPW + (RES ? G::R_IPW : 0), STEPS = 9 * IC / 16;
    static constexpr int SP = STEPS / NI > 0 ? STEPS / NI : 1;
    static_assert(NI * SP <= STEPS, "every instruction has a step");
    uint8_t* st;
    const RwWalk* k;
    int oh0, ow0, xo, ro, wave;
    bool on;
    __device__ __forceinline__ RwSide(uint8_t* st_, const RwWalk& k_, int t, int wave_, bool on_)
        : st(st_), k(&k_), wave(wave_), on(on_) {
        const int th = t % k_.tiles_h, r = t / k_.tiles_h, tw = r % k_.tiles_w;
        const int b = r / k_.tiles_w;
        oh0 = th * TH;
        ow0 = tw * 32;
        xo = ((b * k_.H + oh0 - 1) * k_.W + ow0 - 1) * IC * 2;
        ro = ((b * k_.H + oh0) * k_.W + ow0) * OC * 2;
    }
    __device__ __forceinline__ void operator()(int s) const {
        if (s % SP != 0 || !on) return;
        const int j = s / SP;
        if (j < G::X_IPW) {
            const int ins = wave + j * NW;
            if (ins >= G::X_INS) return;
            const int ih = oh0 - 1 + (k->hpos[j] >> 8), iw = ow0 - 1 + (k->hpos[j] & 255);
            const uint32_t off = ((unsigned)ih < (unsigned)k->H && (unsigned)iw < (unsigned)k->W)
                                     ? (uint32_t)(xo + k->hofs[j]) : kOOB;
            dma16(st + ins * 1024, k->xr, off);
        } else if constexpr (RES) {
            const int i = j - G::X_IPW;
            if (i >= G::R_IPW) return;
            const int ins = wave + i * NW;
            if (ins >= G::R_INS) return;
            const int ih = oh0 + (k->rpos[i] >> 8), iw = ow0 + (k->rpos[i] & 255);
            const uint32_t off = ((unsigned)ih < (unsigned)k->H && (unsigned)iw < (unsigned)k->W)
                                     ? (uint32_t)(ro + k->rofs[i]) : kOOB;
            dma16(st + G::X_BYTES + ins * 1024, k->rr, off);
        }
    }
};

// All of this wave's DMA instructions for tile t into stage st at once.
template <int IC, int OC, int TH, int NW, int NS, bool RES>
__device__ __forceinline__ void rw_issue(uint8_t* st, const RwWalk& k, int t, int wave) {
    const RwSide<IC, OC, TH, NW, NS, RES> side(st, k, t, wave, true);
#pragma unroll
    for (int j = 0; j < RwSide<IC, OC, TH, NW, NS, RES>::NI; ++j) side(j * RwSide<IC, OC, TH, NW, NS, RES>::SP);
}

// Tile t from stage st while tile t+NS-1's DMA goes out into stage nst
// (prefetch: it is in the walk): conv, then wait until at most `younger` of
// this wave's DMA instructions are in flight (those of the tiles after t+1:
// loads complete in issue order, so tile t+1's have landed; this tile's
// stores stay out of the wait), then the epilogue.
template <int IC, int OC, int TH, int NW, int NS, bool RES>
__device__ __forceinline__ void rw_tile(const uint8_t* st, uint8_t* nst, bool prefetch, const half8* wf,
                                        const float* bv, const RwWalk& k, int t, int younger, const ConvArgs& a,
                                        int wave, int lane) {
    using G = RwTile<IC, OC, TH, NW, NS>;
    const int H = k.H, W = k.W;
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int mg = wave / G::WPM, wr = wave - mg * G::WPM;   // wave group (32 output channels), row slot
    const int th = t % k.tiles_h, r = t / k.tiles_h, tw = r % k.tiles_w;
    const int b = r / k.tiles_w, oh0 = th * TH, ow0 = tw * 32;
    const RwSide<IC, OC, TH, NW, NS, RES> side(nst, k, t + NS - 1, wave, prefetch);

    // output row i (columns ow0 .. ow0 + 31) is one MFMA column block; its B
    // operand for tap (kh, kw) is 32 consecutive halo pixels of halo row
    // i + kh from column kw
    float16v acc[G::NB];
#pragma unroll
    for (int q = 0; q < G::NB; ++q)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[q][e] = 0.0f;
    if constexpr (G::F > 0) {
        conv_rows<IC, G::F, G::XW>(wf, st, wr, G::WPM, lrow, lhalf, acc, side);
    } else {
        // fewer rows than waves per group: not every wave runs a conv, so
        // the DMA goes out up front
#pragma unroll
        for (int j = 0; j < side.NI; ++j) side(j * side.SP);
    }
    if (G::R && wr < G::R) conv_rows<IC, 1, G::XW>(wf, st, wr + G::F * G::WPM, G::WPM, lrow, lhalf, acc + G::F);
    wait_vmcnt_le(younger);

    // act(acc + bias [+ residual]) straight from the accumulators: register
    // g*4+e of a lane is channel oc0 + 8g + 4*lhalf + e of pixel column lrow
    const int oc0 = mg * 32, ow = ow0 + lrow;
    half_t* const y = static_cast<half_t*>(a.y);
    const bool relu = a.act == VDK_ACT_RELU;
#pragma unroll
    for (int q = 0; q < G::NB; ++q) {
        const int i = wr + q * G::WPM, oh = oh0 + i;
        if (i >= TH || oh >= H || ow >= W) continue;
        const uint8_t* const rrow = st + G::X_BYTES + (i * 32 + lrow) * G::RBR + oc0 * 2 + lhalf * 8;
        half_t* const yp = y + ((size_t)(b * H + oh) * W + ow) * OC + oc0 + lhalf * 4;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = acc[q][g * 4 + e] + bv[g * 4 + e];
            if constexpr (RES) {
                const half4 rv = *reinterpret_cast<const half4*>(rrow + g * 16);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] += (float)rv[e];
            }
            half4 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = (half_t)(relu ? fmaxf(v[e], 0.0f) : v[e]);
            *reinterpret_cast<half4*>(yp + g * 8) = h;
        }
    }
}

template <int IC, int OC, int TH, int NW, int NS, bool RES>
__global__ __launch_bounds__(NW * 64) void conv3x3_rw_kernel(ConvArgs a, int ntiles, int per_wg) {
    using G = RwTile<IC, OC, TH, NW, NS>;
    static_assert(G::NWM * G::WPM == NW && G::WPM >= 1, "wave groups split the workgroup evenly");
    __shared__ __attribute__((aligned(1024))) uint8_t ring[NS * G::STAGE];

    const int W = a.W;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int t_begin = blockIdx.x * per_wg;
    const int t_end = t_begin + per_wg < ntiles ? t_begin + per_wg : ntiles;
    if (t_begin >= t_end) return;   // the whole workgroup: no barrier is pending

    // this lane's DMA slots (the same for every tile): byte offset from the
    // tile origin and (row << 8 | column), row 255 for padding slots
    int hofs[G::X_IPW], hpos[G::X_IPW], rofs[G::R_IPW], rpos[G::R_IPW];
#pragma unroll
    for (int i = 0; i < G::X_IPW; ++i) {
        const int p = (wave + i * NW) * 64 + lane;
        const int r = p / G::SPRX, cc = p - r * G::SPRX;
        const int hr = r / G::XW, hc = r - hr * G::XW;
        hofs[i] = (hr * W + hc) * IC * 2 + cc * 16;
        hpos[i] = (r < G::XPIX && cc < IC / 8) ? (hr << 8 | hc) : (255 << 8);
    }
#pragma unroll
    for (int i = 0; i < G::R_IPW; ++i) {
        const int p = (wave + i * NW) * 64 + lane;
        const int r = p / G::SPRR, cc = p - r * G::SPRR;
        const int pr = r / 32, pc = r - pr * 32;
        rofs[i] = (pr * W + pc) * OC * 2 + cc * 16;
        rpos[i] = (r < G::RPIX && cc < OC / 8) ? (pr << 8 | pc) : (255 << 8);
    }
    RwWalk k;
    k.hofs = hofs; k.hpos = hpos; k.rofs = rofs; k.rpos = rpos;
    k.xr = dma_rsrc(a.x, (uint32_t)a.npix_in * IC * 2);
    k.rr = dma_rsrc(RES ? (const void*)a.res : (const void*)a.x, RES ? (uint32_t)a.npix * OC * 2 : 0u);
    k.H = a.H;
    k.W = W;
    k.tiles_w = (W + 31) / 32;
    k.tiles_h = (a.H + TH - 1) / TH;
    k.t_end = t_end;
    // this wave's DMA instructions per tile
    k.per_tile = (G::X_INS - wave + NW - 1) / NW + (RES ? (G::R_INS - wave + NW - 1) / NW : 0);

    // the first tile's DMA goes out ahead of the weight loads, which it
    // overlaps
    rw_issue<IC, OC, TH, NW, NS, RES>(ring, k, t_begin, wave);
    // A fragments and biases of this wave's 32 output channels; from the
    // chunk-major weight copy ([IC/16][9][OC][16]) a fragment is one
    // contiguous kilobyte, from the plain layout 32 pieces 9*IC*2 bytes apart
    const int oc0 = (wave / G::WPM) * 32;
    half8 wf[G::NF];
    if (a.wc) {
#pragma unroll
        for (int tap = 0; tap < 9; ++tap)
#pragma unroll
            for (int kk = 0; kk < IC / 16; ++kk)
                wf[tap * (IC / 16) + kk] = *reinterpret_cast<const half8*>(
                    a.wc + ((size_t)(kk * 9 + tap) * OC + oc0 + lrow) * 16 + lhalf * 8);
    } else {
#pragma unroll
        for (int tap = 0; tap < 9; ++tap)
#pragma unroll
            for (int kk = 0; kk < IC / 16; ++kk)
                wf[tap * (IC / 16) + kk] = *reinterpret_cast<const half8*>(
                    a.w + (size_t)((oc0 + lrow) * 9 + tap) * IC + (kk * 2 + lhalf) * 8);
    }
    float bv[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const float4v v = a.bias ? *reinterpret_cast<const float4v*>(a.bias + oc0 + g * 8 + lhalf * 4)
                                 : float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[g * 4 + e] = v[e];
    }
    // a full wait the compiler sees, so the weights count as loaded inside
    // the loop; the tiles after the first go out behind it
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int s = 1; s + 1 < NS; ++s)
        if (t_begin + s < t_end) rw_issue<IC, OC, TH, NW, NS, RES>(ring + s * G::STAGE, k, t_begin + s, wave);
    int slot = 0;
#pragma unroll 1
    for (int t = t_begin; t < t_end; ++t) {
        // every wave's share of tile t has landed (each waited for its own
        // DMA before the barrier) and tile t-1 is done with its stage, which
        // tile t+NS-1 takes over (its DMA goes out during tile t's conv)
        lds_barrier();
        const int prev = slot == 0 ? NS - 1 : slot - 1;
        // DMA instructions issued after tile t+1's: those of tiles t+2 .. t+NS-1
        const int last = t + NS - 1 < t_end - 1 ? t + NS - 1 : t_end - 1;
        const int younger = last > t + 1 ? (last - t - 1) * k.per_tile : 0;
        rw_tile<IC, OC, TH, NW, NS, RES>(ring + slot * G::STAGE, ring + prev * G::STAGE, t + NS - 1 < t_end, wf, bv,
                                         k, t, younger, a, wave, lane);
        slot = slot + 1 == NS ? 0 : slot + 1;
    }
}

template <int IC, int OC, int TH, int NW, int NS>
void launch_rw(const ConvArgs& a, hipStream_t s) {
    const int B = a.npix / (a.Ho * a.Wo);
    const int ntiles = B * cdiv(a.Ho, TH) * cdiv(a.Wo, 32);
    const int per = cdiv(ntiles, device_cu_count());
    if (a.res)
        hipLaunchKernelGGL((conv3x3_rw_kernel<IC, OC, TH, NW, NS, true>), dim3(cdiv(ntiles, per)), dim3(NW * 64), 0, s,
                           a, ntiles, per);
    else
        hipLaunchKernelGGL((conv3x3_rw_kernel<IC, OC, TH, NW, NS, false>), dim3(cdiv(ntiles, per)), dim3(NW * 64), 0,
                           s, a, ntiles, per);
}

// ---------------------------------------------------------------------------
// conv3x3_split_kernel: persistent stride-1 3x3 conv (pad 1) on split-f16
// maps (value = hi + lo, the lo plane x_lo / y_lo elements after the hi one,
// any pixel stride) with f16-exact weights (split 2: w.x_hi + w.x_lo), for
// ERes2Net's narrow Res2Net group convs (src/encoder_eres2net.cpp:111-137).
// The register-weight kernel's scheme: every wave keeps the A fragments of its
// output channels in VGPRs for the whole launch (one set serves both planes),
// each workgroup walks a contiguous range of TH x 32 output tiles (rows
// fastest) through an NS-stage LDS ring whose stage holds one tile's
// (TH+2) x 34 halo as [hi IC | lo IC] pixel rows, and tile t+NS-1's DMA goes
// out spread over tile t's MFMA steps.  Two MFMA shapes:
//   * M16: 16x16x32 MFMAs over 16-pixel column blocks, every wave computing
//     all OC/16 (1 or 2) row blocks of its pixel blocks; K = 32 is one plane's
//     32-channel chunk, or at IC = 16 both planes of a tap at once;
//   * M32: the 32x32x16 blocks of the other conv kernels in the halo kernel's
//     order (plane, 32-channel chunk, tap, 16-channel step), so the results
//     equal the halo kernel's bit for bit; wave groups of 32 output channels.
// Epilogue straight from the accumulators: + bias, [ReLU [min(v, clamp_hi)]],
// hi = f16(v), lo = f16(v - hi), 8-byte stores into both planes.
// ---------------------------------------------------------------------------
template <int IC, int OC, int TH, int NW, int NS, bool M16>
struct SpTile {
    static constexpr int kIC = IC, kOC = OC, kTH = TH, kNW = NW, kNS = NS;
    static constexpr bool kM16 = M16;
    static constexpr int C2 = 2 * IC;                                    // [hi | lo] channels per halo pixel
    static constexpr int RB = PadRow<C2>::RB, SPR = PadRow<C2>::SPR;
    static constexpr int XW = 34, XPIX = (TH + 2) * XW;
    static constexpr int X_INS = (XPIX * SPR + 63) / 64, X_IPW = (X_INS + NW - 1) / NW;
    static constexpr int STAGE = X_INS * 1024;
    static constexpr int PN = M16 ? 16 : 32;                             // pixels per MFMA column block
    static constexpr int MB = M16 ? OC / 16 : 1;                         // row blocks per wave
    static constexpr int NWM = M16 ? 1 : OC / 32, WPM = NW / NWM;        // wave groups, waves per group
    static constexpr int NBT = TH * (32 / PN);                           // column blocks per tile
    static constexpr int BPW = NBT / WPM;                                // ... per wave
    static constexpr int NFT = M16 ? (IC >= 32 ? IC / 32 : 1) : IC / 16; // A fragments per tap and row block
    static constexpr int NF = 9 * NFT * MB;
    static constexpr int NSTEP = M16 ? (IC == 16 ? 9 : 18 * IC / 32) : 36 * IC / 32;
    static constexpr int NBV = M16 ? 4 * MB : 16;                        // bias registers
    static_assert(M16 ? ((OC == 16 || OC == 32) && (IC == 16 || IC % 32 == 0)) : (OC % 32 == 0 && IC % 32 == 0),
                  "supported widths");
    static_assert(NWM * WPM == NW && NBT % WPM == 0 && BPW >= 1, "column blocks split evenly over the waves");
    static_assert(NS >= 2 && NS * STAGE <= 163840, "the ring fits the 160 KB of LDS");
};

// MFMA step s: tap, element offset of its K chunk in the [hi | lo] halo row,
// A fragment (per row block)
struct SpStep {
    int tap, coff, frag;
};
template <int IC, bool M16>
__device__ __forceinline__ constexpr SpStep sp_step(int s) {
    if constexpr (M16) {
        if constexpr (IC == 16) return {s, 0, s};
        const int pc = s / 9, tap = s - pc * 9, p = pc / (IC / 32), c = pc - p * (IC / 32);
        return {tap, p * IC + c * 32, tap * (IC / 32) + c};
    } else {
        constexpr int PER = IC / 32 * 18;
        const int p = s / PER, r = s - p * PER, c = r / 18, r2 = r - c * 18, tap = r2 / 2, kk = r2 - tap * 2;
        return {tap, p * IC + c * 32 + kk * 16, tap * (IC / 16) + c * 2 + kk};
    }
}

__device__ __forceinline__ float4v sp_mfma(const half8& a, const half8& b, const float4v& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float16v sp_mfma(const half8& a, const half8& b, const float16v& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Per-workgroup constants of the split kernel's tile walk; hpos < 0 marks a
// padding slot.
struct SpWalk {
    const int* hofs; const int* hpos;
    int4v xr;
    int tiles_w, tiles_h, per_tile, H, W, xs2;
};

// This wave's DMA instructions for tile t's halo into stage st, instruction j
// issued after MFMA step j * SP of the tile before it.
template <class G>
struct SpSide {
    static constexpr int NI = G::X_IPW, SP = G::NSTEP / NI > 0 ? G::NSTEP / NI : 1;
    static_assert(NI * SP <= G::NSTEP, "every instruction has a step");
    uint8_t* st;
    const SpWalk* k;
    int oh0, ow0, xo, wave;
    bool on;
    __device__ __forceinline__ SpSide(uint8_t* st_, const SpWalk& k_, int t, int wave_, bool on_)
        : st(st_), k(&k_), wave(wave_), on(on_) {
        const int th = t % k_.tiles_h, r = t / k_.tiles_h, tw = r % k_.tiles_w;
        const int b = r / k_.tiles_w;
        oh0 = th * G::kTH;
        ow0 = tw * 32;
        xo = ((b * k_.H + oh0 - 1) * k_.W + ow0 - 1) * k_.xs2;
    }
    __device__ __forceinline__ void operator()(int s) const {
        if (s % SP != 0 || !on) return;
        const int j = s / SP;
        if (j >= NI) return;
        const int ins = wave + j * G::kNW;
        if (ins >= G::X_INS) return;
        const int hp = k->hpos[j];
        const int ih = oh0 - 1 + (hp >> 8), iw = ow0 - 1 + (hp & 255);
        const uint32_t off = (hp >= 0 && (unsigned)ih < (unsigned)k->H && (unsigned)iw < (unsigned)k->W)
                                 ? (uint32_t)(xo + k->hofs[j]) : kOOB;
        dma16(st + ins * 1024, k->xr, off);
    }
};

template <class G>
__device__ __forceinline__ void sp_issue(uint8_t* st, const SpWalk& k, int t, int wave) {
    const SpSide<G> side(st, k, t, wave, true);
#pragma unroll
    for (int j = 0; j < SpSide<G>::NI; ++j) side(j * SpSide<G>::SP);
}

// The convolution of one tile from stage st: the B reads run PD steps ahead
// of the MFMAs; side(s) after step s.
template <class G, class Acc, class Side>
__device__ __forceinline__ void sp_conv(const half8* wf, const uint8_t* st, int wr, int lane,
                                        Acc (&acc)[G::BPW][G::MB], const Side& side) {
    constexpr int PD = 3, BPW = G::BPW, MB = G::MB;
    static_assert(PD < G::NSTEP, "prefetch distance within the step count");
    const int lp = lane % G::PN, kg = lane / G::PN;
    const uint8_t* const base = st + lp * G::RB + kg * 16;
    int boff[BPW];
#pragma unroll
    for (int q = 0; q < BPW; ++q) {
        const int j = wr + q * G::WPM;
        const int i = G::PN == 16 ? j >> 1 : j, cb = G::PN == 16 ? (j & 1) : 0;
        boff[q] = (i * G::XW + cb * G::PN) * G::RB;
    }
    auto load = [&](int s, half8* dst) {
        const SpStep si = sp_step<G::kIC, G::kM16>(s);
        const int kh = si.tap / 3, kw = si.tap - kh * 3;
#pragma unroll
        for (int q = 0; q < BPW; ++q)
            dst[q] = *reinterpret_cast<const half8*>(base + boff[q] + (kh * G::XW + kw) * G::RB + si.coff * 2);
    };
    half8 ring[PD][BPW];
#pragma unroll
    for (int s = 0; s < PD; ++s) load(s, ring[s]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < G::NSTEP; ++s) {
        half8 cur[BPW];
#pragma unroll
        for (int q = 0; q < BPW; ++q) cur[q] = ring[s % PD][q];
        if (s + PD < G::NSTEP) load(s + PD, ring[s % PD]);
        __builtin_amdgcn_sched_barrier(0);
        const int f = sp_step<G::kIC, G::kM16>(s).frag;
#pragma unroll
        for (int q = 0; q < BPW; ++q)
#pragma unroll
            for (int m = 0; m < MB; ++m) acc[q][m] = sp_mfma(wf[f * MB + m], cur[q], acc[q][m]);
        side(s);
    }
}

// Tile t from stage st while tile t+NS-1's DMA goes out into stage nst, then
// (after tile t+1's loads have landed, see rw_tile) the epilogue.
template <class G>
__device__ __forceinline__ void sp_tile(const uint8_t* st, uint8_t* nst, bool prefetch, const half8* wf,
                                        const float* bv, const SpWalk& k, int t, int younger, const ConvArgs& a,
                                        int wave, int lane) {
    using Acc = std::conditional_t<G::kM16, float4v, float16v>;
    constexpr int NE = G::kM16 ? 4 : 16, NG = NE / 4;
    const int mg = wave / G::WPM, wr = wave - mg * G::WPM;
    const int th = t % k.tiles_h, r = t / k.tiles_h, tw = r % k.tiles_w;
    const int b = r / k.tiles_w, oh0 = th * G::kTH, ow0 = tw * 32;
    const SpSide<G> side(nst, k, t + G::kNS - 1, wave, prefetch);
    Acc acc[G::BPW][G::MB];
#pragma unroll
    for (int q = 0; q < G::BPW; ++q)
#pragma unroll
        for (int m = 0; m < G::MB; ++m)
#pragma unroll
            for (int e = 0; e < NE; ++e) acc[q][m][e] = 0.0f;
    sp_conv<G>(wf, st, wr, lane, acc, side);
    wait_vmcnt_le(younger);

    half_t* const y = static_cast<half_t*>(a.y);
    const bool relu = a.act == VDK_ACT_RELU;
    const float chi = a.clamp_hi;
#pragma unroll
    for (int q = 0; q < G::BPW; ++q) {
        const int j = wr + q * G::WPM;
        const int oh = oh0 + (G::kM16 ? j >> 1 : j);
        const int ow = ow0 + (G::kM16 ? (j & 1) * 16 + (lane & 15) : (lane & 31));
        if (oh >= k.H || ow >= k.W) continue;
        half_t* const yp = y + ((size_t)(b * k.H + oh) * k.W + ow) * a.ys;
#pragma unroll
        for (int m = 0; m < G::MB; ++m)
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                // register g*4+e: channel 16m + 4*(lane/16) + e (M16), 32mg + 8g + 4*(lane/32) + e (M32)
                const int oc = chan_off(G::kM16 ? m * 16 + (lane >> 4) * 4 : mg * 32 + g * 8 + (lane >> 5) * 4, a.ygl, a.ygs);
                half4 h, l;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v = acc[q][m][g * 4 + e] + bv[(m * NG + g) * 4 + e];
                    if (relu) {
                        v = fmaxf(v, 0.0f);
                        if (chi > 0.0f) v = fminf(v, chi);
                    }
                    h[e] = (half_t)v;
                    l[e] = (half_t)(v - (float)h[e]);
                }
                *reinterpret_cast<half4*>(yp + oc) = h;
                *reinterpret_cast<half4*>(yp + a.y_lo + oc) = l;
            }
    }
}

template <int IC, int OC, int TH, int NW, int NS, bool M16>
__global__ __launch_bounds__(NW * 64) void conv3x3_split_kernel(ConvArgs a, int ntiles, int per_wg) {
    using G = SpTile<IC, OC, TH, NW, NS, M16>;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[NS * G::STAGE];

    const int W = a.W;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t_begin = blockIdx.x * per_wg;
    const int t_end = t_begin + per_wg < ntiles ? t_begin + per_wg : ntiles;
    if (t_begin >= t_end) return;   // the whole workgroup: no barrier is pending

    // this lane's DMA slots (the same for every tile): byte offset from the
    // tile origin (hi-plane slots, then lo-plane ones) and (row << 8 | column)
    const int xs2 = a.xs * 2;
    int hofs[G::X_IPW], hpos[G::X_IPW];
#pragma unroll
    for (int i = 0; i < G::X_IPW; ++i) {
        const int p = (wave + i * NW) * 64 + lane;
        const int r = p / G::SPR, cc = p - r * G::SPR;
        const int hr = r / G::XW, hc = r - hr * G::XW;
        const bool lo = cc >= IC / 8;
        hofs[i] = (hr * W + hc) * xs2 + (lo ? a.x_lo : 0) * 2 + chan_off((lo ? cc - IC / 8 : cc) * 8, a.xgl, a.xgs) * 2;
        hpos[i] = (r < G::XPIX && cc < G::C2 / 8) ? (hr << 8 | hc) : -1;
    }
    SpWalk k;
    k.hofs = hofs; k.hpos = hpos;
    k.xr = dma_rsrc(a.x, (uint32_t)(((size_t)(a.npix_in - 1) * a.xs + a.x_lo + ((IC >> a.xgl) - 1) * a.xgs +
                                     (1 << a.xgl)) * 2));
    k.H = a.H;
    k.W = W;
    k.xs2 = xs2;
    k.tiles_w = (W + 31) / 32;
    k.tiles_h = (a.H + TH - 1) / TH;
    k.per_tile = (G::X_INS - wave + NW - 1) / NW;   // this wave's DMA instructions per tile

    sp_issue<G>(ring, k, t_begin, wave);
    // A fragments (columns of the weights' hi copy, whose second copy the lo
    // plane uses) and biases of this wave's output channels
    const int mg = wave / G::WPM;
    constexpr int ICW = 2 * IC;
    auto wfrag = [&](int oc, int tap, int col) {
        return a.wc ? *reinterpret_cast<const half8*>(a.wc + (((size_t)(col >> 4) * 9 + tap) * OC + oc) * 16 + (col & 15))
                    : *reinterpret_cast<const half8*>(a.w + ((size_t)oc * 9 + tap) * ICW + col);
    };
    half8 wf[G::NF];
    float bv[G::NBV];
    if constexpr (M16) {
        const int orow = lane & 15, g = lane >> 4;
#pragma unroll
        for (int tap = 0; tap < 9; ++tap)
#pragma unroll
            for (int c = 0; c < G::NFT; ++c)
#pragma unroll
                for (int m = 0; m < G::MB; ++m)
                    wf[(tap * G::NFT + c) * G::MB + m] = wfrag(m * 16 + orow, tap, c * 32 + g * 8);
#pragma unroll
        for (int m = 0; m < G::MB; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) bv[m * 4 + e] = a.bias ? a.bias[m * 16 + g * 4 + e] : 0.0f;
    } else {
        const int orow = lane & 31, g = lane >> 5;
#pragma unroll
        for (int tap = 0; tap < 9; ++tap)
#pragma unroll
            for (int f = 0; f < IC / 16; ++f) wf[tap * (IC / 16) + f] = wfrag(mg * 32 + orow, tap, f * 16 + g * 8);
#pragma unroll
        for (int gg = 0; gg < 4; ++gg)
#pragma unroll
            for (int e = 0; e < 4; ++e) bv[gg * 4 + e] = a.bias ? a.bias[mg * 32 + gg * 8 + g * 4 + e] : 0.0f;
    }
    // a full wait the compiler sees, so the weights count as loaded inside
    // the loop; the tiles after the first go out behind it
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int s = 1; s + 1 < NS; ++s)
        if (t_begin + s < t_end) sp_issue<G>(ring + s * G::STAGE, k, t_begin + s, wave);
    int slot = 0;
#pragma unroll 1
    for (int t = t_begin; t < t_end; ++t) {
        // every wave's share of tile t has landed and tile t-1 is done with
        // its stage, which tile t+NS-1 takes over
        lds_barrier();
        const int prev = slot == 0 ? NS - 1 : slot - 1;
        const int last = t + NS - 1 < t_end - 1 ? t + NS - 1 : t_end - 1;
        const int younger = last > t + 1 ? (last - t - 1) * k.per_tile : 0;
        sp_tile<G>(ring + slot * G::STAGE, ring + prev * G::STAGE, t + NS - 1 < t_end, wf, bv, k, t, younger, a, wave,
                   lane);
        slot = slot + 1 == NS ? 0 : slot + 1;
    }
}

template <int IC, int OC, int TH, int NW, int NS, bool M16>
void launch_sp(const ConvArgs& a, hipStream_t s) {
    const int B = a.npix / (a.Ho * a.Wo);
    const int ntiles = B * cdiv(a.Ho, TH) * cdiv(a.Wo, 32);
    const int per = cdiv(ntiles, device_cu_count());
    hipLaunchKernelGGL((conv3x3_split_kernel<IC, OC, TH, NW, NS, M16>), dim3(cdiv(ntiles, per)), dim3(NW * 64), 0, s,
                       a, ntiles, per);
}

// ---------------------------------------------------------------------------
// conv3x3_band_kernel: stride-1 3x3 conv (pad 1) for the wide layers
// (IC % 16 == 0, OC % 128 == 0).  A workgroup of 8 waves owns a band of TH
// full image rows of one clip and 128 output channels; the band's pixels,
// flattened row-major, form NB = 2*NBW MFMA column blocks of 32 (so a
// 75- or 38-wide map wastes at most a couple of percent of the lanes, where
// 32-wide row tiles would waste 22-40 %).  Per 16-channel chunk of the input
// the workgroup DMAs into LDS
//   * the weights of all 9 taps for its 128 output channels (rows (tap, oc)
//     of 32 bytes, the two 16-byte halves swapped on every other group of 8
//     rows so an operand read of 16 consecutive rows hits 16 distinct bank
//     groups), and
//   * the band's (TH+2) x (W+2) input halo (48-byte rows: 32 bytes of
//     channels + 16 of padding, so 16 consecutive rows start in 16 distinct
//     bank groups and a tap is a constant offset from a lane's base row),
// double-buffered: chunk k+1 is in flight while chunk k runs 9 taps x NBW
// MFMAs per wave (wave w: output channels 32*(w%4).., column blocks
// NBW*(w/4)..).  Every B fragment is read once per tap from the halo instead
// of being re-fetched per tap as an im2col row.  The epilogue stages each
// 32x32 block per wave through LDS and runs the shared epilogue (epi8, store8) on
// 16-byte channel rows.  Products and sums are the other conv kernels'
// (f16 x f16 -> f32, tap-major / channel-minor within a chunk).
// ---------------------------------------------------------------------------
template <int TH, int NBW>
struct BandTile {
    static constexpr int NW = 8, OCB = 128;
    static constexpr int A_BYTES = 9 * OCB * 32, A_INS = A_BYTES / 1024;   // weights of one chunk
    static constexpr int NB = 2 * NBW;                                    // column blocks per band
    static constexpr int MAXW = NB * 32 / TH;                             // widest map a band holds
    static constexpr int XPIX = (TH + 2) * (MAXW + 2);                    // halo pixels, upper bound
    static constexpr int RB = 48;                                         // halo row bytes
    static constexpr int X_INS = (XPIX * 3 + 63) / 64;
    static constexpr int A_IPW = (A_INS + NW - 1) / NW, X_IPW = (X_INS + NW - 1) / NW;
    static constexpr int STAGE = A_BYTES + X_INS * 1024;                  // one pipeline buffer pair
    // epilogue: the band's residual rows (128 channels + 16 bytes of padding)
    // and a 2 KB f16 staging block per wave, in the freed pipeline buffers
    static constexpr int RRB = 272, RES_BYTES = NB * 32 * RRB, SBLK = 32 * 64;
    static_assert(RES_BYTES + NW * SBLK <= 2 * STAGE, "the epilogue fits the pipeline buffers");
};

// Weight slot p of a chunk: row p/2 = (tap, oc), 16-byte half (p & 1) xor
// ((row >> 3) & 1) of the row's 16 channels; recomputed per chunk from the
// lane (a few integer ops) rather than held in registers across the loop.
template <int TH, int NBW>
__device__ __forceinline__ void band_issue(uint8_t* __restrict__ sa, uint8_t* __restrict__ sx, int c0, int oc0,
                                           int IC, const int* xoff, __amdgpu_buffer_rsrc_t wr,
                                           __amdgpu_buffer_rsrc_t xr, int wave, int lane) {
    using G = BandTile<TH, NBW>;
    asm volatile("" : "+v"(lane));
#pragma unroll
    for (int i = 0; i < G::A_IPW; ++i) {
        const int ins = wave + i * G::NW;
        if (ins >= G::A_INS) break;
        const int p = ins * 64 + lane;
        const int row = p >> 1, tap = row >> 7, oc = row & 127;
        const int half = (p & 1) ^ ((row >> 3) & 1);
        const uint32_t off = (uint32_t)((((oc0 + oc) * 9 + tap) * IC + c0) * 2 + half * 16);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void*)(sa + ins * 1024), 16, off, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < G::X_IPW; ++i) {
        const int ins = wave + i * G::NW;
        if (ins >= G::X_INS) break;
        const uint32_t off = xoff[i] < 0 ? kOOB : (uint32_t)(xoff[i] + c0 * 2);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(sx + ins * 1024), 16, off, 0, 0, 0);
    }
}

// One chunk: the next chunk's DMA (into the other buffer pair, passed as
// distinct __restrict__ pointers so the reads below are not made to wait for
// it), then 9 taps x NBW MFMAs with the fragment reads one tap ahead.
template <int TH, int NBW>
__device__ __forceinline__ void band_chunk(const uint8_t* __restrict__ sa, const uint8_t* __restrict__ sx,
                                           uint8_t* __restrict__ sa_n, uint8_t* __restrict__ sx_n, bool prefetch,
                                           int c0n, int oc0, int IC, const int* xoff, __amdgpu_buffer_rsrc_t wr,
                                           __amdgpu_buffer_rsrc_t xr, int abase, int* bb, int hw,
                                           float16v* acc, int wave, int lane) {
    using G = BandTile<TH, NBW>;
    if (prefetch) band_issue<TH, NBW>(sa_n, sx_n, c0n, oc0, IC, xoff, wr, xr, wave, lane);
    // the B bases go behind an empty asm per chunk: otherwise the 9 x NBW
    // (base + tap offset) sums are hoisted out of the chunk loop and spill
#pragma unroll
    for (int j = 0; j < NBW; ++j) asm volatile("" : "+v"(bb[j]));
    // the 9 x NBW MFMAs as one sequence of steps (tap-major); B fragments are
    // read D steps ahead through a D-slot ring, the next tap's A fragment at
    // the first step of the current tap
    constexpr int S = 9 * NBW, D = NBW > 4 ? 2 : 3;
    half8 aq[2], bq[D];
    auto load_a = [&](int tap, int slot) {
        aq[slot] = *reinterpret_cast<const half8*>(sa + abase + tap * G::OCB * 32);
    };
    auto load_b = [&](int st, int slot) {
        const int tap = st / NBW, j = st - tap * NBW;
        const int kh = tap / 3, kw = tap - kh * 3;
        bq[slot] = *reinterpret_cast<const half8*>(sx + bb[j] + (kh * hw + kw) * G::RB);
    };
    load_a(0, 0);
#pragma unroll
    for (int st = 0; st < D; ++st) load_b(st, st);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < S; ++st) {
        const int tap = st / NBW, j = st - tap * NBW;
        const half8 cur = bq[st % D];
        if (st + D < S) load_b(st + D, st % D);
        if (j == 0 && tap + 1 < 9) load_a(tap + 1, (tap + 1) & 1);
        __builtin_amdgcn_sched_barrier(0);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aq[tap & 1], cur, acc[j], 0, 0, 0);
    }
}

template <int TH, int NBW>
__global__ __launch_bounds__(512) void conv3x3_band_kernel(ConvArgs a) {
    using G = BandTile<TH, NBW>;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * G::STAGE];
    uint8_t* const sa0 = smem;
    uint8_t* const sx0 = smem + G::A_BYTES;
    uint8_t* const sa1 = smem + G::STAGE;
    uint8_t* const sx1 = sa1 + G::A_BYTES;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int H = a.H, W = a.W, IC = a.IC, HW = W + 2;
    const int bands = (H + TH - 1) / TH;
    const int b = blockIdx.x / bands, r0 = (blockIdx.x - b * bands) * TH;
    const int oc0 = blockIdx.y * G::OCB;
    const int mb = wave & 3, ng = wave >> 2;
    const int npx = TH * W;   // band pixels (rows past H are computed and dropped)

    // this lane's halo DMA slots, as byte offsets at channel 0 (add 2*c0 per chunk)
    int xoff[G::X_IPW];
#pragma unroll
    for (int i = 0; i < G::X_IPW; ++i) {
        const int p = (wave + i * G::NW) * 64 + lane;
        const int hrow = p / 3, s = p - hrow * 3;
        const int hr = hrow / HW, hc = hrow - hr * HW;
        const int ih = r0 - 1 + hr, iw = hc - 1;
        const bool ok = s < 2 && hr < TH + 2 && ih >= 0 && ih < H && iw >= 0 && iw < W;
        xoff[i] = ok ? (int)(((size_t)(b * H + ih) * W + iw) * a.xs * 2) + s * 16 : -1;
    }
    // operand read bases: A row (tap, mb*32 + lrow) with its halves swapped
    // on odd groups of 8 rows; B halo row of pixel p = block*32 + lrow
    const int abase = (mb * 32 + lrow) * 32 + ((lhalf ^ ((lrow >> 3) & 1)) * 16);
    int bbase[NBW];
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
        int p = (ng * NBW + j) * 32 + lrow;
        if (p >= npx) p = 0;   // masked lane: any valid row, result dropped
        const int r = p / W, c = p - r * W;
        bbase[j] = (r * HW + c) * G::RB + lhalf * 16;
    }
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.w, 0, (int)((size_t)a.OC * 9 * IC * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.x, 0, (int)(((size_t)(a.npix_in - 1) * a.xs + IC) * 2), 0x00020000);

    float16v acc[NBW];
#pragma unroll
    for (int j = 0; j < NBW; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;

    const int nk = IC / 16;
    band_issue<TH, NBW>(sa0, sx0, 0, oc0, IC, xoff, wr, xr, wave, lane);
#pragma unroll 1
    for (int k = 0; k < nk; ++k) {
        // chunk k: this wave's DMA has landed (nothing else is outstanding),
        // then every wave's has, and chunk k-1's reads of the other pair are
        // done.  One chunk per trip with the buffer pair picked per chunk (the
        // inlined chunk keeps its distinct __restrict__ views, so its reads
        // still do not wait for the other pair's DMA), which keeps the
        // accumulators in one set of registers.
        __builtin_amdgcn_s_waitcnt(0);
        lds_barrier();
        const bool odd = k & 1;
        band_chunk<TH, NBW>(odd ? sa1 : sa0, odd ? sx1 : sx0, odd ? sa0 : sa1, odd ? sx0 : sx1, k + 1 < nk,
                            (k + 1) * 16, oc0, IC, xoff, wr, xr, abase, bbase, HW, acc, wave, lane);
    }
    lds_barrier();   // every wave is done reading the buffers the epilogue reuses

    // Epilogue y = act(acc + bias [+ residual]) in the MFMA layout (register
    // g*4+e of a lane: channel 8g + 4*lhalf + e of its 32-channel block,
    // pixel lrow of the column block).  The band's residual rows arrive in one
    // DMA burst into the freed pipeline buffers and the bias sits in
    // registers, so no global load waits behind a store; each finished 32x32
    // block goes through the wave's f16 staging block to 16-byte channel-row
    // stores.
    const bool has_res = a.res != nullptr;
    uint8_t* const sres = smem;
    uint8_t* const sstg = smem + G::RES_BYTES + wave * G::SBLK;
    const int ocw = oc0 + mb * 32;                   // this wave's first output channel
    float bias[16];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) bias[g * 4 + e] = a.bias ? a.bias[ocw + g * 8 + lhalf * 4 + e] : 0.0f;
    if (has_res) {
        const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)a.res, 0, (int)(((size_t)(a.npix - 1) * a.rs + a.OC) * 2), 0x00020000);
        constexpr int SPR = G::RRB / 16;             // 17 slots per row, the last is padding
        const int nins = (npx * SPR + 63) / 64;
        for (int ins = wave; ins < nins; ins += G::NW) {
            const int p = ins * 64 + lane;
            const int px = p / SPR, ch = p - px * SPR;
            const int r = px / W, c = px - r * W;
            const bool ok = ch < 16 && px < npx && r0 + r < H;
            const uint32_t off =
                ok ? (uint32_t)((((size_t)(b * H + r0 + r) * W + c) * a.rs + oc0) * 2 + ch * 16) : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_void*)(sres + ins * 1024), 16, off, 0, 0, 0);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    half_t* const y = static_cast<half_t*>(a.y);
    const bool relu = a.act == VDK_ACT_RELU;
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
        const int p0 = (ng * NBW + j) * 32;
        int pr = p0 + lrow;
        pr = pr < npx ? pr : npx - 1;
        const uint8_t* const rrow = sres + pr * G::RRB + (mb * 32 + lhalf * 4) * 2;
        uint8_t* const srow = sstg + lrow * 64 + lhalf * 8;
        // the block's 4 residual reads go out together (zero without a residual)
        half4 r4[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            r4[g] = has_res ? *reinterpret_cast<const half4*>(rrow + g * 16) : half4{};
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            half4 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float v = acc[j][g * 4 + e] + bias[g * 4 + e] + (float)r4[g][e];
                h[e] = (half_t)(relu ? fmaxf(v, 0.0f) : v);
            }
            *reinterpret_cast<half4*>(srow + (swz<32>(lrow, g) * 16)) = h;
        }
#pragma unroll
        for (int hp = 0; hp < 2; ++hp) {
            const int pix = hp * 16 + (lane >> 2), ch = lane & 3;
            const half8 v8 = *reinterpret_cast<const half8*>(sstg + pix * 64 + swz<32>(pix, ch) * 16);
            const int p = p0 + pix, r = p / W, c = p - r * W;
            if (p < npx && r0 + r < H)
                *reinterpret_cast<half8*>(y + ((size_t)(b * H + r0 + r) * W + c) * a.ys + ocw + ch * 8) = v8;
        }
    }
}

template <int TH, int NBW>
void launch_band(const ConvArgs& a, hipStream_t s) {
    const int B = a.npix / (a.Ho * a.Wo);
    hipLaunchKernelGGL((conv3x3_band_kernel<TH, NBW>), dim3(B * cdiv(a.H, TH), a.OC / 128), dim3(512), 0, s, a);
}

// ---------------------------------------------------------------------------
// conv3x3_bandws_kernel: stride-1 3x3 conv (pad 1) for maps up to MAXW wide
// and OC % 128 == 0, one workgroup per band of TH full rows x 128 output
// channels (flattened 32-pixel MFMA blocks), with the waves split by role:
//  * NCW compute waves in a WMG x WNG grid, each holding 4/WMG 32-channel A
//    blocks x NJ 32-pixel B blocks of accumulators; they only read LDS and
//    run MFMAs, never a global load, so no MFMA stream stalls behind the
//    memory queue;
//  * NP producer waves that move all data: per 16-channel chunk the 9 taps'
//    weights of the 128 channels and the band's input halo, DMA'd
//    (buffer_load ... lds) two chunks ahead into a 3-stage ring, and the
//    residual tile, in two halves, into the two stages the last chunks free;
//  * one barrier per chunk, reached by producers once their own chunk-k loads
//    have landed and by compute waves once they have finished chunk k-1;
//  * halo rows of 32 bytes (16 channels) whose 16-byte halves swap on every
//    other group of 8 rows, so the 16 lanes of a B read cover all 64 banks;
//  * weights read from the chunk-major copy ([IC/16][9][OC][16],
//    vdk_conv_desc.w_chunked) when there is one, so a DMA instruction's 64
//    slots are one contiguous kilobyte instead of pieces of 32 cache lines;
//  * accumulators that start at the bias; the residual added by two MFMAs per
//    32x32 block with identity A operands (products r x 1, one rounding of
//    acc + r), then [ReLU], f16, written over the residual rows, and stored
//    as 16-byte channel chunks.
// Products are f16 x f16 with f32 accumulation in tap-major, channel-minor
// order, like the other conv kernels, with the bias entering first.
// ---------------------------------------------------------------------------
template <int TH, int MAXW, int WMG, int WNG, int NJ, int NP>
struct BandWsTile {
    static constexpr int OCB = 128, NCW = WMG * WNG, MI = 4 / WMG, NW = NCW + NP;
    static constexpr int NB = WNG * NJ;                               // 32-pixel blocks per band
    static constexpr int A_BYTES = 9 * OCB * 32, A_INS = A_BYTES / 1024;
    static constexpr int HWM = MAXW + 2, XPIX = (TH + 2) * HWM;      // halo pixels (widest map)
    static constexpr int X_INS = (XPIX * 2 + 63) / 64;                // 32-byte rows = two 16-byte slots
    static constexpr int STAGE = A_BYTES + X_INS * 1024;
    static constexpr int RRB = 272, SPR = RRB / 16;                   // residual rows: 128 channels + 16 B
    static constexpr int HALF_ROWS = NB * 16;                         // residual rows per free stage
    static constexpr int R_INS = (HALF_ROWS * SPR + 63) / 64;         // DMA instructions per half
    static constexpr int XPP = (X_INS + NP - 1) / NP, RPP = (R_INS + NP - 1) / NP;
    static constexpr int CPR = MI * 4;                                // 16-byte output chunks per row and wave
    static_assert(WMG * MI == 4, "the channel groups cover the 128 channels");
    static_assert(3 * STAGE <= 163840, "three stages fit the 160 KB of LDS");
    static_assert(R_INS * 1024 <= STAGE, "half the residual tile fits one stage");
    static_assert(NB * 32 >= TH * MAXW, "the band's pixel blocks cover TH rows");
    static_assert(A_INS % NP == 0, "the weight instructions split evenly over the producers");
};

// Global byte offset of weight slot p (row p/2 = (tap, oc), 16-byte half
// p & 1, swapped on odd groups of 8 rows) of 16-channel chunk c0, from the
// chunk-major copy or the plain [OC][3][3][IC] layout.
__device__ __forceinline__ uint32_t band_woff(int p, int c0, int oc0, int IC, int OC, bool chunked) {
    const int row = p >> 1, tap = row >> 7, oc = row & 127;
    const int half = (p & 1) ^ ((row >> 3) & 1);
    return chunked ? (uint32_t)((((c0 >> 4) * 9 + tap) * OC + oc0 + oc) * 32 + half * 16)
                   : (uint32_t)((((oc0 + oc) * 9 + tap) * IC + c0) * 2 + half * 16);
}

// n / d for 0 <= n < 2^20 and d >= 1, given inv_d = 1 / d: (n + 1/2) / d lies
// at least 1/(2d) away from an integer, far beyond the float rounding error.
__device__ __forceinline__ int div_small(int n, float inv_d) {
    return (int)(((float)n + 0.5f) * inv_d);
}

template <int TH, int MAXW, int WMG, int WNG, int NJ, int NP>
__global__ __launch_bounds__((WMG * WNG + NP) * 64) void conv3x3_bandws_kernel(ConvArgs a) {
    using G = BandWsTile<TH, MAXW, WMG, WNG, NJ, NP>;
    constexpr int MI = G::MI;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[3 * G::STAGE];
    uint8_t* const st0 = smem;
    uint8_t* const st1 = smem + G::STAGE;
    uint8_t* const st2 = smem + 2 * G::STAGE;
    auto stage = [&](int k) { const int m = k % 3; return m == 0 ? st0 : (m == 1 ? st1 : st2); };

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int H = a.H, W = a.W, IC = a.IC, HW = W + 2;
    const int bands = (H + TH - 1) / TH;
    const int b = blockIdx.x / bands, r0 = (blockIdx.x - b * bands) * TH;
    const int oc0 = blockIdx.y * G::OCB;
    const int npx = TH * W;                           // band pixels (rows past H are computed and dropped)
    const bool has_res = a.res != nullptr;
    const float inv_w = 1.0f / (float)W;
    const int nk = IC / 16;
    uint8_t* const rs0 = stage(nk);                   // residual rows [0, HALF_ROWS): free from chunk nk-2 on
    uint8_t* const rs1 = stage(nk + 1);               // the other half: free from chunk nk-1 on
    auto rrow = [&](int pr) { return pr < G::HALF_ROWS ? rs0 + pr * G::RRB : rs1 + (pr - G::HALF_ROWS) * G::RRB; };

    if (wave >= G::NCW) {
        // ---------------- producers ----------------
        const int p = wave - G::NCW;
        const bool chunked = a.wc != nullptr;
        const float inv_hw = 1.0f / (float)HW;
        int xoff[G::XPP];   // this lane's halo slots as byte offsets at channel 0
#pragma unroll
        for (int i = 0; i < G::XPP; ++i) {
            const int xi = p + NP * i;
            xoff[i] = -1;
            if (xi < G::X_INS) {
                const int s = xi * 64 + lane;
                const int q = s >> 1, hr = div_small(q, inv_hw), hc = q - hr * HW;
                const int ghalf = (s & 1) ^ ((q >> 3) & 1);
                const int ih = r0 - 1 + hr, iw = hc - 1;
                if (hr < TH + 2 && ih >= 0 && ih < H && iw >= 0 && iw < W)
                    xoff[i] = (int)(((size_t)(b * H + ih) * W + iw) * a.xs * 2) + ghalf * 16;
            }
        }
        const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(chunked ? a.wc : a.w), 0, (int)((size_t)a.OC * 9 * IC * 2), 0x00020000);
        const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)a.x, 0, (int)(((size_t)(a.npix_in - 1) * a.xs + IC) * 2), 0x00020000);
        auto issue = [&](uint8_t* __restrict__ nx, int c0) {
#pragma unroll
            for (int i = 0; i < G::A_INS / NP; ++i) {
                const int ins = p + NP * i;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    wr, (lds_void*)(nx + ins * 1024), 16, band_woff(ins * 64 + lane, c0, oc0, IC, a.OC, chunked), 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < G::XPP; ++i) {
                const int xi = p + NP * i;
                if (xi < G::X_INS) {
                    const uint32_t off = xoff[i] < 0 ? kOOB : (uint32_t)(xoff[i] + c0 * 2);
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(nx + (G::A_INS + xi) * 1024), 16, off, 0, 0,
                                                             0);
                }
            }
        };
        auto issue_res = [&](uint8_t* __restrict__ dst, int half) {
            const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
                (void*)a.res, 0, (int)(((size_t)(a.npix - 1) * a.rs + a.OC) * 2), 0x00020000);
#pragma unroll
            for (int i = 0; i < G::RPP; ++i) {
                const int ri = p + NP * i;
                if (ri < G::R_INS) {
                    const int sl = ri * 64 + lane;
                    const int pr = half * G::HALF_ROWS + sl / G::SPR, ch = sl % G::SPR;
                    const int r = div_small(pr, inv_w), c = pr - r * W;
                    const bool ok = ch < 16 && pr < npx && r0 + r < H;
                    const uint32_t off =
                        ok ? (uint32_t)(((((size_t)(b * H + r0 + r) * W + c) * a.rs + oc0) * 2) + ch * 16) : kOOB;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_void*)(dst + ri * 1024), 16, off, 0, 0, 0);
                }
            }
        };
        const int nper = G::A_INS / NP + (p + NP * (G::XPP - 1) < G::X_INS ? G::XPP : G::XPP - 1);   // per chunk
        // chunk 0 alone goes out first, so the compute waves start as soon as
        // it has landed; chunks 1 and 2 follow together after the first
        // barrier, then the ring keeps two chunks ahead
        issue(st0, 0);
#pragma unroll 1
        for (int k = 0; k < nk; ++k) {
            wait_vmcnt_le(k >= 1 && k + 1 < nk ? nper : 0);   // chunk k has landed (chunk k+1 may be in flight)
            lds_barrier();                            // ... and chunk k-1's stage is free
            if (k == 0 && nk > 1) issue(st1, 16);
            if (k + 2 < nk) issue(stage(k + 2), (k + 2) * 16);
            if (has_res && (k == nk - 2 || (nk == 1 && k == 0))) issue_res(rs0, 0);
            if (has_res && k == nk - 1) issue_res(rs1, 1);
        }
        if (has_res) {
            __builtin_amdgcn_s_waitcnt(0);
            lds_barrier();                            // the residual tile has landed
        }
        return;
    }

    // ---------------- compute waves ----------------
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int og = wave % WMG, pg = wave / WMG;       // channel group, pixel group
    const int cg0 = og * MI * 32;                     // the group's first channel within the 128
    // A row (tap, cg0 + i*32 + lrow) with its halves swapped on odd groups of 8
    // rows; B halo row q = qb[j] + (kh * HW + kw) of pixel p = block*32 + lrow
    const int abase = (cg0 + lrow) * 32 + ((lhalf ^ ((lrow >> 3) & 1)) * 16);
    int qb[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        int pp = (pg * NJ + j) * 32 + lrow;
        if (pp >= npx) pp = 0;   // masked lane: any valid row, result dropped
        const int r = div_small(pp, inv_w), c = pp - r * W;
        qb[j] = r * HW + c;
    }
    // the accumulators start at the bias (register g*4+e of a lane: channel
    // 8g + 4*lhalf + e of its 32-row block)
    float16v acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        float16v bv;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4v v = a.bias ? *reinterpret_cast<const float4v*>(a.bias + oc0 + cg0 + i * 32 + g * 8 + lhalf * 4)
                                     : float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int e = 0; e < 4; ++e) bv[g * 4 + e] = v[e];
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = bv;
    }

#pragma unroll 1
    for (int k = 0; k < nk; ++k) {
        lds_barrier();                                // chunk k has landed; chunk k-1's reads are done
        const uint8_t* const cur = stage(k);
        const uint8_t* const xs = cur + G::A_BYTES;
        // the halo bases go behind an empty asm per chunk: otherwise the 9 x NJ
        // (base + tap offset) addresses are hoisted out of the loop and spill
#pragma unroll
        for (int j = 0; j < NJ; ++j) asm volatile("" : "+v"(qb[j]));
        half8 af[2][MI], bf[2][NJ];
        auto load = [&](int tap, int buf) {
            const int toff = (tap / 3) * HW + tap % 3;
#pragma unroll
            for (int i = 0; i < MI; ++i)
                af[buf][i] = *reinterpret_cast<const half8*>(cur + abase + tap * (G::OCB * 32) + i * 1024);
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int q = qb[j] + toff;
                bf[buf][j] = *reinterpret_cast<const half8*>(xs + q * 32 + ((((q >> 3) ^ lhalf) & 1) << 4));
            }
        };
        load(0, 0);
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            const int c = tap & 1;
            if (tap + 1 < 9) load(tap + 1, c ^ 1);
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[c][i], bf[c][j], acc[i][j], 0, 0, 0);
            if (tap + 1 < 9) {
                // one MFMA, then one fragment read with its address VALU, in turn
#pragma unroll
                for (int q = 0; q < MI + NJ; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // VALU
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
                }
                __builtin_amdgcn_sched_group_barrier(0x008, MI * NJ - (MI + NJ), 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (has_res) lds_barrier();                       // the producers' residual tile has landed

    // Epilogue: the residual through identity-operand MFMAs, [ReLU], f16 over
    // the residual rows, then the wave's channel range of its pixel rows out
    // as 16-byte chunks.
    const bool relu = a.act == VDK_ACT_RELU;
    half8 eye[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) eye[h][e] = (half_t)((lrow == h * 16 + lhalf * 8 + e) ? 1.0f : 0.0f);
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        const int cw = cg0 + i * 32;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            uint8_t* const prow = rrow((pg * NJ + j) * 32 + lrow);
            if (has_res) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const half8 rv = *reinterpret_cast<const half8*>(prow + (cw + h * 16 + lhalf * 8) * 2);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(eye[h], rv, acc[i][j], 0, 0, 0);
                }
            }
            uint8_t* const row = prow + (cw + lhalf * 4) * 2;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                half4 hv;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v = acc[i][j][g * 4 + e];
                    hv[e] = (half_t)(relu ? fmaxf(v, 0.0f) : v);
                }
                *reinterpret_cast<half4*>(row + g * 16) = hv;
            }
        }
    }
    half_t* const y = static_cast<half_t*>(a.y) + oc0 + cg0;
    constexpr int NST = NJ * 32 * G::CPR / 64;        // 16-byte stores per wave
    const int ch = lane % G::CPR;
#pragma unroll
    for (int it = 0; it < NST; ++it) {
        const int pr = pg * NJ * 32 + (it * 64 + lane) / G::CPR;
        const half8 v8 = *reinterpret_cast<const half8*>(rrow(pr) + cg0 * 2 + ch * 16);
        const int r = div_small(pr, inv_w), c = pr - r * W;
        if (pr < npx && r0 + r < H)
            *reinterpret_cast<half8*>(y + ((size_t)(b * H + r0 + r) * W + c) * a.ys + ch * 8) = v8;
    }
}

template <int TH, int MAXW, int WMG, int WNG, int NJ, int NP>
void launch_bandws(const ConvArgs& a, hipStream_t s) {
    const int B = a.npix / (a.Ho * a.Wo);
    hipLaunchKernelGGL((conv3x3_bandws_kernel<TH, MAXW, WMG, WNG, NJ, NP>), dim3(B * cdiv(a.H, TH), a.OC / 128),
                       dim3((WMG * WNG + NP) * 64), 0, s, a);
}


template <int BM, int BN, int WM, int WN, int KC>
void launch_igemm(const ConvArgs& a, hipStream_t s) {
    constexpr int NT = (BM / WM) * (BN / WN) * 64;
    dim3 grid(cdiv(a.npix, BN), cdiv(a.OC, BM));
    if (a.segsum && a.in_scale)   // segment sums: the f16-weight variants only
        hipLaunchKernelGGL((conv_igemm_kernel<BM, BN, WM, WN, KC, true, false, true>), grid, dim3(NT), 0, s, a);
    else if (a.segsum)
        hipLaunchKernelGGL((conv_igemm_kernel<BM, BN, WM, WN, KC, false, false, true>), grid, dim3(NT), 0, s, a);
    else if (a.in_scale && a.wq)
        hipLaunchKernelGGL((conv_igemm_kernel<BM, BN, WM, WN, KC, true, true>), grid, dim3(NT), 0, s, a);
    else if (a.in_scale)
        hipLaunchKernelGGL((conv_igemm_kernel<BM, BN, WM, WN, KC, true>), grid, dim3(NT), 0, s, a);
    else if (a.wq)
        hipLaunchKernelGGL((conv_igemm_kernel<BM, BN, WM, WN, KC, false, true>), grid, dim3(NT), 0, s, a);
    else
        hipLaunchKernelGGL((conv_igemm_kernel<BM, BN, WM, WN, KC, false>), grid, dim3(NT), 0, s, a);
}

struct TileCfg {
    int bm, bn, kc;
    void (*launch)(const ConvArgs&, hipStream_t);
    bool halo;       // 3x3 stride-1 pad-1 dilation-1 only
    int rw_ic = 0;   // register-weight kernels: exactly IC = rw_ic and OC = bm, plain epilogue
    int band_w = 0;  // band kernels: W <= band_w, OC % 128 == 0, IC % 16 == 0
    int sp_ic = 0;   // split-f16 register-weight kernels: exactly IC = sp_ic and OC = bm, split 2
    bool gemm = false;   // the GEMM kernel with producer / compute waves: no reflect / q8_0
    bool gemm_ext = false;   // ... and its prologue / segment-sum variants (1x1, no padding)
};

// Entries 0-13 are the register-staged kernel (any layout; the only one with
// KC=16 for IC % 32 != 0), 14-25 the LDS-DMA kernel, 26-32 the halo kernel,
// 33-52 LDS-DMA tiles with 8 waves per workgroup, 53-56 the register-weight
// persistent 3x3 kernel, 57-59 the band kernel for wide 3x3 layers, 60-61
// narrow LDS-DMA tiles, 62-63 narrow register-staged tiles, 64-65 the band
// kernel with producer / compute waves (128-channel groups, maps up to 75 /
// 38 wide), 66-69 the register-weight kernel with 3- and 4-stage rings,
// 70-75 the split-f16 register-weight kernel (ERes2Net's group convs), 76-79
// the producer / compute band kernel on one-row bands (the same sums in the
// same order as its 5-row bands, so the same bits, on 5x the workgroups), 80
// the register-staged 64x64 tile with 64-channel chunks, 81-84 the 1x1 GEMM
// kernel with producer / compute waves, 85-88 narrow tiles of that kernel
// with the prologue / segment-sum variants.

// Tile table.  Wave tiles are WM x WN = (bm / waves_m) x (bn / waves_n) with
// 4 waves per workgroup; entries are selected per layer by pick_tile().
const TileCfg kTiles[] = {
    {32, 256, 32, launch_igemm<32, 256, 32, 64, 32>},     // 0: OC=32 layers
    {64, 256, 32, launch_igemm<64, 256, 64, 64, 32>},     // 1
    {64, 128, 32, launch_igemm<64, 128, 32, 64, 32>},     // 2
    {128, 128, 32, launch_igemm<128, 128, 64, 64, 32>},   // 3
    {128, 128, 64, launch_igemm<128, 128, 64, 64, 64>},   // 4
    {128, 64, 32, launch_igemm<128, 64, 64, 32, 32>},     // 5
    {128, 64, 64, launch_igemm<128, 64, 64, 32, 64>},     // 6
    {128, 256, 32, launch_igemm<128, 256, 64, 128, 32>},  // 7
    {256, 128, 32, launch_igemm<256, 128, 128, 64, 32>},  // 8
    {64, 256, 32, launch_igemm<64, 256, 32, 128, 32>},    // 9
    {32, 128, 32, launch_igemm<32, 128, 32, 32, 32>},     // 10
    {32, 256, 16, launch_igemm<32, 256, 32, 64, 16>},     // 11: IC % 32 != 0
    {64, 128, 16, launch_igemm<64, 128, 32, 64, 16>},     // 12
    {128, 64, 16, launch_igemm<128, 64, 64, 32, 16>},     // 13
    {32, 256, 32, launch_dma<32, 256, 32, 64, 32, 2>},    // 14: DMA ring variants
    {64, 128, 64, launch_dma<64, 128, 32, 64, 64, 2>},    // 15
    {64, 256, 32, launch_dma<64, 256, 64, 64, 32, 2>},    // 16
    {128, 128, 64, launch_dma<128, 128, 64, 64, 64, 2>},  // 17
    {128, 64, 64, launch_dma<128, 64, 64, 32, 64, 2>},    // 18
    {128, 64, 64, launch_dma<128, 64, 64, 32, 64, 3>},    // 19
    {256, 128, 64, launch_dma<256, 128, 128, 64, 64, 2>}, // 20
    {64, 256, 64, launch_dma<64, 256, 64, 64, 64, 2>},    // 21
    {32, 256, 32, launch_dma<32, 256, 32, 64, 32, 3>},    // 22
    {64, 128, 64, launch_dma<64, 128, 32, 64, 64, 3>},    // 23
    {64, 256, 32, launch_dma<64, 256, 64, 64, 32, 3>},    // 24
    {128, 256, 64, launch_dma<128, 256, 64, 128, 64, 2>}, // 25
    {32, 256, 32, launch_halo<32, 32, 4, 64>, true},      // 26: halo tiles
    {32, 256, 32, launch_halo<32, 32, 8, 32>, true},      // 27
    {32, 128, 32, launch_halo<32, 32, 4, 32>, true},      // 28
    {32, 128, 64, launch_halo<32, 64, 4, 32>, true},      // 29
    {64, 128, 32, launch_halo<64, 32, 4, 32>, true},      // 30
    {64, 128, 64, launch_halo<64, 64, 2, 64>, true},      // 31
    {32, 256, 64, launch_halo<32, 64, 4, 64>, true},      // 32
    {128, 256, 64, launch_dma<128, 256, 64, 64, 64, 2>},  // 33: 8-wave DMA tiles
    {256, 128, 64, launch_dma<256, 128, 64, 64, 64, 2>},  // 34
    {128, 128, 64, launch_dma<128, 128, 64, 64, 64, 3>},  // 35
    {128, 256, 32, launch_dma<128, 256, 64, 64, 32, 2>},  // 36
    {128, 256, 64, launch_dma<128, 256, 64, 64, 64, 3>},  // 37
    {256, 256, 64, launch_dma<256, 256, 128, 64, 64, 2>}, // 38
    {128, 128, 32, launch_dma<128, 128, 64, 64, 32, 2>},  // 39
    {128, 128, 64, launch_dma<128, 128, 64, 32, 64, 2>},  // 40: 8 waves, 64x32 wave tiles
    {128, 256, 32, launch_dma<128, 256, 64, 64, 32, 4>},  // 41: deeper rings
    {128, 256, 32, launch_dma<128, 256, 64, 64, 32, 6>},  // 42
    {256, 128, 32, launch_dma<256, 128, 64, 64, 32, 4>},  // 43
    {256, 128, 32, launch_dma<256, 128, 64, 64, 32, 6>},  // 44
    {128, 128, 32, launch_dma<128, 128, 64, 32, 32, 4>},  // 45
    {128, 128, 32, launch_dma<128, 128, 64, 32, 32, 6>},  // 46
    {128, 64, 32, launch_dma<128, 64, 64, 32, 32, 2>},    // 47: small-footprint tiles
    {128, 64, 32, launch_dma<128, 64, 64, 32, 32, 3>},    // 48
    {128, 64, 32, launch_dma<128, 64, 64, 32, 32, 4>},    // 49
    {256, 64, 32, launch_dma<256, 64, 64, 64, 32, 2>},    // 50
    {256, 64, 64, launch_dma<256, 64, 64, 64, 64, 2>},    // 51
    {128, 32, 64, launch_dma<128, 32, 32, 32, 64, 2>},    // 52
    {64, 128, 64, launch_rw<64, 64, 4, 8, 2>, true, 64},  // 53: register-weight persistent 3x3
    {64, 192, 64, launch_rw<64, 64, 6, 8, 2>, true, 64},  // 54
    {64, 64, 64, launch_rw<64, 64, 2, 8, 2>, true, 64},   // 55
    {32, 128, 32, launch_rw<32, 32, 4, 8, 2>, true, 32},  // 56
    {128, 384, 16, launch_band<5, 6>, true, 0, BandTile<5, 6>::MAXW},   // 57: band kernels
    {128, 192, 16, launch_band<5, 3>, true, 0, BandTile<5, 3>::MAXW},   // 58
    {128, 320, 16, launch_band<4, 5>, true, 0, BandTile<4, 5>::MAXW},   // 59
    {32, 64, 32, launch_dma<32, 64, 32, 32, 32, 2>},      // 60: narrow DMA tiles (OC = 32, few pixels)
    {32, 128, 32, launch_dma<32, 128, 32, 32, 32, 2>},    // 61
    {128, 32, 32, launch_igemm<128, 32, 64, 32, 32>},     // 62: register-staged, more workgroups
    {64, 64, 32, launch_igemm<64, 64, 32, 32, 32>},       // 63
    {128, 384, 16, launch_bandws<5, 75, 2, 4, 3, 4>, true, 0, 75},   // 64: producer / compute band kernels
    {128, 192, 16, launch_bandws<5, 38, 2, 2, 3, 4>, true, 0, 38},   // 65
    {64, 128, 64, launch_rw<64, 64, 4, 8, 3>, true, 64},  // 66: register-weight kernel, deeper rings
    {64, 64, 64, launch_rw<64, 64, 2, 8, 4>, true, 64},   // 67
    {32, 128, 32, launch_rw<32, 32, 4, 8, 4>, true, 32},  // 68
    {32, 256, 32, launch_rw<32, 32, 8, 8, 3>, true, 32},  // 69
    {16, 256, 32, launch_sp<32, 16, 8, 8, 3, true>, true, 0, 0, 32},    // 70: split-f16 register-weight 3x3
    {16, 256, 16, launch_sp<16, 16, 8, 8, 4, true>, true, 0, 0, 16},    // 71
    {32, 256, 32, launch_sp<32, 32, 8, 8, 3, false>, true, 0, 0, 32},   // 72
    {32, 64, 64, launch_sp<64, 32, 2, 4, 4, true>, true, 0, 0, 64},     // 73
    {32, 128, 64, launch_sp<64, 32, 4, 4, 2, false>, true, 0, 0, 64},   // 74
    {64, 128, 64, launch_sp<64, 64, 4, 8, 2, false>, true, 0, 0, 64},   // 75
    {128, 96, 16, launch_bandws<1, 75, 4, 1, 3, 4>, true, 0, 75},   // 76: one-row bands (small batches)
    {128, 96, 16, launch_bandws<1, 75, 4, 3, 1, 4>, true, 0, 75},   // 77
    {128, 64, 16, launch_bandws<1, 38, 4, 1, 2, 4>, true, 0, 38},   // 78
    {128, 64, 16, launch_bandws<1, 38, 4, 2, 1, 4>, true, 0, 38},   // 79
    {64, 64, 64, launch_igemm<64, 64, 32, 32, 64>},       // 80: register-staged, 64-channel chunks
    {128, 256, 64, launch_gemm_ws<128, 256, 2, 4, 64, 3, 4>, false, 0, 0, 0, true},   // 81: 1x1 GEMMs, producer / compute waves
    {128, 384, 32, launch_gemm_ws<128, 384, 2, 4, 32, 4, 4>, false, 0, 0, 0, true},   // 82
    {256, 128, 64, launch_gemm_ws<256, 128, 4, 2, 64, 3, 4>, false, 0, 0, 0, true},   // 83
    {128, 288, 64, launch_gemm_ws<128, 288, 2, 3, 64, 3, 4>, false, 0, 0, 0, true},   // 84
    {128, 64, 32, launch_gemm_ws<128, 64, 2, 2, 32, 4, 2, true>, false, 0, 0, 0, true, true},   // 85: narrow GEMMs
    {128, 64, 64, launch_gemm_ws<128, 64, 2, 2, 64, 3, 2, true>, false, 0, 0, 0, true, true},   // 86
    {128, 32, 32, launch_gemm_ws<128, 32, 4, 1, 32, 4, 2, true>, false, 0, 0, 0, true, true},   // 87
    {64, 64, 32, launch_gemm_ws<64, 64, 2, 2, 32, 4, 2, true>, false, 0, 0, 0, true, true},     // 88
    {128, 256, 64, launch_gemm_ws<128, 256, 2, 4, 64, 3, 4, true>, false, 0, 0, 0, true, true},   // 89: wide, + prologue
    {256, 128, 64, launch_gemm_ws<256, 128, 4, 2, 64, 3, 4, true>, false, 0, 0, 0, true, true},   // 90
    {128, 384, 32, launch_gemm_ws<128, 384, 2, 4, 32, 4, 4, true>, false, 0, 0, 0, true, true},   // 91
};
constexpr int kNumTiles = (int)(sizeof(kTiles) / sizeof(kTiles[0]));

bool is_s1_3x3(const ConvArgs& a) {
    return a.KH == 3 && a.KW == 3 && a.sh == 1 && a.sw == 1 && a.ph == 1 && a.pw == 1 && a.dh == 1 && a.dw == 1;
}

constexpr int kFirstDma = 14;   // then the halo tiles from 26, 8-wave DMA tiles from 33

// The register-weight kernels take the plain epilogue only: bias, residual,
// ReLU or none, dense f16 NHWC in and out.
bool plain_epilogue(const ConvArgs& a) {
    return !a.gate && !a.post_scale && !a.tanh_after && !a.ax && !a.y_f32 && !a.y_tr && !a.bias_bs && !a.split &&
           (a.act == VDK_ACT_NONE || (a.act == VDK_ACT_RELU && a.clamp_hi <= 0.0f)) && a.xs == a.IC &&
           a.ys == a.OC && (!a.res || a.rs == a.OC) && !a.res_f32 && !a.res_after && !a.y2 && !a.reflect;
}

// The split-f16 register-weight kernels: f16-exact weights (split 2), bias
// and ReLU [clamp] or none, no residual; 16-byte aligned input rows and
// planes, 8-byte aligned output ones, byte offsets within 31 bits.
bool split_epilogue(const ConvArgs& a) {
    const auto al = [](const void* p, int n) { return ((uintptr_t)p & (uintptr_t)(n - 1)) == 0; };
    return a.split == 2 && !a.gate && !a.post_scale && !a.tanh_after && !a.ax && !a.y_f32 && !a.y_tr && !a.bias_bs &&
           (a.act == VDK_ACT_NONE || a.act == VDK_ACT_RELU) && !a.res && !a.y2 && !a.reflect && !a.in_scale &&
           !a.segsum && !a.wq && a.xs % 8 == 0 && a.x_lo % 8 == 0 && a.ys % 4 == 0 && a.y_lo % 4 == 0 &&
           al(a.x, 16) && al(a.y, 8) && al(a.w, 16) && al(a.wc, 16) && al(a.bias, 4) &&
           ((size_t)a.npix_in * a.xs + a.x_lo + ((a.IC >> a.xgl) - 1) * a.xgs + (1 << a.xgl)) * 2 < ((size_t)1 << 31);
}

// The register-staged (igemm) entries: 0-13 and 62-63.
bool igemm_tile(int idx) { return idx < kFirstDma || idx == 62 || idx == 63 || idx == 80; }

bool tile_fits(const TileCfg& t, const ConvArgs& a) {
    const int idx = (int)(&t - kTiles);
    if (t.halo && !is_s1_3x3(a)) return false;
    // the input prologue lives in the register-staged kernel's operand loads
    // and the LDS-DMA kernel's B fragments (up to 1024 input channels: their
    // scale / shift stage in LDS)
    if (a.in_scale && (t.halo || t.rw_ic || t.band_w || a.IC > 1024)) return false;
    // reflect padding lives in the LDS-DMA kernel's pixel offsets (one row
    // of at most 32 taps)
    if (a.reflect && (igemm_tile(idx) || t.halo || a.KH * a.KW > 32)) return false;
    // q8_0 weights are dequantised in the register-staged kernel's weight loads
    if (a.wq && !igemm_tile(idx)) return false;
    // segment sums live in the staged epilogue of the register-staged
    // kernel (f16 weights); pixel tiles at most seg_len wide keep most pixels
    // in the two segments the epilogue sums locally
    if (a.segsum && (!(igemm_tile(idx) || t.gemm_ext) || a.wq || t.bn > a.seg_len)) return false;
    // the LDS-DMA kernels keep one bit per tap in a 32-bit in-image mask, or
    // the in-image tap range for a single row of taps; longer 2-D kernels
    // take the register-staged kernel
    if (a.KH * a.KW > 32 && a.KH != 1 && !igemm_tile(idx)) return false;
    if (t.sp_ic) return a.IC == t.sp_ic && a.OC == t.bm && split_epilogue(a);
    // the GEMM kernel: split-f16 inputs for 1x1 convs only (the plane terms
    // are consecutive chunks of one tap), channel groups whole per chunk
    // (prologue / segment sums: the EXT tiles, 1x1 without padding, up to
    // 1024 input channels, pixel tiles at most seg_len wide)
    if (t.gemm) {
        const bool one = a.KH * a.KW == 1 && a.ph == 0 && a.pw == 0;
        if ((a.in_scale || a.segsum) && !(t.gemm_ext && one && !a.split)) return false;
        if (a.in_scale && a.IC > 1024) return false;
        if (a.segsum && t.bn > a.seg_len) return false;
        return (!a.split || a.KH * a.KW == 1) && !a.reflect && !a.wq && t.kc % (1 << a.xgl) == 0 &&
               a.IC % t.kc == 0 && a.xs % 8 == 0 && (!a.split || a.x_lo % 8 == 0);
    }
    // 16-channel group strides: the LDS-DMA kernel's offsets and the shared store
    if ((a.xgs != (1 << a.xgl) || a.ygs != (1 << a.ygl)) && (igemm_tile(idx) || t.halo || t.rw_ic || t.band_w))
        return false;
    // a DMA chunk covers whole groups
    if (a.xgl == 5 && t.kc % 32 != 0) return false;
    if (t.rw_ic) return a.IC == t.rw_ic && a.OC == t.bm && plain_epilogue(a);
    if (t.band_w) return plain_epilogue(a) && a.W <= t.band_w && a.OC % t.bm == 0 && a.IC % 16 == 0;
    // split: the DMA and halo kernels only (IC % kc == 0 below keeps a chunk inside one plane)
    if (a.split && (igemm_tile(idx) || idx >= 62)) return false;
    return a.IC % t.kc == 0;
}

// Optional override for tuning sweeps: VDK_CONV_TILE=<index into kTiles>.
int tile_override() {
    static const int v = [] {
        const char* e = std::getenv("VDK_CONV_TILE");
        return (e && *e) ? std::atoi(e) : -1;
    }();
    return v;
}

// Per-layer-class defaults, from a sweep of every ResNet34 conv shape at
// batch 64 on MI355X (64-channel 3x3 stride-1 layers with the plain
// epilogue: the register-weight kernel; 128-channel ones whose map is 39-76
// wide: the band kernel, 256+-channel ones on maps up to 38 wide: the
// 3-block band; the strided / 1x1 32 -> 64 convs: the register-staged 64x128
// tile; other narrow 3x3 stride-1 layers: the 32-channel halo tile;
// 128 output channels: the 128x128 DMA tile with KC = 32; the rest: DMA
// implicit GEMM with the widest OC tile that divides OC; IC % 32 != 0: the
// register-staged kernel with KC = 16).  OC that no tile divides runs on
// 32-wide tiles with the surplus rows masked.
int pick_tile(const ConvArgs& a) {
    const int o = tile_override();
    if (o >= 0 && o < kNumTiles && tile_fits(kTiles[o], a)) return o;
    const int bm = a.OC % 128 == 0 ? 128 : (a.OC % 64 == 0 ? 64 : 32);
    if (a.in_scale) {   // register-staged tiles for a few ten thousand pixels (CAM++'s
        // linear1: the LDS-DMA tiles, faster in isolation, measured slower in the model):
        // 64-channel chunks from 256 input channels (half the chunk steps, each a
        // load round trip) on the 64x64 tile (B=32 x 499 frames: 12.8 / 16.6 /
        // 19.9 -> 12.0 / 15.8 / 19.5 us at 256 / 512 / 768 channels against the
        // 128x64 one), else the 64x64 tile with 32-channel chunks
        // the GEMM kernel's narrow tiles from 800 channels (B=32 x 499 frames,
        // interleaved: 800 22.5 -> 21.2 us, 1024 23.5 -> 22.1 us)
        // CAM++'s 1024 -> 512 transits (B=32 x 499 frames): the GEMM kernel's
        // 256x128 prologue tile, 55.5 -> 31.8 us (512 -> 256: no gain)
        if (a.KH * a.KW == 1 && a.IC >= 1024 && a.OC >= 512 && a.OC % 256 == 0 && !a.segsum &&
            tile_fits(kTiles[90], a))
            return 90;
        // the 512 -> 256 transit on the 128x64 LDS-DMA tile (in-model: 21.3 -> 16.8 us)
        if (a.KH * a.KW == 1 && a.IC == 512 && a.OC == 256 && !a.segsum && tile_fits(kTiles[18], a)) return 18;
        if (a.IC >= 800 && a.OC == 128 && a.npix < 65536) {
            if (a.IC % 64 == 0 && tile_fits(kTiles[86], a)) return 86;
            if (tile_fits(kTiles[85], a)) return 85;
        }
        if (a.IC >= 256 && a.IC % 64 == 0 && a.OC == 128 && a.npix < 65536 && tile_fits(kTiles[80], a)) return 80;
        if (a.IC % 32 == 0) return bm >= 64 ? (a.npix < 32768 ? 63 : (bm == 128 ? 5 : 2)) : 10;
        return bm == 128 ? 13 : (bm == 64 ? 12 : 11);
    }
    if (a.KH * a.KW > 32 && a.KH != 1) {   // register-staged kernel only
        if (a.IC % 32 == 0) return bm == 128 ? 5 : (bm == 64 ? 2 : 10);
        return a.IC % 16 == 0 ? (bm == 128 ? 13 : (bm == 64 ? 12 : 11)) : -1;
    }
    if (a.KH == 1 && !a.split) {
        // 1-D convs over time-major maps (wav2vec2, ECAPA), from a sweep of
        // the wav2vec2 / ECAPA layer shapes at batch 64 on MI355X: long
        // kernels (a 128-tap positional conv) on the 128x32 tile, wide 1x1
        // GEMMs on the 128x256 8-wave tile (768 outputs: the 256x128 one),
        // the big strided feature convs on the 256x256 tile
        // (re-checked with random data: zeros draw less MFMA power and run
        // at higher clocks, which had favoured some tiles)
        if (a.KW > 32 && a.IC % 64 == 0) return 52;
        // 1x1 GEMMs on the producer / compute wave kernel, from a sweep of the
        // ECAPA (64 x 398 frames) and wav2vec2 (64 x 149 frames) layer shapes
        // with random data: MFA 3072 -> 1536 313 -> 238 us, asp.tdnn 4608 ->
        // 128 64 -> 49 us, the TDNNs 1024 -> 1024 84 -> 78 us, wav2vec2 ff2
        // 62 -> 49 us (base) / 115 -> 90 us (large), out-projections 23.5 ->
        // 20.3 / 39.8 -> 31.7 us (the 768- / 1024-input ff1 and qkv GEMMs
        // measured no faster and stay on the LDS-DMA tile).  The
        // 128 x 384 tile where it covers a 9536-pixel map in one round of
        // workgroups, 128 x 288 for the 25472-pixel TDNNs (712 workgroups:
        // 2.8 rounds where 128 x 256 makes 3.1), 256 x 128 for 768 outputs
        // and from 2048 input channels (the MFA's 3072 -> 1536: 272 -> 253
        // us against 128 x 256 once the producers' loads went out
        // branch-free), 128 x 256 for narrower outputs from 2048 channels
        if (a.KW == 1 && tile_fits(kTiles[81], a)) {
            if (a.OC == 768 && a.IC >= 768) return 83;
            // (in-model sweep, every fitting tile timed in place: wav2vec2-base's
            // qkv 768 -> 2304 on the 8-wave LDS-DMA tile, 60.9 -> 55.8 us; ECAPA's
            // 1024 -> 1024 TDNNs the same, 88.5 -> 84.6 us)
            if (a.npix < 16384 && a.OC == 2304 && a.IC == 768 && tile_fits(kTiles[40], a)) return 40;
            if (a.npix < 16384 && (a.OC == 1024 || a.OC == 2304) && tile_fits(kTiles[82], a)) return 82;
            if (a.npix >= 16384 && a.OC == 1024 && a.IC == 1024 && tile_fits(kTiles[40], a)) return 40;
            if (a.IC >= 2048) return a.OC % 256 == 0 ? 83 : 81;
        }
        // the same kernel for wav2vec2's strided feature convs (512 -> 512,
        // 3 / 2 taps, stride 2, exact GELU; 64 x 3 s clips, interleaved
        // timing): from 64k output pixels and under 16k the 256 x 128 tile
        // (conv1 .. conv3: 617 -> 583, 322 -> 306, 157 -> 148 us against
        // 128 x 256; conv6: 21.2 us), 2-tap ones of 16k-32k pixels the
        // 128 x 384 tile (conv5: 34.6 us)
        if (a.sw == 2 && a.KW <= 3 && a.IC == 512 && a.OC == 512 && tile_fits(kTiles[83], a)) {
            if (a.npix >= 65536 || a.npix < 16384) return 83;
            if (a.KW == 2 && a.npix >= 16384 && a.npix < 32768 && tile_fits(kTiles[82], a)) return 82;
        }
        // ECAPA's block0 (k = 5 over the 96 padded mel channels, 1024 out) on
        // the 128x256 8-wave tile (52.9 against 69.2 us at batch 64 x 4 s),
        // and asp.tdnn's 1536 -> 128 GEMM on the 128x64 tile (398 workgroups
        // instead of 199: 25.0 against 38.7 us)
        if (a.KW == 5 && a.IC % 32 == 0 && a.OC >= 512 && a.OC % 128 == 0 && tile_fits(kTiles[36], a)) return 36;
        // CAM++'s TDNN (k = 5, stride 2, 320 -> 128) on the 128x32 tile (in-model: 30.2 -> 19.2 us)
        if (a.KW == 5 && a.sw == 2 && a.OC == 128 && a.IC % 64 == 0 && tile_fits(kTiles[52], a)) return 52;
        if (a.KW == 1 && a.IC >= 1024 && a.OC == 128 && a.IC % 64 == 0 && tile_fits(kTiles[18], a)) return 18;
        if (a.KW == 1 && a.IC == 768 && a.OC == 768 && tile_fits(kTiles[40], a)) return 40;
        if (a.KW == 1 && a.IC >= 512 && a.OC == 768 && a.IC % 64 == 0) return 34;
        if (a.KW == 1 && a.IC >= 2048 && a.OC >= 1536 && a.OC % 256 == 0 && a.IC % 64 == 0) return 38;
        if (a.KW == 1 && a.IC >= 512 && a.OC >= 512 && a.OC % 128 == 0 && a.IC % 32 == 0) return 36;
        if (a.KW <= 4 && a.OC % 256 == 0 && a.IC % 64 == 0 && a.npix >= 131072) return 38;
        if (a.KW <= 4 && a.OC % 256 == 0 && a.IC % 64 == 0 && a.npix >= 32768 && tile_fits(kTiles[40], a))
            return 40;
        // ECAPA's Res2Net group convs (B=64 x 398 frames, reflect padding and
        // the second output): the 128x32 tile, 796 workgroups (13.0 against
        // 15.1 us for the 128x128 one at dilation 2, 12.9 / 13.9 at 4)
        if (a.KW == 3 && a.IC == 128 && a.OC == 128 && tile_fits(kTiles[52], a)) return 52;
        if (a.KW == 3 && a.OC == 32 && a.IC % 32 == 0) return 60;     // CAM++'s gated linear_local
    }
    // CAM++'s FCM: 32 -> 32 convs with a frequency stride (measured in the
    // model): the 1x1 shortcuts and the 40 -> 20 3x3 on the 128x32
    // register-staged tile, the 80 -> 40 and the final 20 -> 10 3x3s on the
    // narrow 32x64 DMA tile
    if (!a.split && a.IC == 32 && a.OC == 32 && (a.sh != 1 || a.sw != 1)) {
        if (a.KH * a.KW == 1) return 10;
        if (a.H <= 20) return 60;
        if (a.H <= 40) return 10;   // the second stage's 40 -> 20 conv (B=32 x 10 s: 48.1 -> 43.4 us)
        if (tile_fits(kTiles[60], a)) return 60;   // 80 -> 40 (in-model: 87.2 -> 80.5 us)
    }
    // the FCM blocks' stride-1 conv2 (+ the shortcut): the 32-channel
    // register-weight tile at every batch (B=32 x 10 s, 40 rows: 54.4 -> 45.6 us;
    // in the model fcm_conv1 + fcm_conv2 0.256 -> 0.219 ms per step)
    if (!a.split && is_s1_3x3(a) && a.IC == 32 && a.OC == 32 && a.res && tile_fits(kTiles[69], a)) return 69;
    if (a.split && is_s1_3x3(a)) {   // ERes2Net's split-f16 group convs (random-data sweeps)
        // f16-exact weights: the split-f16 register-weight kernel
        if (a.OC == 16 && a.IC == 32 && tile_fits(kTiles[70], a)) return 70;
        if (a.OC == 16 && a.IC == 16 && tile_fits(kTiles[71], a)) return 71;
        if (a.OC == 32 && a.IC == 32 && tile_fits(kTiles[72], a)) return 72;
        if (a.OC == 32 && a.IC == 64 && tile_fits(kTiles[74], a)) return 74;
        if (a.OC == 64 && a.IC == 64 && tile_fits(kTiles[75], a)) return 75;
        // up to 64 output channels: the halo kernel (each input pixel fetched
        // once per chunk for all 9 taps; 2.5-2.8x faster than the DMA tiles
        // on the 16-64-channel layers), 8-row tiles on the 1998-frame maps
        if (a.OC <= 32 && a.IC % 32 == 0 && tile_fits(kTiles[a.W >= 1000 ? 27 : 28], a)) return a.W >= 1000 ? 27 : 28;
        if (a.OC == 64 && a.IC % 32 == 0 && tile_fits(kTiles[30], a)) return 30;
        // layer 4's 10-row maps: the halo tile (in-model sweep, 41.8 -> 37.7 us)
        if (a.IC == 128 && a.OC == 128 && a.H <= 10 && tile_fits(kTiles[26], a)) return 26;
        if (a.IC == 128 && a.OC == 128 && tile_fits(kTiles[40], a)) return 40;
    }
    if (a.split && a.KH == 3 && a.KW == 3 && a.sh == 2 && a.sw == 2) {   // ERes2Net's cross-stage downsamples
        if (a.IC == 64 && a.OC == 128 && tile_fits(kTiles[36], a)) return 36;
        if (a.IC == 128 && a.OC == 256 && tile_fits(kTiles[34], a)) return 34;
        if (a.IC == 256 && a.OC == 512 && tile_fits(kTiles[40], a)) return 40;
    }
    if (a.split && a.KH * a.KW == 1) {
        // ERes2Net's split-f16 1x1s from an in-model sweep (B=16 x 20 s, every
        // fitting tile timed in place on the model's buffers): the widening /
        // narrowing convs and the AFF local_att convs
        auto fit = [&](int t) { return tile_fits(kTiles[t], a) ? t : -1; };
        int t = -1;
        if (a.sh == 1 && a.sw == 1) {
            if (a.IC == 32 && a.OC == 64 && a.split == 2) t = fit(61);              // 37.9 -> 29.4 us
            else if (a.IC == 32 && a.OC == 128) t = fit(a.H <= 10 ? 61 : 47);      // 31.1 -> 19.3 / 244.8 -> 230.1
            else if (a.IC == 64 && a.OC == 256) t = fit(47);                       // 162.4 -> 131.9
            else if (a.IC == 128 && a.OC == 32) t = fit(60);                       // 27.4 -> 23.6
            else if (a.IC == 256 && a.OC == 32) t = fit(a.H <= 10 ? 60 : 22);      // 25.2 -> 18.3 / 197.0 -> 184.2
            else if (a.IC == 1024 && a.OC == 128) t = fit(18);                     // 71.5 -> 54.0
            else if (a.IC == 128 && a.OC == 512) t = fit(47);                      // 85.1 -> 73.4
            else if (a.IC == 512 && a.OC == 64) t = fit(23);                       // 96.4 -> 91.6
        } else if (a.sh == 2 && a.sw == 2) {   // the shortcuts' stride-2 1x1s
            if (a.IC == 128 && a.OC == 256) t = fit(36);                           // 79.5 -> 68.4
            else if (a.IC == 64 && a.OC == 64) t = fit(16);                        // 89.1 -> 82.5
            else if (a.IC == 256 && a.OC == 512) t = fit(40);                      // 54.6 -> 50.4
        }
        if (t >= 0) return t;
    }
    if (a.split && a.KH * a.KW == 1 && a.sh == 1 && a.sw == 1) {   // ERes2Net's split-f16 1x1s (same sweep;
        // the 128 -> 64, 128 -> 256 and 256 -> 512 rules re-swept interleaved
        // at B=16 x 20 s with three-term weights: 133 -> 129, 125 -> 120 and
        // 76 -> 64 us)
        if (a.IC == 64 && a.OC == 32) return 61;
        if (a.IC == 128 && a.OC == 64) return 16;
        if (a.IC == 256 && a.OC == 128) return 45;
        if (a.IC == 128 && a.OC == 256) return 40;
        if (a.IC == 256 && a.OC == 512) return 40;
    }
    if (is_s1_3x3(a) && a.IC == 64 && a.OC == 64 && plain_epilogue(a)) return 66;   // 3-stage ring
    // small batches (5-row bands on under 48 workgroups): one-row bands, the
    // same bits on 5x the workgroups; measured on ResNet34's maps: 128->128
    // 22.1 -> 11.1 us at batch 1, 23.1 -> 15.0 us at batch 8, slower from
    // batch 16 (64 workgroups); 256->256 23.8 -> 14.8 us at batch 1
    const long bands5 = (long)(a.npix / (a.Ho * a.Wo)) * cdiv(a.H, 5) * (a.OC / 128);
    if (is_s1_3x3(a) && a.OC == 128 && a.W > BandTile<5, 3>::MAXW && bands5 < 48 && tile_fits(kTiles[77], a))
        return 77;
    if (is_s1_3x3(a) && a.OC >= 256 && a.W <= BandTile<5, 3>::MAXW && bands5 < 48 && tile_fits(kTiles[78], a))
        return 78;
    if (is_s1_3x3(a) && a.OC == 128 && a.W > BandTile<5, 3>::MAXW && tile_fits(kTiles[64], a)) return 64;
    if (is_s1_3x3(a) && a.OC == 128 && a.W > BandTile<5, 3>::MAXW && tile_fits(kTiles[57], a)) return 57;
    if (is_s1_3x3(a) && a.OC >= 256 && a.W <= BandTile<5, 3>::MAXW && tile_fits(kTiles[65], a)) return 65;
    if (is_s1_3x3(a) && a.OC >= 256 && a.W <= BandTile<5, 3>::MAXW && tile_fits(kTiles[58], a)) return 58;
    // ResNet's stride-2 convs at small batches (under 8192 output pixels, e.g.
    // batch 1), measured: the 3x3s from 64 / 128 channels on the 128x32 DMA
    // tile (18.8 -> 9.6 / 13.7 us), the rest on the 64x64 register-staged tile
    // (32 -> 64 3x3 10.8 -> 7.0 us, the 1x1 shortcuts 9.1 -> 4.5 and 7.3 -> 5.1)
    if (!a.split && a.KH == a.KW && a.sh == 2 && a.sw == 2 && a.npix < 8192 && a.IC % 32 == 0 && a.OC % 64 == 0) {
        if (a.KH == 3 && a.IC % 64 == 0 && a.OC % 128 == 0 && tile_fits(kTiles[52], a)) return 52;
        if (tile_fits(kTiles[63], a)) return 63;
    }
    // ResNet's stride-2 3x3s from 64 / 128 channels at batch 64 on the GEMM
    // producer / compute kernel (interleaved timing: 32.5 -> 29.3 us on the
    // 128 x 384 tile, 28.3 -> 26.3 us on 256 x 128)
    if (!a.split && a.KH == 3 && a.KW == 3 && a.sh == 2 && a.sw == 2 && a.npix >= 16384) {
        if (a.IC == 64 && a.OC == 128 && tile_fits(kTiles[82], a)) return 82;
        if (a.IC == 128 && a.OC == 256 && tile_fits(kTiles[83], a)) return 83;
    }
    // ResNet's stride-2 32->64 pair (random-data sweep): the 1x1 on the 64x64
    // register-staged tile, the 3x3 on the 64x128 one
    if (!a.split && !is_s1_3x3(a) && a.IC == 32 && a.OC == 64) return a.KH * a.KW == 1 ? 63 : 2;
    if (!a.split && is_s1_3x3(a) && a.IC % 32 == 0 && a.IC <= 64 && a.OC <= 64) return 28;
    if (a.IC % 32 == 0 && a.OC == 128) return 39;   // 128x128 tile, KC = 32
    if (a.IC % 64 == 0) return bm == 128 ? 18 : (bm == 64 ? 15 : 14);
    if (a.IC % 32 == 0) return bm >= 64 ? 16 : 14;
    if (a.split) return -1;
    if (a.IC % 16 == 0) return bm == 128 ? 13 : (bm == 64 ? 12 : 11);
    return -1;
}

template <int OC>
__global__ __launch_bounds__(256) void stem_conv3x3_kernel(const float* __restrict__ feats,
                                                           const float* __restrict__ rmean, int B, int H, int W,
                                                           const float* __restrict__ w,
                                                           const float* __restrict__ bias, int relu, int split,
                                                           half_t* __restrict__ y) {
    // OC/8 threads per output pixel, 8 channels each: the OC/8 lanes of a pixel
    // write its OC*2 bytes as consecutive 16-byte chunks.
    constexpr int G = OC / 8;
    __shared__ float sw[OC * 9], sb[OC];
    for (int i = threadIdx.x; i < OC * 9; i += 256) sw[i] = w[i];
    for (int i = threadIdx.x; i < OC; i += 256) sb[i] = bias[i];
    __syncthreads();
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    const long HW = (long)H * W;
    const long P = idx / G;
    const int g = (int)(idx - P * G);
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
            xv[kh * 3 + kw] = (ih >= 0 && ih < H && iw >= 0 && iw < W)
                                  ? feats[((long)b * H + ih) * W + iw] - (rmean ? rmean[(long)b * H + ih] : 0.0f)
                                  : 0.0f;
        }
    half8 hv, lv;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int oc = g * 8 + e;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 9; ++k) acc += sw[oc * 9 + k] * xv[k];
        float v = acc + sb[oc];
        if (relu) v = fmaxf(v, 0.0f);
        hv[e] = (half_t)v;
        lv[e] = (half_t)(v - (float)hv[e]);
    }
    if (split) {   // [hi(OC) | lo(OC)] per pixel
        *reinterpret_cast<half8*>(y + P * 2 * OC + g * 8) = hv;
        *reinterpret_cast<half8*>(y + P * 2 * OC + OC + g * 8) = lv;
    } else {
        *reinterpret_cast<half8*>(y + P * OC + g * 8) = hv;
    }
}

// The stem as f32 MFMA (v_mfma_f32_32x32x2_f32: f32 products and sums, the
// precision of the f32 FMA loop above).  A wavefront walks up to kStemRuns
// runs of 32 consecutive output pixels of one row; per run the GEMM rows are
// the output channels (OC/32 blocks), the columns its 32 pixels and K the 9
// taps padded to 10: five K=2 MFMAs per block whose B operand lane l reads
// tap 2q + l/32 of pixel l%32 straight from the features (the three input
// rows stay in the L1), loaded one run ahead.  The accumulators (+bias,
// [ReLU]) are rounded to f16 (and the split-f16 remainder) into a per-wave LDS
// tile that leaves as 16-byte channel chunks, so each store instruction
// writes 16 whole pixels.
constexpr int kStemRuns = 10;

template <int OC, bool SPLIT>
__global__ __launch_bounds__(256) void stem_mfma_kernel(const float* __restrict__ feats,
                                                        const float* __restrict__ rmean, int B, int H, int W,
                                                        const float* __restrict__ w, const float* __restrict__ bias,
                                                        int relu, half_t* __restrict__ y, int rpw) {
    constexpr int NOB = OC / 32, PITCH = OC * 2 + 16;   // LDS row: OC f16 channels + 16 bytes
    static_assert(OC % 32 == 0, "whole 32-channel MFMA blocks");
    __shared__ __attribute__((aligned(16))) uint8_t stile[4][SPLIT ? 2 : 1][32 * PITCH];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 31, kk = lane >> 5;
    const int ntb = (W + 31) >> 5, nch = (ntb + rpw - 1) / rpw;
    const int item = blockIdx.x * 4 + wave;
    if (item >= B * H * nch) return;   // no barrier below: a wave may leave alone
    const int row = item / nch, r0 = (item - row * nch) * rpw;
    const int r1 = r0 + rpw < ntb ? r0 + rpw : ntb;
    const int b = row / H, h = row - b * H;
    float wa[NOB][5];
    float16v bv[NOB];   // the accumulators start at the bias (register g*4+e: channel 8g + 4*kk + e)
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) {
#pragma unroll
        for (int q = 0; q < 5; ++q) {
            const int tap = 2 * q + kk;
            wa[ob][q] = tap < 9 ? w[(ob * 32 + j) * 9 + tap] : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) bv[ob][r] = bias[ob * 32 + (r >> 2) * 8 + kk * 4 + (r & 3)];
    }
    // the CMN means of the three input rows (rows outside the map stay zero
    // padding, so their mean is never applied)
    // the CMN means of the three input rows (0 outside the map), then the one
    // this lane's tap q takes (selects, not an indexed array: an indexed
    // private array would be placed in LDS)
    float mu0 = 0.0f, mu1 = 0.0f, mu2 = 0.0f;
    if (rmean) {
        if (h >= 1) mu0 = rmean[(size_t)b * H + h - 1];
        mu1 = rmean[(size_t)b * H + h];
        if (h + 1 < H) mu2 = rmean[(size_t)b * H + h + 1];
    }
    float muq[5];
#pragma unroll
    for (int q = 0; q < 5; ++q) {
        const int kh = (2 * q + kk) / 3;
        muq[q] = kh == 0 ? mu0 : (kh == 1 ? mu1 : mu2);
    }
    // raw values, and the mean each one takes when it is used (0 for the
    // zero padding), so the loads of the next run stay in flight meanwhile
    auto load = [&](int r, float* xb, float* mb) {
        const int t0 = r * 32;
#pragma unroll
        for (int q = 0; q < 5; ++q) {
            const int tap = 2 * q + kk, kh = tap / 3, kw = tap - kh * 3;
            const int ih = h - 1 + kh, iw = t0 + j - 1 + kw;
            const bool in = tap < 9 && ih >= 0 && ih < H && iw >= 0 && iw < W;
            xb[q] = in ? feats[((size_t)b * H + ih) * W + iw] : 0.0f;
            mb[q] = in ? muq[q] : 0.0f;
        }
    };
    uint8_t* const hi = stile[wave][0];
    uint8_t* const lo = stile[wave][SPLIT ? 1 : 0];
    constexpr int CPP = OC / 8;                  // 16-byte chunks per pixel
    constexpr int PPI = 64 / CPP;                // pixels per store instruction
    constexpr int ostride = SPLIT ? 2 * OC : OC;
    float xn[5], mn[5];
    load(r0, xn, mn);
    for (int r = r0; r < r1; ++r) {
        float xb[5];
#pragma unroll
        for (int q = 0; q < 5; ++q) xb[q] = xn[q] - mn[q];   // the CMN subtraction (x - 0 = x without it)
        if (r + 1 < r1) load(r + 1, xn, mn);
#pragma unroll
        for (int ob = 0; ob < NOB; ++ob) {
            float16v acc = bv[ob];
#pragma unroll
            for (int q = 0; q < 5; ++q) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(wa[ob][q], xb[q], acc, 0, 0, 0);
            // register g*4+e: channel ob*32 + 8g + 4*kk + e of pixel j
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int c = ob * 32 + g * 8 + kk * 4;
                half4 hv, lv;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v = acc[g * 4 + e];
                    if (relu) v = fmaxf(v, 0.0f);
                    hv[e] = (half_t)v;
                    if constexpr (SPLIT) lv[e] = (half_t)(v - (float)hv[e]);
                }
                *reinterpret_cast<half4*>(hi + j * PITCH + c * 2) = hv;
                if constexpr (SPLIT) *reinterpret_cast<half4*>(lo + j * PITCH + c * 2) = lv;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int t0 = r * 32;
        const size_t pix0 = (size_t)row * W + t0;
#pragma unroll
        for (int it = 0; it < 32 / PPI; ++it) {
            const int p = it * PPI + lane / CPP, ch = lane % CPP;
            if (t0 + p < W) {
                half_t* const dst = y + (pix0 + p) * ostride + ch * 8;
                *reinterpret_cast<half8*>(dst) = *reinterpret_cast<const half8*>(hi + p * PITCH + ch * 16);
                if constexpr (SPLIT)
                    *reinterpret_cast<half8*>(dst + OC) = *reinterpret_cast<const half8*>(lo + p * PITCH + ch * 16);
            }
        }
        // this run's tile reads are issued before the next run's writes (in-order LDS per wavefront)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Run-time tile tuning: mismatching f16 values between two outputs of npix
// pixels x OC channels at pixel stride ys.
__global__ __launch_bounds__(256) void count_diff_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                                         int npix, int OC, int ys, unsigned* __restrict__ out) {
    const long n = (long)npix * OC;
    unsigned c = 0;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        const long p = i / OC, k = i - p * OC;
        c += a[p * ys + k] != b[p * ys + k];
    }
    if (c) atomicAdd(out, c);
}

std::atomic<int> g_autotune{-1};   // -1: not yet read from VDK_CONV_AUTOTUNE
bool autotune_on() {
    int v = g_autotune.load();
    if (v < 0) {
        const char* e = std::getenv("VDK_CONV_AUTOTUNE");
        v = (e && *e && *e != '0') ? 1 : 0;
        int expect = -1;
        g_autotune.compare_exchange_strong(expect, v);
        v = g_autotune.load();
    }
    return v == 1;
}
struct TuneCache {
    std::mutex mu;
    std::unordered_map<std::string, int> best;
};
TuneCache& tune_cache() {
    static TuneCache c;
    return c;
}
std::string tune_key(const ConvArgs& a) {
    char k[400];
    snprintf(k, sizeof k, "%d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d",
             a.H, a.W, a.IC, a.Ho, a.Wo, a.OC, a.KH, a.KW, a.sh, a.sw, a.ph, a.pw, a.dh, a.dw, a.act, a.xs, a.ys,
             a.rs, a.npix, a.npix_in, a.reflect, a.bias != nullptr, a.res != nullptr, a.gate != nullptr,
             a.post_scale != nullptr, a.in_scale != nullptr, a.wc != nullptr, a.wq != nullptr, a.res_f32, a.res_after,
             a.tanh_after);
    return k;
}
// The tuner handles convs whose output is plain f16 rows (no second output,
// segment sums, split-f16, f32 / transposed store or AFF operands) that do
// not overlap an input.
bool tunable(const ConvArgs& a) {
    if (a.split || a.y2 || a.segsum || a.y_f32 || a.y_tr || a.ax || a.xgl != 4 || a.ygl != 4 || a.xgs != 16 ||
        a.ygs != 16)
        return false;
    const auto* y0 = static_cast<const uint8_t*>(a.y);
    const uint8_t* y1 = y0 + 2 * ((size_t)(a.npix - 1) * a.ys + a.OC);
    auto overlaps = [&](const void* p, size_t bytes) {
        const auto* q = static_cast<const uint8_t*>(p);
        return p && q < y1 && y0 < q + bytes;
    };
    return !overlaps(a.x, 2 * ((size_t)(a.npix_in - 1) * a.xs + a.IC)) &&
           !overlaps(a.res, (a.res_f32 ? 4 : 2) * ((size_t)(a.npix - 1) * a.rs + a.OC));
}
// Times every tile that fits (into scratch outputs) and returns the fastest
// whose output equals the default tile's bit for bit (so the choice changes
// neither the results nor their independence of the batch); synchronises s.
int tune_tile(const ConvArgs& a, int t_default, hipStream_t s) {
    const size_t ybytes = 2 * ((size_t)(a.npix - 1) * a.ys + a.OC);
    void *ya = nullptr, *yb = nullptr;
    unsigned* cnt = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int best = t_default;
    auto cleanup = [&] {
        if (ya) (void)hipFree(ya);
        if (yb) (void)hipFree(yb);
        if (cnt) (void)hipFree(cnt);
        if (e0) (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
    };
    if (hipMalloc(&ya, ybytes) != hipSuccess || hipMalloc(&yb, ybytes) != hipSuccess ||
        hipMalloc((void**)&cnt, sizeof(unsigned)) != hipSuccess || hipEventCreate(&e0) != hipSuccess ||
        hipEventCreate(&e1) != hipSuccess) {
        cleanup();
        (void)hipGetLastError();
        return t_default;
    }
    auto time_tile = [&](int t, void* y) {
        ConvArgs b = a;
        b.y = y;
        kTiles[t].launch(b, s);   // warm
        float best_ms = 1e30f;
        for (int rep = 0; rep < 3; ++rep) {
            VDK_HIP(hipEventRecord(e0, s));
            kTiles[t].launch(b, s);
            VDK_HIP(hipEventRecord(e1, s));
            VDK_HIP(hipEventSynchronize(e1));
            float ms = 0.0f;
            VDK_HIP(hipEventElapsedTime(&ms, e0, e1));
            best_ms = std::min(best_ms, ms);
        }
        return best_ms;
    };
    try {
        VDK_HIP(hipMemsetAsync(ya, 0, ybytes, s));
        VDK_HIP(hipMemsetAsync(yb, 0, ybytes, s));
        float best_ms = time_tile(t_default, ya);
        for (int t = 0; t < kNumTiles; ++t) {
            if (t == t_default || !tile_fits(kTiles[t], a)) continue;
            const float ms = time_tile(t, yb);
            VDK_HIP(hipMemsetAsync(cnt, 0, sizeof(unsigned), s));
            const long n = (long)a.npix * a.OC;
            hipLaunchKernelGGL(count_diff_kernel, dim3((unsigned)std::min<long>(cdiv(n, 256), 4096)), dim3(256), 0, s,
                               static_cast<const uint16_t*>(ya), static_cast<const uint16_t*>(yb), a.npix, a.OC, a.ys,
                               cnt);
            unsigned diff = 1;
            VDK_HIP(hipMemcpyAsync(&diff, cnt, sizeof(unsigned), hipMemcpyDeviceToHost, s));
            VDK_HIP(hipStreamSynchronize(s));
            if (diff == 0 && ms < best_ms) {
                best_ms = ms;
                best = t;
            }
        }
    } catch (...) {
        cleanup();
        throw;
    }
    cleanup();
    return best;
}

}  // namespace
}  // namespace vdk

using namespace vdk;

namespace {
int conv_impl(const vdk_conv_desc& d, void* stream) {
    return guarded([&] {
        require(d.x && (d.w || d.w_q8_0) && d.y, "conv2d: NULL device pointer");
        require(d.batch > 0 && d.H > 0 && d.W > 0, "conv2d: empty input");
        require(d.IC > 0 && d.IC % 16 == 0, "conv2d: IC must be a positive multiple of 16");
        require(d.OC > 0 && d.OC % 8 == 0, "conv2d: OC must be a positive multiple of 8");
        require(d.KH >= 1 && d.KW >= 1 && d.KH * d.KW <= 256, "conv2d: kernel size out of range (KH*KW <= 256)");
        const int sh = d.stride_h ? d.stride_h : 1, sw = d.stride_w ? d.stride_w : 1;
        const int dh = d.dil_h ? d.dil_h : 1, dw = d.dil_w ? d.dil_w : 1;
        require(sh >= 1 && sw >= 1 && dh >= 1 && dw >= 1 && d.pad_h >= 0 && d.pad_w >= 0,
                "conv2d: invalid stride/pad/dilation");
        const int ekh = (d.KH - 1) * dh + 1, ekw = (d.KW - 1) * dw + 1;
        require(d.H + 2 * d.pad_h >= ekh && d.W + 2 * d.pad_w >= ekw, "conv2d: output would be empty");
        const int Ho = (d.H + 2 * d.pad_h - ekh) / sh + 1, Wo_full = (d.W + 2 * d.pad_w - ekw) / sw + 1;
        require(d.out_w >= 0 && d.out_w <= Wo_full, "conv2d: out_w exceeds the output width");
        const int Wo = d.out_w > 0 ? d.out_w : Wo_full;
        const int xs = d.x_stride ? d.x_stride : d.IC, ys = d.y_stride ? d.y_stride : d.OC;
        const int rs = d.res_stride ? d.res_stride : d.OC;
        require(xs >= d.IC && ys >= d.OC && rs >= d.OC, "conv2d: pixel stride smaller than the channel count");
        require(xs % 8 == 0 && ys % 8 == 0 && rs % 8 == 0, "conv2d: pixel strides must be multiples of 8");
        require((long)d.batch * Ho * Wo < (1L << 31) && (long)d.batch * d.H * d.W * xs < (1L << 30) &&
                    (long)d.batch * Ho * Wo * ys < (1L << 31) &&
                    (long)d.OC * d.KH * d.KW * d.IC * (d.split == 2 ? 2 : (d.split ? 3 : 1)) < (1L << 30),
                "conv2d: too many pixels for one launch");
        require(aligned16(d.x) && aligned16(d.w) && aligned16(d.y) && (!d.residual || aligned16(d.residual)),
                "conv2d: device pointers must be 16-byte aligned");
        require(!d.post_scale == !d.post_shift, "conv2d: post_scale and post_shift go together");
        require(aligned16(d.bias) && aligned16(d.gate) && aligned16(d.post_scale) && aligned16(d.post_shift) &&
                    d.bias_batch_stride % 4 == 0,
                "conv2d: bias / gate / post-affine vectors must be 16-byte aligned");
        require(!d.gate || (d.gate_seg > 0 && d.gate_nseg > 0 && (Wo + d.gate_seg - 1) / d.gate_seg <= d.gate_nseg),
                "conv2d: gate needs gate_seg > 0 and enough segments for the output width");
        require(!d.y_time_major || !d.residual, "conv2d: a time-major store takes no residual");
        require(!d.res_f32 || (d.residual && !d.split), "conv2d: an f32 residual needs a residual and no split-f16");
        require(!d.in_scale == !d.in_shift, "conv2d: in_scale and in_shift go together");
        require(!d.in_scale || (d.KH == 1 && d.KW == 1 && d.pad_h == 0 && d.pad_w == 0 && !d.split &&
                                aligned16(d.in_scale) && aligned16(d.in_shift)),
                "conv2d: the input prologue needs a 1x1 conv without padding and 16-byte aligned vectors");
        require(d.split >= 0 && d.split <= 2, "conv2d: split must be 0, 1 or 2");
        const int xgn = d.x_group ? d.x_group : 16, ygn = d.y_group ? d.y_group : 16;   // channels per group
        const int xgs = d.x_group_stride ? d.x_group_stride : xgn, ygs = d.y_group_stride ? d.y_group_stride : ygn;
        require((xgn == 16 || xgn == 32) && (ygn == 16 || ygn == 32), "conv2d: channel groups are 16 or 32 wide");
        // grouped split layouts: each group's lo half sits inside the group stride
        const bool xg = xgs != xgn, yg = ygs != ygn;
        require((!xg && !yg) ||
                    (d.split && d.IC % xgn == 0 && d.OC % ygn == 0 && xgs % 8 == 0 && ygs % 8 == 0 &&
                     (!xg || (d.x_lo >= xgn && d.x_lo + xgn <= xgs && (d.IC / xgn - 1) * xgs + xgn + d.x_lo <= xs)) &&
                     (!yg || (d.y_lo >= ygn && d.y_lo + ygn <= ygs && (d.OC / ygn - 1) * ygs + ygn + d.y_lo <= ys))),
                "conv2d: group strides need split-f16, whole groups, lo halves inside the group stride and groups "
                "inside the pixel stride");
        require(!d.split || (!d.y_f32 && !d.y_time_major && (xg || d.x_lo >= d.IC) && (yg || d.y_lo >= d.OC) &&
                             (!d.residual || d.res_lo >= d.OC) && d.x_lo % 8 == 0 && d.y_lo % 8 == 0 &&
                             d.res_lo % 8 == 0 && (d.IC % 32 == 0 || (d.split == 2 && d.IC == 16))),
                "conv2d: split-f16 needs IC % 32 == 0 (or 16 with split 2), f16 output and lo offsets past the "
                "channels");
        require(!d.reflect_pad || (d.KH == 1 && d.pad_h == 0 && d.pad_w < d.W),
                "conv2d: reflect padding is for 1-D convs (KH = 1) with pad_w < W");
        const int y2s = d.y2_stride ? d.y2_stride : d.OC, r2s = d.res2_stride ? d.res2_stride : d.OC;
        require(!d.y2 || (d.res2 && !d.split && !d.y_f32 && !d.y_time_major && aligned16(d.y2) &&
                          aligned16(d.res2) && y2s >= d.OC && r2s >= d.OC && y2s % 8 == 0 && r2s % 8 == 0),
                "conv2d: the second output needs res2, f16 NHWC output, 16-byte alignment and strides >= OC");
        require(!d.w_q8_0 || (d.KH == 1 && d.KW == 1 && d.IC % 32 == 0 && !d.split &&
                               (reinterpret_cast<uintptr_t>(d.w_q8_0) & 3) == 0 &&
                               (long)d.OC * (d.IC / 32) * 34 < (1L << 31)),
                "conv2d: q8_0 weights are for 1x1 convs with IC % 32 == 0 and no split-f16");
        require(!d.aff_x == !d.aff_ds, "conv2d: aff_x and aff_ds go together");
        const int axs = d.aff_x_stride ? d.aff_x_stride : d.OC, adss = d.aff_ds_stride ? d.aff_ds_stride : d.OC;
        require(!d.aff_x || (!d.y_f32 && !d.y_time_major && !d.y2 && !yg && aligned16(d.aff_x) && aligned16(d.aff_ds) &&
                             axs >= d.OC && adss >= d.OC && axs % 8 == 0 && adss % 8 == 0 &&
                             (!d.split || (d.aff_x_lo >= d.OC && d.aff_ds_lo >= d.OC && d.aff_x_lo % 8 == 0 &&
                                           d.aff_ds_lo % 8 == 0)) &&
                             (long)d.batch * Ho * Wo * std::max(axs, adss) < (1L << 31)),
                "conv2d: the AFF combine needs x and ds at the output's pixels (16-byte aligned, strides >= OC, "
                "lo offsets past the channels with split) and an f16 NHWC output");
        ConvArgs a{};
        a.ax = static_cast<const half_t*>(d.aff_x);
        a.ads = static_cast<const half_t*>(d.aff_ds);
        a.axs = axs; a.adss = adss; a.ax_lo = d.aff_x_lo; a.ads_lo = d.aff_ds_lo;
        a.wq = static_cast<const uint8_t*>(d.w_q8_0);
        require(!d.seg_sum || (Ho == 1 && d.seg_len > 0 && !d.split && !d.y_f32 && !d.y_time_major && !d.y2 &&
                               (reinterpret_cast<uintptr_t>(d.seg_sum) & 7) == 0),
                "conv2d: seg_sum needs H_out = 1, seg_len > 0, an f16 output (no split, time-major store or y2) and "
                "8-byte alignment");
        a.segsum = d.seg_sum;
        a.seg_len = d.seg_sum ? d.seg_len : 1;
        a.seg_n = d.seg_sum ? (Wo + d.seg_len - 1) / d.seg_len : 1;
        a.reflect = d.reflect_pad ? 1 : 0;
        a.y2 = static_cast<half_t*>(d.y2);
        a.r2 = static_cast<const half_t*>(d.res2);
        a.y2s = y2s; a.r2s = r2s;
        a.x = static_cast<const half_t*>(d.x);
        a.w = static_cast<const half_t*>(d.w);
        a.wc = static_cast<const half_t*>(d.w_chunked);
        a.bias = d.bias;
        a.res = static_cast<const half_t*>(d.residual);
        a.y = d.y;
        a.post_scale = d.post_scale;
        a.post_shift = d.post_shift;
        a.gate = d.gate;
        a.gate_seg = d.gate ? d.gate_seg : 1;
        a.gate_nseg = d.gate ? d.gate_nseg : 1;
        a.H = d.H; a.W = d.W; a.IC = d.IC; a.Ho = Ho; a.Wo = Wo; a.OC = d.OC;
        a.KH = d.KH; a.KW = d.KW;
        a.sh = sh; a.sw = sw; a.ph = d.pad_h; a.pw = d.pad_w; a.dh = dh; a.dw = dw;
        require(d.act >= VDK_ACT_NONE && d.act <= VDK_ACT_GELU, "conv2d: unknown activation");
        a.act = d.act;
        a.clamp_hi = d.act == VDK_ACT_RELU ? d.clamp_hi : 0.0f;
        a.tanh_after = d.tanh_after ? 1 : 0;
        a.y_f32 = d.y_f32 ? 1 : 0;
        a.y_tr = d.y_time_major ? 1 : 0;
        a.xs = xs; a.ys = ys; a.rs = rs;
        a.bias_bs = d.bias_batch_stride;
        a.split = d.split;
        a.x_lo = d.x_lo; a.r_lo = d.res_lo; a.y_lo = d.y_lo;
        a.xgs = xgs; a.ygs = ygs;
        a.xgl = xgn == 32 ? 5 : 4; a.ygl = ygn == 32 ? 5 : 4;
        a.res_f32 = d.res_f32 ? 1 : 0;
        a.res_after = d.res_after_act ? 1 : 0;
        a.in_scale = d.in_scale;
        a.in_shift = d.in_shift;
        a.npix = d.batch * Ho * Wo;
        a.npix_in = d.batch * d.H * d.W;
        hipStream_t s = static_cast<hipStream_t>(stream);
        int t = d.tile;
        if (t < 0) {
            t = pick_tile(a);
            require(t >= 0, "conv2d: no kernel for this channel count");
            if (autotune_on() && tunable(a)) {
                TuneCache& tc = tune_cache();
                const std::string key = tune_key(a);
                std::lock_guard<std::mutex> lock(tc.mu);
                auto it = tc.best.find(key);
                if (it != tc.best.end()) {
                    t = it->second;
                } else {
                    t = tune_tile(a, t, s);
                    tc.best.emplace(key, t);
                }
            }
        } else {
            require(t < kNumTiles, "conv2d: tile index out of range");
        }
        require(tile_fits(kTiles[t], a), "conv2d: tile " + std::to_string(t) + " does not fit this shape");
        kTiles[t].launch(a, s);
        VDK_HIP(hipGetLastError());
    });
}

vdk_conv_desc plain_desc(const void* d_x, int batch, int H, int W, int IC, const void* d_w, int OC, int KH, int KW,
                         int stride, int pad, const float* d_bias, const void* d_residual, int relu, void* d_y,
                         int tile) {
    vdk_conv_desc d{};
    d.x = d_x; d.batch = batch; d.H = H; d.W = W; d.IC = IC;
    d.w = d_w; d.OC = OC; d.KH = KH; d.KW = KW;
    d.stride_h = d.stride_w = stride;
    d.pad_h = d.pad_w = pad;
    d.dil_h = d.dil_w = 1;
    d.bias = d_bias; d.residual = d_residual; d.act = relu ? VDK_ACT_RELU : VDK_ACT_NONE; d.y = d_y; d.tile = tile;
    return d;
}

// The fields of a descriptor that decide which tiles apply (shape, layout,
// which epilogue stages are present); pointers only by presence.
ConvArgs shape_args(const vdk_conv_desc& d) {
    ConvArgs a{};
    a.split = d.split;
    a.IC = d.IC; a.OC = d.OC; a.KH = d.KH; a.KW = d.KW;
    a.sh = d.stride_h ? d.stride_h : 1; a.sw = d.stride_w ? d.stride_w : 1;
    a.ph = d.pad_h; a.pw = d.pad_w;
    a.dh = d.dil_h ? d.dil_h : 1; a.dw = d.dil_w ? d.dil_w : 1;
    a.H = d.H; a.W = d.W;
    a.xs = d.x_stride ? d.x_stride : d.IC;
    a.ys = d.y_stride ? d.y_stride : d.OC;
    a.rs = d.res_stride ? d.res_stride : d.OC;
    a.res = static_cast<const half_t*>(d.residual);
    a.res_f32 = d.res_f32 ? 1 : 0;
    a.res_after = d.res_after_act ? 1 : 0;
    a.in_scale = d.in_scale;
    a.in_shift = d.in_shift;
    a.gate = d.gate;
    a.post_scale = d.post_scale;
    a.act = d.act;
    a.clamp_hi = d.act == VDK_ACT_RELU ? d.clamp_hi : 0.0f;
    a.tanh_after = d.tanh_after ? 1 : 0;
    a.y_f32 = d.y_f32 ? 1 : 0;
    a.y_tr = d.y_time_major ? 1 : 0;
    a.bias_bs = d.bias_batch_stride;
    a.reflect = d.reflect_pad ? 1 : 0;
    a.y2 = static_cast<half_t*>(d.y2);
    a.wq = static_cast<const uint8_t*>(d.w_q8_0);
    a.segsum = d.seg_sum;
    a.seg_len = d.seg_sum && d.seg_len > 0 ? d.seg_len : 1;
    a.ax = static_cast<const half_t*>(d.aff_x);
    a.ads = static_cast<const half_t*>(d.aff_ds);
    a.xgl = d.x_group == 32 ? 5 : 4;
    a.ygl = d.y_group == 32 ? 5 : 4;
    a.xgs = d.x_group_stride ? d.x_group_stride : 1 << a.xgl;
    a.ygs = d.y_group_stride ? d.y_group_stride : 1 << a.ygl;
    return a;
}

}  // namespace

extern "C" int vdk_conv2d_ex(const vdk_conv_desc* d, void* stream) {
    if (!d) {
        set_error("conv2d: descriptor is NULL");
        return 1;
    }
    return conv_impl(*d, stream);
}

extern "C" int vdk_conv2d_nhwc(const void* d_x, int batch, int H, int W, int IC, const void* d_w, int OC, int KH,
                               int KW, int stride, int pad, const float* d_bias, const void* d_residual, int relu,
                               void* d_y, void* stream) {
    return conv_impl(plain_desc(d_x, batch, H, W, IC, d_w, OC, KH, KW, stride, pad, d_bias, d_residual, relu, d_y, -1),
                     stream);
}

extern "C" int vdk_conv2d_nhwc_tile(const void* d_x, int batch, int H, int W, int IC, const void* d_w, int OC,
                                    int KH, int KW, int stride, int pad, const float* d_bias, const void* d_residual,
                                    int relu, void* d_y, void* stream, int tile) {
    return conv_impl(plain_desc(d_x, batch, H, W, IC, d_w, OC, KH, KW, stride, pad, d_bias, d_residual, relu, d_y,
                                tile), stream);
}

extern "C" void vdk_conv_pack_chunked(const unsigned short* w, int OC, int KH, int KW, int IC, unsigned short* out) {
    const int taps = KH * KW;
    for (int oc = 0; oc < OC; ++oc)
        for (int t = 0; t < taps; ++t)
            for (int ic = 0; ic < IC; ++ic)
                out[(((size_t)(ic >> 4) * taps + t) * OC + oc) * 16 + (ic & 15)] = w[((size_t)oc * taps + t) * IC + ic];
}

extern "C" int vdk_conv2d_tile_count(void) { return kNumTiles; }

extern "C" int vdk_conv2d_tile_fits(int tile, int IC, int OC, int KH, int KW, int stride, int pad) {
    if (tile < 0 || tile >= kNumTiles) return 0;
    const vdk_conv_desc d = plain_desc(nullptr, 1, 1, 1, IC, nullptr, OC, KH, KW, stride, pad, nullptr, nullptr, 0,
                                       nullptr, tile);
    return tile_fits(kTiles[tile], shape_args(d)) ? 1 : 0;
}

extern "C" int vdk_conv_set_autotune(int on) {
    g_autotune.store(on ? 1 : 0);
    return 0;
}

extern "C" int vdk_conv_tuned_tile(const vdk_conv_desc* d) {
    if (!d || d->batch <= 0) return -1;
    ConvArgs a = shape_args(*d);   // + the fields conv_impl derives
    const int ekh = (d->KH - 1) * a.dh + 1, ekw = (d->KW - 1) * a.dw + 1;
    a.Ho = (d->H + 2 * d->pad_h - ekh) / a.sh + 1;
    const int Wo_full = (d->W + 2 * d->pad_w - ekw) / a.sw + 1;
    a.Wo = d->out_w > 0 ? d->out_w : Wo_full;
    a.npix = d->batch * a.Ho * a.Wo;
    a.npix_in = d->batch * d->H * d->W;
    a.bias = d->bias;
    a.wc = static_cast<const half_t*>(d->w_chunked);
    TuneCache& tc = tune_cache();
    std::lock_guard<std::mutex> lock(tc.mu);
    auto it = tc.best.find(tune_key(a));
    return it == tc.best.end() ? -1 : it->second;
}

extern "C" int vdk_conv2d_tile_fits_ex(int tile, const vdk_conv_desc* d) {
    if (tile < 0 || tile >= kNumTiles || !d) return 0;
    return tile_fits(kTiles[tile], shape_args(*d)) ? 1 : 0;
}

extern "C" int vdk_stem_conv3x3_ex(const float* d_feats, const float* d_row_mean, int batch, int H, int W,
                                   const float* d_w, const float* d_bias, int OC, int relu, int split, void* d_y,
                                   void* stream) {
    return guarded([&] {
        require(d_feats && d_w && d_bias && d_y, "stem: NULL device pointer");
        require(batch > 0 && H > 0 && W > 0, "stem: empty input");
        require((long)batch * H * W < (1L << 31), "stem: too many pixels for one launch");
        require(aligned16(d_y), "stem: output must be 16-byte aligned");
        hipStream_t s = static_cast<hipStream_t>(stream);
        const long n = (long)batch * H * W * (OC / 8);
        require(n < (1L << 31), "stem: too many pixels for one launch");
        half_t* y = static_cast<half_t*>(d_y);
        const int sp = split ? 1 : 0;
        // 32 / 64 channels: f32 MFMA, one wavefront per rpw (up to kStemRuns)
        // 32-pixel runs of a row; small batches take fewer runs per wavefront
        // until there are 2048 wavefronts (each run's arithmetic is the same)
        int rpw = kStemRuns;
        while (rpw > 1 && (long)batch * H * cdiv(cdiv(W, 32), rpw) < 2048) rpw = (rpw + 1) / 2;
        const long runs = (long)batch * H * cdiv(cdiv(W, 32), rpw);
        switch (OC) {
            case 16: hipLaunchKernelGGL(stem_conv3x3_kernel<16>, dim3(cdiv(n, 256)), dim3(256), 0, s, d_feats, d_row_mean, batch, H, W, d_w, d_bias, relu, sp, y); break;
            case 32:
                if (sp) hipLaunchKernelGGL((stem_mfma_kernel<32, true>), dim3(cdiv(runs, 4)), dim3(256), 0, s, d_feats, d_row_mean, batch, H, W, d_w, d_bias, relu, y, rpw);
                else hipLaunchKernelGGL((stem_mfma_kernel<32, false>), dim3(cdiv(runs, 4)), dim3(256), 0, s, d_feats, d_row_mean, batch, H, W, d_w, d_bias, relu, y, rpw);
                break;
            case 64:
                if (sp) hipLaunchKernelGGL((stem_mfma_kernel<64, true>), dim3(cdiv(runs, 4)), dim3(256), 0, s, d_feats, d_row_mean, batch, H, W, d_w, d_bias, relu, y, rpw);
                else hipLaunchKernelGGL((stem_mfma_kernel<64, false>), dim3(cdiv(runs, 4)), dim3(256), 0, s, d_feats, d_row_mean, batch, H, W, d_w, d_bias, relu, y, rpw);
                break;
            default: throw Error("stem: OC must be 16, 32 or 64");
        }
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_stem_conv3x3(const float* d_feats, int batch, int H, int W, const float* d_w, const float* d_bias,
                                int OC, int relu, void* d_y, void* stream) {
    return vdk_stem_conv3x3_ex(d_feats, nullptr, batch, H, W, d_w, d_bias, OC, relu, 0, d_y, stream);
}

extern "C" int vdk_resblock3x3_variant(const void* d_x, int batch, int H, int W, int C, const void* d_w1,
                                       const float* d_b1, const void* d_w2, const float* d_b2, void* d_y,
                                       int variant, void* stream) {
    return guarded([&] {
        require(d_x && d_w1 && d_b1 && d_w2 && d_b2 && d_y, "resblock3x3: NULL device pointer");
        require(batch > 0 && H > 0 && W > 0, "resblock3x3: empty input");
        require(C == 32, "resblock3x3: only C = 32 has a fused kernel");
        const size_t bytes = (size_t)batch * H * W * C * 2;
        require(bytes < (1ull << 31), "resblock3x3: too many pixels for one launch");
        const uintptr_t xa = reinterpret_cast<uintptr_t>(d_x), ya = reinterpret_cast<uintptr_t>(d_y);
        require(xa + bytes <= ya || ya + bytes <= xa, "resblock3x3: y must not overlap x");
        require(aligned16(d_x) && aligned16(d_w1) && aligned16(d_w2) && aligned16(d_y) && aligned16(d_b1) &&
                    aligned16(d_b2), "resblock3x3: device pointers must be 16-byte aligned");
        require(variant >= -1 && variant <= 2, "resblock3x3: variant out of range");
        const auto* x = static_cast<const half_t*>(d_x);
        const auto* w1 = static_cast<const half_t*>(d_w1);
        const auto* w2 = static_cast<const half_t*>(d_w2);
        auto* y = static_cast<half_t*>(d_y);
        hipStream_t s = static_cast<hipStream_t>(stream);
        switch (variant) {
            case 1: launch_resblock<6, 8, 1>(x, w1, d_b1, w2, d_b2, y, batch, H, W, s); break;
            case 2: launch_resblock<14, 8, 1>(x, w1, d_b1, w2, d_b2, y, batch, H, W, s); break;
            default:
                // small batches (under 128 10-row tiles: ResNet34 batch 1): 6-row
                // tiles, more workgroups (every tile height gives the same bits);
                // measured 9.6 -> 8.7 us at batch 1, slower at batch 2
                if (variant < 0 && (long)batch * cdiv(H, 10) * cdiv(W, 30) < 128)
                    launch_resblock<6, 8, 1>(x, w1, d_b1, w2, d_b2, y, batch, H, W, s);
                else
                    launch_resblock<10, 8, 1>(x, w1, d_b1, w2, d_b2, y, batch, H, W, s);
                break;
        }
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_resblock3x3(const void* d_x, int batch, int H, int W, int C, const void* d_w1, const float* d_b1,
                               const void* d_w2, const float* d_b2, void* d_y, void* stream) {
    return vdk_resblock3x3_variant(d_x, batch, H, W, C, d_w1, d_b1, d_w2, d_b2, d_y, -1, stream);
}

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

// ---------------------------------------------------------------------------
// res2_pair_kernel: the two chained Res2Net 3x3 convs of a plain (non-AFF)
// scale-2 block with 16-channel chunks (src/encoder_eres2net.cpp:111-137,
// ERes2Net's layer 1) in one launch, split-f16 with f16-exact weights:
//   sp0 = min(relu(conv_a(c0) + b_a), clamp),
//   sp1 = min(relu(conv_b(sp0 + c1) + b_b), clamp).
// Maps are pixel rows of 16-channel groups [hi 16 | lo 16] (64 bytes): the
// input row's groups 0, 1 hold c0, c1 and the output row's groups 0, 1
// receive sp0, sp1, so the launch reads and writes whole 128-byte lines.  A
// persistent workgroup walks TH x 30 output tiles (rows fastest) through a
// ring of (TH+4) x 34 input halos, each DMA'd two tiles ahead; per tile
// conv_a runs over the (TH+2) x 32 region around the tile into LDS (zero
// outside the image: conv_b's zero padding) and the tile's own sp0 goes
// out, then conv_b reads c1 from the halo and sp0 from LDS.  Both run on
// 16x16x32 MFMAs (16 output channels x 16 pixels) with the K grouping of the
// one-conv kernel: conv_a [c0 hi | c0 lo] per tap, conv_b [c1 hi | sp0 hi]
// for every tap, then [c1 lo | sp0 lo] (its input sp0 + c1 is the two
// 16-channel halves of one 32-channel MFMA operand with the weights
// repeated), so sp0 and sp1 equal the two one-conv launches bit for bit.
// ---------------------------------------------------------------------------
namespace pair {
constexpr int TH = 4, TW = 30, NW = 8, NS = 3;
constexpr int XW = 34, XH = TH + 4, XPIX = XH * XW;     // input halo (tile origin - 2)
constexpr int RBX = 144, SPRX = 9;                      // [c0h c0l c1h c1l] + 16 bytes of padding
constexpr int X_INS = (XPIX * SPRX + 63) / 64, X_IPW = (X_INS + NW - 1) / NW;
constexpr int STAGE = X_INS * 1024;
constexpr int IW = 32, IH = TH + 2, IPIX = IH * IW;     // sp0 region (tile origin - 1)
constexpr int RBT = 80;                                 // [sp0h sp0l] + 16 bytes of padding
constexpr int NBA = IH * 2, NBB = TH * 2;               // 16-pixel column blocks of conv_a / conv_b
constexpr int BPA = (NBA + NW - 1) / NW, BPB = (NBB + NW - 1) / NW;
// one spare row: conv_b's discarded columns 30, 31 read up to two pixels past the region
constexpr int INTER_BYTES = (IPIX + IW) * RBT;
constexpr int SP = 18 / X_IPW;                          // conv_b steps between DMA instructions
static_assert(NS * STAGE + INTER_BYTES <= 163840, "the ring and the sp0 region fit the 160 KB of LDS");
static_assert(SP >= 1 && X_IPW * SP <= 18, "every DMA instruction has a conv_b step");
}  // namespace pair

__device__ __forceinline__ void wait_vm_le(int n) {
    switch (n) {
#define VDK_VM(N) case N: wait_vmcnt<N>(); break;
        VDK_VM(0) VDK_VM(1) VDK_VM(2) VDK_VM(3) VDK_VM(4) VDK_VM(5) VDK_VM(6) VDK_VM(7) VDK_VM(8)
#undef VDK_VM
        default: __builtin_amdgcn_s_waitcnt(0); break;
    }
}

struct PairWalk {
    const int* hofs; const int* hpos;
    int4v xr;
    int tiles_w, tiles_h, H, W, xs2;
};

// This wave's DMA instructions for tile t's halo into stage st.
struct PairDma {
    uint8_t* st;
    const PairWalk* k;
    int oh0, ow0, xo, wave;
    bool on;
    __device__ __forceinline__ PairDma(uint8_t* st_, const PairWalk& k_, int t, int wave_, bool on_)
        : st(st_), k(&k_), wave(wave_), on(on_) {
        const int th = t % k_.tiles_h, r = t / k_.tiles_h, tw = r % k_.tiles_w, b = r / k_.tiles_w;
        oh0 = th * pair::TH;
        ow0 = tw * pair::TW;
        xo = ((b * k_.H + oh0 - 2) * k_.W + ow0 - 2) * k_.xs2;
    }
    __device__ __forceinline__ void issue(int j) const {
        const int ins = wave + j * pair::NW;
        if (!on || ins >= pair::X_INS) return;
        const int hp = k->hpos[j];
        const int ih = oh0 - 2 + (hp >> 8), iw = ow0 - 2 + (hp & 255);
        const uint32_t off = (hp >= 0 && (unsigned)ih < (unsigned)k->H && (unsigned)iw < (unsigned)k->W)
                                 ? (uint32_t)(xo + k->hofs[j]) : kOOB;
        dma16(st + ins * 1024, k->xr, off);
    }
};

__device__ __forceinline__ void split_relu_clamp(const float4v& acc, const float* bv, float chi, half4& h, half4& l) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float v = fmaxf(acc[e] + bv[e], 0.0f);
        if (chi > 0.0f) v = fminf(v, chi);
        h[e] = (half_t)v;
        l[e] = (half_t)(v - (float)h[e]);
    }
}

// The block's conv3 (1x1 over [sp0 | sp1] -> 64 channels, split-f16 weights
// [hi | hi (| lo)] per input channel, bias, + residual, ReLU, clamp) fused
// after conv_b: sp1 goes to LDS instead of memory, and wave w computes output
// row w/2, channels 32 (w%2) .. on 32x32x16 MFMAs in the LDS-DMA kernel's
// order (K chunks hi.w_hi, lo.w_hi [, hi.w_lo], each sp0 then sp1) with its
// epilogue (+ bias, + residual hi, + lo, ReLU, clamp), so y equals the pair
// followed by that conv bit for bit.
struct PairConv3 {
    const half_t* w;          // [64][terms * 32]
    const float* b;
    int terms;
    const half_t* res; int rs, r_lo;
    half_t* y; int ys, y_lo;
};

// conv_a of tile (b, oh0, ow0) over its (TH+2) x 32 sp0 region, from the
// [c0 | c1] halo st into inter as [sp0 hi | sp0 lo] rows, zero outside the
// image (conv_b's zero padding).  Block j = region row j/2, columns
// 16*(j%2) ..; the B reads run PD steps ahead of the MFMAs.  With Y the
// tile's own sp0 also goes to y (the pair without conv3).
template <bool Y>
__device__ __forceinline__ void pair_conv_a(const uint8_t* st, uint8_t* inter, const half8* fa, const float* bva,
                                            float chi, int b, int oh0, int ow0, int H, int W, half_t* y, int ys,
                                            int wave, int lane) {
    using namespace pair;
    constexpr int PD = 4;
    const int lp = lane & 15, kg = lane >> 4;
    float4v acc[BPA];
    int aoff[BPA];
#pragma unroll
    for (int q = 0; q < BPA; ++q) {
        acc[q] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
        const int j = wave + q * NW < NBA ? wave + q * NW : 0;   // a spare block reads block 0
        aoff[q] = ((j >> 1) * XW + (j & 1) * 16 + lp) * RBX + kg * 16;
    }
    auto load_a = [&](int tap, half8* dst) {
        const int kh = tap / 3, kw = tap - kh * 3;
#pragma unroll
        for (int q = 0; q < BPA; ++q) dst[q] = *reinterpret_cast<const half8*>(st + aoff[q] + (kh * XW + kw) * RBX);
    };
    {
        half8 ring_a[PD][BPA];
#pragma unroll
        for (int s = 0; s < PD; ++s) load_a(s, ring_a[s]);
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            half8 cur[BPA];
#pragma unroll
            for (int q = 0; q < BPA; ++q) cur[q] = ring_a[tap % PD][q];
            if (tap + PD < 9) load_a(tap + PD, ring_a[tap % PD]);
#pragma unroll
            for (int q = 0; q < BPA; ++q)
                if (wave + q * NW < NBA)
                    acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[tap], cur[q], acc[q], 0, 0, 0);
        }
    }
#pragma unroll
    for (int q = 0; q < BPA; ++q) {
        const int j = wave + q * NW;
        if (j >= NBA) continue;
        const int r = j >> 1, col = (j & 1) * 16 + lp;
        const int gh = oh0 - 1 + r, gw = ow0 - 1 + col;
        half4 h, l;
        split_relu_clamp(acc[q], bva, chi, h, l);
        const bool in = (unsigned)gh < (unsigned)H && (unsigned)gw < (unsigned)W;
        if (!in) h = l = half4{0, 0, 0, 0};
        uint8_t* const tp = inter + (r * IW + col) * RBT + kg * 8;
        *reinterpret_cast<half4*>(tp) = h;
        *reinterpret_cast<half4*>(tp + 32) = l;
        if (Y && in && r >= 1 && r <= TH && col >= 1 && col <= TW) {
            half_t* const yp = y + ((size_t)(b * H + gh) * W + gw) * ys + kg * 4;
            *reinterpret_cast<half4*>(yp) = h;
            *reinterpret_cast<half4*>(yp + 16) = l;
        }
    }
}

// conv_b of the tile into cb: block j = output row j/2, columns 16*(j%2) ..
// (30, 31 are discarded); lanes of K half 0 read c1 from the halo st, of
// half 1 sp0 from inter.  side(s) runs after step s's MFMAs.
template <class Side>
__device__ __forceinline__ void pair_conv_b(const uint8_t* st, const uint8_t* inter, const half8* fb, float4v* cb,
                                            int wave, int lane, const Side& side) {
    using namespace pair;
    constexpr int PD = 4;
    const int lp = lane & 15, kg = lane >> 4;
    const bool fromx = kg < 2;
    const int srow = fromx ? XW * RBX : IW * RBT, scol = fromx ? RBX : RBT;
    const uint8_t* bbase[BPB];
#pragma unroll
    for (int q = 0; q < BPB; ++q) {
        cb[q] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
        const int j = wave + q * NW < NBB ? wave + q * NW : 0;
        const int i = j >> 1, c = (j & 1) * 16 + lp;
        bbase[q] = fromx ? st + ((i + 1) * XW + c + 1) * RBX + 64 + kg * 16 : inter + (i * IW + c) * RBT + (kg - 2) * 16;
    }
    auto load_b = [&](int s, half8* dst) {
        const int p = s / 9, tap = s - p * 9, kh = tap / 3, kw = tap - kh * 3;
#pragma unroll
        for (int q = 0; q < BPB; ++q) dst[q] = *reinterpret_cast<const half8*>(bbase[q] + kh * srow + kw * scol + p * 32);
    };
    half8 ring_b[PD][BPB];
#pragma unroll
    for (int s = 0; s < PD; ++s) load_b(s, ring_b[s]);
#pragma unroll
    for (int s = 0; s < 18; ++s) {
        half8 cur[BPB];
#pragma unroll
        for (int q = 0; q < BPB; ++q) cur[q] = ring_b[s % PD][q];
        if (s + PD < 18) load_b(s + PD, ring_b[s % PD]);
#pragma unroll
        for (int q = 0; q < BPB; ++q)
            if (wave + q * NW < NBB) cb[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fb[s % 9], cur[q], cb[q], 0, 0, 0);
        side(s);
    }
}

// sp1 of the tile's 4 x 32 pixels (columns 30, 31 unused) into s1t as
// [sp1 hi | sp1 lo] rows
__device__ __forceinline__ void pair_sp1_to_lds(const float4v* cb, const float* bvb, float chi, uint8_t* s1t, int wave,
                                                int lane) {
    using namespace pair;
    const int lp = lane & 15, kg = lane >> 4;
#pragma unroll
    for (int q = 0; q < BPB; ++q) {
        const int j = wave + q * NW;
        if (j >= NBB) continue;
        const int i = j >> 1, c = (j & 1) * 16 + lp;
        half4 h, l;
        split_relu_clamp(cb[q], bvb, chi, h, l);
        uint8_t* const tp = s1t + (i * 32 + c) * RBT + kg * 8;
        *reinterpret_cast<half4*>(tp) = h;
        *reinterpret_cast<half4*>(tp + 32) = l;
    }
}

// conv3 for this wave's 32 outputs: output row crow = wave / 2, pixel l32,
// channels 32 (wave % 2) ..; B = sp0 at region (crow + 1, l32 + 1), sp1 at
// tile (crow, l32), K steps (term, half); + bias, + residual hi, + lo, ReLU,
// clamp, split store at yp (nothing when !ok).  f3(st) is K step st's A
// fragment, bv3(i) the bias of the lane's i-th output (register g * 4 + e).
template <class F3, class BV3>
__device__ __forceinline__ void pair_conv3(const uint8_t* inter, const uint8_t* s1t, const F3& f3, const BV3& bv3,
                                           int terms, const half4* rh, const half4* rl, bool ok, half_t* yp, int y_lo,
                                           float chi, int wave, int lane) {
    using namespace pair;
    const int l32 = lane & 31, lh = lane >> 5, ob = wave & 1, crow = wave >> 1;
    float16v a3;
#pragma unroll
    for (int e = 0; e < 16; ++e) a3[e] = 0.0f;
    const uint8_t* const b0 = inter + ((crow + 1) * IW + l32 + 1) * RBT + lh * 16;
    const uint8_t* const b1 = s1t + (crow * 32 + l32) * RBT + lh * 16;
#pragma unroll
    for (int st = 0; st < 6; ++st) {
        if (st >= terms * 2) break;
        const int term = st >> 1, half = st & 1;
        const int po = term == 1 ? 32 : 0;   // term 1 multiplies the lo halves
        const half8 bf = *reinterpret_cast<const half8*>((half ? b1 : b0) + po);
        a3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(f3(st), bf, a3, 0, 0, 0);
    }
    if (ok) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int oc = ob * 32 + g * 8 + lh * 4;
            half4 h, l;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float v = a3[g * 4 + e] + bv3(g * 4 + e);
                v += (float)rh[g][e];
                v += (float)rl[g][e];
                v = fmaxf(v, 0.0f);
                if (chi > 0.0f) v = fminf(v, chi);
                h[e] = (half_t)v;
                l[e] = (half_t)(v - (float)h[e]);
            }
            *reinterpret_cast<half4*>(yp + oc) = h;
            *reinterpret_cast<half4*>(yp + y_lo + oc) = l;
        }
    }
}

// conv3's weights (A fragments of K steps (term, half)) and bias for this
// wave's 32 output channels
__device__ __forceinline__ void pair_conv3_weights(const PairConv3& c3, half8* f3, float* bv3, int wave, int lane) {
    const int l32 = lane & 31, lh = lane >> 5, ob = wave & 1;
    const int icw = c3.terms * 32;
#pragma unroll
    for (int st = 0; st < 6; ++st)
        if (st < c3.terms * 2)
            f3[st] = *reinterpret_cast<const half8*>(c3.w + (size_t)(ob * 32 + l32) * icw + st * 16 + lh * 8);
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) bv3[g * 4 + e] = c3.b ? c3.b[ob * 32 + g * 8 + lh * 4 + e] : 0.0f;
}

template <bool C3>
__global__ __launch_bounds__(pair::NW * 64) void res2_pair_kernel(
    const half_t* __restrict__ x, int xs, half_t* __restrict__ y, int ys, const half_t* __restrict__ wa,
    const float* __restrict__ ba, const half_t* __restrict__ wb, const float* __restrict__ bb, float chi, int H,
    int W, int npix, int ntiles, int per_wg, PairConv3 c3) {
    using namespace pair;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[NS * STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t inter[INTER_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t s1t[C3 ? TH * 32 * RBT : 16];   // sp1 rows [hi 16 | lo 16]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t_begin = blockIdx.x * per_wg;
    const int t_end = t_begin + per_wg < ntiles ? t_begin + per_wg : ntiles;
    if (t_begin >= t_end) return;   // the whole workgroup: no barrier is pending

    // DMA slots of this lane (the same for every tile): halo pixel row r,
    // 16-byte slot cc of its 128 bytes [c0h c0l c1h c1l]
    int hofs[X_IPW], hpos[X_IPW];
#pragma unroll
    for (int i = 0; i < X_IPW; ++i) {
        const int p = (wave + i * NW) * 64 + lane;
        const int r = p / SPRX, cc = p - r * SPRX;
        const int hr = r / XW, hc = r - hr * XW;
        hofs[i] = ((hr * W + hc) * xs + cc * 8) * 2;
        hpos[i] = (r < XPIX && cc < 8) ? (hr << 8 | hc) : -1;
    }
    PairWalk k;
    k.hofs = hofs; k.hpos = hpos;
    k.xr = dma_rsrc(x, (uint32_t)(((size_t)(npix - 1) * xs + 64) * 2));
    k.H = H; k.W = W; k.xs2 = xs * 2;
    k.tiles_w = (W + TW - 1) / TW;
    k.tiles_h = (H + TH - 1) / TH;
    const int per_tile = (X_INS - wave + NW - 1) / NW;   // this wave's DMA instructions per tile

    {
        const PairDma d(ring, k, t_begin, wave, true);
#pragma unroll
        for (int j = 0; j < X_IPW; ++j) d.issue(j);
    }
    // A fragments: K = 32 is two 16-channel halves with the same weights
    const int orow = lane & 15, kg = lane >> 4, lp = lane & 15;
    half8 fa[9], fb[9];
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
        fa[tap] = *reinterpret_cast<const half8*>(wa + (orow * 9 + tap) * 16 + (kg & 1) * 8);
        fb[tap] = *reinterpret_cast<const half8*>(wb + (orow * 9 + tap) * 16 + (kg & 1) * 8);
    }
    float bva[4], bvb[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        bva[e] = ba ? ba[kg * 4 + e] : 0.0f;
        bvb[e] = bb ? bb[kg * 4 + e] : 0.0f;
    }
    const int l32 = lane & 31, lh = lane >> 5, ob = wave & 1, crow = wave >> 1;
    half8 f3[6];
    float bv3[16];
    if constexpr (C3) pair_conv3_weights(c3, f3, bv3, wave, lane);
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int s = 1; s + 1 < NS; ++s)
        if (t_begin + s < t_end) {
            const PairDma d(ring + s * STAGE, k, t_begin + s, wave, true);
#pragma unroll
            for (int j = 0; j < X_IPW; ++j) d.issue(j);
        }

    int slot = 0;
#pragma unroll 1
    for (int t = t_begin; t < t_end; ++t) {
        // tile t's halo has landed for every wave; tile t-1 is done with the
        // sp0 region and with its stage, which tile t+NS-1 takes over
        lds_barrier();
        const int prev = slot == 0 ? NS - 1 : slot - 1;
        const uint8_t* const st = ring + slot * STAGE;
        const PairDma nd(ring + prev * STAGE, k, t + NS - 1, wave, t + NS - 1 < t_end);
        const int th = t % k.tiles_h, rr = t / k.tiles_h, tw = rr % k.tiles_w, b = rr / k.tiles_w;
        const int oh0 = th * TH, ow0 = tw * TW;
        // conv3's residual for this wave's 32 outputs, loaded before the next
        // tiles' DMA goes out (a later load would wait for that DMA too)
        const int c3h = oh0 + crow, c3w = ow0 + l32;
        const bool ok = C3 && l32 < TW && c3h < H && c3w < W;
        const size_t P = (size_t)(b * H + (ok ? c3h : 0)) * W + (ok ? c3w : 0);
        half4 rh[4], rl[4];
        if constexpr (C3) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int oc = ob * 32 + g * 8 + lh * 4;
                rh[g] = *reinterpret_cast<const half4*>(c3.res + P * c3.rs + oc);
                rl[g] = *reinterpret_cast<const half4*>(c3.res + P * c3.rs + c3.r_lo + oc);
            }
        }

        pair_conv_a<!C3>(st, inter, fa, bva, chi, b, oh0, ow0, H, W, y, ys, wave, lane);
        lds_barrier();

        float4v cb[BPB];
        pair_conv_b(st, inter, fb, cb, wave, lane, [&](int s) {
            if (s % SP == 0 && s / SP < X_IPW) nd.issue(s / SP);
        });
        // tile t+1's loads have landed (this wave's): only tile t+2's may be in flight
        const int last = t + NS - 1 < t_end - 1 ? t + NS - 1 : t_end - 1;
        wait_vm_le(last > t + 1 ? (last - t - 1) * per_tile : 0);
        if constexpr (!C3) {
#pragma unroll
            for (int q = 0; q < BPB; ++q) {
                const int j = wave + q * NW;
                if (j >= NBB) continue;
                const int i = j >> 1, c = (j & 1) * 16 + lp;
                const int oh = oh0 + i, ow = ow0 + c;
                if (c >= TW || oh >= H || ow >= W) continue;
                half4 h, l;
                split_relu_clamp(cb[q], bvb, chi, h, l);
                half_t* const yp = y + ((size_t)(b * H + oh) * W + ow) * ys + 32 + kg * 4;
                *reinterpret_cast<half4*>(yp) = h;
                *reinterpret_cast<half4*>(yp + 16) = l;
            }
        } else {
            pair_sp1_to_lds(cb, bvb, chi, s1t, wave, lane);
            lds_barrier();
            pair_conv3(inter, s1t, [&](int st) { return f3[st]; }, [&](int i) { return bv3[i]; }, c3.terms, rh, rl, ok,
                       c3.y + P * c3.ys, c3.y_lo, chi, wave, lane);
        }
        slot = slot + 1 == NS ? 0 : slot + 1;
    }
}

// ---------------------------------------------------------------------------
// res2_bottleneck_kernel: a whole layer-1 block of ERes2Net
// (src/encoder_eres2net.cpp:111-137: conv1 -> Res2Net pair -> conv3 + shortcut)
// in one launch, split-f16 with f16-exact conv1 / conv_a / conv_b weights:
//   c = min(relu(conv1(x) + b1), clamp)            1x1, IC1 -> 32 = [c0 | c1]
//   sp0 = min(relu(conv_a(c0) + ba), clamp),  sp1 = min(relu(conv_b(sp0 + c1) + bb), clamp)
//   y = min(relu(conv3([sp0 | sp1]) + b3 + res), clamp)
// where res is x itself (64 input channels, no shortcut conv) or a given map
// (the block's shortcut output).  Per tile the x halo ((TH+4) x 34 pixels of
// [hi IC1 | lo IC1]) is DMA'd into LDS and conv1 runs over it into the
// [c0 | c1] halo (zero outside the image) with the LDS-DMA conv kernel's MFMA
// shape, K order (hi plane, then lo plane, 16 channels a step) and epilogue;
// conv_a, conv_b and conv3 then run as in res2_pair_kernel.  So y equals
// conv1 followed by vdk_res2_pair3x3_conv3 bit for bit, while HBM sees x read
// once and y written once: the chunks c0 / c1 never leave the chip.  The next
// tile's x halo is DMA'd while conv_a, conv_b and conv3 run.
// ---------------------------------------------------------------------------
namespace bott {
template <int IC1, int T1>
struct Geo {
    static constexpr int RB = IC1 * 4 + 16;                            // [hi IC1 | lo IC1] + 16 bytes of padding
    static constexpr int SPR = RB / 16;                                // 16-byte slots per row (the last is padding)
    static constexpr int INS = (pair::XPIX * SPR + 63) / 64;           // DMA instructions per x halo
    static constexpr int IPW = (INS + pair::NW - 1) / pair::NW;
    static constexpr int BYTES = INS * 1024;
    static constexpr int KP = IC1 / 16;                                // conv1 K steps of 16 per plane
    static constexpr int KS = T1 * KP;                                 // ... over the T1 terms
};
constexpr int NB1 = (pair::XPIX + 31) / 32;                            // conv1 blocks of 32 halo pixels
constexpr int CH_BYTES = pair::XPIX * pair::RBX;                       // the [c0 | c1] halo
}  // namespace bott

template <int IC1, int T1, bool RESX>
__global__ __launch_bounds__(pair::NW * 64) void res2_bottleneck_kernel(
    const half_t* __restrict__ x, int xs, int x_lo, const half_t* __restrict__ w1, const float* __restrict__ b1,
    const half_t* __restrict__ wa, const float* __restrict__ ba, const half_t* __restrict__ wb,
    const float* __restrict__ bb, float chi, int H, int W, int npix, int ntiles, int per_wg, PairConv3 c3) {
    using namespace pair;
    using G = bott::Geo<IC1, T1>;
    static_assert(!RESX || IC1 == 64, "x is the residual only when it has the block's 64 output channels");
    static_assert(G::BYTES + bott::CH_BYTES + INTER_BYTES + TH * 32 * RBT + 512 + 12288 <= 163840, "LDS");
    __shared__ __attribute__((aligned(1024))) uint8_t xh[G::BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t chalo[bott::CH_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t inter[INTER_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t s1t[TH * 32 * RBT];
    // biases (conv1 32, conv_a 16, conv_b 16, conv3 64) and conv3's A
    // fragments [ob][K step][lane] in LDS: the registers hold the conv1 /
    // conv_a / conv_b fragments and the phases' accumulators
    __shared__ __attribute__((aligned(16))) float sbias[128];
    __shared__ __attribute__((aligned(16))) half8 sf3[2 * 6 * 64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t_begin = blockIdx.x * per_wg;
    const int t_end = t_begin + per_wg < ntiles ? t_begin + per_wg : ntiles;
    if (t_begin >= t_end) return;   // the whole workgroup: no barrier is pending
    const int tiles_w = (W + TW - 1) / TW, tiles_h = (H + TH - 1) / TH;

    // x halo DMA slots of this lane (the same for every tile): halo pixel
    // (hr, hc) and 16-byte slot cc of its row, as hr << 16 | hc << 8 | cc,
    // -1 for the padding slots
    int slot[G::IPW];
#pragma unroll
    for (int i = 0; i < G::IPW; ++i) {
        const int p = (wave + i * NW) * 64 + lane;
        const int r = p / G::SPR, cc = p - r * G::SPR;
        const int hr = r / XW, hc = r - hr * XW;
        slot[i] = (r < XPIX && cc < G::SPR - 1) ? (hr << 16 | hc << 8 | cc) : -1;
    }
    const int4v xr = dma_rsrc(x, (uint32_t)(((size_t)(npix - 1) * xs + x_lo + IC1) * 2));
    auto issue_x = [&](int t) {
        const int th = t % tiles_h, rr = t / tiles_h, tw = rr % tiles_w, b = rr / tiles_w;
        const int ih0 = th * TH - 2, iw0 = tw * TW - 2;
#pragma unroll
        for (int i = 0; i < G::IPW; ++i) {
            const int ins = wave + i * NW;
            if (ins >= G::INS) break;   // wave-uniform
            const int sp = slot[i];
            const int ih = ih0 + (sp >> 16), iw = iw0 + ((sp >> 8) & 255), cc = sp & 255;
            const int ch = cc < IC1 / 8 ? cc * 8 : x_lo + (cc - IC1 / 8) * 8;
            const uint32_t off = (sp >= 0 && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W)
                                     ? (uint32_t)((((b * H + ih) * W + iw) * xs + ch) * 2) : kOOB;
            dma16(xh + ins * 1024, xr, off);
        }
    };
    issue_x(t_begin);

    // conv1: one 32-channel MFMA block, A fragments of its K steps over
    // x_hi . w_hi, x_lo . w_hi (, x_hi . w_lo) with the weights [hi | hi (| lo)]
    const int l32 = lane & 31, lh = lane >> 5, ob = wave & 1, crow = wave >> 1;
    half8 f1[G::KS];
#pragma unroll
    for (int s = 0; s < G::KS; ++s) f1[s] = *reinterpret_cast<const half8*>(w1 + l32 * (T1 * IC1) + s * 16 + lh * 8);
    if (tid < 128) {
        const float* const src = tid < 32 ? b1 : tid < 48 ? ba : tid < 64 ? bb : c3.b;
        const int i = tid < 32 ? tid : tid < 48 ? tid - 32 : tid < 64 ? tid - 48 : tid - 64;
        sbias[tid] = src ? src[i] : 0.0f;
    }
    if (wave < 2) {
        half8 f3[6];
        float unused[16];
        pair_conv3_weights(c3, f3, unused, wave, lane);
#pragma unroll
        for (int st = 0; st < 6; ++st) sf3[(wave * 6 + st) * 64 + lane] = f3[st];
    }
    // conv_a / conv_b: K = 32 is two 16-channel halves with the same weights
    const int orow = lane & 15, kg = lane >> 4;
    half8 fa[9], fb[9];
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
        fa[tap] = *reinterpret_cast<const half8*>(wa + (orow * 9 + tap) * 16 + (kg & 1) * 8);
        fb[tap] = *reinterpret_cast<const half8*>(wb + (orow * 9 + tap) * 16 + (kg & 1) * 8);
    }
    __builtin_amdgcn_s_waitcnt(0);   // weights, and this wave's share of the first x halo

#pragma unroll 1
    for (int t = t_begin; t < t_end; ++t) {
        // tile t's x halo has landed for every wave (each waited for its own
        // DMA); tile t-1 is done with the [c0 | c1] halo, sp0 and sp1
        lds_barrier();
        const int th = t % tiles_h, rr = t / tiles_h, tw = rr % tiles_w, b = rr / tiles_w;
        const int oh0 = th * TH, ow0 = tw * TW;
        const int c3h = oh0 + crow, c3w = ow0 + l32;
        const bool ok = l32 < TW && c3h < H && c3w < W;
        const size_t P = (size_t)(b * H + (ok ? c3h : 0)) * W + (ok ? c3w : 0);
        // conv3's residual for this wave's 32 outputs (channels ob*32 + g*8 + lh*4 ..)
        half4 rh[4], rl[4];
        if constexpr (RESX) {
            const uint8_t* const xp = xh + ((crow + 2) * XW + l32 + 2) * G::RB;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int oc = ob * 32 + g * 8 + lh * 4;
                rh[g] = *reinterpret_cast<const half4*>(xp + oc * 2);
                rl[g] = *reinterpret_cast<const half4*>(xp + IC1 * 2 + oc * 2);
            }
        } else {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int oc = ob * 32 + g * 8 + lh * 4;
                rh[g] = *reinterpret_cast<const half4*>(c3.res + P * c3.rs + oc);
                rl[g] = *reinterpret_cast<const half4*>(c3.res + P * c3.rs + c3.r_lo + oc);
            }
        }

        // conv1 over the halo: block j = halo pixels 32 j .. 32 j + 31 (the
        // halo's rows run on), lane column l32; the last block's spare
        // columns read the last pixel and are not stored
#pragma unroll 1
        for (int j = wave; j < bott::NB1; j += NW) {
            const int pp = j * 32 + l32;
            const int pr = pp < XPIX ? pp : XPIX - 1;
            const uint8_t* const bp = xh + pr * G::RB + lh * 16;
            // step s reads the hi plane, then the lo plane, then (3 terms) the hi plane again
            constexpr int PD = 4;
            auto bload = [&](int s) { return *reinterpret_cast<const half8*>(bp + (s % (2 * G::KP)) * 32); };
            half8 ring[PD];
#pragma unroll
            for (int s = 0; s < PD; ++s) ring[s] = bload(s);
            float16v acc;
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
#pragma unroll
            for (int s = 0; s < G::KS; ++s) {
                const half8 cur = ring[s % PD];
                if (s + PD < G::KS) ring[s % PD] = bload(s + PD);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(f1[s], cur, acc, 0, 0, 0);
            }
            if (pp < XPIX) {
                const int hr = pp / XW, hc = pp - hr * XW;
                const int gh = oh0 - 2 + hr, gw = ow0 - 2 + hc;
                const bool in = (unsigned)gh < (unsigned)H && (unsigned)gw < (unsigned)W;
                uint8_t* const cp = chalo + pp * RBX;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    // channels 8 g + 4 lh .. + 3: chunk g / 2, channel (g % 2) * 8 + 4 lh of the chunk
                    const float4v bq = *reinterpret_cast<const float4v*>(sbias + g * 8 + lh * 4);
                    const float bv[4] = {bq[0], bq[1], bq[2], bq[3]};
                    const float4v a4 = float4v{acc[g * 4], acc[g * 4 + 1], acc[g * 4 + 2], acc[g * 4 + 3]};
                    half4 h, l;
                    split_relu_clamp(a4, bv, chi, h, l);
                    if (!in) h = l = half4{0, 0, 0, 0};
                    uint8_t* const tp = cp + (g >> 1) * 64 + ((g & 1) * 8 + lh * 4) * 2;
                    *reinterpret_cast<half4*>(tp) = h;
                    *reinterpret_cast<half4*>(tp + 32) = l;
                }
            }
        }
        lds_barrier();   // the [c0 | c1] halo is complete; the x halo buffer is free
        if (t + 1 < t_end) issue_x(t + 1);

        {
            const float4v q = *reinterpret_cast<const float4v*>(sbias + 32 + kg * 4);
            const float bva[4] = {q[0], q[1], q[2], q[3]};
            pair_conv_a<false>(chalo, inter, fa, bva, chi, b, oh0, ow0, H, W, nullptr, 0, wave, lane);
        }
        lds_barrier();
        float4v cb[BPB];
        pair_conv_b(chalo, inter, fb, cb, wave, lane, [](int) {});
        {
            const float4v q = *reinterpret_cast<const float4v*>(sbias + 48 + kg * 4);
            const float bvb[4] = {q[0], q[1], q[2], q[3]};
            pair_sp1_to_lds(cb, bvb, chi, s1t, wave, lane);
        }
        // this wave's DMA of tile t+1's x halo has landed before the next barrier
        __builtin_amdgcn_s_waitcnt(0);
        lds_barrier();
        const half8* const f3l = sf3 + ob * 6 * 64 + lane;
        const float* const b3l = sbias + 64 + ob * 32 + lh * 4;
        pair_conv3(inter, s1t, [&](int st) { return f3l[st * 64]; }, [&](int i) { return b3l[(i >> 2) * 8 + (i & 3)]; },
                   c3.terms, rh, rl, ok, c3.y + P * c3.ys, c3.y_lo, chi, wave, lane);
    }
}

int cu_count() {
    static const int n = [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        return cus;
    }();
    return n;
}

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

extern "C" int vdk_res2_pair3x3(const void* d_x, int x_stride, void* d_y, int y_stride, int batch, int H, int W,
                                const void* d_wa, const float* d_ba, const void* d_wb, const float* d_bb,
                                float clamp_hi, void* stream) {
    return guarded([&] {
        require(d_x && d_y && d_wa && d_wb, "res2_pair3x3: NULL device pointer");
        require(batch > 0 && H > 0 && W > 0, "res2_pair3x3: empty map");
        require(x_stride >= 64 && y_stride >= 64 && x_stride % 8 == 0 && y_stride % 8 == 0,
                "res2_pair3x3: pixel strides must hold the two 32-element groups and be multiples of 8");
        require(al16(d_x) && al16(d_y) && al16(d_wa) && al16(d_wb) && al16(d_ba) && al16(d_bb),
                "res2_pair3x3: device pointers must be 16-byte aligned");
        const long npix = (long)batch * H * W;
        require(npix * x_stride * 2 < (1L << 31) && npix * y_stride < (1L << 31) && W < 8192,
                "res2_pair3x3: map too large for one launch");
        const int ntiles = batch * cdiv(H, pair::TH) * cdiv(W, pair::TW);
        const int per = cdiv(ntiles, cu_count());
        hipLaunchKernelGGL(res2_pair_kernel<false>, dim3(cdiv(ntiles, per)), dim3(pair::NW * 64), 0,
                           static_cast<hipStream_t>(stream), static_cast<const half_t*>(d_x), x_stride,
                           static_cast<half_t*>(d_y), y_stride, static_cast<const half_t*>(d_wa), d_ba,
                           static_cast<const half_t*>(d_wb), d_bb, clamp_hi, H, W, (int)npix, ntiles, per,
                           PairConv3{});
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_res2_pair3x3_conv3(const void* d_x, int x_stride, int batch, int H, int W, const void* d_wa,
                                      const float* d_ba, const void* d_wb, const float* d_bb, const void* d_w3,
                                      const float* d_b3, int terms3, const void* d_res, int res_stride, int res_lo,
                                      void* d_y, int y_stride, int y_lo, float clamp_hi, void* stream) {
    return guarded([&] {
        require(d_x && d_wa && d_wb && d_w3 && d_res && d_y, "res2_pair3x3_conv3: NULL device pointer");
        require(batch > 0 && H > 0 && W > 0, "res2_pair3x3_conv3: empty map");
        require(terms3 == 2 || terms3 == 3, "res2_pair3x3_conv3: conv3 weights have 2 or 3 terms");
        require(x_stride >= 64 && x_stride % 8 == 0 && res_stride >= 64 && res_stride % 4 == 0 && res_lo >= 64 &&
                    res_lo % 4 == 0 && y_stride >= 64 && y_stride % 4 == 0 && y_lo >= 64 && y_lo % 4 == 0,
                "res2_pair3x3_conv3: strides / lo offsets must hold the 64 channels and keep 8-byte alignment");
        require(al16(d_x) && al16(d_wa) && al16(d_wb) && al16(d_w3) && al16(d_ba) && al16(d_bb) && al16(d_b3) &&
                    (reinterpret_cast<uintptr_t>(d_res) & 7) == 0 && (reinterpret_cast<uintptr_t>(d_y) & 7) == 0,
                "res2_pair3x3_conv3: x / weights / biases 16-byte, residual / y 8-byte aligned");
        const long npix = (long)batch * H * W;
        require(npix * x_stride * 2 < (1L << 31) && W < 8192, "res2_pair3x3_conv3: map too large for one launch");
        const int ntiles = batch * cdiv(H, pair::TH) * cdiv(W, pair::TW);
        const int per = cdiv(ntiles, cu_count());
        PairConv3 c3{static_cast<const half_t*>(d_w3), d_b3, terms3, static_cast<const half_t*>(d_res), res_stride,
                     res_lo, static_cast<half_t*>(d_y), y_stride, y_lo};
        hipLaunchKernelGGL(res2_pair_kernel<true>, dim3(cdiv(ntiles, per)), dim3(pair::NW * 64), 0,
                           static_cast<hipStream_t>(stream), static_cast<const half_t*>(d_x), x_stride, nullptr, 0,
                           static_cast<const half_t*>(d_wa), d_ba, static_cast<const half_t*>(d_wb), d_bb, clamp_hi,
                           H, W, (int)npix, ntiles, per, c3);
        VDK_HIP(hipGetLastError());
    });
}

extern "C" int vdk_res2_bottleneck(const void* d_x, int x_stride, int x_lo, int ic1, int batch, int H, int W,
                                   const void* d_w1, int terms1, const float* d_b1, const void* d_wa, const float* d_ba,
                                   const void* d_wb, const float* d_bb, const void* d_w3, const float* d_b3,
                                   int terms3, const void* d_res, int res_stride, int res_lo, void* d_y, int y_stride,
                                   int y_lo, float clamp_hi, void* stream) {
    return guarded([&] {
        require(d_x && d_w1 && d_wa && d_wb && d_w3 && d_y, "res2_bottleneck: NULL device pointer");
        require(batch > 0 && H > 0 && W > 0, "res2_bottleneck: empty map");
        require(ic1 == 32 || ic1 == 64, "res2_bottleneck: conv1 takes 32 or 64 input channels");
        require(d_res || ic1 == 64, "res2_bottleneck: x is the residual only with 64 channels");
        require((terms1 == 2 || terms1 == 3) && (terms3 == 2 || terms3 == 3),
                "res2_bottleneck: conv1 / conv3 weights have 2 or 3 terms");
        if (!d_res) {
            d_res = d_x;
            res_stride = x_stride;
            res_lo = x_lo;
        }
        require(x_stride % 8 == 0 && x_lo % 8 == 0 && x_lo >= ic1 && x_stride >= x_lo + ic1,
                "res2_bottleneck: x rows are [hi | lo] planes of the input channels, 8-element aligned");
        require(res_stride >= 64 && res_stride % 4 == 0 && res_lo >= 64 && res_lo % 4 == 0 && y_stride >= 64 &&
                    y_stride % 4 == 0 && y_lo >= 64 && y_lo % 4 == 0,
                "res2_bottleneck: residual / y strides and lo offsets must hold the 64 channels, 8-byte aligned");
        require(al16(d_x) && al16(d_w1) && al16(d_wa) && al16(d_wb) && al16(d_w3) && al16(d_b1) && al16(d_ba) &&
                    al16(d_bb) && al16(d_b3) && (reinterpret_cast<uintptr_t>(d_res) & 7) == 0 &&
                    (reinterpret_cast<uintptr_t>(d_y) & 7) == 0,
                "res2_bottleneck: x / weights / biases 16-byte, residual / y 8-byte aligned");
        const long npix = (long)batch * H * W;
        require(npix * x_stride * 2 < (1L << 31) && W < 200 * 1024, "res2_bottleneck: map too large for one launch");
        const uintptr_t xa = reinterpret_cast<uintptr_t>(d_x), ya = reinterpret_cast<uintptr_t>(d_y);
        const uintptr_t xb = (uintptr_t)(npix * x_stride * 2), yb = (uintptr_t)(npix * y_stride * 2);
        require(xa + xb <= ya || ya + yb <= xa, "res2_bottleneck: y must not overlap x (other tiles read its halo)");
        const int ntiles = batch * cdiv(H, pair::TH) * cdiv(W, pair::TW);
        const int per = cdiv(ntiles, cu_count());
        const PairConv3 c3{static_cast<const half_t*>(d_w3), d_b3, terms3, static_cast<const half_t*>(d_res),
                           res_stride, res_lo, static_cast<half_t*>(d_y), y_stride, y_lo};
        const bool resx = d_res == d_x;
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(cdiv(ntiles, per)), dim3(pair::NW * 64), 0, static_cast<hipStream_t>(stream),
                               static_cast<const half_t*>(d_x), x_stride, x_lo, static_cast<const half_t*>(d_w1), d_b1,
                               static_cast<const half_t*>(d_wa), d_ba, static_cast<const half_t*>(d_wb), d_bb,
                               clamp_hi, H, W, (int)npix, ntiles, per, c3);
        };
        if (ic1 == 64 && resx) terms1 == 2 ? go(res2_bottleneck_kernel<64, 2, true>) : go(res2_bottleneck_kernel<64, 3, true>);
        else if (ic1 == 64) terms1 == 2 ? go(res2_bottleneck_kernel<64, 2, false>) : go(res2_bottleneck_kernel<64, 3, false>);
        else terms1 == 2 ? go(res2_bottleneck_kernel<32, 2, false>) : go(res2_bottleneck_kernel<32, 3, false>);
        VDK_HIP(hipGetLastError());
    });
}

// fbank.hip - Kaldi FBank front end on gfx950.
//
// Follows vd::FBank::compute (src/fbank.cpp:121-205): snip_edges framing,
// per-frame DC removal, pre-emphasis with replicate padding, povey window,
// zero-pad to n_fft, power spectrum, triangular mel filters, log with a
// FLT_EPSILON floor, then per-utterance CMN.  The arithmetic keeps the
// reference's precision split: framing steps in f32, window product, FFT, mel
// sums and log in f64 (MI355X runs f64 at full vector rate, and f64 keeps the
// log of low-energy mel bins within 1e-4 of the reference).
//
// Layout: one wavefront per frame, several frames per wavefront in turn (the
// next frame's samples in flight during the current one), 4 wavefronts per
// workgroup; the 512-point FFT is register resident (radix 8, two LDS
// exchanges) and transforms two frames at once (one as the real, one as the
// imaginary part; their spectra separated through the mirror bins).  A workgroup's log-mel values collect in an LDS tile and leave
// as runs of consecutive frames per mel row, and the workgroups of a clip run
// on one XCD, so each output line is written once through one L2.  CMN: the
// frames pass also writes each workgroup's per-mel sums, a small kernel adds
// them into the per-clip means, and either a coalesced pass subtracts them or
// the consumer of the features does as it loads them.
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstring>
#include <vector>

#include "common.hpp"
#include "vdk.h"

namespace vdk {
namespace {

constexpr int kFbMaxWaves = 4;   // frames (wavefronts) per workgroup at n_fft <= 512
constexpr double kPi = 3.14159265358979323846;

struct FbankDev {
    // byte offsets of the tables inside the table block (copied to LDS)
    int off_window, off_tw_re, off_tw_im, off_mel_start, off_mel_len, off_mel_off, off_mel_w, off_mel_lane;
    int mel_q;              // mels per lane in the mel_lane table (512-point path)
    int n_mels, n_fft, log2n, pow2, win, hop, T, n_samples;
    int waves;              // frames processed concurrently per workgroup (one per wavefront)
    float preemph;
};

// Output side of the frames kernels.  CMN sums are fixed point (value * 2^36
// rounded to a 64-bit integer), so they are exact whatever the grouping of
// frames into workgroups (which changes with the batch size).
constexpr double kCmnScale = 68719476736.0;   // 2^36
struct FbankOut {
    float* feats;               // [B][n_mels][T] log-mel energies (before CMN)
    long long* part;            // [B][gc][n_mels] per-workgroup CMN sums, or NULL
    int gc;                     // workgroups per clip
};

struct TableLayout {
    size_t window, tw_re, tw_im, mel_start, mel_len, mel_off, mel_lane, mel_w, total;
    int nnz;
};

constexpr int kMelQ = 8;   // at most this many mels per lane in the mel_lane table

// The mel bins of the 512-point path split over the 64 lanes of a wavefront
// by filter length (longest first, each to the lane with the least work so
// far), so no lane runs far more filter taps than the others: table
// [kMelQ][64] of mel indices, -1 past a lane's list; returns the longest list.
int mel_lanes(const std::vector<int>& len, std::vector<int>& lane_tab) {
    const int n = (int)len.size();
    std::vector<int> order(n), load(64, 0), count(64, 0);
    for (int m = 0; m < n; ++m) order[m] = m;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return len[a] > len[b]; });
    lane_tab.assign(kMelQ * 64, -1);
    int q = 0;
    for (int m : order) {
        int best = 0;
        for (int l = 1; l < 64; ++l)
            if (load[l] + count[l] < load[best] + count[best]) best = l;   // + 1 per mel: its log and store
        require(count[best] < kMelQ, "fbank: too many mel bins for the 512-point path");
        lane_tab[count[best] * 64 + best] = m;
        load[best] += len[m];
        ++count[best];
        q = count[best] > q ? count[best] : q;
    }
    return q;
}

double mel_scale(double f) { return 1127.0 * std::log(1.0 + f / 700.0); }

// Host copy of the triangular filters (src/fbank.cpp:137-158) in sparse form.
void mel_sparse(const vdk_fbank_cfg& c, std::vector<int>& start, std::vector<int>& len,
                std::vector<int>& off, std::vector<double>& w) {
    const int half = c.n_fft / 2;
    const double lo = c.low_freq;
    const double hi = c.high_freq > 0.0f ? (double)c.high_freq : c.sample_rate / 2.0;
    const double mlo = mel_scale(lo), mhi = mel_scale(hi);
    const double step = (mhi - mlo) / (c.n_mels + 1);
    start.assign(c.n_mels, 0);
    len.assign(c.n_mels, 0);
    off.assign(c.n_mels, 0);
    w.clear();
    for (int m = 0; m < c.n_mels; ++m) {
        const double l = mlo + m * step, ce = mlo + (m + 1) * step, r = mlo + (m + 2) * step;
        int first = -1, last = -1;
        std::vector<double> row(half + 1, 0.0);
        for (int k = 0; k <= half; ++k) {
            const double mf = mel_scale((double)k * c.sample_rate / c.n_fft);
            double v = 0.0;
            if (mf > l && mf <= ce) v = (mf - l) / (ce - l);
            else if (mf > ce && mf < r) v = (r - mf) / (r - ce);
            row[k] = v;
            if (v != 0.0) {
                if (first < 0) first = k;
                last = k;
            }
        }
        off[m] = (int)w.size();
        if (first >= 0) {
            start[m] = first;
            len[m] = last - first + 1;
            for (int k = first; k <= last; ++k) w.push_back(row[k]);
        }
    }
}

TableLayout layout(const vdk_fbank_cfg& c, int nnz) {
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    TableLayout t{};
    size_t o = 0;
    t.window = o;    o = al(o + sizeof(double) * c.win_length);
    t.tw_re = o;     o = al(o + sizeof(double) * (c.n_fft / 2 + 1));
    t.tw_im = o;     o = al(o + sizeof(double) * (c.n_fft / 2 + 1));
    t.mel_start = o; o = al(o + sizeof(int) * c.n_mels);
    t.mel_len = o;   o = al(o + sizeof(int) * c.n_mels);
    t.mel_off = o;   o = al(o + sizeof(int) * c.n_mels);
    t.mel_lane = o;  o = al(o + sizeof(int) * kMelQ * 64);
    t.mel_w = o;     o = al(o + sizeof(double) * (nnz > 0 ? nnz : 1));
    t.total = o;
    t.nnz = nnz;
    return t;
}

void check_cfg(const vdk_fbank_cfg* c) {
    require(c != nullptr, "fbank: cfg is NULL");
    require(c->win_length > 0 && c->hop_length > 0 && c->n_mels > 0 && c->sample_rate > 0,
            "fbank: invalid window/hop/mel configuration");
    require(c->n_fft >= c->win_length, "fbank: n_fft must be >= win_length");
    require(c->n_fft <= 1024, "fbank: n_fft above 1024 is not supported");
}

__device__ __forceinline__ double wave_sum(double v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Wavefront-scope LDS ordering: one wave owns one frame, so the FFT stages
// need no workgroup barrier, only program order on the LDS accesses.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One workgroup copies the constant tables (window, twiddles, packed mel
// filters; `tab_bytes` from the host layout) into LDS once, then each of its
// wavefronts processes `fpw` consecutive frames.
__global__ __launch_bounds__(kFbMaxWaves * 64) void fbank_frames_kernel(FbankDev p, const uint8_t* __restrict__ tables,
                                                                     int tab_bytes, int fpw,
                                                                     const float* __restrict__ pcm,
                                                                     float* __restrict__ feats) {
#pragma clang fp contract(off)
    extern __shared__ double smem[];
    uint8_t* tab = reinterpret_cast<uint8_t*>(smem);
    for (int i = threadIdx.x * 16; i < tab_bytes; i += blockDim.x * 16)
        *reinterpret_cast<uint4*>(tab + i) = *reinterpret_cast<const uint4*>(tables + i);
    __syncthreads();
    const double* window = reinterpret_cast<const double*>(tab + p.off_window);
    const double* tw_re = reinterpret_cast<const double*>(tab + p.off_tw_re);
    const double* tw_im = reinterpret_cast<const double*>(tab + p.off_tw_im);
    const int* mel_start = reinterpret_cast<const int*>(tab + p.off_mel_start);
    const int* mel_len = reinterpret_cast<const int*>(tab + p.off_mel_len);
    const int* mel_off = reinterpret_cast<const int*>(tab + p.off_mel_off);
    const double* mel_w = reinterpret_cast<const double*>(tab + p.off_mel_w);

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = blockIdx.y;
    const int nfft = p.n_fft, half = nfft >> 1;
    double* re = smem + tab_bytes / 8 + (size_t)wave * (2 * nfft + nfft / 2);
    double* im = re + nfft;
    float* raw = reinterpret_cast<float*>(im + nfft);

    for (int f = 0; f < fpw; ++f) {
        const int t = (blockIdx.x * p.waves + wave) * fpw + f;
        if (t >= p.T) break;                       // uniform per wavefront
        const float* src = pcm + (size_t)b * p.n_samples + (size_t)t * p.hop;
        // remove_dc_offset: double sum of the frame (src/fbank.cpp:170-174)
        double s = 0.0;
        for (int i = lane; i < p.win; i += 64) s += (double)src[i];
        s = wave_sum(s);
        const float mean = (float)(s / p.win);
        for (int i = lane; i < p.win; i += 64) raw[i] = src[i] - mean;
        wave_sync();
        // pre-emphasis with replicate padding, window in double, zero pad, and
        // the bit-reversed placement of the FFT input (src/fbank.cpp:176-183)
        for (int i = lane; i < nfft; i += 64) {
            float v = 0.0f;
            if (i < p.win) {
                const float cur = raw[i];
                const float prev = raw[i > 0 ? i - 1 : 0];
                const float y = cur - p.preemph * prev;
                v = (float)((double)y * window[i]);
            }
            const int j = p.pow2 ? (int)(__builtin_bitreverse32((unsigned)i) >> (32 - p.log2n)) : i;
            re[j] = (double)v;
            im[j] = 0.0;
        }
        wave_sync();
        if (p.pow2) {
            // iterative radix-2 decimation in time; a stage's butterflies are independent
            for (int lg = 1; lg <= p.log2n; ++lg) {
                const int h = 1 << (lg - 1);
                const int tws = nfft >> lg;            // twiddle stride n_fft / len
                for (int q = lane; q < half; q += 64) {
                    const int pos = q & (h - 1);
                    const int a = ((q >> (lg - 1)) << lg) + pos, c = a + h;
                    const double wr = tw_re[pos * tws], wi = tw_im[pos * tws];
                    const double xr = wr * re[c] - wi * im[c];
                    const double xi = wr * im[c] + wi * re[c];
                    const double ar = re[a], ai = im[a];
                    re[c] = ar - xr;
                    im[c] = ai - xi;
                    re[a] = ar + xr;
                    im[a] = ai + xi;
                }
                wave_sync();
            }
            for (int k = lane; k <= half; k += 64) {
                const double r = re[k], i2 = im[k];
                im[k] = r * r + i2 * i2;                 // power spectrum into im[]
            }
        } else {
            // naive DFT for non power-of-two sizes (src/fbank.cpp:97-107)
            for (int k = lane; k <= half; k += 64) {
                double r = 0.0, i2 = 0.0;
                for (int n = 0; n < nfft; ++n) {
                    const double a = -2.0 * kPi * k * n / nfft;
                    r += re[n] * cos(a);
                    i2 += re[n] * sin(a);
                }
                im[k] = r * r + i2 * i2;
            }
        }
        wave_sync();
        const double* ps = im;
        for (int m = lane; m < p.n_mels; m += 64) {
            double e = 0.0;
            const int st = mel_start[m], n = mel_len[m];
            const double* w = mel_w + mel_off[m];
            for (int k = 0; k < n; ++k) e += w[k] * ps[st + k];
            const double fl = (double)FLT_EPSILON;
            feats[((size_t)b * p.n_mels + m) * p.T + t] = (float)log(e > fl ? e : fl);
        }
        wave_sync();
    }
}

// ---------------------------------------------------------------------------
// 512-point path (the size every speaker encoder uses): a register-resident
// radix-8 FFT.  With n = a + 64 b and k = c + 8 d (a in [0,64), b, c in [0,8)):
//   X[c + 8 d] = sum_a W64^(a d) * W512^(a c) * sum_b x[a + 64 b] W8^(b c)
// and the 64-point DFT over a = a0 + 8 a1, d = d0 + 8 d1 splits the same way.
// Lane a does the first 8-point DFT on its 8 samples; two LDS exchanges
// (rows padded so each 16-lane group of a ds_*_b128 hits distinct banks) hand
// the next 8-point DFTs to lane (c, a0) and then lane (c, d0), which ends up
// holding X[c + 8 d0 + 64 d1] for d1 = 0..7.
// ---------------------------------------------------------------------------
struct cplx {
    double r, i;
};

__device__ __forceinline__ cplx cmul(cplx a, cplx b) { return {a.r * b.r - a.i * b.i, a.r * b.i + a.i * b.r}; }

// In-place 8-point DFT, natural order in and out: X[k] = sum_n x[n] W8^(n k).
__device__ __forceinline__ void dft8(cplx* x) {
    const double h = 0.70710678118654752440;   // sqrt(2)/2
    // radix-2 DIT on bit-reversed input order
    cplx v[8] = {x[0], x[4], x[2], x[6], x[1], x[5], x[3], x[7]};
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        const cplx a = v[j], b = v[j + 1];
        v[j] = {a.r + b.r, a.i + b.i};
        v[j + 1] = {a.r - b.r, a.i - b.i};
    }
#pragma unroll
    for (int j = 0; j < 8; j += 4) {
        const cplx a0 = v[j], b0 = v[j + 2];
        v[j] = {a0.r + b0.r, a0.i + b0.i};
        v[j + 2] = {a0.r - b0.r, a0.i - b0.i};
        const cplx a1 = v[j + 1], b1 = {v[j + 3].i, -v[j + 3].r};   // * W4^1 = -i
        v[j + 1] = {a1.r + b1.r, a1.i + b1.i};
        v[j + 3] = {a1.r - b1.r, a1.i - b1.i};
    }
    const cplx w1 = {h, -h}, w3 = {-h, -h};
    const cplx t0 = v[4], t1 = cmul(v[5], w1), t2 = {v[6].i, -v[6].r}, t3 = cmul(v[7], w3);
    x[0] = {v[0].r + t0.r, v[0].i + t0.i};
    x[4] = {v[0].r - t0.r, v[0].i - t0.i};
    x[1] = {v[1].r + t1.r, v[1].i + t1.i};
    x[5] = {v[1].r - t1.r, v[1].i - t1.i};
    x[2] = {v[2].r + t2.r, v[2].i + t2.i};
    x[6] = {v[2].r - t2.r, v[2].i - t2.i};
    x[3] = {v[3].r + t3.r, v[3].i + t3.i};
    x[7] = {v[3].r - t3.r, v[3].i - t3.i};
}

// The exchanges move the real parts through a per-wave buffer of doubles,
// then the imaginary parts through the same buffer (half the LDS of a complex
// buffer, so more workgroups fit on a CU).  Rows of 72 doubles keep each
// half-wave of a ds_*_b64 on distinct banks for all three access patterns.
constexpr int kX1 = 72;   // exchange-1 row stride (doubles): row c, column a
constexpr int kX2 = 9;    // exchange-2: index c * 72 + d0 * 9 + a0

// CMN sums of one workgroup's frames: per mel, the fixed-point sum of its
// log values (`tile` [nf][pitch]) into part[b][g][m].
__device__ __forceinline__ void cmn_part(const FbankOut& o, const float* tile, int pitch, int nf, int n_mels, int b,
                                         int g) {
    for (int m = threadIdx.x; m < n_mels; m += blockDim.x) {
        long long s = 0;
        for (int lf = 0; lf < nf; ++lf) s += __double2ll_rn((double)tile[lf * pitch + m] * kCmnScale);
        o.part[((size_t)b * o.gc + g) * n_mels + m] = s;
    }
}

// The workgroup's tile [nf][pitch] out to feats rows: consecutive threads
// write consecutive frames of one mel row.
__device__ __forceinline__ void store_tile(float* feats, const float* tile, int pitch, int nf, int F, int n_mels,
                                           int T, int b, int t0) {
    for (int i = threadIdx.x; i < n_mels * F; i += blockDim.x) {
        const int m = i / F, lf = i - m * F;
        if (lf < nf) feats[((size_t)b * n_mels + m) * T + t0 + lf] = tile[lf * pitch + m];
    }
}

// The window and the twiddles are per-lane constants, read once from the
// table block into registers; only the mel tables (from off_mel_start on) are
// copied to LDS, which leaves room for three workgroups per CU.
__global__ __launch_bounds__(kFbMaxWaves * 64) void fbank512_kernel(FbankDev p, const uint8_t* __restrict__ tables,
                                                                   int tab_bytes, int fpw,
                                                                   const float* __restrict__ pcm, FbankOut o) {
#pragma clang fp contract(off)
    extern __shared__ double smem[];
    uint8_t* tab = reinterpret_cast<uint8_t*>(smem);
    const int mel0 = p.off_mel_start, mel_bytes = tab_bytes - mel0;   // both multiples of 256
    for (int i = threadIdx.x * 16; i < mel_bytes; i += blockDim.x * 16)
        *reinterpret_cast<uint4*>(tab + i) = *reinterpret_cast<const uint4*>(tables + mel0 + i);
    __syncthreads();
    const double* window = reinterpret_cast<const double*>(tables + p.off_window);
    const double* tw_re = reinterpret_cast<const double*>(tables + p.off_tw_re);   // cos(-2 pi j / 512)
    const double* tw_im = reinterpret_cast<const double*>(tables + p.off_tw_im);
    const int* mel_start = reinterpret_cast<const int*>(tab + p.off_mel_start - mel0);
    const int* mel_len = reinterpret_cast<const int*>(tab + p.off_mel_len - mel0);
    const int* mel_off = reinterpret_cast<const int*>(tab + p.off_mel_off - mel0);
    const int* mel_lane = reinterpret_cast<const int*>(tab + p.off_mel_lane - mel0);
    const double* mel_w = reinterpret_cast<const double*>(tab + p.off_mel_w - mel0);

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int F = p.waves * fpw;                   // frames per workgroup
    const int lid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int b = lid / o.gc, g = lid - b * o.gc, t0 = g * F;
    cplx* const xbase = reinterpret_cast<cplx*>(smem + mel_bytes / 8);
    cplx* const tw1 = xbase;                       // [c][lane]: W512^(lane c)
    cplx* const tw2 = xbase + 8 * 64;              // [c][a0]: W64^(a0 c) = W512^(8 a0 c)
    double* const xall = reinterpret_cast<double*>(xbase + 8 * 64 + 8 * 8);
    double* xch = xall + (size_t)wave * (8 * kX1);
    double* ps = xch;                              // reused after the last exchange (257 bins)
    const int pitch = p.n_mels + 1;                // odd pitch: the row-wise tile reads hit distinct banks
    float* tile = reinterpret_cast<float*>(xall + (size_t)p.waves * (8 * kX1));   // [F][pitch]

    // the twiddles, constant over frames, in LDS (in registers they would
    // take 64 VGPRs and a wave per SIMD): W512^(a c) for lane a and
    // W64^(a0 d0) = W512^(8 a0 d0) for lane (c, a0) = (lane / 8, lane % 8)
    auto w512 = [&](int j) {
        return cplx{j < 256 ? tw_re[j] : -tw_re[j - 256], j < 256 ? tw_im[j] : -tw_im[j - 256]};
    };
    for (int i = threadIdx.x; i < 8 * 64 + 8 * 8; i += blockDim.x) {
        if (i < 8 * 64) tw1[i] = w512(((i & 63) * (i >> 6)) & 511);
        else tw2[i - 8 * 64] = w512((8 * ((i - 8 * 64) & 7) * ((i - 8 * 64) >> 3)) & 511);
    }
    __syncthreads();
    const int a0 = lane & 7, cl = lane >> 3;

    double win[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) win[j] = lane + 64 * j < p.win ? window[lane + 64 * j] : 0.0;
    // samples n = lane + 64 j of frame t (zero past the window)
    auto load = [&](int t, float* xs) {
        const float* src = pcm + (size_t)b * p.n_samples + (size_t)t * p.hop;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int n = lane + 64 * j;
            xs[j] = n < p.win ? src[n] : 0.0f;
        }
    };
    const int tw0 = t0 + wave * fpw;               // this wave's frames: tw0 .. tw0 + fpw - 1
    // Frames go through the FFT in pairs: frame t as the real part and frame
    // t + 1 as the imaginary part of one complex 512-point input z, so
    // Z = A + iB with A, B the frames' spectra, and with m = (512 - k) mod 512
    //   A[k] = (Z[k] + conj Z[m]) / 2,   B[k] = (Z[k] - conj Z[m]) / 2i
    // (A and B are Hermitian): one FFT per two frames.  A pair past the
    // wave's last frame (or the clip's) runs with B = 0 and drops its output.
    // DC removal, pre-emphasis and window of one frame's samples
    // (src/fbank.cpp:170-183): y[j] for sample n = lane + 64 j
    auto prep = [&](const float* xs, double* y) {
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < 8; ++j) s += (double)xs[j];
        s = wave_sum(s);
        const float mean = (float)(s / p.win);
        // sample n - 1 is lane - 1's value, or lane 63's of the previous j
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int n = lane + 64 * j;
            const float up = __shfl(xs[j], (lane + 63) & 63);
            const float wrap =
                j > 0 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(xs[j > 0 ? j - 1 : 0]), 63)) : xs[0];
            const float prev_raw = lane > 0 ? up : wrap;
            y[j] = 0.0;
            if (n < p.win) {
                const float cur = xs[j] - mean;
                const float prev = prev_raw - mean;
                const float e = cur - p.preemph * prev;
                y[j] = (double)(float)((double)e * win[j]);
            }
        }
    };
    const int tend = tw0 + fpw < p.T ? tw0 + fpw : p.T;   // this wave's frames end here
    float xa[8], xb[8];
    if (tw0 < tend) load(tw0, xa);
    if (tw0 + 1 < tend) load(tw0 + 1, xb);
    for (int t = tw0; t < tend; t += 2) {          // uniform per wavefront
        const bool two = t + 1 < tend;
        float na[8], nb[8];                        // the next pair's samples, in flight meanwhile
        if (t + 2 < tend) load(t + 2, na);
        if (t + 3 < tend) load(t + 3, nb);
        double ya[8], yb[8];
        prep(xa, ya);
        if (two) {
            prep(xb, yb);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) yb[j] = 0.0;
        }
        cplx v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = {ya[j], yb[j]};
        // pass 1: 8-point DFT over b, twiddle W512^(a c); store row c, column a
        dft8(v);
#pragma unroll
        for (int c = 0; c < 8; ++c) v[c] = cmul(v[c], tw1[c * 64 + lane]);
        // pass 2: lane (c, a0) gathers a = a0 + 8 a1, DFT over a1 -> d0, twiddle W64^(a0 d0)
        {
            cplx u[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) xch[c * kX1 + lane] = v[c].r;
            wave_sync();
#pragma unroll
            for (int a1 = 0; a1 < 8; ++a1) u[a1].r = xch[cl * kX1 + a0 + 8 * a1];
            wave_sync();
#pragma unroll
            for (int c = 0; c < 8; ++c) xch[c * kX1 + lane] = v[c].i;
            wave_sync();
#pragma unroll
            for (int a1 = 0; a1 < 8; ++a1) u[a1].i = xch[cl * kX1 + a0 + 8 * a1];
            wave_sync();
#pragma unroll
            for (int a1 = 0; a1 < 8; ++a1) v[a1] = u[a1];
        }
        dft8(v);
#pragma unroll
        for (int d0 = 0; d0 < 8; ++d0) v[d0] = cmul(v[d0], tw2[d0 * 8 + a0]);
        // pass 3: lane (c, d0) gathers a0, DFT over a0 -> d1: Z[c + 8 d0 + 64 d1]
        const int d0 = a0;
        {
            cplx u[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) xch[cl * kX1 + k * kX2 + a0] = v[k].r;
            wave_sync();
#pragma unroll
            for (int q = 0; q < 8; ++q) u[q].r = xch[cl * kX1 + d0 * kX2 + q];
            wave_sync();
#pragma unroll
            for (int k = 0; k < 8; ++k) xch[cl * kX1 + k * kX2 + a0] = v[k].i;
            wave_sync();
#pragma unroll
            for (int q = 0; q < 8; ++q) u[q].i = xch[cl * kX1 + d0 * kX2 + q];
            wave_sync();
#pragma unroll
            for (int q = 0; q < 8; ++q) v[q] = u[q];
        }
        dft8(v);
        // Z in natural order through the buffer (real parts, then imaginary
        // parts), each lane reading bins k = lane + 64 j (j < 4, and 256 for
        // lane 0) and their mirrors m = 512 - k; then the two power spectra
        // |A[k]|^2 = ((Zr_k + Zr_m)^2 + (Zi_k - Zi_m)^2) / 4 and
        // |B[k]|^2 = ((Zi_k + Zi_m)^2 + (Zr_k - Zr_m)^2) / 4 for k <= 256.
        double zr[5], zrm[5], zi[5], zim[5];
        auto zidx = [](int k) { return k + (k >> 6); };   // rows of 64 padded by one: lanes of a write spread over banks
#pragma unroll
        for (int d1 = 0; d1 < 8; ++d1) xch[zidx(cl + 8 * d0 + 64 * d1)] = v[d1].r;
        wave_sync();
#pragma unroll
        for (int j = 0; j < 5; ++j) {
            const int k = j < 4 ? lane + 64 * j : 256;
            zr[j] = xch[zidx(k)];
            zrm[j] = xch[zidx((512 - k) & 511)];
        }
        wave_sync();
#pragma unroll
        for (int d1 = 0; d1 < 8; ++d1) xch[zidx(cl + 8 * d0 + 64 * d1)] = v[d1].i;
        wave_sync();
#pragma unroll
        for (int j = 0; j < 5; ++j) {
            const int k = j < 4 ? lane + 64 * j : 256;
            zi[j] = xch[zidx(k)];
            zim[j] = xch[zidx((512 - k) & 511)];
        }
        wave_sync();
        double* const psa = ps;                    // [257]
        double* const psb = ps + 288;              // [257]
#pragma unroll
        for (int j = 0; j < 5; ++j) {
            const int k = j < 4 ? lane + 64 * j : 256;
            if (j < 4 || lane == 0) {
                const double ar = 0.5 * (zr[j] + zrm[j]), ai = 0.5 * (zi[j] - zim[j]);
                const double br = 0.5 * (zi[j] + zim[j]), bi = 0.5 * (zr[j] - zrm[j]);
                psa[k] = ar * ar + ai * ai;
                psb[k] = br * br + bi * bi;
            }
        }
        wave_sync();
        // mel sums in the reference's order (src/fbank.cpp:187-191), each lane
        // over its mels from the length-balanced table; the log of the f64
        // energy rounded to f32 (v_log_f32, within a few f32 ulps of the f64
        // log rounded to f32)
        float* trow = tile + (t - t0) * pitch;
        for (int q = 0; q < p.mel_q; ++q) {
            const int m = mel_lane[q * 64 + lane];
            if (m < 0) continue;
            double ea = 0.0, eb = 0.0;
            const int st = mel_start[m], n = mel_len[m];
            const double* w = mel_w + mel_off[m];
            for (int k = 0; k < n; ++k) {
                const double wk = w[k];
                ea += wk * psa[st + k];
                eb += wk * psb[st + k];
            }
            const double fl = (double)FLT_EPSILON;
            constexpr float kLn2 = 0.693147180559945309f;
            trow[m] = __builtin_amdgcn_logf((float)(ea > fl ? ea : fl)) * kLn2;
            if (two) trow[pitch + m] = __builtin_amdgcn_logf((float)(eb > fl ? eb : fl)) * kLn2;
        }
        wave_sync();
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            xa[j] = na[j];
            xb[j] = nb[j];
        }
    }
    __syncthreads();
    const int nf = p.T - t0 < F ? p.T - t0 : F;
    store_tile(o.feats, tile, pitch, nf, F, p.n_mels, p.T, b, t0);
    if (o.part) cmn_part(o, tile, pitch, nf, p.n_mels, b, g);
}

// CMN means of the generic path's features (src/fbank.cpp:194-201): one
// workgroup per (mel bin, clip), a double tree reduction over time; the mean
// goes to `mean` (may be NULL) and, with `apply`, is subtracted in place.
__global__ __launch_bounds__(256) void fbank_cmn_kernel(float* __restrict__ feats, int n_mels, int T,
                                                        float* __restrict__ mean, int apply) {
    __shared__ double part[4];
    float* row = feats + ((size_t)blockIdx.y * n_mels + blockIdx.x) * T;
    double s = 0.0;
    for (int t = threadIdx.x; t < T; t += 256) s += (double)row[t];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    const double tot = part[0] + part[1] + part[2] + part[3];
    const float mu = (float)(tot / T);
    if (mean && threadIdx.x == 0) mean[(size_t)blockIdx.y * n_mels + blockIdx.x] = mu;
    if (apply)
        for (int t = threadIdx.x; t < T; t += 256) row[t] = row[t] - mu;
}

// CMN means from the frames pass's per-workgroup sums: 16 lanes per (clip,
// mel) row, each adding every 16th workgroup's sum, then a butterfly over the
// 16 lanes (integer sums: exact in any order), then / 2^36 / T.
__global__ __launch_bounds__(256) void fbank_mean_kernel(const long long* __restrict__ part, int gc, int n_mels,
                                                         int rows, int T, float* __restrict__ mean) {
    const int i = blockIdx.x * 16 + (threadIdx.x >> 4), l = threadIdx.x & 15;
    long long s = 0;
    if (i < rows) {
        const int b = i / n_mels, m = i - b * n_mels;
        const long long* p = part + (size_t)b * gc * n_mels + m;
        for (int g = l; g < gc; g += 16) s += p[(size_t)g * n_mels];
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 16);
    if (i < rows && l == 0) mean[i] = (float)((double)s / kCmnScale / T);
}

// feats[b][m][t] -= mean[b][m]: the CMN subtraction (f32) over the whole map.
__global__ __launch_bounds__(256) void fbank_sub_mean_kernel(float* __restrict__ feats, const float* __restrict__ mean,
                                                             long n, int T) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    feats[i] = feats[i] - mean[i / T];
}

}  // namespace
}  // namespace vdk

using namespace vdk;

extern "C" size_t vdk_fbank_tables_size(const vdk_fbank_cfg* cfg) {
    try {
        check_cfg(cfg);
        std::vector<int> st, ln, of;
        std::vector<double> w;
        mel_sparse(*cfg, st, ln, of, w);
        return layout(*cfg, (int)w.size()).total;
    } catch (const std::exception& e) {
        set_error(e.what());
        return 0;
    }
}

extern "C" int vdk_fbank_tables_fill(const vdk_fbank_cfg* cfg, void* d_tables) {
    return guarded([&] {
        check_cfg(cfg);
        require(d_tables != nullptr, "fbank: tables pointer is NULL");
        const vdk_fbank_cfg& c = *cfg;
        std::vector<int> st, ln, of;
        std::vector<double> w;
        mel_sparse(c, st, ln, of, w);
        const TableLayout L = layout(c, (int)w.size());
        std::vector<uint8_t> host(L.total, 0);
        double* win = reinterpret_cast<double*>(host.data() + L.window);
        for (int i = 0; i < c.win_length; ++i)   // povey window (src/fbank.cpp:132-135)
            win[i] = std::pow(0.5 - 0.5 * std::cos(2.0 * kPi * i / (c.win_length - 1)), 0.85);
        double* twr = reinterpret_cast<double*>(host.data() + L.tw_re);
        double* twi = reinterpret_cast<double*>(host.data() + L.tw_im);
        for (int j = 0; j < c.n_fft / 2; ++j) {
            const double a = -2.0 * kPi * j / c.n_fft;
            twr[j] = std::cos(a);
            twi[j] = std::sin(a);
        }
        std::memcpy(host.data() + L.mel_start, st.data(), sizeof(int) * c.n_mels);
        std::memcpy(host.data() + L.mel_len, ln.data(), sizeof(int) * c.n_mels);
        std::memcpy(host.data() + L.mel_off, of.data(), sizeof(int) * c.n_mels);
        if (c.n_mels <= kMelQ * 64) {
            std::vector<int> lanes;
            mel_lanes(ln, lanes);
            std::memcpy(host.data() + L.mel_lane, lanes.data(), sizeof(int) * lanes.size());
        }
        if (!w.empty()) std::memcpy(host.data() + L.mel_w, w.data(), sizeof(double) * w.size());
        VDK_HIP(hipMemcpy(d_tables, host.data(), L.total, hipMemcpyHostToDevice));
    });
}

namespace {

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

int fbank_frames(const vdk_fbank_cfg& c, int n_samples) { return 1 + (n_samples - c.win_length) / c.hop_length; }

// CMN workspace: per-workgroup sums [B][ceil(T/4)][n_mels] (workgroups hold at
// least 4 frames) and the means [B][n_mels] when the caller takes none.
size_t work_bytes(const vdk_fbank_cfg& c, int batch, int n_samples) {
    const int T = n_samples >= c.win_length ? fbank_frames(c, n_samples) : 1;
    return al256(8 * (size_t)batch * cdiv(T, 4) * c.n_mels) + al256(4 * (size_t)batch * c.n_mels);
}

void fbank_run(const vdk_fbank_cfg* cfg, const void* d_tables, const float* d_pcm, int batch, int n_samples,
               float* d_feats, float* d_mean, void* d_work, size_t work_size, hipStream_t s) {
    check_cfg(cfg);
    require(d_tables && d_pcm && d_feats, "fbank: NULL device pointer");
    require(batch > 0, "fbank: batch must be positive");
    require(n_samples >= cfg->win_length, "voicedetect: FBank produced no frames");
    const vdk_fbank_cfg& c = *cfg;
    require(!c.cmn || (d_work && work_size >= work_bytes(c, batch, n_samples) &&
                       (reinterpret_cast<uintptr_t>(d_work) & 255) == 0),
            "fbank: CMN needs a 256-byte aligned workspace of vdk_fbank_workspace_size bytes");
    std::vector<int> st, ln, of;
    std::vector<double> w;
    mel_sparse(c, st, ln, of, w);
    const TableLayout L = layout(c, (int)w.size());
    FbankDev p;
    p.off_window = (int)L.window;
    p.off_tw_re = (int)L.tw_re;
    p.off_tw_im = (int)L.tw_im;
    p.off_mel_start = (int)L.mel_start;
    p.off_mel_len = (int)L.mel_len;
    p.off_mel_off = (int)L.mel_off;
    p.off_mel_w = (int)L.mel_w;
    p.off_mel_lane = (int)L.mel_lane;
    p.mel_q = 0;
    p.n_mels = c.n_mels;
    p.n_fft = c.n_fft;
    p.pow2 = (c.n_fft & (c.n_fft - 1)) == 0;
    p.log2n = 0;
    while ((1 << p.log2n) < c.n_fft) ++p.log2n;
    p.win = c.win_length;
    p.hop = c.hop_length;
    p.T = 1 + (n_samples - c.win_length) / c.hop_length;
    p.n_samples = n_samples;
    p.preemph = c.preemph;
    p.waves = c.n_fft <= 512 ? kFbMaxWaves : 2;
    const bool radix8 = c.n_fft == 512 && c.win_length <= 512 && c.n_mels <= kMelQ * 64;
    if (radix8) {
        std::vector<int> lanes;
        p.mel_q = mel_lanes(ln, lanes);
    }
    // frames per wavefront: enough to amortise the table copy, while
    // keeping >= ~4 workgroups per CU at batch 64
    int fpw = p.T >= 256 ? 4 : (p.T >= 64 ? 2 : 1);
    // the 512-point path transforms frames in pairs (2j, 2j + 1) of the clip:
    // an even count per wavefront keeps every pair in one wavefront, so a
    // frame's bits never depend on the batch
    const int min_fpw = radix8 ? 2 : 1;
    fpw = fpw < min_fpw ? min_fpw : fpw;
    // small batches: fewer frames per wavefront until the launch covers
    // the CUs (each frame's arithmetic is the same whatever the grouping)
    while (fpw > min_fpw && (long)batch * cdiv(p.T, p.waves * fpw) < 256) fpw /= 2;
    const int gc = cdiv(p.T, p.waves * fpw);
    const size_t per_wave = radix8 ? (size_t)8 * kX1 * sizeof(double)
                                   : (size_t)(2 * c.n_fft + c.n_fft / 2) * sizeof(double);
    const size_t tile = radix8 ? (size_t)p.waves * fpw * (c.n_mels + 1) * sizeof(float) : 0;
    const size_t twid = radix8 ? (size_t)(8 * 64 + 8 * 8) * sizeof(cplx) : 0;
    const size_t shmem = (radix8 ? L.total - L.mel_start : L.total) + twid + (size_t)p.waves * per_wave + tile;
    require(shmem <= 160 * 1024, "fbank: configuration needs more LDS than a workgroup has");
    long long* const part = c.cmn ? static_cast<long long*>(d_work) : nullptr;
    float* const mean = d_mean ? d_mean
                               : (c.cmn ? reinterpret_cast<float*>(static_cast<uint8_t*>(d_work) +
                                                                   al256(8 * (size_t)batch * cdiv(p.T, 4) * c.n_mels))
                                        : nullptr);
    if (radix8) {
        if (shmem > 64 * 1024)
            VDK_HIP(hipFuncSetAttribute((const void*)fbank512_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)shmem));
        FbankOut o{d_feats, part, gc};
        hipLaunchKernelGGL(fbank512_kernel, dim3(batch * gc), dim3(p.waves * 64), shmem, s, p,
                           static_cast<const uint8_t*>(d_tables), (int)L.total, fpw, d_pcm, o);
        VDK_HIP(hipGetLastError());
        if (c.cmn) {
            const int rows = batch * c.n_mels;
            hipLaunchKernelGGL(fbank_mean_kernel, dim3(cdiv(rows, 16)), dim3(256), 0, s, part, gc, c.n_mels, rows,
                               p.T, mean);
            VDK_HIP(hipGetLastError());
        }
        if (c.cmn && !d_mean) {   // the means subtracted here, in place
            const long n = (long)batch * c.n_mels * p.T;
            hipLaunchKernelGGL(fbank_sub_mean_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, d_feats, mean, n, p.T);
            VDK_HIP(hipGetLastError());
        }
    } else {
        dim3 grid(gc, batch);
        if (shmem > 64 * 1024)
            VDK_HIP(hipFuncSetAttribute((const void*)fbank_frames_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)shmem));
        hipLaunchKernelGGL(fbank_frames_kernel, grid, dim3(p.waves * 64), shmem, s, p,
                           static_cast<const uint8_t*>(d_tables), (int)L.total, fpw, d_pcm, d_feats);
        VDK_HIP(hipGetLastError());
        if (c.cmn) {
            hipLaunchKernelGGL(fbank_cmn_kernel, dim3(c.n_mels, batch), dim3(256), 0, s, d_feats, c.n_mels, p.T,
                               d_mean, d_mean ? 0 : 1);
            VDK_HIP(hipGetLastError());
        }
    }
}

}  // namespace

extern "C" size_t vdk_fbank_workspace_size(const vdk_fbank_cfg* cfg, int batch, int n_samples) {
    if (!cfg || batch <= 0 || n_samples <= 0) {
        set_error("fbank: bad workspace query");
        return 0;
    }
    return cfg->cmn ? work_bytes(*cfg, batch, n_samples) : 0;
}

extern "C" int vdk_fbank_ex(const vdk_fbank_cfg* cfg, const void* d_tables, const float* d_pcm, int batch,
                            int n_samples, float* d_feats, float* d_mean, void* d_work, size_t work_size,
                            void* stream) {
    return guarded([&] {
        fbank_run(cfg, d_tables, d_pcm, batch, n_samples, d_feats, d_mean, d_work, work_size,
                  static_cast<hipStream_t>(stream));
    });
}

extern "C" int vdk_fbank(const vdk_fbank_cfg* cfg, const void* d_tables, const float* d_pcm,
                         int batch, int n_samples, float* d_feats, void* stream) {
    return guarded([&] {
        require(cfg != nullptr && batch > 0, "fbank: cfg is NULL or batch not positive");
        hipStream_t s = static_cast<hipStream_t>(stream);
        void* work = nullptr;
        const size_t bytes = cfg->cmn && n_samples >= cfg->win_length ? work_bytes(*cfg, batch, n_samples) : 0;
        if (bytes) VDK_HIP(hipMallocAsync(&work, bytes, s));
        try {
            fbank_run(cfg, d_tables, d_pcm, batch, n_samples, d_feats, nullptr, work, bytes, s);
        } catch (...) {
            if (work) (void)hipFreeAsync(work, s);
            throw;
        }
        if (work) VDK_HIP(hipFreeAsync(work, s));
    });
}

extern "C" int vdk_fbank_sub_mean(float* d_feats, const float* d_mean, int batch, int n_mels, int T, void* stream) {
    return guarded([&] {
        require(d_feats && d_mean && batch > 0 && n_mels > 0 && T > 0, "fbank_sub_mean: bad arguments");
        const long n = (long)batch * n_mels * T;
        hipLaunchKernelGGL(fbank_sub_mean_kernel, dim3(cdiv(n, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                           d_feats, d_mean, n, T);
        VDK_HIP(hipGetLastError());
    });
}

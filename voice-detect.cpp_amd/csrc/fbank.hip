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
// Layout: one wavefront per frame (4 frames per 256-thread workgroup), the
// frame's complex spectrum in LDS (2 x n_fft doubles), radix-2 butterflies
// spread over the 64 lanes; a second kernel does CMN with one workgroup per
// (clip, mel bin) and a double-precision tree reduction over time.
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
    const double* window;   // [win]
    const double* tw_re;    // [n_fft/2]  cos(-2 pi j / n_fft)
    const double* tw_im;    // [n_fft/2]  sin(-2 pi j / n_fft)
    const int* mel_start;   // [n_mels] first non-zero bin
    const int* mel_len;     // [n_mels] number of non-zero bins
    const int* mel_off;     // [n_mels] offset into mel_w
    const double* mel_w;    // packed non-zero filter weights
    int n_mels, n_fft, log2n, pow2, win, hop, T, n_samples;
    int waves;              // frames per workgroup (LDS stays <= 40 KB)
    float preemph;
};

struct TableLayout {
    size_t window, tw_re, tw_im, mel_start, mel_len, mel_off, mel_w, total;
    int nnz;
};

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

__global__ __launch_bounds__(kFbMaxWaves * 64) void fbank_frames_kernel(FbankDev p, const float* __restrict__ pcm,
                                                                     float* __restrict__ feats) {
#pragma clang fp contract(off)
    extern __shared__ double smem[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = blockIdx.x * p.waves + wave;
    const int b = blockIdx.y;
    const bool valid = t < p.T;
    const int nfft = p.n_fft;
    double* re = smem + (size_t)wave * 2 * nfft;
    double* im = re + nfft;
    float* raw = reinterpret_cast<float*>(smem + (size_t)p.waves * 2 * nfft) + (size_t)wave * nfft;

    const float* src = pcm + (size_t)b * p.n_samples + (size_t)(valid ? t : 0) * p.hop;
    // remove_dc_offset: double sum of the frame (src/fbank.cpp:170-174)
    double s = 0.0;
    if (valid)
        for (int i = lane; i < p.win; i += 64) s += (double)src[i];
    s = wave_sum(s);
    const float mean = (float)(s / p.win);
    for (int i = lane; i < p.win; i += 64) raw[i] = valid ? src[i] - mean : 0.0f;
    __syncthreads();
    // pre-emphasis with replicate padding, window in double, zero pad, and the
    // bit-reversed placement of the FFT input (src/fbank.cpp:176-183)
    for (int i = lane; i < nfft; i += 64) {
        float v = 0.0f;
        if (i < p.win) {
            const float cur = raw[i];
            const float prev = raw[i > 0 ? i - 1 : 0];
            const float y = cur - p.preemph * prev;
            v = (float)((double)y * p.window[i]);
        }
        const int j = p.pow2 ? (int)(__builtin_bitreverse32((unsigned)i) >> (32 - p.log2n)) : i;
        re[j] = (double)v;
        im[j] = 0.0;
    }
    __syncthreads();
    const int half = nfft >> 1;
    if (p.pow2) {
        // iterative radix-2 decimation in time; every butterfly of a stage is independent
        for (int lg = 1; lg <= p.log2n; ++lg) {
            const int h = 1 << (lg - 1);
            const int tws = nfft >> lg;            // twiddle stride n_fft / len
            for (int q = lane; q < half; q += 64) {
                const int pos = q & (h - 1);
                const int a = ((q >> (lg - 1)) << lg) + pos, c = a + h;
                const double wr = p.tw_re[pos * tws], wi = p.tw_im[pos * tws];
                const double xr = wr * re[c] - wi * im[c];
                const double xi = wr * im[c] + wi * re[c];
                re[c] = re[a] - xr;
                im[c] = im[a] - xi;
                re[a] = re[a] + xr;
                im[a] = im[a] + xi;
            }
            __syncthreads();
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
    __syncthreads();
    const double* ps = im;
    for (int m = lane; m < p.n_mels; m += 64) {
        double e = 0.0;
        const int st = p.mel_start[m], n = p.mel_len[m];
        const double* w = p.mel_w + p.mel_off[m];
        for (int k = 0; k < n; ++k) e += w[k] * ps[st + k];
        const double fl = (double)FLT_EPSILON;
        if (valid) feats[((size_t)b * p.n_mels + m) * p.T + t] = (float)log(e > fl ? e : fl);
    }
}

// Per-utterance CMN (src/fbank.cpp:194-201): one workgroup per (mel bin, clip).
__global__ __launch_bounds__(256) void fbank_cmn_kernel(float* __restrict__ feats, int n_mels, int T) {
    __shared__ double part[4];
    float* row = feats + ((size_t)blockIdx.y * n_mels + blockIdx.x) * T;
    double s = 0.0;
    for (int t = threadIdx.x; t < T; t += 256) s += (double)row[t];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    const double tot = part[0] + part[1] + part[2] + part[3];
    const float mu = (float)(tot / T);
    for (int t = threadIdx.x; t < T; t += 256) row[t] = row[t] - mu;
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
        if (!w.empty()) std::memcpy(host.data() + L.mel_w, w.data(), sizeof(double) * w.size());
        VDK_HIP(hipMemcpy(d_tables, host.data(), L.total, hipMemcpyHostToDevice));
    });
}

extern "C" int vdk_fbank(const vdk_fbank_cfg* cfg, const void* d_tables, const float* d_pcm,
                         int batch, int n_samples, float* d_feats, void* stream) {
    return guarded([&] {
        check_cfg(cfg);
        require(d_tables && d_pcm && d_feats, "fbank: NULL device pointer");
        require(batch > 0, "fbank: batch must be positive");
        require(n_samples >= cfg->win_length, "voicedetect: FBank produced no frames");
        const vdk_fbank_cfg& c = *cfg;
        std::vector<int> st, ln, of;
        std::vector<double> w;
        mel_sparse(c, st, ln, of, w);
        const TableLayout L = layout(c, (int)w.size());
        const uint8_t* base = static_cast<const uint8_t*>(d_tables);
        FbankDev p;
        p.window = reinterpret_cast<const double*>(base + L.window);
        p.tw_re = reinterpret_cast<const double*>(base + L.tw_re);
        p.tw_im = reinterpret_cast<const double*>(base + L.tw_im);
        p.mel_start = reinterpret_cast<const int*>(base + L.mel_start);
        p.mel_len = reinterpret_cast<const int*>(base + L.mel_len);
        p.mel_off = reinterpret_cast<const int*>(base + L.mel_off);
        p.mel_w = reinterpret_cast<const double*>(base + L.mel_w);
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
        const size_t shmem = (size_t)p.waves * (2 * c.n_fft * sizeof(double) + c.n_fft * sizeof(float));
        hipStream_t s = static_cast<hipStream_t>(stream);
        dim3 grid(cdiv(p.T, p.waves), batch);
        hipLaunchKernelGGL(fbank_frames_kernel, grid, dim3(p.waves * 64), shmem, s, p, d_pcm, d_feats);
        VDK_HIP(hipGetLastError());
        if (c.cmn) {
            hipLaunchKernelGGL(fbank_cmn_kernel, dim3(c.n_mels, batch), dim3(256), 0, s, d_feats, c.n_mels, p.T);
            VDK_HIP(hipGetLastError());
        }
    });
}

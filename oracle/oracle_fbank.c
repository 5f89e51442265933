/*
 * oracle_fbank.c - CPU restatement of the reference Kaldi FBank front end.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Built with -ffp-contract=off so
 * the float framing steps round exactly like separate multiply/subtract.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>

static const double kPi = 3.14159265358979323846;

/* ------------------------------------------------------------------ FBank */

int orc_fbank_frames(int n_samples, const orc_fbank_cfg* c) {
    /* src/fbank.cpp:127-130: snip_edges drops the trailing partial frame. */
    if (c->win_length <= 0 || c->hop_length <= 0 || n_samples < c->win_length) return 0;
    return 1 + (n_samples - c->win_length) / c->hop_length;
}

void orc_povey_window(int win, double* w) {
    /* src/fbank.cpp:132-135: (0.5 - 0.5 cos(2 pi i / (N-1)))^0.85 */
    for (int i = 0; i < win; ++i)
        w[i] = pow(0.5 - 0.5 * cos(2.0 * kPi * i / (win - 1)), 0.85);
}

static double mel_of(double f) { return 1127.0 * log(1.0 + f / 700.0); }

void orc_mel_filters(const orc_fbank_cfg* c, double* fb) {
    /* src/fbank.cpp:137-158: triangles equally spaced on the mel scale over
     * [low, high], n_mels + 2 edge points; the Nyquist bin gets zero weight. */
    const int half = c->n_fft / 2;
    const double lo = c->low_freq;
    const double hi = c->high_freq > 0.0f ? (double)c->high_freq : c->sample_rate / 2.0;
    const double mlo = mel_of(lo), mhi = mel_of(hi);
    const double step = (mhi - mlo) / (c->n_mels + 1);
    for (int m = 0; m < c->n_mels; ++m) {
        const double left = mlo + m * step, centre = mlo + (m + 1) * step, right = mlo + (m + 2) * step;
        for (int k = 0; k <= half; ++k) {
            const double mf = mel_of((double)k * c->sample_rate / c->n_fft);
            double v = 0.0;
            if (mf > left && mf <= centre) v = (mf - left) / (centre - left);
            else if (mf > centre && mf < right) v = (right - mf) / (right - centre);
            fb[(size_t)m * (half + 1) + k] = v;
        }
    }
}

/* In-place iterative radix-2 decimation-in-time FFT of length n (power of 2). */
static void fft_radix2(double* re, double* im, int n) {
    for (int i = 1, j = 0; i < n; ++i) {          /* bit-reversal permutation */
        int bit = n >> 1;
        for (; j & bit; bit >>= 1) j ^= bit;
        j |= bit;
        if (i < j) {
            double t = re[i]; re[i] = re[j]; re[j] = t;
            t = im[i]; im[i] = im[j]; im[j] = t;
        }
    }
    for (int len = 2; len <= n; len <<= 1) {
        const int h = len >> 1;
        for (int j = 0; j < h; ++j) {
            const double a = -2.0 * kPi * j / len;
            const double wr = cos(a), wi = sin(a);
            for (int s = j; s < n; s += len) {
                const double xr = wr * re[s + h] - wi * im[s + h];
                const double xi = wr * im[s + h] + wi * re[s + h];
                re[s + h] = re[s] - xr; im[s + h] = im[s] - xi;
                re[s] += xr;            im[s] += xi;
            }
        }
    }
}

void orc_powspec(const float* frame, int frame_len, int n_fft, int use_dft, double* out) {
    /* src/fbank.cpp:92-118: |X_k|^2 for k = 0..n_fft/2 of the zero-padded frame;
     * radix-2 FFT for power-of-two sizes, the naive DFT otherwise. */
    const int half = n_fft / 2;
    const int pow2 = n_fft > 0 && (n_fft & (n_fft - 1)) == 0;
    if (use_dft || !pow2) {
        for (int k = 0; k <= half; ++k) {
            double r = 0.0, i = 0.0;
            for (int t = 0; t < frame_len && t < n_fft; ++t) {
                const double a = -2.0 * kPi * k * t / n_fft;
                r += frame[t] * cos(a);
                i += frame[t] * sin(a);
            }
            out[k] = r * r + i * i;
        }
        return;
    }
    double* re = calloc((size_t)n_fft, sizeof(double));
    double* im = calloc((size_t)n_fft, sizeof(double));
    for (int t = 0; t < frame_len && t < n_fft; ++t) re[t] = frame[t];
    fft_radix2(re, im, n_fft);
    for (int k = 0; k <= half; ++k) out[k] = re[k] * re[k] + im[k] * im[k];
    free(re);
    free(im);
}

int orc_fbank(const float* pcm, int n_samples, const orc_fbank_cfg* c, float* out) {
    /* src/fbank.cpp:121-205 */
    const int win = c->win_length, hop = c->hop_length, nfft = c->n_fft, nmel = c->n_mels;
    if (win <= 0 || hop <= 0 || nfft < win || nmel <= 0) return 0;
    const int T = orc_fbank_frames(n_samples, c);
    if (T <= 0) return 0;
    const int half = nfft / 2;
    double* window = malloc(sizeof(double) * win);
    double* fb = malloc(sizeof(double) * (size_t)nmel * (half + 1));
    float* raw = malloc(sizeof(float) * win);
    float* frame = malloc(sizeof(float) * nfft);
    double* ps = malloc(sizeof(double) * (half + 1));
    orc_povey_window(win, window);
    orc_mel_filters(c, fb);
    const double floor_e = FLT_EPSILON;
    for (int t = 0; t < T; ++t) {
        const float* src = pcm + (size_t)t * hop;
        double mean = 0.0;                                   /* remove_dc_offset (double sum) */
        for (int i = 0; i < win; ++i) mean += src[i];
        mean /= win;
        for (int i = 0; i < win; ++i) raw[i] = src[i] - (float)mean;
        for (int i = win - 1; i > 0; --i) raw[i] -= c->preemph * raw[i - 1];  /* pre-emphasis */
        raw[0] -= c->preemph * raw[0];                        /* replicate pad at i = 0 */
        for (int i = 0; i < nfft; ++i)                        /* window in double, store f32 */
            frame[i] = i < win ? (float)(raw[i] * window[i]) : 0.0f;
        orc_powspec(frame, nfft, nfft, 0, ps);
        for (int m = 0; m < nmel; ++m) {
            double e = 0.0;
            const double* row = fb + (size_t)m * (half + 1);
            for (int k = 0; k <= half; ++k) e += row[k] * ps[k];
            out[(size_t)m * T + t] = (float)log(e > floor_e ? e : floor_e);
        }
    }
    if (c->cmn) {                                            /* per-utterance CMN */
        for (int m = 0; m < nmel; ++m) {
            double s = 0.0;
            for (int t = 0; t < T; ++t) s += out[(size_t)m * T + t];
            const float mu = (float)(s / T);
            for (int t = 0; t < T; ++t) out[(size_t)m * T + t] -= mu;
        }
    }
    free(window); free(fb); free(raw); free(frame); free(ps);
    return T;
}


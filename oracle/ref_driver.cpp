// ref_driver.cpp - C entry points around the reference's own FBank and WAV
// loader, compiled from the reference sources where they lie (see Makefile,
// target `ref`) into oracle/_ref/.  TEST INFRASTRUCTURE ONLY: used to write the
// golden FBank vectors under tests/golden/ and to pin the oracle's FBank and
// this repository's WAV reader against the reference implementation.
//
// Binds: vd::FBank::compute (src/fbank.cpp:121-205),
//        vd::load_audio_16k_mono (src/audio_io.cpp:25-38),
//        vd::resample_linear (src/audio_io.cpp:9-23).
#include "audio_io.hpp"
#include "fbank.hpp"

#include <cstring>
#include <vector>

extern "C" {

// Returns T (frames) and writes feat-major [n_mels][T] into out (capacity in
// floats); returns -1 if out is too small.
int ref_fbank(const float* pcm, int n_samples, int n_mels, int n_fft, int win, int hop,
              float preemph, float low_freq, float high_freq, int cmn,
              float* out, long cap) {
    vd::VoiceDetectConfig cfg;
    cfg.n_mels = (uint32_t)n_mels;
    cfg.n_fft = (uint32_t)n_fft;
    cfg.win_length = (uint32_t)win;
    cfg.hop_length = (uint32_t)hop;
    cfg.preemph = preemph;
    cfg.fbank_low_freq = low_freq;
    cfg.fbank_high_freq = high_freq;
    cfg.fbank_cmn = cmn != 0;
    std::vector<float> x(pcm, pcm + n_samples);
    int T = 0;
    std::vector<float> f = vd::FBank(cfg).compute(x, T);
    if ((long)f.size() > cap) return -1;
    if (!f.empty()) std::memcpy(out, f.data(), f.size() * sizeof(float));
    return T;
}

// Decode + downmix + resample a WAV to 16 kHz mono.  Returns the sample count
// (copies at most cap samples), or -1 on failure.
long ref_load_wav(const char* path, float* out, long cap) {
    vd::Audio a;
    if (!vd::load_audio_16k_mono(path, a)) return -1;
    long n = (long)a.samples.size();
    std::memcpy(out, a.samples.data(), (size_t)(n < cap ? n : cap) * sizeof(float));
    return n;
}

long ref_resample(const float* in, long n, int in_sr, int out_sr, float* out, long cap) {
    std::vector<float> x(in, in + n);
    std::vector<float> y = vd::resample_linear(x, in_sr, out_sr);
    long m = (long)y.size();
    std::memcpy(out, y.data(), (size_t)(m < cap ? m : cap) * sizeof(float));
    return m;
}

}  // extern "C"

// audio.cpp - WAV decode, downmix and linear resampling on the host.
//
// Behaviour of vd::load_audio_16k_mono / vd::resample_linear
// (src/audio_io.cpp:9-38): decode any PCM/float WAV to f32 with dr_wav's
// integer scalings (u8: x/127.5 - 1 as x*(2/255) - 1, s16: x/32768,
// s24: x/8388608, s32: x/2147483648), average the channels in double, then
// linearly resample to 16 kHz.  Written from the RIFF/WAVE format description.
#include "audio.hpp"

#include <cmath>
#include <cstring>
#include <fstream>

#include "common.hpp"
#include "vdk.h"

namespace vdk {

std::vector<float> resample_linear(const std::vector<float>& in, int in_sr, int out_sr) {
    if (in_sr == out_sr || in.empty()) return in;
    require(in_sr > 0 && out_sr > 0, "voicedetect: invalid sample rate");
    const double ratio = (double)out_sr / (double)in_sr;
    const size_t n_out = (size_t)std::floor(in.size() * ratio);
    std::vector<float> out(n_out);
    for (size_t i = 0; i < n_out; ++i) {
        const double src = i / ratio;
        const size_t i0 = (size_t)src;
        const double frac = src - (double)i0;
        const float a = in[i0];
        const float b = i0 + 1 < in.size() ? in[i0 + 1] : a;
        out[i] = (float)(a + (b - a) * frac);
    }
    return out;
}

namespace {

uint32_t rd32(const uint8_t* p) { uint32_t v; std::memcpy(&v, p, 4); return v; }
uint16_t rd16(const uint8_t* p) { uint16_t v; std::memcpy(&v, p, 2); return v; }

}  // namespace

bool load_wav_mono(const std::string& path, std::vector<float>& mono, int& sample_rate) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    std::vector<uint8_t> b((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    if (b.size() < 12 || std::memcmp(b.data(), "RIFF", 4) || std::memcmp(b.data() + 8, "WAVE", 4)) return false;
    uint16_t fmt = 0, ch = 0, bits = 0;
    uint32_t sr = 0;
    const uint8_t* data = nullptr;
    size_t data_len = 0;
    size_t pos = 12;
    while (pos + 8 <= b.size()) {
        const uint8_t* c = b.data() + pos;
        const uint32_t len = rd32(c + 4);
        const size_t body = pos + 8;
        const size_t avail = b.size() - body;
        if (!std::memcmp(c, "fmt ", 4) && len >= 16 && avail >= 16) {
            fmt = rd16(c + 8);
            ch = rd16(c + 10);
            sr = rd32(c + 12);
            bits = rd16(c + 22);
            if (fmt == 0xFFFE && len >= 26 && avail >= 26) fmt = rd16(c + 32);  // extensible: sub-format tag
        } else if (!std::memcmp(c, "data", 4)) {
            data = c + 8;
            data_len = len < avail ? len : avail;
        }
        pos = body + len + (len & 1);
    }
    if (!data || ch == 0 || sr == 0) return false;
    const size_t bps = bits / 8;
    if (bps == 0) return false;
    const size_t frames = data_len / (bps * ch);
    mono.assign(frames, 0.0f);
    for (size_t i = 0; i < frames; ++i) {
        double acc = 0.0;
        for (uint16_t k = 0; k < ch; ++k) {
            const uint8_t* s = data + (i * ch + k) * bps;
            float v;
            if (fmt == 1 && bits == 8) {
                v = (float)s[0] * 0.00784313725490196078f - 1.0f;
            } else if (fmt == 1 && bits == 16) {
                v = (float)(int16_t)rd16(s) * 0.000030517578125f;
            } else if (fmt == 1 && bits == 24) {
                int32_t x = (int32_t)((uint32_t)s[0] << 8 | (uint32_t)s[1] << 16 | (uint32_t)s[2] << 24) >> 8;
                v = (float)(x * 0.00000011920928955078125);
            } else if (fmt == 1 && bits == 32) {
                v = (float)((int32_t)rd32(s) / 2147483648.0);
            } else if (fmt == 3 && bits == 32) {
                std::memcpy(&v, s, 4);
            } else if (fmt == 3 && bits == 64) {
                double d;
                std::memcpy(&d, s, 8);
                v = (float)d;
            } else {
                return false;
            }
            acc += v;
        }
        mono[i] = (float)(acc / ch);
    }
    sample_rate = (int)sr;
    return true;
}

bool load_audio_16k_mono(const std::string& path, std::vector<float>& out) {
    std::vector<float> mono;
    int sr = 0;
    if (!load_wav_mono(path, mono, sr)) return false;
    out = resample_linear(mono, sr, 16000);
    return true;
}

}  // namespace vdk

extern "C" long vdk_load_wav_16k(const char* path, float* out, long cap) {
    if (!path) return -1;
    try {
        std::vector<float> x;
        if (!vdk::load_audio_16k_mono(path, x)) return -1;
        const long n = (long)x.size();
        if (out && cap > 0) std::memcpy(out, x.data(), sizeof(float) * (size_t)(n < cap ? n : cap));
        return n;
    } catch (...) {
        return -1;
    }
}

extern "C" long vdk_resample_linear(const float* in, long n, int in_sr, int out_sr, float* out, long cap) {
    if (!in || n < 0) return -1;
    try {
        std::vector<float> y = vdk::resample_linear(std::vector<float>(in, in + n), in_sr, out_sr);
        const long m = (long)y.size();
        if (out && cap > 0) std::memcpy(out, y.data(), sizeof(float) * (size_t)(m < cap ? m : cap));
        return m;
    } catch (...) {
        return -1;
    }
}

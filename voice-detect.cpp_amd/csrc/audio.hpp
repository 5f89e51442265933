// audio.hpp - host WAV loading and resampling (src/audio_io.hpp equivalents).
#pragma once

#include <string>
#include <vector>

namespace vdk {

// Linear resampler, identity when in_sr == out_sr (src/audio_io.cpp:9-23).
std::vector<float> resample_linear(const std::vector<float>& in, int in_sr, int out_sr);
// Decode a WAV and average its channels; false on an unreadable/unsupported file.
bool load_wav_mono(const std::string& path, std::vector<float>& mono, int& sample_rate);
// load_wav_mono + resample to 16 kHz (src/audio_io.cpp:25-38).
bool load_audio_16k_mono(const std::string& path, std::vector<float>& out);

}  // namespace vdk

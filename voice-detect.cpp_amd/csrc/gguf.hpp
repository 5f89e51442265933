// gguf.hpp - GGUF v2/v3 reader for the speaker-encoder models.
//
// Reads what vd::ModelLoader::load consumes (src/model_loader.cpp:114-215):
// `voicedetect.*` key/values (u32, i32, f32, bool, string, string/i32 arrays)
// and named F32 / F16 / Q8_0 tensors with ggml `ne` dims (fastest first).
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace vdk {

enum GgmlType : uint32_t { GGML_F32 = 0, GGML_F16 = 1, GGML_Q8_0 = 8 };

struct GgufValue {
    enum Kind { NONE, INT, FLOAT, BOOL, STR, ARR_STR, ARR_INT, ARR_FLOAT } kind = NONE;
    int64_t i = 0;
    double f = 0.0;
    bool b = false;
    std::string s;
    std::vector<std::string> as;
    std::vector<int64_t> ai;
    std::vector<double> af;
};

struct GgufTensor {
    std::string name;
    uint32_t type = 0;
    std::vector<int64_t> ne;   // fastest dim first
    const uint8_t* data = nullptr;
    size_t nbytes = 0;
    int64_t nelements() const;
};

class GgufFile {
public:
    // Throws vdk::Error on a missing file or a malformed/unsupported header.
    explicit GgufFile(const std::string& path);

    bool has(const std::string& key) const { return kv_.count(key) != 0; }
    uint32_t u32(const std::string& key, uint32_t def) const;
    float f32(const std::string& key, float def) const;
    bool boolean(const std::string& key, bool def) const;
    std::string str(const std::string& key, const std::string& def = "") const;
    std::vector<std::string> str_arr(const std::string& key) const;
    std::vector<int32_t> i32_arr(const std::string& key) const;

    const GgufTensor* tensor(const std::string& name) const;
    // Tensor as f32 (F16 widened exactly, Q8_0 dequantised q * d); throws if absent.
    std::vector<float> to_f32(const std::string& name) const;

private:
    std::vector<uint8_t> buf_;
    std::map<std::string, GgufValue> kv_;
    std::map<std::string, GgufTensor> tensors_;
};

}  // namespace vdk

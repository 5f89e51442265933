// gguf.cpp - GGUF reader (see gguf.hpp).
#include "gguf.hpp"

#include <algorithm>
#include <climits>
#include <cstring>
#include <fstream>

#include "common.hpp"

namespace vdk {

namespace {

enum : uint32_t { T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 };

struct Reader {
    const uint8_t* p;
    const uint8_t* end;
    template <class T>
    T get() {
        if ((size_t)(end - p) < sizeof(T)) throw Error("gguf: truncated file");
        T v;
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if ((uint64_t)(end - p) < n) throw Error("gguf: truncated string");
        std::string s(reinterpret_cast<const char*>(p), (size_t)n);
        p += n;
        return s;
    }
};

size_t scalar_size(uint32_t t) {
    switch (t) {
        case T_U8: case T_I8: case T_BOOL: return 1;
        case T_U16: case T_I16: return 2;
        case T_U32: case T_I32: case T_F32: return 4;
        case T_U64: case T_I64: case T_F64: return 8;
        default: return 0;
    }
}

bool read_number(Reader& r, uint32_t t, int64_t& i, double& f) {
    switch (t) {
        case T_U8: i = r.get<uint8_t>(); f = (double)i; return true;
        case T_I8: i = r.get<int8_t>(); f = (double)i; return true;
        case T_U16: i = r.get<uint16_t>(); f = (double)i; return true;
        case T_I16: i = r.get<int16_t>(); f = (double)i; return true;
        case T_U32: i = r.get<uint32_t>(); f = (double)i; return true;
        case T_I32: i = r.get<int32_t>(); f = (double)i; return true;
        case T_U64: i = (int64_t)r.get<uint64_t>(); f = (double)i; return true;
        case T_I64: i = r.get<int64_t>(); f = (double)i; return true;
        case T_F32: f = r.get<float>(); i = (int64_t)f; return true;
        case T_F64: f = r.get<double>(); i = (int64_t)f; return true;
        case T_BOOL: i = r.get<uint8_t>() != 0; f = (double)i; return true;
        default: return false;
    }
}

GgufValue read_value(Reader& r, uint32_t t) {
    GgufValue v;
    if (t == T_STR) {
        v.kind = GgufValue::STR;
        v.s = r.str();
    } else if (t == T_ARR) {
        const uint32_t et = r.get<uint32_t>();
        const uint64_t n = r.get<uint64_t>();
        if (et == T_STR) {
            v.kind = GgufValue::ARR_STR;
            for (uint64_t k = 0; k < n; ++k) v.as.push_back(r.str());
        } else if (scalar_size(et)) {
            const bool fl = et == T_F32 || et == T_F64;
            v.kind = fl ? GgufValue::ARR_FLOAT : GgufValue::ARR_INT;
            for (uint64_t k = 0; k < n; ++k) {
                int64_t i;
                double f;
                read_number(r, et, i, f);
                v.ai.push_back(i);
                v.af.push_back(f);
            }
        } else {
            throw Error("gguf: unsupported array element type");
        }
    } else if (t == T_BOOL) {
        v.kind = GgufValue::BOOL;
        v.b = r.get<uint8_t>() != 0;
        v.i = v.b;
    } else if (scalar_size(t)) {
        read_number(r, t, v.i, v.f);
        v.kind = (t == T_F32 || t == T_F64) ? GgufValue::FLOAT : GgufValue::INT;
    } else {
        throw Error("gguf: unsupported value type");
    }
    return v;
}

size_t tensor_bytes(uint32_t type, int64_t n) {
    switch (type) {
        case GGML_F32: return 4 * (size_t)n;
        case GGML_F16: return 2 * (size_t)n;
        case GGML_Q8_0:
            if (n % 32) throw Error("gguf: Q8_0 tensor size not a multiple of 32");
            return (size_t)(n / 32) * 34;
        default: throw Error("gguf: unsupported tensor type " + std::to_string(type));
    }
}

}  // namespace

int64_t GgufTensor::nelements() const {
    int64_t n = 1;
    for (int64_t d : ne) n *= d;   // dims and their product are range-checked at load
    return n;
}

GgufFile::GgufFile(const std::string& path) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) throw Error("gguf open failed: " + path);
    const std::streamsize n = f.tellg();
    f.seekg(0);
    buf_.resize((size_t)n);
    if (n > 0 && !f.read(reinterpret_cast<char*>(buf_.data()), n)) throw Error("gguf read failed: " + path);
    Reader r{buf_.data(), buf_.data() + buf_.size()};
    if (r.get<uint32_t>() != 0x46554747u) throw Error("not a GGUF file: " + path);
    const uint32_t ver = r.get<uint32_t>();
    if (ver != 2 && ver != 3) throw Error("unsupported GGUF version");
    const uint64_t nt = r.get<uint64_t>(), nkv = r.get<uint64_t>();
    for (uint64_t k = 0; k < nkv; ++k) {
        std::string key = r.str();
        const uint32_t t = r.get<uint32_t>();
        kv_[key] = read_value(r, t);
    }
    uint64_t align = 32;
    if (kv_.count("general.alignment")) align = (uint64_t)kv_["general.alignment"].i;
    if (align == 0 || (align & (align - 1)) || align > (1u << 24)) throw Error("gguf: bad alignment");
    struct Info { std::string name; std::vector<int64_t> ne; uint32_t type; uint64_t off; };
    std::vector<Info> infos;
    for (uint64_t k = 0; k < nt; ++k) {
        Info in;
        in.name = r.str();
        const uint32_t nd = r.get<uint32_t>();
        if (nd > 4) throw Error("gguf: tensor rank above 4");
        for (uint32_t d = 0; d < nd; ++d) {
            // ggml dims are int64; anything negative or past INT32_MAX is a
            // corrupt header (the encoders index tensors with int)
            const uint64_t v = r.get<uint64_t>();
            if (v > (uint64_t)INT32_MAX) throw Error("gguf: tensor dimension out of range: " + in.name);
            in.ne.push_back((int64_t)v);
        }
        in.type = r.get<uint32_t>();
        in.off = r.get<uint64_t>();
        infos.push_back(in);
    }
    const size_t hdr = (size_t)(r.p - buf_.data());
    const size_t base = (hdr + align - 1) / align * align;
    const size_t size = buf_.size();
    for (const Info& in : infos) {
        GgufTensor t;
        t.name = in.name;
        t.type = in.type;
        t.ne = in.ne;
        // element count without overflow; every element takes at least one
        // byte of the file (F32 4, F16 2, Q8_0 34/32), which bounds nbytes too
        int64_t n = 1;
        for (int64_t d : in.ne)
            if (__builtin_mul_overflow(n, d, &n)) throw Error("gguf: tensor size overflows: " + in.name);
        if ((uint64_t)n > (uint64_t)size) throw Error("gguf: tensor larger than the file: " + in.name);
        t.nbytes = tensor_bytes(in.type, n);
        if (in.off % align) throw Error("gguf: tensor offset not aligned: " + in.name);
        if (base > size || in.off > size - base || t.nbytes > size - base - in.off)
            throw Error("gguf: tensor data out of range: " + in.name);
        t.data = buf_.data() + base + in.off;
        tensors_[in.name] = t;
    }
}

uint32_t GgufFile::u32(const std::string& key, uint32_t def) const {
    auto it = kv_.find(key);
    return it == kv_.end() ? def : (uint32_t)it->second.i;
}

float GgufFile::f32(const std::string& key, float def) const {
    auto it = kv_.find(key);
    return it == kv_.end() ? def : (float)it->second.f;
}

bool GgufFile::boolean(const std::string& key, bool def) const {
    auto it = kv_.find(key);
    return it == kv_.end() ? def : it->second.i != 0;
}

std::string GgufFile::str(const std::string& key, const std::string& def) const {
    auto it = kv_.find(key);
    return (it == kv_.end() || it->second.kind != GgufValue::STR) ? def : it->second.s;
}

std::vector<std::string> GgufFile::str_arr(const std::string& key) const {
    auto it = kv_.find(key);
    if (it == kv_.end() || it->second.kind != GgufValue::ARR_STR) return {};
    return it->second.as;
}

std::vector<int32_t> GgufFile::i32_arr(const std::string& key) const {
    auto it = kv_.find(key);
    if (it == kv_.end() || it->second.kind != GgufValue::ARR_INT) return {};
    return std::vector<int32_t>(it->second.ai.begin(), it->second.ai.end());
}

const GgufTensor* GgufFile::tensor(const std::string& name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

std::vector<float> GgufFile::to_f32(const std::string& name) const {
    const GgufTensor* t = tensor(name);
    if (!t) throw Error("voicedetect: missing tensor '" + name + "'");
    const int64_t n = t->nelements();
    std::vector<float> out((size_t)n);
    if (t->type == GGML_F32) {
        std::memcpy(out.data(), t->data, (size_t)n * 4);
    } else if (t->type == GGML_F16) {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(t->data);
        for (int64_t i = 0; i < n; ++i) out[(size_t)i] = half_bits_to_float(h[i]);
    } else if (t->type == GGML_Q8_0) {
        for (int64_t blk = 0; blk < n / 32; ++blk) {
            const uint8_t* bp = t->data + blk * 34;
            uint16_t dh;
            std::memcpy(&dh, bp, 2);
            const float d = half_bits_to_float(dh);
            const int8_t* q = reinterpret_cast<const int8_t*>(bp + 2);
            for (int k = 0; k < 32; ++k) out[(size_t)(blk * 32 + k)] = (float)q[k] * d;
        }
    } else {
        throw Error("voicedetect: unsupported tensor type for '" + name + "'");
    }
    return out;
}

}  // namespace vdk

extern "C" int vdk_gguf_tensor_f32(const char* path, const char* name, float* out, long long n) {
    return vdk::guarded([&] {
        vdk::require(path && name && out, "gguf: NULL argument");
        const vdk::GgufFile g(path);
        const vdk::GgufTensor* t = g.tensor(name);
        vdk::require(t != nullptr, std::string("gguf: no tensor '") + name + "'");
        vdk::require(t->nelements() == n, std::string("gguf: tensor '") + name + "' has a different element count");
        const std::vector<float> v = g.to_f32(name);
        std::copy(v.begin(), v.end(), out);
    });
}

// weights.hpp - reading GGUF conv / linear weights into kernel layouts.
//
// A manifest conv weight arrives in one of the reference converter's forms
// (scripts/convert_voicedetect_to_gguf.py quant_plan): F32/F16 with ggml
// ne = [KW, KH, IC, OC] (Conv2d) or [K, IC, OC] (Conv1d), or a 1x1 weight
// squeezed to a 2-D [IC, OC] matrix (F16 / Q8_0 blocks along IC).  read_conv
// dequantises any of them to f32 [OC][IC][KH][KW]; pack_conv_f16 reorders to
// the conv kernels' f16 [OC][KH][KW][ICp] with an optional input-channel
// permutation and zero channels up to ICp.
#pragma once

#include <functional>
#include <string>
#include <vector>

#include "common.hpp"
#include "gguf.hpp"

namespace vdk {

struct HostConv {
    int oc = 0, ic = 0, kh = 1, kw = 1;
    std::vector<float> w;   // [OC][IC][KH][KW]
};

inline HostConv read_conv(const GgufFile& g, const std::string& name) {
    const GgufTensor* t = g.tensor(name);
    require(t != nullptr, "voicedetect: missing tensor '" + name + "'");
    HostConv c;
    if (t->ne.size() == 2) {
        c.ic = (int)t->ne[0]; c.oc = (int)t->ne[1];
    } else if (t->ne.size() == 3) {
        c.kw = (int)t->ne[0]; c.ic = (int)t->ne[1]; c.oc = (int)t->ne[2];
    } else if (t->ne.size() == 4) {
        c.kw = (int)t->ne[0]; c.kh = (int)t->ne[1]; c.ic = (int)t->ne[2]; c.oc = (int)t->ne[3];
    } else {
        throw Error("voicedetect: conv weight '" + name + "' must be 2-D, 3-D or 4-D");
    }
    c.w = g.to_f32(name);
    require(c.w.size() == (size_t)c.oc * c.ic * c.kh * c.kw, "voicedetect: tensor '" + name + "' has the wrong size");
    return c;
}

// f16 [OC][KH][KW][icp]; source channel i lands at ic_map(i) (identity if empty).
inline std::vector<uint16_t> pack_conv_f16(const HostConv& c, int icp,
                                           const std::function<int(int)>& ic_map = nullptr) {
    std::vector<uint16_t> p((size_t)c.oc * c.kh * c.kw * icp, 0);
    for (int o = 0; o < c.oc; ++o)
        for (int i = 0; i < c.ic; ++i) {
            const int d = ic_map ? ic_map(i) : i;
            for (int kh = 0; kh < c.kh; ++kh)
                for (int kw = 0; kw < c.kw; ++kw)
                    p[(((size_t)o * c.kh + kh) * c.kw + kw) * icp + d] =
                        float_to_half_bits(c.w[(((size_t)o * c.ic + i) * c.kh + kh) * c.kw + kw]);
        }
    return p;
}

// Whether f16 holds every weight exactly (the split-f16 lo halves are all 0).
inline bool conv_f16_exact(const HostConv& c) {
    for (float v : c.w)
        if (half_bits_to_float(float_to_half_bits(v)) != v) return false;
    return true;
}

// Split-f16 weights: f16 [OC][KH][KW][terms*icp] holding [hi | hi | lo] per tap
// (hi = f16(w), lo = f16(w - hi)), or [hi | hi] when terms = 2 (weights that
// conv_f16_exact accepts, whose lo halves are 0); rows oc_pad > oc are zero.
inline std::vector<uint16_t> pack_conv_f16_split(const HostConv& c, int icp, int oc_pad = 0,
                                                 const std::function<int(int)>& ic_map = nullptr, int terms = 3) {
    require(terms == 2 || terms == 3, "voicedetect: split-f16 weights have 2 or 3 terms");
    const int ocp = oc_pad > c.oc ? oc_pad : c.oc;
    const size_t row = (size_t)terms * icp;
    std::vector<uint16_t> p((size_t)ocp * c.kh * c.kw * row, 0);
    for (int o = 0; o < c.oc; ++o)
        for (int i = 0; i < c.ic; ++i) {
            const int d = ic_map ? ic_map(i) : i;
            for (int kh = 0; kh < c.kh; ++kh)
                for (int kw = 0; kw < c.kw; ++kw) {
                    const float v = c.w[(((size_t)o * c.ic + i) * c.kh + kh) * c.kw + kw];
                    const uint16_t hi = float_to_half_bits(v);
                    const uint16_t lo = float_to_half_bits(v - half_bits_to_float(hi));
                    uint16_t* q = &p[(((size_t)o * c.kh + kh) * c.kw + kw) * row];
                    q[d] = hi;
                    q[icp + d] = hi;
                    if (terms == 3) q[2 * icp + d] = lo;
                }
        }
    return p;
}

}  // namespace vdk

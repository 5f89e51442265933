// runtime.cpp - error state, host half conversion and the vdk device helpers.
#include <cstring>

#include "common.hpp"
#include "vdk.h"

namespace vdk {

namespace {
thread_local std::string g_error;
}

void set_error(const std::string& msg) { g_error = msg; }
const char* get_error() { return g_error.c_str(); }
void clear_error() { g_error.clear(); }

float half_bits_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    const uint32_t exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {  // subnormal: renormalise
            int e = -1;
            do { ++e; mant <<= 1; } while ((mant & 0x400) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mant & 0x3ff) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t float_to_half_bits(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000;
    const uint32_t absx = x & 0x7fffffff;
    if (absx >= 0x7f800000u)  // inf / nan
        return (uint16_t)(sign | 0x7c00 | (absx > 0x7f800000u ? 0x200 : 0));
    if (absx >= 0x477ff000u)  // rounds to >= 65520 -> inf
        return (uint16_t)(sign | 0x7c00);
    if (absx < 0x38800000u) {  // below the smallest normal half: subnormal or zero
        if (absx < 0x33000000u) return (uint16_t)sign;  // < 2^-25 rounds to 0
        const uint32_t e = absx >> 23;
        const uint32_t m = (absx & 0x7fffff) | 0x800000;
        const int shift = 126 - (int)e;  // 14 + (113 - e) - ... : mantissa >> (shift)
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((absx >> 13) - (112u << 10));
    const uint32_t rem = absx & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) ++h;
    return (uint16_t)(sign | h);
}

}  // namespace vdk

using namespace vdk;

extern "C" int vdk_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

extern "C" int vdk_set_device(int device) {
    return guarded([&] { VDK_HIP(hipSetDevice(device)); });
}

extern "C" void* vdk_malloc(size_t bytes) {
    void* p = nullptr;
    if (guarded([&] { VDK_HIP(hipMalloc(&p, bytes)); }) != 0) return nullptr;
    return p;
}

extern "C" int vdk_free(void* p) {
    return guarded([&] { if (p) VDK_HIP(hipFree(p)); });
}

extern "C" int vdk_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    return guarded([&] { VDK_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice)); });
}

extern "C" int vdk_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    return guarded([&] { VDK_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost)); });
}

extern "C" int vdk_memcpy_d2d(void* dst, const void* src, size_t bytes) {
    return guarded([&] { VDK_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice)); });
}

extern "C" int vdk_memset(void* dst, int value, size_t bytes) {
    return guarded([&] { VDK_HIP(hipMemset(dst, value, bytes)); });
}

extern "C" int vdk_synchronize(void) {
    return guarded([&] { VDK_HIP(hipDeviceSynchronize()); });
}

extern "C" const char* vdk_last_error(void) { return get_error(); }

extern "C" void vdk_f32_to_f16(const float* in, unsigned short* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = float_to_half_bits(in[i]);
}

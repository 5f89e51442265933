// common.hpp - shared types and error plumbing for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>

namespace vdk {

typedef _Float16 half_t;
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

// Thread-local last error for the C ABI.
void set_error(const std::string& msg);
const char* get_error();
void clear_error();

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess)
        throw Error(std::string(what) + ": " + hipGetErrorString(e));
}

#define VDK_HIP(call) ::vdk::hip_check((call), #call)

inline void require(bool ok, const std::string& msg) {
    if (!ok) throw Error(msg);
}

// Run `body` and translate exceptions into the C-ABI status convention.
template <class F>
int guarded(F&& body) {
    try {
        body();
        clear_error();
        return 0;
    } catch (const std::exception& e) {
        set_error(e.what());
        return 1;
    } catch (...) {
        set_error("unknown error");
        return 1;
    }
}

// IEEE half <-> float on the host (round to nearest even).
float half_bits_to_float(uint16_t h);
uint16_t float_to_half_bits(float f);

inline int cdiv(long a, long b) { return (int)((a + b - 1) / b); }

}  // namespace vdk

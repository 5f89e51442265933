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

// ---- device helpers shared by the kernels ----

typedef __attribute__((address_space(3))) void lds_void;
typedef int int4v __attribute__((ext_vector_type(4)));

constexpr uint32_t kOOB = 0x80000000u;   // any buffer offset >= num_records reads as zero

// Spread consecutive workgroup ids over the 8 XCDs in contiguous ranges so that
// neighbouring tiles (which share input rows or output lines) run under the
// same L2: workgroups are dispatched to the XCDs round robin.
__device__ __forceinline__ int xcd_swizzle(int bid, int nb) {
    const int per = nb >> 3;
    if (bid >= (per << 3)) return bid;
    return (bid & 7) * per + (bid >> 3);
}

// Workgroup barrier over LDS traffic only: this wave's LDS reads and writes
// complete (lgkmcnt(0)) before s_barrier, while its global stores and LDS DMA
// stay in flight.  (A workgroup-scope release fence would also drain vmcnt,
// because LDS DMA counts as a pending LDS write.)
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_s_waitcnt(0xC07F);   // vmcnt 63, expcnt 7, lgkmcnt 0
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// s_waitcnt until at most N vector memory operations of this wave are in
// flight (expcnt and lgkmcnt left at their "no wait" maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit field");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// s_waitcnt until at most n (a run-time count) vector memory operations of
// this wave are in flight; counts without a case wait for all of them.
__device__ __forceinline__ void wait_vmcnt_le(int n) {
    // s_waitcnt with vmcnt = n (6-bit field split [3:0] / [15:14]), expcnt and
    // lgkmcnt left at their "no wait" maxima.
    switch (n) {
#define VDK_VM(N) case N: __builtin_amdgcn_s_waitcnt(((N) & 15) | (((N) >> 4) << 14) | (7 << 4) | (15 << 8)); break;
        VDK_VM(0) VDK_VM(1) VDK_VM(2) VDK_VM(3) VDK_VM(4) VDK_VM(5) VDK_VM(6) VDK_VM(7) VDK_VM(8)
        VDK_VM(9) VDK_VM(10) VDK_VM(11) VDK_VM(12) VDK_VM(13) VDK_VM(14) VDK_VM(15) VDK_VM(16)
        VDK_VM(18) VDK_VM(20) VDK_VM(21) VDK_VM(24) VDK_VM(26) VDK_VM(27) VDK_VM(28) VDK_VM(30) VDK_VM(32)
        VDK_VM(36) VDK_VM(39) VDK_VM(40) VDK_VM(42) VDK_VM(45) VDK_VM(48) VDK_VM(54) VDK_VM(56) VDK_VM(60)
#undef VDK_VM
        default: __builtin_amdgcn_s_waitcnt(0); break;
    }
}

// Buffer resource words of [base, base + bytes) for dma16 (raw buffer,
// offsets at or past `bytes` read as zero).
__device__ __forceinline__ int4v dma_rsrc(const void* base, uint32_t bytes) {
    const uint64_t p = (uint64_t)(uintptr_t)base;
    return int4v{(int)(uint32_t)p, (int)(uint32_t)(p >> 32), (int)bytes, 0x00020000};
}

// One 16-byte-per-lane DMA (buffer_load ... lds) from the buffer at byte
// offset voff to LDS lds_dst + 16 * lane (lds_dst is wave-uniform).  Written
// as inline assembly, so the compiler does not see it as a write to LDS and
// never makes LDS reads wait for it: the caller orders it with vmcnt waits
// and barriers of its own.
__device__ __forceinline__ void dma16(uint8_t* lds_dst, int4v rsrc, uint32_t voff) {
    const uint32_t m0v = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)lds_dst);
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(m0v) : "memory");
}

}  // namespace vdk

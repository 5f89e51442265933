// arena.hpp - host staging of a model's device weight arena.
//
// Tensors are appended 256-byte aligned into one host buffer; upload() makes a
// single device allocation, copies the buffer and binds every registered
// pointer to its device address.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <vector>

#include "common.hpp"

namespace vdk {

class ArenaBuilder {
public:
    size_t put(const void* src, size_t bytes) {
        const size_t off = (host_.size() + 255) & ~(size_t)255;
        host_.resize(off + bytes);
        if (bytes) std::memcpy(host_.data() + off, src, bytes);
        return off;
    }
    template <class T>
    void put(const std::vector<T>& v, T** dst) {
        fixes_.push_back({put(v.data(), v.size() * sizeof(T)), reinterpret_cast<void**>(dst)});
    }
    template <class T>
    void put(const std::vector<T>& v, void** dst) {
        fixes_.push_back({put(v.data(), v.size() * sizeof(T)), dst});
    }
    // One hipMalloc + copy; binds every registered pointer.  Returns the arena.
    void* upload() {
        void* arena = nullptr;
        VDK_HIP(hipMalloc(&arena, host_.empty() ? 256 : host_.size()));
        if (!host_.empty()) VDK_HIP(hipMemcpy(arena, host_.data(), host_.size(), hipMemcpyHostToDevice));
        uint8_t* base = static_cast<uint8_t*>(arena);
        for (const Fix& f : fixes_) *f.dst = base + f.off;
        return arena;
    }

private:
    struct Fix { size_t off; void** dst; };
    std::vector<uint8_t> host_;
    std::vector<Fix> fixes_;
};

}  // namespace vdk

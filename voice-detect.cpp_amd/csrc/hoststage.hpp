// hoststage.hpp - host PCM into the device through pinned staging.
//
// The drop-in entry points (voicedetect_capi_embed_pcm_batch and friends,
// src/voicedetect_capi.cpp:61-178) take PCM in ordinary pageable host memory.
// A pageable hipMemcpy stages it through the driver's own buffers on one CPU
// thread; here the batch is copied into a pinned buffer by a few threads,
// chunk by chunk, and each chunk's DMA is queued as soon as its copy is done,
// so the DMA of chunk k runs while chunk k+1 is copied.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

#include "common.hpp"

namespace vdk {

// memcpy split over the caller and `n` persistent worker threads.
class CopyPool {
public:
    explicit CopyPool(int n) {
        for (int i = 0; i < n; ++i) th_.emplace_back([this] { work(); });
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> g(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto& t : th_) t.join();
    }
    CopyPool(const CopyPool&) = delete;
    CopyPool& operator=(const CopyPool&) = delete;

    void copy(void* dst, const void* src, size_t bytes) {
        constexpr size_t kPart = 256 << 10;
        const int parts = (int)std::max<size_t>(1, (bytes + kPart - 1) / kPart);
        if (th_.empty() || parts == 1) {
            std::memcpy(dst, src, bytes);
            return;
        }
        {
            std::lock_guard<std::mutex> g(mu_);
            dst_ = static_cast<uint8_t*>(dst);
            src_ = static_cast<const uint8_t*>(src);
            bytes_ = bytes;
            part_ = (bytes + parts - 1) / parts;
            parts_ = parts;
            next_.store(0);
            left_ = parts;
            ++gen_;
        }
        cv_.notify_all();
        run_parts();
        std::unique_lock<std::mutex> l(mu_);
        done_.wait(l, [this] { return left_ == 0; });
    }

private:
    void run_parts() {
        for (;;) {
            const int p = next_.fetch_add(1);
            if (p >= parts_) return;
            const size_t off = (size_t)p * part_;
            std::memcpy(dst_ + off, src_ + off, std::min(part_, bytes_ - off));
            std::lock_guard<std::mutex> g(mu_);
            if (--left_ == 0) done_.notify_all();
        }
    }
    void work() {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> l(mu_);
                cv_.wait(l, [&] { return stop_ || gen_ != seen; });
                if (stop_) return;
                seen = gen_;
            }
            run_parts();
        }
    }

    std::vector<std::thread> th_;
    std::mutex mu_;
    std::condition_variable cv_, done_;
    uint8_t* dst_ = nullptr;
    const uint8_t* src_ = nullptr;
    size_t bytes_ = 0, part_ = 0;
    int parts_ = 0, left_ = 0;
    std::atomic<int> next_{0};
    uint64_t gen_ = 0;
    bool stop_ = false;
};

// A pinned host buffer that grows on demand (hipHostMalloc; freed with the owner).
class PinnedBuffer {
public:
    PinnedBuffer() = default;
    ~PinnedBuffer() {
        if (p_) (void)hipHostFree(p_);
    }
    PinnedBuffer(const PinnedBuffer&) = delete;
    PinnedBuffer& operator=(const PinnedBuffer&) = delete;
    void* get(size_t bytes) {
        if (bytes > cap_) {
            if (p_) VDK_HIP(hipHostFree(p_));
            p_ = nullptr;
            cap_ = 0;
            VDK_HIP(hipHostMalloc(&p_, bytes, hipHostMallocDefault));
            cap_ = bytes;
        }
        return p_;
    }

private:
    void* p_ = nullptr;
    size_t cap_ = 0;
};

// Host rows [rows][row_bytes] to the device buffer on `s`: copied into pinned
// memory in about `chunks` pieces of whole rows, each piece's DMA queued right
// after its copy.  The pinned buffer is not reused within a call, and the
// caller waits on `s` before the next call overwrites it.
inline void stage_h2d(CopyPool& pool, PinnedBuffer& pin, void* d_dst, const void* src, int rows, size_t row_bytes,
                      int chunks, hipStream_t s) {
    const size_t total = (size_t)rows * row_bytes;
    uint8_t* p = static_cast<uint8_t*>(pin.get(total));
    const int per = std::max(1, (rows + chunks - 1) / chunks);
    for (int r0 = 0; r0 < rows; r0 += per) {
        const size_t off = (size_t)r0 * row_bytes, n = (size_t)std::min(per, rows - r0) * row_bytes;
        pool.copy(p + off, static_cast<const uint8_t*>(src) + off, n);
        VDK_HIP(hipMemcpyAsync(static_cast<uint8_t*>(d_dst) + off, p + off, n, hipMemcpyHostToDevice, s));
    }
}

}  // namespace vdk

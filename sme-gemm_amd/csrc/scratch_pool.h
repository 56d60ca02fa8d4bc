// Grow-only scratch buffers keyed by (device, stream), for the device-pointer
// entry points: a kernel they enqueue, or a HIP graph that captured it, may
// still read its buffer long after the call returned, so a buffer that a later
// call outgrows is retired -- kept allocated until the pool is destroyed --
// never freed or reused. Calls on different streams get different buffers, so
// they cannot race; calls on one stream are ordered by that stream.
//
// Host-only and independent of HIP: the allocator is a template parameter, so
// the growth rule is exercised on the CPU (tests/cpp/scratch_pool_test.cpp).
#pragma once

#include <cstddef>
#include <mutex>
#include <vector>

namespace smg {

template <class Alloc>
class ScratchPool {
public:
    explicit ScratchPool(Alloc a = Alloc()) : alloc_(a) {}
    ~ScratchPool() {
        for (Entry &e : live_) alloc_.release(e.device, e.buf);
        for (Entry &e : retired_) alloc_.release(e.device, e.buf);
    }
    ScratchPool(const ScratchPool &) = delete;
    ScratchPool &operator=(const ScratchPool &) = delete;

    // A buffer of at least `bytes` for work on (device, stream); nullptr when
    // the allocator fails (the previous buffer, if any, is kept).
    void *get(int device, const void *stream, size_t bytes) {
        std::lock_guard<std::mutex> lk(mu_);
        for (Entry &e : live_) {
            if (e.device != device || e.stream != stream) continue;
            if (e.cap >= bytes) return e.buf;
            void *nb = alloc_.acquire(device, grown(bytes));
            if (!nb) return nullptr;
            retired_.push_back(e);
            e.buf = nb;
            e.cap = grown(bytes);
            return nb;
        }
        void *nb = alloc_.acquire(device, grown(bytes));
        if (!nb) return nullptr;
        live_.push_back(Entry{device, stream, nb, grown(bytes)});
        return nb;
    }

    size_t live_count() const { std::lock_guard<std::mutex> lk(mu_); return live_.size(); }
    size_t retired_count() const { std::lock_guard<std::mutex> lk(mu_); return retired_.size(); }

private:
    struct Entry {
        int device;
        const void *stream;
        void *buf;
        size_t cap;
    };
    // sizes round up to whole MiB so small growth steps share an allocation
    static size_t grown(size_t bytes) {
        return ((bytes ? bytes : 1) + ((size_t)1 << 20) - 1) >> 20 << 20;
    }

    Alloc alloc_;
    mutable std::mutex mu_;
    std::vector<Entry> live_;
    std::vector<Entry> retired_;
};

}  // namespace smg

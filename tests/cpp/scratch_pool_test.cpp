// The device-pointer scratch pool's growth rule (sme-gemm_amd/csrc/scratch_pool.h),
// checked on the CPU with a recording allocator: a buffer handed out for a
// (device, stream) stays valid -- never freed, never handed to another stream --
// until the pool itself goes away, however the sizes asked for grow. Built and
// run by tests/test_host_logic.py under AddressSanitizer and UBSan.
#include <cassert>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <set>
#include <thread>
#include <vector>

#include "../../sme-gemm_amd/csrc/scratch_pool.h"

struct Recorder {
    std::vector<void *> *live;
    int *acquired;
    int *released;
    bool fail_next = false;
    void *acquire(int, size_t bytes) {
        if (fail_next) return nullptr;
        void *p = std::malloc(bytes);
        std::memset(p, 0xA5, bytes);  // ASan flags any use after release
        live->push_back(p);
        ++*acquired;
        return p;
    }
    void release(int, void *p) {
        ++*released;
        std::free(p);
    }
};

int main() {
    std::vector<void *> live;
    int acquired = 0, released = 0;
    {
        smg::ScratchPool<Recorder> pool(Recorder{&live, &acquired, &released});
        const void *s1 = (const void *)0x10, *s2 = (const void *)0x20;
        void *a = pool.get(0, s1, 1000);
        assert(a);
        std::memset(a, 1, 1000);
        // same stream, fits: the same buffer
        assert(pool.get(0, s1, 1 << 20) == a);
        // another stream: its own buffer
        void *b = pool.get(0, s2, 10);
        assert(b && b != a);
        // another device, same stream handle: its own buffer
        void *c = pool.get(1, s1, 10);
        assert(c && c != a && c != b);
        // growth: a new buffer; the old one is retired, still readable
        void *a2 = pool.get(0, s1, (3 << 20) + 5);
        assert(a2 && a2 != a);
        for (int i = 0; i < 1000; i++) assert(((unsigned char *)a)[i] == 1);
        assert(pool.retired_count() == 1 && pool.live_count() == 3);
        // a smaller request after growth keeps the grown buffer
        assert(pool.get(0, s1, 100) == a2);
        // a failed growth keeps the current buffer and retires nothing
        Recorder failing{&live, &acquired, &released, true};
        smg::ScratchPool<Recorder> pool2(failing);
        assert(pool2.get(0, s1, 10) == nullptr);
        assert(pool2.live_count() == 0);
        // many threads, many streams: every stream ends with a distinct buffer
        std::vector<std::thread> th;
        std::vector<void *> got(16);
        for (int t = 0; t < 16; t++)
            th.emplace_back([&, t] {
                for (int r = 1; r <= 8; r++) got[t] = pool.get(2, (const void *)(uintptr_t)(0x100 + t), (size_t)r << 19);
            });
        for (auto &x : th) x.join();
        std::set<void *> distinct(got.begin(), got.end());
        assert(distinct.size() == 16 && !distinct.count(nullptr));
        assert(released == 0);  // nothing freed while the pool lives
    }
    assert(released == acquired);  // everything freed once, when the pool goes
    std::printf("scratch pool ok: %d buffers\n", acquired);
    return 0;
}

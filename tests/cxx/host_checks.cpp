// Host-only checks of library logic that needs no GPU, built with g++ (and
// the sanitizers) by tests/test_host_logic.py:
//   trips FIRST N STEP ...  prints mi::strided_trips for each triple (the
//                           trip count the row-band and LayerNorm-backward
//                           kernels use), one per line;
//   pool                    drives mi::WorkspacePool from 8 threads with a
//                           mock allocator and checks that no buffer handed
//                           out is freed before release();
//   slots                   8 threads, each with its own per-thread slot
//                           (mi::thread_slot()) and the shared slot: a
//                           thread's slot buffer is never another thread's,
//                           the shared slot is one buffer for all, capture
//                           refuses growth per slot, release() frees every
//                           slot of the device and no other device's.
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <random>
#include <set>
#include <thread>
#include <vector>

#include "mi_index.hpp"
#include "workspace_pool.hpp"

namespace {

std::mutex g_live_mu;
std::set<void*> g_live;
std::atomic<int> g_allocs{0};

struct MockAlloc {
    int alloc(void** p, size_t bytes) {
        *p = std::malloc(bytes);
        if (*p == nullptr) return 2;
        std::memset(*p, 0, bytes);
        std::lock_guard<std::mutex> l(g_live_mu);
        g_live.insert(*p);
        ++g_allocs;
        return 0;
    }
    void free(void* p) {
        {
            std::lock_guard<std::mutex> l(g_live_mu);
            if (g_live.erase(p) != 1) {
                std::fprintf(stderr, "free of a pointer not allocated\n");
                std::abort();
            }
        }
        std::free(p);  // a later touch of p is a heap-use-after-free under ASan
    }
};

int fail(const char* msg) {
    std::fprintf(stderr, "FAIL: %s\n", msg);
    return 1;
}

int pool_test() {
    mi::WorkspacePool<MockAlloc> pool;
    const int dev = 3;
    std::atomic<int> errors{0};
    std::vector<std::thread> th;
    for (int t = 0; t < 8; ++t) {
        th.emplace_back([&, t] {
            std::mt19937 rng(1234 + t);
            for (int i = 0; i < 400; ++i) {
                const size_t want = 1 + rng() % (48u << 20);
                int err = -7;
                unsigned char* p = static_cast<unsigned char*>(
                    pool.get(dev, mi::WorkspacePool<MockAlloc>::kShared, want, false, -2, &err));
                if (p == nullptr || err != 0) {
                    ++errors;
                    continue;
                }
                // a "kernel" that uses the buffer some time after the call
                p[0] = static_cast<unsigned char>(t);
                p[want - 1] = static_cast<unsigned char>(i);
                std::this_thread::sleep_for(std::chrono::microseconds(rng() % 50));
                p[want / 2] ^= 1;
                p[want - 1] ^= p[0];
            }
        });
    }
    for (auto& x : th) x.join();
    if (errors) return fail("get returned an error");
    const size_t cur = pool.bytes(dev);
    if (cur < (48u << 20) - (1u << 20)) return fail("pool smaller than the largest request");
    // geometric growth: at most log2(48 MiB / 1 MiB) + 1 buffers
    if (g_allocs.load() > 8) return fail("too many allocations for geometric growth");
    if (pool.retired_count(dev) + 1 != static_cast<size_t>(g_allocs.load()))
        return fail("a grown buffer was freed before release()");
    // capture: a request that fits is served, a larger one is refused
    int err = 0;
    if (pool.get(dev, 0, 1024, true, -2, &err) == nullptr || err != 0)
        return fail("fitting request refused during capture");
    if (pool.get(dev, 0, cur + 1, true, -2, &err) != nullptr || err != -2)
        return fail("growth allowed during capture");
    pool.release(dev);
    if (!g_live.empty()) return fail("release() left buffers allocated");
    if (pool.bytes(dev) != 0) return fail("release() left a current buffer");
    // usable again after release
    if (pool.get(dev, 0, 100, false, -2, &err) == nullptr) return fail("no buffer after release");
    pool.release(dev);
    std::printf("pool ok: %d allocations\n", g_allocs.load());
    return 0;
}

int slots_test() {
    using Pool = mi::WorkspacePool<MockAlloc>;
    Pool pool;
    const int dev = 5, other = 6;
    constexpr int kThreads = 8;
    std::atomic<int> errors{0};
    std::mutex mu;
    std::vector<std::set<void*>> own(kThreads);  // every buffer each thread's slot handed out
    std::set<void*> shared;
    std::vector<int> slot_of(kThreads, 0);
    std::vector<std::thread> th;
    for (int t = 0; t < kThreads; ++t) {
        th.emplace_back([&, t] {
            const int slot = mi::thread_slot();
            if (slot < 1 || slot != mi::thread_slot()) ++errors;  // >= 1, fixed per thread
            std::mt19937 rng(77 + t);
            for (int i = 0; i < 200; ++i) {
                const size_t want = 1 + rng() % (8u << 20);
                int err = -7;
                void* p = pool.get(dev, slot, want, false, -2, &err);
                void* q = pool.get(dev, Pool::kShared, want / 2 + 1, false, -2, &err);
                if (p == nullptr || q == nullptr || err != 0) {
                    ++errors;
                    continue;
                }
                std::memset(p, t, want);  // this thread's "kernel" fills its whole buffer
                std::lock_guard<std::mutex> l(mu);
                own[t].insert(p);
                shared.insert(q);
                slot_of[t] = slot;
            }
        });
    }
    for (auto& x : th) x.join();
    if (errors) return fail("get or thread_slot misbehaved");
    std::set<int> slots(slot_of.begin(), slot_of.end());
    if (slots.size() != kThreads) return fail("two threads share a slot");
    for (int a = 0; a < kThreads; ++a)
        for (int b = a + 1; b < kThreads; ++b)
            for (void* p : own[a])
                if (own[b].count(p)) return fail("a slot buffer reached two threads");
    for (int a = 0; a < kThreads; ++a)
        for (void* p : own[a])
            if (shared.count(p)) return fail("a thread's slot buffer is the shared one");
    // the shared slot is one buffer at a time: all handed-out shared buffers
    // are its current one or retired ones, geometric growth keeps them few
    if (shared.size() > 8) return fail("shared slot grew too often");
    // capture refuses growth per slot; a fitting request is served
    int err = 0;
    const int s0 = slot_of[0];
    if (pool.get(dev, s0, pool.bytes(dev, s0) + 1, true, -2, &err) != nullptr || err != -2)
        return fail("per-thread slot grew during capture");
    if (pool.get(dev, s0, 16, true, -2, &err) == nullptr || err != 0)
        return fail("fitting per-thread request refused during capture");
    // another device's buffers survive this device's release
    void* keep = pool.get(other, s0, 4096, false, -2, &err);
    if (keep == nullptr) return fail("no buffer on the other device");
    pool.release(dev);
    if (pool.bytes(dev) != 0) return fail("release left the shared slot");
    for (int s : slots)
        if (pool.bytes(dev, s) != 0) return fail("release left a per-thread slot");
    {
        std::lock_guard<std::mutex> l(g_live_mu);
        if (g_live.size() != 1 || !g_live.count(keep)) return fail("release freed the wrong buffers");
    }
    pool.release(other);
    if (!g_live.empty()) return fail("buffers left after releasing both devices");
    std::printf("slots ok: %zu slots\n", slots.size());
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc >= 2 && std::strcmp(argv[1], "pool") == 0) return pool_test();
    if (argc >= 2 && std::strcmp(argv[1], "slots") == 0) return slots_test();
    if (argc >= 2 && std::strcmp(argv[1], "trips") == 0) {
        for (int i = 2; i + 2 < argc; i += 3) {
            const long long first = std::atoll(argv[i]), n = std::atoll(argv[i + 1]),
                            step = std::atoll(argv[i + 2]);
            std::printf("%u\n", mi::strided_trips(static_cast<unsigned>(first),
                                                   static_cast<unsigned>(n),
                                                   static_cast<unsigned>(step)));
        }
        return 0;
    }
    std::fprintf(stderr, "usage: host_checks pool | slots | trips FIRST N STEP ...\n");
    return 2;
}

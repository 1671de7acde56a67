// Per-device workspace bookkeeping of the library, independent of HIP so
// that host tests can drive it with a mock allocator.
//
// A workspace buffer, once handed out, is never freed behind a caller's back:
// kernels already queued, a launch being issued on another thread, or an
// instantiated graph may still reference it.  Growth therefore retires the
// old buffer (kept alive) and allocates a larger one; nothing is released
// until release() is called by a caller who guarantees that no pending or
// replayable work references any workspace buffer.  Geometric growth bounds
// the retired memory by the size of the current buffer.
//
// Buffers are kept per (device, slot).  Slot kShared serves calls on
// explicit streams and on the null stream: calls that share it must not run
// concurrently on different streams of one device (the caller serialises
// them, as one stream does).  Calls on the per-thread default stream
// (hipStreamPerThread, the reference's `--default-stream per-thread`) run
// concurrently when two host threads issue them, so each calling thread has
// its own slot (thread_slot(), numbered from 1 on a thread's first use).  A
// thread's slot stays allocated after the thread exits, until release().
#pragma once

#include <atomic>
#include <cstddef>
#include <map>
#include <mutex>
#include <vector>

namespace mi {

// The calling thread's workspace slot for per-thread-stream calls: a
// process-wide number >= 1, fixed on the thread's first call.
inline int thread_slot() {
    static std::atomic<int> next{1};
    thread_local const int slot = next.fetch_add(1, std::memory_order_relaxed);
    return slot;
}

// Alloc provides
//   int  alloc(void** p, size_t bytes);   // 0 on success, else an error code
//   void free(void* p);
template <class Alloc>
class WorkspacePool {
  public:
    static constexpr int kMaxDevices = 64;
    static constexpr int kShared = 0;
    static constexpr size_t kGrain = size_t(1) << 20;

    explicit WorkspacePool(Alloc a = Alloc()) : alloc_(a) {}

    // Returns a buffer of at least `bytes` for (device `dev`, slot `slot`),
    // growing that slot's buffer if needed (refused with `capture_err` while
    // `capturing`).  On failure returns nullptr and stores the allocator's
    // error (or capture_err) in *err.
    void* get(int dev, int slot, size_t bytes, bool capturing, int capture_err, int* err) {
        std::lock_guard<std::mutex> lock(mu_);
        Dev& d = at(dev, slot);
        if (d.cur != nullptr && d.bytes >= bytes) {
            *err = 0;
            return d.cur;
        }
        if (capturing) {
            *err = capture_err;
            return nullptr;
        }
        size_t want = bytes > 2 * d.bytes ? bytes : 2 * d.bytes;
        want = (want + kGrain - 1) / kGrain * kGrain;
        if (want == 0) want = kGrain;
        void* p = nullptr;
        const int rc = alloc_.alloc(&p, want);
        if (rc != 0 || p == nullptr) {
            *err = rc != 0 ? rc : -1;
            return nullptr;
        }
        if (d.cur != nullptr) d.retired.push_back(d.cur);
        d.cur = p;
        d.bytes = want;
        *err = 0;
        return p;
    }

    size_t bytes(int dev, int slot = kShared) {
        std::lock_guard<std::mutex> lock(mu_);
        return at(dev, slot).bytes;
    }

    size_t retired_count(int dev, int slot = kShared) {
        std::lock_guard<std::mutex> lock(mu_);
        return at(dev, slot).retired.size();
    }

    // Frees every buffer of `dev` (current and retired, every slot).  The
    // caller guarantees that nothing pending or replayable references them.
    void release(int dev) {
        std::lock_guard<std::mutex> lock(mu_);
        drop(shared_[dev]);
        for (auto& kv : threads_)
            if (kv.first % kMaxDevices == dev) drop(kv.second);
    }

  private:
    struct Dev {
        void* cur = nullptr;
        size_t bytes = 0;
        std::vector<void*> retired;
    };

    // std::map keeps references to its elements valid across inserts.
    Dev& at(int dev, int slot) {
        if (slot == kShared) return shared_[dev];
        return threads_[static_cast<long long>(slot) * kMaxDevices + dev];
    }

    void drop(Dev& d) {
        for (void* p : d.retired) alloc_.free(p);
        d.retired.clear();
        if (d.cur != nullptr) alloc_.free(d.cur);
        d.cur = nullptr;
        d.bytes = 0;
    }

    Alloc alloc_;
    std::mutex mu_;
    Dev shared_[kMaxDevices];
    std::map<long long, Dev> threads_;
};

}  // namespace mi

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
#pragma once

#include <cstddef>
#include <mutex>
#include <vector>

namespace mi {

// Alloc provides
//   int  alloc(void** p, size_t bytes);   // 0 on success, else an error code
//   void free(void* p);
template <class Alloc>
class WorkspacePool {
  public:
    static constexpr int kMaxDevices = 64;
    static constexpr size_t kGrain = size_t(1) << 20;

    explicit WorkspacePool(Alloc a = Alloc()) : alloc_(a) {}

    // Returns a buffer of at least `bytes` for device `dev`, growing the pool
    // if needed (refused with `capture_err` while `capturing`).  On failure
    // returns nullptr and stores the allocator's error (or capture_err) in
    // *err.
    void* get(int dev, size_t bytes, bool capturing, int capture_err, int* err) {
        std::lock_guard<std::mutex> lock(mu_);
        Dev& d = dev_[dev];
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

    size_t bytes(int dev) {
        std::lock_guard<std::mutex> lock(mu_);
        return dev_[dev].bytes;
    }

    size_t retired_count(int dev) {
        std::lock_guard<std::mutex> lock(mu_);
        return dev_[dev].retired.size();
    }

    // Frees every buffer of `dev` (current and retired).  The caller
    // guarantees that nothing pending or replayable references them.
    void release(int dev) {
        std::lock_guard<std::mutex> lock(mu_);
        Dev& d = dev_[dev];
        for (void* p : d.retired) alloc_.free(p);
        d.retired.clear();
        if (d.cur != nullptr) alloc_.free(d.cur);
        d.cur = nullptr;
        d.bytes = 0;
    }

  private:
    struct Dev {
        void* cur = nullptr;
        size_t bytes = 0;
        std::vector<void*> retired;
    };
    Alloc alloc_;
    std::mutex mu_;
    Dev dev_[kMaxDevices];
};

}  // namespace mi

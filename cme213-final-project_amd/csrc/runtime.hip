// Host runtime of the C ABI: error slot, memory helpers, and the per-device
// workspace used by the deterministic two-pass reductions.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "mi_common.hpp"

namespace mi {

namespace {
thread_local char g_err[512] = "no error";

constexpr int kMaxDevices = 64;
std::mutex g_ws_mutex;
void* g_ws_ptr[kMaxDevices] = {};
size_t g_ws_bytes[kMaxDevices] = {};
}  // namespace

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(static_cast<int>(e), "%s: launch failed: %s", what,
                         hipGetErrorString(e));
    return MI_OK;
}

static int grow_workspace_locked(int dev, size_t bytes, hipStream_t stream) {
    if (g_ws_bytes[dev] >= bytes) return MI_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (stream != nullptr && hipStreamIsCapturing(stream, &cs) == hipSuccess &&
        cs != hipStreamCaptureStatusNone)
        return set_error(MI_ERR_CAPTURE_ALLOC,
                         "workspace of %zu bytes needed during graph capture "
                         "(have %zu); call mi_workspace_reserve first",
                         bytes, g_ws_bytes[dev]);
    // Grow geometrically so a sequence of slightly larger shapes does not
    // reallocate every call.  The old buffer may still be read by queued
    // kernels, so drain the device before releasing it.
    size_t want = round_up(bytes > 2 * g_ws_bytes[dev] ? bytes : 2 * g_ws_bytes[dev],
                           size_t(1) << 20);
    if (g_ws_ptr[dev] != nullptr) {
        hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess)
            return set_error(static_cast<int>(e), "workspace: sync failed: %s",
                             hipGetErrorString(e));
        (void)hipFree(g_ws_ptr[dev]);
        g_ws_ptr[dev] = nullptr;
        g_ws_bytes[dev] = 0;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess)
        return set_error(static_cast<int>(e), "workspace: hipMalloc(%zu) failed: %s",
                         want, hipGetErrorString(e));
    g_ws_ptr[dev] = p;
    g_ws_bytes[dev] = want;
    return MI_OK;
}

void* workspace_get(size_t bytes, hipStream_t stream, int* err) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        *err = set_error(static_cast<int>(e), "hipGetDevice failed: %s", hipGetErrorString(e));
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        *err = set_error(MI_ERR_INVALID_ARG, "device %d out of range", dev);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    int rc = grow_workspace_locked(dev, bytes, stream);
    if (rc != MI_OK) {
        *err = rc;
        return nullptr;
    }
    *err = MI_OK;
    return g_ws_ptr[dev];
}

}  // namespace mi

using mi::set_error;

#define MI_HIP_TRY(call, what)                                                     \
    do {                                                                           \
        hipError_t e_ = (call);                                                    \
        if (e_ != hipSuccess)                                                      \
            return set_error(static_cast<int>(e_), "%s: %s", what,                 \
                             hipGetErrorString(e_));                               \
    } while (0)

extern "C" {

const char* mi_last_error(void) { return mi::g_err; }

const char* mi_version(void) { return "cme213_amd 0.1 gfx950"; }

int mi_device_count(int* count) {
    if (count == nullptr) return set_error(MI_ERR_INVALID_ARG, "count is NULL");
    MI_HIP_TRY(hipGetDeviceCount(count), "hipGetDeviceCount");
    return MI_OK;
}

int mi_set_device(int device) {
    MI_HIP_TRY(hipSetDevice(device), "hipSetDevice");
    return MI_OK;
}

int mi_malloc(void** ptr, size_t bytes) {
    if (ptr == nullptr) return set_error(MI_ERR_INVALID_ARG, "ptr is NULL");
    MI_HIP_TRY(hipMalloc(ptr, bytes == 0 ? 1 : bytes), "hipMalloc");
    return MI_OK;
}

int mi_free(void* ptr) {
    MI_HIP_TRY(hipFree(ptr), "hipFree");
    return MI_OK;
}

int mi_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    MI_HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
    return MI_OK;
}

int mi_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    MI_HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return MI_OK;
}

int mi_memset_zero(void* ptr, size_t bytes, void* stream) {
    MI_HIP_TRY(hipMemsetAsync(ptr, 0, bytes, mi::to_stream(stream)), "hipMemsetAsync");
    return MI_OK;
}

int mi_stream_sync(void* stream) {
    MI_HIP_TRY(hipStreamSynchronize(mi::to_stream(stream)), "hipStreamSynchronize");
    return MI_OK;
}

int mi_device_sync(void) {
    MI_HIP_TRY(hipDeviceSynchronize(), "hipDeviceSynchronize");
    return MI_OK;
}

int mi_workspace_reserve(size_t bytes) {
    int err = MI_OK;
    (void)mi::workspace_get(bytes, nullptr, &err);
    return err;
}

size_t mi_workspace_bytes(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= mi::kMaxDevices) return 0;
    std::lock_guard<std::mutex> lock(mi::g_ws_mutex);
    return mi::g_ws_bytes[dev];
}

}  // extern "C"

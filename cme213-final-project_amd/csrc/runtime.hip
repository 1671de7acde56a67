// Host runtime of the C ABI: error slot, memory helpers, and the per-device
// workspace used by the deterministic two-pass reductions.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "mi_common.hpp"
#include "workspace_pool.hpp"

namespace mi {

namespace {
thread_local char g_err[512] = "no error";

struct HipAlloc {
    int alloc(void** p, size_t bytes) { return static_cast<int>(hipMalloc(p, bytes)); }
    void free(void* p) { (void)hipFree(p); }
};

WorkspacePool<HipAlloc> g_ws;
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

static int current_device(int* dev) {
    hipError_t e = hipGetDevice(dev);
    if (e != hipSuccess)
        return set_error(static_cast<int>(e), "hipGetDevice failed: %s", hipGetErrorString(e));
    if (*dev < 0 || *dev >= WorkspacePool<HipAlloc>::kMaxDevices)
        return set_error(MI_ERR_INVALID_ARG, "device %d out of range", *dev);
    return MI_OK;
}

// The workspace slot of a call on `stream`: the calling thread's own slot on
// the per-thread default stream (two host threads' per-thread streams run
// concurrently), else the device's shared slot.
static int stream_slot(hipStream_t stream) {
    return stream == hipStreamPerThread ? thread_slot() : WorkspacePool<HipAlloc>::kShared;
}

// Growth never frees the buffer it replaces (queued kernels, a launch on
// another thread or an instantiated graph may still use it) and never
// synchronises: the old buffer is retired and kept until
// mi_workspace_release().
void* workspace_get(size_t bytes, hipStream_t stream, int* err) {
    int dev = 0;
    if (int rc = current_device(&dev)) {
        *err = rc;
        return nullptr;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool capturing = stream != nullptr &&
                           hipStreamIsCapturing(stream, &cs) == hipSuccess &&
                           cs != hipStreamCaptureStatusNone;
    const int slot = stream_slot(stream);
    int rc = MI_OK;
    void* p = g_ws.get(dev, slot, bytes, capturing, MI_ERR_CAPTURE_ALLOC, &rc);
    if (p == nullptr) {
        if (rc == MI_ERR_CAPTURE_ALLOC)
            *err = set_error(MI_ERR_CAPTURE_ALLOC,
                             "workspace of %zu bytes needed during graph capture (have %zu); "
                             "call mi_workspace_reserve (mi_workspace_reserve_stream for the "
                             "per-thread stream) first",
                             bytes, g_ws.bytes(dev, slot));
        else
            *err = set_error(rc, "workspace: hipMalloc of %zu bytes failed: %s", bytes,
                             hipGetErrorString(static_cast<hipError_t>(rc)));
        return nullptr;
    }
    *err = MI_OK;
    return p;
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

int mi_workspace_reserve_stream(size_t bytes, void* stream) {
    hipStream_t st = mi::to_stream(stream);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (st != nullptr && hipStreamIsCapturing(st, &cs) == hipSuccess &&
        cs != hipStreamCaptureStatusNone)
        return set_error(MI_ERR_CAPTURE_ALLOC,
                         "mi_workspace_reserve_stream: the stream is capturing; reserve before "
                         "capture");
    int err = MI_OK;
    (void)mi::workspace_get(bytes, st, &err);
    return err;
}

static size_t workspace_bytes_of(hipStream_t stream) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 ||
        dev >= mi::WorkspacePool<mi::HipAlloc>::kMaxDevices)
        return 0;
    return mi::g_ws.bytes(dev, mi::stream_slot(stream));
}

size_t mi_workspace_bytes(void) { return workspace_bytes_of(nullptr); }

size_t mi_workspace_bytes_stream(void* stream) {
    return workspace_bytes_of(mi::to_stream(stream));
}

int mi_workspace_release(void) {
    int dev = 0;
    if (int rc = mi::current_device(&dev)) return rc;
    MI_HIP_TRY(hipDeviceSynchronize(), "mi_workspace_release: hipDeviceSynchronize");
    mi::g_ws.release(dev);
    return MI_OK;
}

}  // extern "C"

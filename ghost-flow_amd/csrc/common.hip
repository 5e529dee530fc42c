// common.hip -- error state, lazy device init, pointer checks, scratch.
#include "common.hpp"

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

namespace gfh {

namespace {
thread_local std::string g_last_error = "No error";
std::atomic<int> g_pointer_checks{1};
std::once_flag g_init_once;
int g_init_status = GFH_UNKNOWN;
std::string g_init_message;
}  // namespace

int set_error(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

void clear_error() { g_last_error = "No error"; }

const char *last_error() { return g_last_error.c_str(); }

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(GFH_COMPUTATION_FAILED, "%s: launch failed: %s", what, hipGetErrorString(e));
    return GFH_SUCCESS;
}

int ensure_init() {
    std::call_once(g_init_once, [] {
        int n = 0;
        hipError_t e = hipGetDeviceCount(&n);
        if (e != hipSuccess || n == 0) {
            g_init_status = GFH_COMPUTATION_FAILED;
            g_init_message = std::string("no HIP device available: ") +
                             (e != hipSuccess ? hipGetErrorString(e) : "device count is 0");
            return;
        }
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) {
            g_init_status = GFH_COMPUTATION_FAILED;
            g_init_message = "hipGetDevice failed";
            return;
        }
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
            g_init_status = GFH_COMPUTATION_FAILED;
            g_init_message = "hipGetDeviceProperties failed";
            return;
        }
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
            g_init_status = GFH_COMPUTATION_FAILED;
            g_init_message = std::string("kernels are built for gfx950, device is ") + prop.gcnArchName;
            return;
        }
        g_init_status = GFH_SUCCESS;
    });
    if (g_init_status != GFH_SUCCESS) return set_error(g_init_status, "%s", g_init_message.c_str());
    return GFH_SUCCESS;
}

int check_device_ptr(const void *p, const char *name) {
    if (!g_pointer_checks.load(std::memory_order_relaxed)) return GFH_SUCCESS;
    hipPointerAttribute_t attr;
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();  // do not leave the lookup failure for the next launch check
        return set_error(GFH_INVALID_DATA, "%s is not a device pointer (%s)", name, hipGetErrorString(e));
    }
    if (attr.type != hipMemoryTypeDevice && attr.type != hipMemoryTypeManaged)
        return set_error(GFH_INVALID_DATA, "%s is not device memory (memory type %d)", name, (int)attr.type);
    return GFH_SUCCESS;
}

int require_ptr(const void *p, const char *name) {
    if (!p) return set_error(GFH_NULL_POINTER, "%s is NULL", name);
    return check_device_ptr(p, name);
}

int require_range(const void *p, size_t bytes, const char *name) {
    if (!p) {
        if (bytes == 0) return GFH_SUCCESS;
        return set_error(GFH_NULL_POINTER, "%s is NULL", name);
    }
    if (!g_pointer_checks.load(std::memory_order_relaxed)) return GFH_SUCCESS;
    GFH_TRY(check_device_ptr(p, name));
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    hipError_t e = hipMemGetAddressRange(&base, &size, const_cast<void *>(p));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return set_error(GFH_INVALID_DATA, "%s: no device allocation contains this address (%s)", name,
                         hipGetErrorString(e));
    }
    const uintptr_t lo = reinterpret_cast<uintptr_t>(base);
    const uintptr_t hi = lo + size;
    const uintptr_t at = reinterpret_cast<uintptr_t>(p);
    if (at < lo || bytes > hi - at)
        return set_error(GFH_INVALID_SHAPE, "%s: %zu bytes needed but only %zu remain in its allocation", name,
                         bytes, (size_t)(hi - at));
    return GFH_SUCCESS;
}

int optional_range(const void *p, size_t bytes, const char *name) {
    if (!p) return GFH_SUCCESS;
    return require_range(p, bytes, name);
}

namespace {

// Zeroes a new counter buffer on its stream.  A fill kernel rather than
// hipMemsetAsync: where a stream is captured into a graph, memset nodes have
// given wrong results on replays after the first.
__global__ void zero_counters_kernel(int *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

// The library's per-stream buffers (and stream-ordered scratch) are
// allocated on first use.  On a stream that is being captured into a graph
// that allocation would become part of the graph, so it is refused: the
// caller runs the call once on the stream before capturing it (or passes a
// workspace), and the captured calls then allocate nothing.
int refuse_during_capture(hipStream_t s, const char *what) {
    if (s == nullptr) return GFH_SUCCESS;  // the legacy default stream is never captured
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) {
        (void)hipGetLastError();
        return GFH_SUCCESS;
    }
    if (st != hipStreamCaptureStatusNone)
        return set_error(GFH_ALLOCATION_FAILED,
                         "%s: the stream is being captured into a graph; run the call once on this stream before "
                         "capturing it (per-stream buffers are allocated on first use) or pass a workspace",
                         what);
    return GFH_SUCCESS;
}

}  // namespace

Scratch::~Scratch() {
    if (owned_ && p_) (void)hipFreeAsync(p_, s_);
}

int Scratch::acquire(void *user, size_t user_bytes, size_t need, hipStream_t s) {
    if (need == 0) need = 16;
    if (user) {
        if (user_bytes < need)
            return set_error(GFH_INVALID_SHAPE, "workspace of %zu bytes is smaller than the %zu required",
                             user_bytes, need);
        GFH_TRY(check_device_ptr(user, "workspace"));
        p_ = user;
        owned_ = false;
        return GFH_SUCCESS;
    }
    GFH_TRY(refuse_during_capture(s, "workspace"));
    hipError_t e = hipMallocAsync(&p_, need, s);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        p_ = nullptr;
        return set_error(GFH_ALLOCATION_FAILED, "hipMallocAsync(%zu) failed: %s", need, hipGetErrorString(e));
    }
    owned_ = true;
    s_ = s;
    return GFH_SUCCESS;
}

namespace {
struct StreamState {
    int *counters = nullptr;
    size_t ncounters = 0;
    void *ws = nullptr;
    size_t ws_bytes = 0;
};
std::mutex g_state_mu;
std::map<std::pair<int, hipStream_t>, StreamState> g_states;
std::vector<void *> g_retired;  // outgrown buffers (maybe still in use by queued work), freed at shutdown

int current_state(hipStream_t s, StreamState **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return set_error(GFH_COMPUTATION_FAILED, "hipGetDevice failed");
    }
    *out = &g_states[std::make_pair(dev, s)];
    return GFH_SUCCESS;
}
}  // namespace

int stream_counters(hipStream_t s, size_t count, int **out) {
    std::lock_guard<std::mutex> lock(g_state_mu);
    StreamState *st = nullptr;
    GFH_TRY(current_state(s, &st));
    if (st->ncounters < count) {
        GFH_TRY(refuse_during_capture(s, "split-K counters"));
        size_t want = 4096;
        while (want < count) want *= 2;
        int *p = nullptr;
        hipError_t e = hipMallocAsync(reinterpret_cast<void **>(&p), want * sizeof(int), s);
        if (e == hipSuccess) {
            hipLaunchKernelGGL(zero_counters_kernel, dim3((unsigned)((want + 255) / 256)), dim3(256), 0, s, p, want);
            e = hipGetLastError();
        }
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return set_error(GFH_ALLOCATION_FAILED, "counter buffer allocation failed: %s", hipGetErrorString(e));
        }
        if (st->counters) g_retired.push_back(st->counters);
        st->counters = p;
        st->ncounters = want;
    }
    *out = st->counters;
    return GFH_SUCCESS;
}

int device_cu_count() {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cache[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

int stream_workspace(hipStream_t s, size_t bytes, void **out) {
    std::lock_guard<std::mutex> lock(g_state_mu);
    StreamState *st = nullptr;
    GFH_TRY(current_state(s, &st));
    if (st->ws_bytes < bytes) {
        GFH_TRY(refuse_during_capture(s, "split-K workspace"));
        size_t want = (size_t)1 << 20;
        while (want < bytes) want *= 2;
        void *p = nullptr;
        hipError_t e = hipMallocAsync(&p, want, s);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return set_error(GFH_ALLOCATION_FAILED, "workspace allocation (%zu bytes) failed: %s", want,
                             hipGetErrorString(e));
        }
        if (st->ws) g_retired.push_back(st->ws);
        st->ws = p;
        st->ws_bytes = want;
    }
    *out = st->ws;
    return GFH_SUCCESS;
}

void release_stream_state() {
    std::lock_guard<std::mutex> lock(g_state_mu);
    if (g_states.empty() && g_retired.empty()) return;
    (void)hipDeviceSynchronize();
    for (auto &kv : g_states) {
        if (kv.second.counters) (void)hipFree(kv.second.counters);
        if (kv.second.ws) (void)hipFree(kv.second.ws);
    }
    for (void *p : g_retired) (void)hipFree(p);
    g_states.clear();
    g_retired.clear();
}

int set_pointer_checks(int enabled) {
    g_pointer_checks.store(enabled ? 1 : 0);
    return GFH_SUCCESS;
}

}  // namespace gfh

// km_runtime.cpp - error reporting, backend selection and staging memory.
#include "km_runtime.hpp"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <strings.h>

#include "kmamba_cuda_utils.h"
#include "kmamba_km.h"

namespace {
thread_local char g_err[512] = "";

std::once_flag g_backend_once;
std::once_flag g_probe_once;
int g_device_count = 0;
int g_usable = 0;
char g_probe_msg[256] = "";

void probe_devices() {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        std::snprintf(g_probe_msg, sizeof g_probe_msg, "hipGetDeviceCount: %s (count %d)",
                      hipGetErrorString(e), n);
        (void)hipGetLastError();
        g_device_count = 0;
        g_usable = 0;
        return;
    }
    g_device_count = n;
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, 0);
    g_usable = (e == hipSuccess) ? 1 : 0;
    if (!g_usable)
        std::snprintf(g_probe_msg, sizeof g_probe_msg, "hipGetDeviceProperties: %s",
                      hipGetErrorString(e));
}

void parse_backend_env() {
    const char *env = std::getenv("KMAMBA_BACKEND");
    if (!env || strcasecmp(env, "auto") == 0) {
        kmamba_backend_preference = KMAMBA_BACKEND_AUTO;
    } else if (strcasecmp(env, "cpu") == 0) {
        kmamba_backend_preference = KMAMBA_BACKEND_CPU;
        std::fprintf(stderr, "[k-mamba] Backend forced to CPU via environment "
                             "(this library has no CPU compute path)\n");
    } else if (strcasecmp(env, "gpu") == 0 || strcasecmp(env, "cuda") == 0) {
        kmamba_backend_preference = KMAMBA_BACKEND_GPU;
        std::fprintf(stderr, "[k-mamba] Backend forced to GPU via environment\n");
    } else {
        std::fprintf(stderr, "[k-mamba] Warning: Unknown KMAMBA_BACKEND='%s', using auto\n", env);
        kmamba_backend_preference = KMAMBA_BACKEND_AUTO;
    }
}

std::mutex g_stage_mu;
void *g_stage_ptr[64] = {};
size_t g_stage_size[64] = {};
}  // namespace

extern "C" {

KMambaBackend kmamba_backend_preference = KMAMBA_BACKEND_AUTO;

int kmamba_cuda_available(void) {
    std::call_once(g_probe_once, probe_devices);
    if (!g_usable && g_probe_msg[0]) km::set_error("%s", g_probe_msg);
    return g_usable;
}

int kmamba_cuda_device_count(void) {
    std::call_once(g_probe_once, probe_devices);
    return g_device_count;
}

int kmamba_cuda_current_device(void) {
    if (!kmamba_cuda_available()) return -1;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return -1;
    return dev;
}

void kmamba_backend_init(void) { std::call_once(g_backend_once, parse_backend_env); }

KMambaBackend kmamba_backend_select(void) {
    kmamba_backend_init();
    switch (kmamba_backend_preference) {
    case KMAMBA_BACKEND_CPU:
        return KMAMBA_BACKEND_CPU;
    case KMAMBA_BACKEND_GPU:
        if (!kmamba_cuda_available()) {
            std::fprintf(stderr, "[k-mamba] Error: GPU requested but not available\n");
            return KMAMBA_BACKEND_CPU;
        }
        return KMAMBA_BACKEND_GPU;
    case KMAMBA_BACKEND_AUTO:
    default:
        return kmamba_cuda_available() ? KMAMBA_BACKEND_GPU : KMAMBA_BACKEND_CPU;
    }
}

const char *km_last_error(void) { return g_err; }
void km_clear_error(void) { g_err[0] = '\0'; }
const char *km_version(void) { return "libkmamba-mi355x 0.1 (gfx950)"; }

size_t km_device_bytes_held(void) {
    size_t total = km::Workspace::held();
    std::lock_guard<std::mutex> guard(g_stage_mu);
    for (int d = 0; d < 64; ++d) total += g_stage_size[d];
    return total;
}

size_t km_release_stream(void *stream) {
    km::clear_error();
    return km::Workspace::release(static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace km {

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

bool gpu_ready() {
    if (kmamba_backend_select() != KMAMBA_BACKEND_GPU) {
        if (kmamba_backend_preference == KMAMBA_BACKEND_CPU)
            set_error("KMAMBA_BACKEND=cpu: libkmamba has no CPU compute path");
        else if (g_probe_msg[0])
            set_error("no usable HIP device (%s)", g_probe_msg);
        else
            set_error("no usable HIP device");
        return false;
    }
    return true;
}

bool is_device_ptr(const void *p) {
    if (!p) return false;
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();   // unregistered host memory reports an error
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

void *Staging::reserve(size_t bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        set_error("staging: no current HIP device");
        return nullptr;
    }
    if (g_stage_size[dev] >= bytes && g_stage_ptr[dev]) return g_stage_ptr[dev];
    if (g_stage_ptr[dev]) {
        (void)hipDeviceSynchronize();
        (void)hipFree(g_stage_ptr[dev]);
        g_stage_ptr[dev] = nullptr;
        g_stage_size[dev] = 0;
    }
    size_t want = align_up(bytes, size_t(1) << 20);
    void *p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
        (void)hipGetLastError();
        set_error("staging: hipMalloc(%zu) failed", want);
        return nullptr;
    }
    g_stage_ptr[dev] = p;
    g_stage_size[dev] = want;
    return p;
}

namespace {
// Workspace blocks keyed by (device, stream, use): launches on different
// streams never share one, nested entry points on one stream use different
// uses, and a block is only freed (to grow it) after its own stream has
// drained.
struct WsEntry {
    int dev;
    hipStream_t stream;
    WsUse use;
    void *ptr;
    size_t size;
    unsigned long long last;   // g_ws_tick at the last reserve
};
constexpr int kMaxWs = 64;
std::mutex g_ws_mu;
WsEntry g_ws[kMaxWs];
int g_ws_n = 0;
unsigned long long g_ws_tick = 0;

// Frees entry i (its device drained first: the entry's stream may be gone)
// and removes it from the table. Called under g_ws_mu.
void ws_drop(int i) {
    WsEntry &e = g_ws[i];
    if (e.ptr) {
        int cur = 0;
        (void)hipGetDevice(&cur);
        if (e.dev != cur) (void)hipSetDevice(e.dev);
        (void)hipDeviceSynchronize();
        (void)hipFree(e.ptr);
        if (e.dev != cur) (void)hipSetDevice(cur);
    }
    g_ws[i] = g_ws[--g_ws_n];
}
}  // namespace

void *Workspace::reserve(size_t bytes, hipStream_t stream, WsUse use, bool *fresh, size_t *got) {
    std::lock_guard<std::mutex> guard(g_ws_mu);
    if (fresh) *fresh = false;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
        set_error("workspace: no current HIP device");
        return nullptr;
    }
    int idx = -1;
    for (int i = 0; i < g_ws_n; ++i)
        if (g_ws[i].dev == dev && g_ws[i].stream == stream && g_ws[i].use == use) idx = i;
    if (idx < 0) {
        if (g_ws_n == kMaxWs) {
            // Evict the least recently used block of another (device, stream):
            // blocks of this stream may be in use by the calling entry point.
            int lru = -1;
            for (int i = 0; i < g_ws_n; ++i)
                if (!(g_ws[i].dev == dev && g_ws[i].stream == stream) &&
                    (lru < 0 || g_ws[i].last < g_ws[lru].last))
                    lru = i;
            if (lru < 0) {
                set_error("workspace: table full");
                return nullptr;
            }
            ws_drop(lru);
        }
        idx = g_ws_n++;
        g_ws[idx] = WsEntry{dev, stream, use, nullptr, 0, 0};
    }
    WsEntry *e = &g_ws[idx];
    e->last = ++g_ws_tick;
    if (e->size >= bytes && e->ptr) {
        if (got) *got = e->size;
        return e->ptr;
    }
    if (e->ptr) {
        (void)hipStreamSynchronize(stream);   // earlier kernels on this stream may use the old block
        (void)hipFree(e->ptr);
        e->ptr = nullptr;
        e->size = 0;
    }
    const size_t want = align_up(bytes > 0 ? bytes : 1, size_t(1) << 20);
    void *p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
        (void)hipGetLastError();
        set_error("workspace: hipMalloc(%zu) failed", want);
        return nullptr;
    }
    e->ptr = p;
    e->size = want;
    if (fresh) *fresh = true;
    if (got) *got = want;
    return p;
}

size_t Workspace::release(hipStream_t stream) {
    std::lock_guard<std::mutex> guard(g_ws_mu);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    size_t freed = 0;
    bool synced = false;
    for (int i = g_ws_n - 1; i >= 0; --i) {
        if (g_ws[i].dev != dev || g_ws[i].stream != stream) continue;
        if (!synced) {
            (void)hipStreamSynchronize(stream);
            synced = true;
        }
        freed += g_ws[i].size;
        (void)hipFree(g_ws[i].ptr);
        g_ws[i] = g_ws[--g_ws_n];
    }
    return freed;
}

void *Workspace::find(hipStream_t stream, WsUse use) {
    std::lock_guard<std::mutex> guard(g_ws_mu);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    for (int i = 0; i < g_ws_n; ++i)
        if (g_ws[i].dev == dev && g_ws[i].stream == stream && g_ws[i].use == use) return g_ws[i].ptr;
    return nullptr;
}

size_t Workspace::held() {
    std::lock_guard<std::mutex> guard(g_ws_mu);
    size_t total = 0;
    for (int i = 0; i < g_ws_n; ++i) total += g_ws[i].size;
    return total;
}

namespace {
void *g_pin_ptr = nullptr;
size_t g_pin_size = 0;
}  // namespace

void *PinnedStaging::reserve(size_t bytes) {
    if (g_pin_size >= bytes && g_pin_ptr) return g_pin_ptr;
    if (g_pin_ptr) {
        (void)hipDeviceSynchronize();   // a copy may still read the old block
        (void)hipHostFree(g_pin_ptr);
        g_pin_ptr = nullptr;
        g_pin_size = 0;
    }
    const size_t want = align_up(bytes, size_t(1) << 20);
    void *p = nullptr;
    if (hipHostMalloc(&p, want, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        set_error("pinned staging: hipHostMalloc(%zu) failed", want);
        return nullptr;
    }
    g_pin_ptr = p;
    g_pin_size = want;
    return p;
}

void Staging::lock() { g_stage_mu.lock(); }
void Staging::unlock() { g_stage_mu.unlock(); }

}  // namespace km

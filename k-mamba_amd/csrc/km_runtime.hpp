// km_runtime.hpp - internal runtime helpers of libkmamba (not installed).
//
// Thread-local error reporting, HIP error checks that return -1 instead of
// exiting (the reference's OM_CHECK exits the process, include/scan.h:18-26),
// host/device pointer classification, and the per-device staging workspace
// used by the host-pointer entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>
#include <functional>

namespace km {

void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// True when the library may use the GPU: KMAMBA_BACKEND is not "cpu" and a
// HIP device is present. Sets an error message otherwise.
bool gpu_ready();

// True when p is device or managed memory that kernels may dereference.
bool is_device_ptr(const void *p);

// Per-device staging arena for the host-pointer API. reserve() grows it (the
// only allocation on these paths) and returns a base pointer; the caller
// carves sub-buffers with carve(). Not reentrant across threads for the same
// device: a mutex serialises host-pointer calls.
struct Staging {
    static void *reserve(size_t bytes);      // nullptr on failure (error set)
    static void lock();
    static void unlock();
};

// Pinned host staging buffer (hipHostMalloc, process-wide, grow-only) for
// packing many small host arrays into one DMA. Use under Staging::lock(); the
// buffer may be reused once the copy that read it has completed.
struct PinnedStaging {
    static void *reserve(size_t bytes);      // nullptr on failure (error set)
};

// What a workspace block is for. Each use has its own block, so an entry
// point that holds one block (the Mamba-1 block's activations) can call
// another that reserves scratch (the Scan1D split's segment states) on the
// same stream without the two aliasing.
enum class WsUse : int {
    Scan1DSplit = 0,   // segment end states, incoming states, flags
    Scan1DBwd,         // checkpoints and per-workgroup partial sums
    Scan1DM1,          // M = 1 backward's per-workgroup ddelta partials
    ScanNDPlan,        // per-level fallback's plan offsets
    ScanNDM3,          // Mamba-3 branch: plan offsets and rotated states
    ScanNDFlow,        // dataflow counters, status, epoch and flags (kept)
    ScanNDBwd,         // adjoint plan, neighbours, partials
    ConvBwd,           // dkernel / dbias partial slots
    Block,             // Mamba-1 block activations
    Model,             // stacked model activations, head, logits
    Count
};

// Scratch for kernels that need device memory beyond their inputs and
// outputs (e.g. the Scan1D backward's partial sums), used when the caller
// passes no workspace. One block per (device, stream, use): grows on demand
// (after draining that stream) and is reused by later calls on the same
// stream, so calls on different streams never share it. When the table is
// full, the least recently used block of another (device, stream) is freed
// after its device drains. `fresh` (optional) is set when the returned block
// was just allocated (its contents are undefined); `got` (optional) receives
// the block's size, at least `bytes`. Host threads that enqueue
// on one stream concurrently must serialise their calls.
struct Workspace {
    static void *reserve(size_t bytes, hipStream_t stream, WsUse use, bool *fresh = nullptr,
                         size_t *got = nullptr);   // nullptr on failure (error set)
    // Frees every block of (current device, stream) after draining the
    // stream. Returns the bytes freed.
    static size_t release(hipStream_t stream);
    // Device bytes held by all blocks (every device and stream).
    static size_t held();
    // The block of (current device, stream, use), or nullptr; allocates
    // nothing.
    static void *find(hipStream_t stream, WsUse use);
};

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Copies between pageable host memory and device memory through a ring of
// pinned slots of about kPipeSlotBytes: each slot's DMA, on a non-blocking
// copy stream, overlaps the host memcpy of the next slot, which is split
// over a small pool of host threads. Calls from several threads serialise.
constexpr size_t kPipeSlotBytes = size_t(8) << 20;
// Host -> device; the copies start after the work already enqueued on
// `stream`, and the call returns when they have completed.
int host_pipe_upload(void *dst_dev, const void *src_host, size_t bytes, hipStream_t stream);
// Device -> host in whole rows of row_bytes; returns when dst_host holds
// every byte. If `ready` is given, the piece that ends at row r is enqueued
// once the event ready(r) (nullptr: no wait), recorded when rows [0, r) of
// src_dev are written, has completed.
int host_pipe_download(void *dst_host, const void *src_dev, size_t bytes, size_t row_bytes,
                       const std::function<hipEvent_t(size_t)> &ready);
// Synchronous copies of the host-pointer entry points, ordered like
// hipMemcpy after the work on the null stream: pageable buffers of 4 MB or
// more go through the pinned ring, the rest (and pinned memory) through
// hipMemcpy.
hipError_t copy_h2d(void *dst_dev, const void *src_host, size_t bytes);
hipError_t copy_d2h(void *dst_host, const void *src_dev, size_t bytes);
// Runs f(0..n-1) over the same host thread pool; returns when all are done.
void host_parallel_for(size_t n, const std::function<void(size_t)> &f);

// Bump allocator over a reserved staging block.
struct Carver {
    char *base;
    size_t off = 0;
    explicit Carver(void *b) : base(static_cast<char *>(b)) {}
    template <typename T> T *take(size_t count) {
        T *p = reinterpret_cast<T *>(base + off);
        off = align_up(off + count * sizeof(T), 256);
        return p;
    }
};

// Host <-> device helpers for the staging path: copy when the pointer is host
// memory, pass through when it is already device memory.
struct Staged {
    const void *host;   // caller pointer
    void *dev;          // device pointer used by kernels
    size_t bytes;
    bool copied;
};

}  // namespace km

#define KM_HIP_TRY(call)                                                        \
    do {                                                                        \
        hipError_t _e = (call);                                                 \
        if (_e != hipSuccess) {                                                 \
            ::km::set_error("%s:%d: %s failed: %s", __FILE__, __LINE__, #call,  \
                            hipGetErrorString(_e));                             \
            return -1;                                                          \
        }                                                                       \
    } while (0)

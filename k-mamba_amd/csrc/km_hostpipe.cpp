// km_hostpipe.cpp - copies between pageable host memory and the device
// through a ring of pinned slots.
//
// A copy from pageable memory cannot be a single DMA: the bytes have to pass
// through pinned memory. Done naively (one host memcpy, then one DMA) the two
// run back to back, and the host memcpy runs on one thread. Here the transfer
// is cut into slot-sized pieces: the DMA of one piece (on a non-blocking copy
// stream) overlaps the host memcpy of the next, and each host memcpy is split
// over a small pool of host threads. A download piece may also wait on an
// event of the producing stream, so it starts as soon as the rows it carries
// are written, while later rows are still being computed.
#include "km_runtime.hpp"

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include <unistd.h>

namespace km {
namespace {

// Runs f(0..n-1) on the calling thread and the pool's workers and returns
// when every index is done. The pool is created on first use and never torn
// down (its threads are detached and sleep on a condition variable), so no
// thread object is destroyed while running at process exit. A process forked
// after the pool started has none of its threads: it builds its own.
class CopyPool {
  public:
    static CopyPool &get() {
        static std::mutex mu;
        static CopyPool *pool = nullptr;
        static pid_t owner = 0;
        std::lock_guard<std::mutex> g(mu);
        if (!pool || owner != getpid()) {
            pool = new CopyPool();   // a forked child's inherited pool is left as is
            owner = getpid();
        }
        return *pool;
    }
    int threads() const { return nworkers_ + 1; }

    void run(size_t n, const std::function<void(size_t)> &f) {
        if (n == 0) return;
        if (nworkers_ == 0 || n == 1) {
            for (size_t i = 0; i < n; ++i) f(i);
            return;
        }
        std::lock_guard<std::mutex> one_job(job_mu_);   // one job at a time
        {
            std::lock_guard<std::mutex> g(mu_);
            fn_ = &f;
            n_ = n;
            next_.store(0);
            pending_ = nworkers_;
            ++gen_;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> g(mu_);
        done_cv_.wait(g, [&] { return pending_ == 0; });
        fn_ = nullptr;
    }

  private:
    CopyPool() {
        const unsigned hc = std::thread::hardware_concurrency();
        nworkers_ = static_cast<int>(std::min(7u, hc > 1 ? hc - 1 : 0u));
        for (int i = 0; i < nworkers_; ++i) std::thread([this] { loop(); }).detach();
    }
    void work() {
        for (;;) {
            const size_t i = next_.fetch_add(1);
            if (i >= n_) break;
            (*fn_)(i);
        }
    }
    void loop() {
        unsigned long seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> g(mu_);
                cv_.wait(g, [&] { return gen_ != seen; });
                seen = gen_;
            }
            work();
            std::lock_guard<std::mutex> g(mu_);
            if (--pending_ == 0) done_cv_.notify_one();
        }
    }

    int nworkers_ = 0;
    std::mutex job_mu_, mu_;
    std::condition_variable cv_, done_cv_;
    const std::function<void(size_t)> *fn_ = nullptr;
    size_t n_ = 0;
    std::atomic<size_t> next_{0};
    int pending_ = 0;
    unsigned long gen_ = 0;
};

// One pinned ring per process (grow-only) and one copy stream per device,
// used under g_pipe_mu.
constexpr int kSlots = 6;
std::mutex g_pipe_mu;
char *g_ring = nullptr;
size_t g_slot = 0;
hipEvent_t g_slot_ev[kSlots] = {};
hipEvent_t g_start_ev = nullptr;
hipStream_t g_copy_stream[64] = {};

bool ring_reserve(size_t slot_bytes) {
    if (!g_start_ev) {
        for (int i = 0; i <= kSlots; ++i)
            if (hipEventCreateWithFlags(i < kSlots ? &g_slot_ev[i] : &g_start_ev, hipEventDisableTiming) !=
                hipSuccess) {
                (void)hipGetLastError();
                set_error("host pipe: hipEventCreate failed");
                return false;
            }
    }
    if (g_ring && g_slot >= slot_bytes) return true;
    if (g_ring) {
        for (int i = 0; i < kSlots; ++i) (void)hipEventSynchronize(g_slot_ev[i]);
        (void)hipHostFree(g_ring);
        g_ring = nullptr;
        g_slot = 0;
    }
    void *p = nullptr;
    const size_t want = align_up(slot_bytes, size_t(1) << 20);
    if (hipHostMalloc(&p, want * kSlots, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        set_error("host pipe: hipHostMalloc(%zu) failed", want * kSlots);
        return false;
    }
    g_ring = static_cast<char *>(p);
    g_slot = want;
    return true;
}

hipStream_t copy_stream() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        set_error("host pipe: no current HIP device");
        return nullptr;
    }
    if (!g_copy_stream[dev] && hipStreamCreateWithFlags(&g_copy_stream[dev], hipStreamNonBlocking) != hipSuccess) {
        (void)hipGetLastError();
        g_copy_stream[dev] = nullptr;
        set_error("host pipe: hipStreamCreate failed");
    }
    return g_copy_stream[dev];
}

// memcpy split over the pool in pieces of at least 256 KB.
void pool_memcpy(void *dst, const void *src, size_t bytes) {
    CopyPool &pool = CopyPool::get();
    const size_t parts = std::max<size_t>(1, std::min<size_t>(pool.threads(), bytes >> 18));
    const size_t step = align_up((bytes + parts - 1) / parts, 4096);
    pool.run(parts, [&](size_t i) {
        const size_t off = i * step;
        if (off < bytes)
            std::memcpy(static_cast<char *>(dst) + off, static_cast<const char *>(src) + off,
                        std::min(step, bytes - off));
    });
}

}  // namespace

void host_parallel_for(size_t n, const std::function<void(size_t)> &f) { CopyPool::get().run(n, f); }

int host_pipe_upload(void *dst_dev, const void *src_host, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return 0;
    std::lock_guard<std::mutex> guard(g_pipe_mu);
    hipStream_t cs = copy_stream();
    if (!cs || !ring_reserve(kPipeSlotBytes)) return -1;
    const size_t S = g_slot;
    const size_t pieces = (bytes + S - 1) / S;
    // The copies follow the work already enqueued on `stream` (which may still
    // read the destination). The host waits for it rather than the copy
    // stream: a copy queued behind a wait on another stream's event has run
    // as a blit kernel on the compute units instead of on a DMA engine.
    KM_HIP_TRY(hipEventRecord(g_start_ev, stream));
    KM_HIP_TRY(hipEventSynchronize(g_start_ev));
    for (size_t j = 0; j < pieces; ++j) {
        const int k = static_cast<int>(j % kSlots);
        const size_t off = j * S, len = std::min(S, bytes - off);
        KM_HIP_TRY(hipEventSynchronize(g_slot_ev[k]));   // the last DMA that read slot k, of any call
        pool_memcpy(g_ring + k * S, static_cast<const char *>(src_host) + off, len);
        KM_HIP_TRY(hipMemcpyAsync(static_cast<char *>(dst_dev) + off, g_ring + k * S, len,
                                  hipMemcpyHostToDevice, cs));
        KM_HIP_TRY(hipEventRecord(g_slot_ev[k], cs));
    }
    KM_HIP_TRY(hipEventSynchronize(g_slot_ev[(pieces - 1) % kSlots]));   // the last piece, so all
    return 0;
}

int host_pipe_download(void *dst_host, const void *src_dev, size_t bytes, size_t row_bytes,
                       const std::function<hipEvent_t(size_t)> &ready) {
    if (bytes == 0) return 0;
    std::lock_guard<std::mutex> guard(g_pipe_mu);
    hipStream_t cs = copy_stream();
    // Pieces are whole rows, so each waits on the event of the last row it carries.
    const size_t rows_per = std::max<size_t>(1, kPipeSlotBytes / row_bytes);
    if (!cs || !ring_reserve(rows_per * row_bytes)) return -1;
    const size_t S = rows_per * row_bytes;
    const size_t pieces = (bytes + S - 1) / S;
    auto issue = [&](size_t j) -> int {
        const int k = static_cast<int>(j % kSlots);
        const size_t off = j * S, len = std::min(S, bytes - off);
        if (ready) {
            // Rows [0, end) written; waited for on the host (see upload).
            hipEvent_t ev = ready((off + len + row_bytes - 1) / row_bytes);
            if (ev) KM_HIP_TRY(hipEventSynchronize(ev));
        }
        KM_HIP_TRY(hipMemcpyAsync(g_ring + k * S, static_cast<const char *>(src_dev) + off, len,
                                  hipMemcpyDeviceToHost, cs));
        KM_HIP_TRY(hipEventRecord(g_slot_ev[k], cs));
        return 0;
    };
    for (size_t j = 0; j < pieces && j < kSlots; ++j)
        if (issue(j) != 0) return -1;
    for (size_t j = 0; j < pieces; ++j) {
        const int k = static_cast<int>(j % kSlots);
        const size_t off = j * S, len = std::min(S, bytes - off);
        KM_HIP_TRY(hipEventSynchronize(g_slot_ev[k]));
        pool_memcpy(static_cast<char *>(dst_host) + off, g_ring + k * S, len);
        if (j + kSlots < pieces && issue(j + kSlots) != 0) return -1;
    }
    return 0;
}

namespace {
// Pageable host memory: what hipMemcpy would stage through its own buffers.
bool pageable(const void *p) {
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();   // unregistered host memory reports an error
        return true;
    }
    return attr.type != hipMemoryTypeHost && attr.type != hipMemoryTypeDevice &&
           attr.type != hipMemoryTypeManaged;
}
constexpr size_t kPipeMinBytes = size_t(4) << 20;   // below: one hipMemcpy
}  // namespace

hipError_t copy_h2d(void *dst_dev, const void *src_host, size_t bytes) {
    if (bytes < kPipeMinBytes || !pageable(src_host))
        return hipMemcpy(dst_dev, src_host, bytes, hipMemcpyHostToDevice);
    return host_pipe_upload(dst_dev, src_host, bytes, nullptr) == 0 ? hipSuccess : hipErrorUnknown;
}

hipError_t copy_d2h(void *dst_host, const void *src_dev, size_t bytes) {
    if (bytes < kPipeMinBytes || !pageable(dst_host))
        return hipMemcpy(dst_host, src_dev, bytes, hipMemcpyDeviceToHost);
    // As hipMemcpy: after the work already enqueued on the null stream.
    const hipError_t e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) return e;
    // Rows of one byte: pieces of one ring slot each.
    return host_pipe_download(dst_host, src_dev, bytes, 1, nullptr) == 0 ? hipSuccess : hipErrorUnknown;
}

}  // namespace km

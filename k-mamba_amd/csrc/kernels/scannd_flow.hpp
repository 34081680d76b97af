// scannd_flow.hpp - the dataflow schedule shared by the ScanND forward tiles
// (scannd.hip) and the ScanND backward's adjoint sweep (scannd_bwd.hip).
//
// One persistent launch per step: a tile waits only for its own axis
// neighbours (predecessors in the forward, successors in the adjoint sweep)
// instead of a whole band. Channel groups never depend on each other, so XCD
// x owns the groups [cg_lo[x], cg_lo[x + 1]) for every tile: each producer /
// consumer pair shares one XCD's L2 (coherent for all its CUs), and no data
// crosses XCDs inside the launch. Each workgroup reads the XCD it runs on
// from the hardware and takes items (tile in schedule order, then a run of
// channel groups) from that XCD's counter, so an item is only ever taken by
// a running workgroup and every item it depends on was taken before it: the
// waits always end.
//
// Hand-off: the producer waits until its stores are acknowledged by the L2
// (vmcnt 0), then publishes flags[tile * ncg + cg] = epoch (this launch's
// number) with an agent-scope store; the consumer polls the flag with
// agent-scope loads and reads the producer's states with agent-coherent
// loads (sc1: past its own L1, from the shared L2). A wait polls at most
// `spin` times. If it runs out, the wave does not compute its tile: it
// writes NaN into the tile's states (and outputs), so every tile that
// depends on it turns NaN too and no output is silently wrong, and it sets
// the launch's status word.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>

namespace km {

// Number of pairs (u, v), 0 <= u < n1, 0 <= v < n2, with u + v = s.
__device__ __forceinline__ int count2(int s, int n1, int n2) {
    const int lo = max(0, s - (n2 - 1)), hi = min(s, n1 - 1);
    return hi >= lo ? hi - lo + 1 : 0;
}

// Tile band b, ordinal o of a grid of ntile[0..nd) tiles: the o-th tile, in
// lexicographic order of the tile index tuple, whose indices sum to b
// (2 <= nd <= 4). Leading axes pick their index by counting the tuples of
// the remaining axes; the last two axes follow in closed form.
__device__ inline bool band_tile_n(int nd, const int *ntile, int band, int ordinal, int *ti) {
    int s = band, o = ordinal;
    for (int a = 0; a + 2 < nd; ++a) {
        bool found = false;
        for (int v = 0; v < ntile[a] && v <= s; ++v) {
            int c;
            if (a + 3 == nd) {
                c = count2(s - v, ntile[a + 1], ntile[a + 2]);
            } else {
                c = 0;
                for (int w = 0; w < ntile[a + 1] && w <= s - v; ++w)
                    c += count2(s - v - w, ntile[a + 2], ntile[a + 3]);
            }
            if (o < c) {
                ti[a] = v;
                s -= v;
                found = true;
                break;
            }
            o -= c;
        }
        if (!found) return false;
    }
    const int n1 = ntile[nd - 2], n2 = ntile[nd - 1];
    if (o >= count2(s, n1, n2)) return false;
    ti[nd - 2] = max(0, s - (n2 - 1)) + o;
    ti[nd - 1] = s - ti[nd - 2];
    return true;
}

constexpr int kMaxFlowBands = 768;
constexpr unsigned kFlowSpinDefault = 1u << 20;
struct FlowArgs {
    unsigned *flags;                     // [ntiles * ncg] epoch of the last finish
    unsigned *counter;                   // [8] items taken per XCD, zero at launch
    unsigned *status;                    // nonzero when a wait ran out (zero at launch)
    const unsigned *epoch;               // this launch's epoch (set by flow_reset)
    unsigned spin;                       // polls per wait before giving up
    int nbands;
    int cg_lo[9];                        // channel groups of XCD x: [cg_lo[x], cg_lo[x + 1])
    int band_start[kMaxFlowBands + 1];   // first tile (band order) of each band
};

// True once the producer published this launch's epoch; false when the
// budget ran out first. Lane 0 polls; the result is wave-uniform.
__device__ __forceinline__ bool flow_wait(const unsigned *flag, unsigned epoch, unsigned spin) {
    int done = 0;
    if ((threadIdx.x & 63) == 0) {
        for (unsigned i = 0; i < spin; ++i) {
            if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == epoch) {
                done = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    return __builtin_amdgcn_readfirstlane(done) != 0;
}

// The XCD the calling wave runs on (HW_REG_XCC_ID).
__device__ __forceinline__ int flow_xcd() {
    return static_cast<int>(__builtin_amdgcn_s_getreg(20 | (3 << 11))) & 7;
}

// Band of tile tb (schedule order): the last b with band_start[b] <= tb.
__device__ __forceinline__ int flow_band(const FlowArgs &f, int tb) {
    int lo = 0, hi = f.nbands - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (f.band_start[mid] <= tb) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// Workgroups of Q = blockDim.x / 64 waves, one channel group per wave of an
// item (Q = kFlowQ when it divides every XCD's group count, else 1).
constexpr int kFlowQ = 4;
inline int flow_q(const FlowArgs &f) {
    for (int x = 0; x < 8; ++x)
        if ((f.cg_lo[x + 1] - f.cg_lo[x]) % kFlowQ != 0) return 1;
    return kFlowQ;
}

// Dataflow state header (u32 words): per-XCD item counters (0-7), the
// status word (8), the epoch (9); completion flags from word kFlowHead.
constexpr size_t kFlowHead = 16;
constexpr int kFlowStatus = 8, kFlowEpoch = 9;

// Dataflow state supplied by the caller instead of the stream's block (the
// allocation-free entry point): a device buffer of `cap` words laid out as
// above and the device's XCD count.
struct FlowBuf {
    unsigned *buf;
    size_t cap;
    int nxcc;
};

// Host side (scannd.hip).
// True when grids of nd dims may use the dataflow schedule on the current
// device: 2+ dims, 8 XCDs, and KM_SCANND_SCHED is not "band".
bool flow_wanted(int nd);
// Binds fa's counters, status, epoch and flags (and its spin budget) to the
// dataflow state of stream s, or to ext's buffer, for a launch with nflags
// flags, and enqueues the reset that starts the launch's epoch. Returns 1
// when bound, 0 when the launch must use another schedule (no state block
// could be had), -1 on an error (set). *kind: 1 stream block, 2 ext buffer.
int flow_bind(hipStream_t s, size_t nflags, FlowBuf *ext, FlowArgs &fa, int *kind);
// Records which dataflow state the latest launch on s used, for
// km_scannd_status: kind 0 none, 1 the stream's block, 2 the buffer at word
// (kept: the caller keeps it alive until the status is read).
void note_flow(hipStream_t s, int kind, const unsigned *word = nullptr);
// Enqueues the zeroing of words u32 words at p on s (a fill kernel).
void flow_zero(unsigned *p, size_t words, hipStream_t s);

}  // namespace km

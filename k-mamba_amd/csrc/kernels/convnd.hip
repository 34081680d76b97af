// convnd.hip - dense per-channel causal ND convolution for gfx950.
//
//   out[n, d] = bias[d] + sum_{k in [0,K)^N} in[n - (K-1-k), d] * W[k, d]
// (reference src/convnd.c:83-126; taps below 0 on any axis are skipped,
// summed in row-major kernel order). Backward (src/convnd.c:135-202):
//   dinput[s, d]  = sum_k dy[s + (K-1-k), d] * W[k, d]   (taps past the end skipped)
//   dkernel[k, d] = sum_n dy[n, d] * in[n - (K-1-k), d]
//   dbias[d]      = sum_n dy[n, d]
//
// Design: the 64 lanes of a wave are 64 channels, so every point row of a
// tensor is one coalesced 256-byte access. A wave sweeps a strip of points
// along the last axis and keeps, for each tap row it reads, a K-wide window
// in registers: each step loads one new value per row instead of K.
//  - 2D and 3D (K <= 4 / K <= 3), the line-group kernels: a wave covers four
//    adjacent lines along axis N-2, which share their tap rows
//    (K^(N-2) x (K+3) rows for four lines instead of 4 x K^(N-1)). The
//    forward and dinput (anti-causal taps of dy) are one kernel; dkernel /
//    dbias accumulate per wave, are summed per workgroup in LDS and stored to
//    one slot per workgroup in the library workspace, and a second kernel
//    adds the slots in a fixed order (no atomics, run-to-run identical).
//    Where both windows fit the registers (2D, 3D with K = 2) the backward
//    is one line-group pass computing dinput and the dkernel terms together,
//    so dy is read once.
//  - Other shapes with N <= 3: one line per wave; the backward fuses dinput
//    and dkernel and adds dkernel per workgroup with fp32 atomics.
//  - Anything else: one thread per (point, channel), taps from memory.
// Lines that share inputs are adjacent in the task order, and workgroups are
// renumbered so that consecutive tasks run on the same XCD and find each
// other's rows in that XCD's L2.
#include <algorithm>

#include "km_device.hpp"
#include "../km_runtime.hpp"
#include "convnd.h"
#include "wavefront_nd.h"
#include "wavefront_plan.h"
#include "kmamba_km.h"

namespace km {

constexpr int kConvMaxNd = 8;
constexpr int ipow(int b, int e) { return e == 0 ? 1 : b * ipow(b, e - 1); }
constexpr int kStrip = 64;        // points per wave along the last axis
constexpr int kConvWaves = 4;     // waves per workgroup

struct ConvArgs {
    const float *in, *W, *bias;
    float *out;
    const float *dy;
    float *din, *dW, *db;         // dW, db: fp32 accumulators zeroed by the launcher
    long P;                        // points per batch element
    long batch;
    int nd, D, K, KV;
    int dims[kConvMaxNd];
    long stride[kConvMaxNd];
    long lines, njb, groups, tasks;
    long louter, ngrp;             // line groups: tuples of axes < nd-2, groups along nd-2
    int strip_l;                   // strip length of the line-group kernels (16, 32 or 64)
    long njb_l, tasks_l;
};

constexpr int kConvR = 4;          // output lines per wave in the line-group kernel

// Workgroup id in an order where consecutive ids share an XCD: the hardware
// deals workgroups to the 8 XCDs round-robin, so XCD x runs ids x, x+8, ...;
// this maps them to one contiguous range of tasks per XCD.
__device__ __forceinline__ long xcd_block(long b, long nb) {
    const long q = nb / 8, r = nb % 8, x = b % 8;
    return x * q + (x < r ? x : r) + b / 8;
}

struct TaskPos {
    long batch, line, j0;
    int d;
    bool dvalid;
    int lc[kConvMaxNd];            // leading coordinates of the line
    long line_off;                 // point offset of (line, j = 0)
};

__device__ __forceinline__ bool task_pos(const ConvArgs &p, long task, TaskPos &t) {
    if (task >= p.tasks) return false;
    const long g = task % p.groups;
    long rest = task / p.groups;
    const long jb = rest % p.njb;
    rest /= p.njb;
    t.line = rest % p.lines;
    t.batch = rest / p.lines;
    t.j0 = jb * kStrip;
    t.d = static_cast<int>(g * 64) + static_cast<int>(threadIdx.x & 63);
    t.dvalid = t.d < p.D;
    long rem = t.line, off = 0;
    for (int a = p.nd - 2; a >= 0; --a) {
        t.lc[a] = static_cast<int>(rem % p.dims[a]);
        rem /= p.dims[a];
        off += t.lc[a] * p.stride[a];
    }
    t.line_off = off;
    return true;
}

// Point offsets (within the batch element) of the K^(N-1) leading tap rows
// of a line, -1 where a tap leaves the grid. dir = -1: causal taps
// (coordinate - (K-1-k)); dir = +1: anti-causal taps (coordinate + (K-1-k)).
template <int ND, int K>
__device__ __forceinline__ void lead_rows(const ConvArgs &p, const TaskPos &t, int dir,
                                          long (&rows)[(ND > 1) ? ipow(K, ND - 1) : 1]) {
    constexpr int KL = (ND > 1) ? ipow(K, ND - 1) : 1;
#pragma unroll
    for (int a = 0; a < KL; ++a) {
        int rem = a;
        long off = 0;
        bool ok = true;
#pragma unroll
        for (int ax = ND - 2; ax >= 0; --ax) {
            const int ka = rem % K;
            rem /= K;
            const int c = t.lc[ax] + dir * (K - 1 - ka);
            ok = ok && c >= 0 && c < p.dims[ax];
            off += static_cast<long>(c) * p.stride[ax];
        }
        rows[a] = ok ? off : -1;
    }
}

// The strip kernels address one batch element through raw buffer resources
// with 32-bit byte offsets (the launcher keeps P*D*4 below 2^31). Taps that
// leave the grid along a leading axis use an offset with bit 31 set, past the
// window, which loads 0; outputs of lanes past D or columns past the line end
// are stored at such an offset and dropped. Every load and store is thus
// unconditional and the strip loop has a fixed trip count: it is unrolled
// and software-pipelined by hand in chunks of CU columns, the loads of chunk
// c+1 issued before the arithmetic and stores of chunk c (the compiler does
// not move loads above stores through buffer resources it cannot tell
// apart).
constexpr unsigned kConvDrop = 0x80000000u;
// Columns per chunk: enough loads in flight per wave, few enough registers.
constexpr int conv_chunk(int loads_per_column) { return loads_per_column <= 3 ? 8 : (loads_per_column <= 9 ? 4 : 2); }

__device__ __forceinline__ int conv_off(unsigned base, int j, int rowbytes) {
    return static_cast<int>(base + static_cast<unsigned>(j * rowbytes));
}

// Workgroup sum of the per-wave dkernel / dbias partials acc[0..KV], then one
// atomic per (tap, channel). Waves of one workgroup may belong to different
// channel groups (task % groups): the first wave of each group adds the
// partials of the waves in that group. Every wave of the workgroup calls
// this (it holds a barrier); ntasks bounds the task ids of the launch.
template <int KV>
__device__ __forceinline__ void conv_wg_reduce(const ConvArgs &p, float (&red)[kConvWaves][KV + 1][64],
                                               const float (&acc)[KV + 1], int wave, int lane, long blk,
                                               long ntasks, bool active, int dc) {
#pragma unroll
    for (int k = 0; k <= KV; ++k) red[wave][k][lane] = active ? acc[k] : 0.f;
    __syncthreads();
    if (!active) return;
    const long g = (blk * kConvWaves + wave) % p.groups;
    for (int v = 0; v < wave; ++v) {
        const long tv = blk * kConvWaves + v;
        if (tv < ntasks && tv % p.groups == g) return;
    }
    for (int k = 0; k <= KV; ++k) {
        float s = 0.f;
        for (int v = 0; v < kConvWaves; ++v) {
            const long tv = blk * kConvWaves + v;
            if (tv < ntasks && tv % p.groups == g) s += red[v][k][lane];
        }
        if (k < KV) unsafeAtomicAdd(p.dW + static_cast<long>(k) * p.D + dc, s);
        else if (p.db) unsafeAtomicAdd(p.db + dc, s);
    }
}

template <int ND, int K>
__global__ void __launch_bounds__(64 * kConvWaves) convnd_fwd_strip(ConvArgs p) {
    constexpr int KL = (ND > 1) ? ipow(K, ND - 1) : 1;
    constexpr int KV = KL * K;
    using F = bio<f32_t>;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const long blk = xcd_block(blockIdx.x, gridDim.x);
    TaskPos t;
    if (!task_pos(p, blk * kConvWaves + wave, t)) return;
    const int dc = t.dvalid ? t.d : p.D - 1;
    const int J = p.dims[ND - 1];
    const long bbase = t.batch * p.P;
    const auto rin = make_rsrc(p.in + bbase * p.D, p.P * p.D * 4);
    const auto rout = make_rsrc(p.out + bbase * p.D, p.P * p.D * 4);
    const int rb = p.D * 4;                          // bytes per point row
    const int j0 = static_cast<int>(t.j0);

    float w[KV];
#pragma unroll
    for (int k = 0; k < KV; ++k) w[k] = p.W[static_cast<long>(k) * p.D + dc];
    const float b0 = p.bias ? p.bias[dc] : 0.f;
    long rows[KL];
    lead_rows<ND, K>(p, t, -1, rows);
    unsigned ro[KL];
#pragma unroll
    for (int a = 0; a < KL; ++a)
        ro[a] = rows[a] >= 0 ? static_cast<unsigned>((rows[a] * p.D + dc) * 4) : kConvDrop;
    const unsigned oo = t.dvalid ? static_cast<unsigned>((t.line_off * p.D + dc) * 4) : kConvDrop;

    // win[a][c]: input of leading tap row a at column j - (K-1) + c; columns
    // before 0 are zero (the row offset would land in the previous line).
    float win[KL][K];
#pragma unroll
    for (int a = 0; a < KL; ++a) {
#pragma unroll
        for (int c = 0; c < K - 1; ++c) {
            const int j = j0 - (K - 1) + c;
            const float v = F::ld(rin, conv_off(ro[a], j < 0 ? 0 : j, rb), 0);
            win[a][c + 1] = j >= 0 ? v : 0.f;
        }
    }
    constexpr int CU = conv_chunk(KL);
    static_assert(kStrip % (2 * CU) == 0, "strip is whole chunk pairs");
    float n0[CU][KL], n1[CU][KL];                    // chunk buffers
    auto load_chunk = [&](int ch, float (&bx)[CU][KL]) {
#pragma unroll
        for (int u = 0; u < CU; ++u)
#pragma unroll
            for (int a = 0; a < KL; ++a) bx[u][a] = F::ld(rin, conv_off(ro[a], j0 + ch * CU + u, rb), 0);
    };
    auto run_chunk = [&](int ch, const float (&bx)[CU][KL]) {
#pragma unroll
        for (int u = 0; u < CU; ++u) {
            const int j = j0 + ch * CU + u;
#pragma unroll
            for (int a = 0; a < KL; ++a) {
#pragma unroll
                for (int c = 0; c < K - 1; ++c) win[a][c] = win[a][c + 1];
                win[a][K - 1] = bx[u][a];
            }
            float s = b0;
#pragma unroll
            for (int kl = 0; kl < KV; ++kl) s += win[kl / K][kl % K] * w[kl];
            F::st(rout, j < J ? conv_off(oo, j, rb) : static_cast<int>(kConvDrop), 0, s);
        }
    };
    // Past the strip the prefetch reads the next columns (in bounds or 0),
    // unused.
    load_chunk(0, n0);
#pragma unroll 1
    for (int ch = 0; ch < kStrip / CU; ch += 2) {
        load_chunk(ch + 1, n1);
        run_chunk(ch, n0);
        load_chunk(ch + 2, n0);
        run_chunk(ch + 1, n1);
    }
}

template <int ND, int K>
__global__ void __launch_bounds__(64 * kConvWaves) convnd_bwd_strip(ConvArgs p) {
    constexpr int KL = (ND > 1) ? ipow(K, ND - 1) : 1;
    constexpr int KV = KL * K;
    using F = bio<f32_t>;
    __shared__ float red[kConvWaves][KV + 1][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const long blk = xcd_block(blockIdx.x, gridDim.x);
    TaskPos t;
    const bool live = task_pos(p, blk * kConvWaves + wave, t);
    float acc[KV + 1];
#pragma unroll
    for (int k = 0; k <= KV; ++k) acc[k] = 0.f;
    int dc = 0;
    if (live) {
        dc = t.dvalid ? t.d : p.D - 1;
        const int J = p.dims[ND - 1];
        const long bbase = t.batch * p.P;
        const auto rin = make_rsrc(p.in + bbase * p.D, p.P * p.D * 4);
        const auto rdy = make_rsrc(p.dy + bbase * p.D, p.P * p.D * 4);
        const auto rdin = make_rsrc(p.din + bbase * p.D, p.P * p.D * 4);
        const int rb = p.D * 4;
        const int j0 = static_cast<int>(t.j0);
        float w[KV];
#pragma unroll
        for (int k = 0; k < KV; ++k) w[k] = p.W[static_cast<long>(k) * p.D + dc];
        long rin_[KL], rdy_[KL];
        lead_rows<ND, K>(p, t, -1, rin_);
        lead_rows<ND, K>(p, t, +1, rdy_);
        unsigned oi[KL], og[KL];
#pragma unroll
        for (int a = 0; a < KL; ++a) {
            oi[a] = rin_[a] >= 0 ? static_cast<unsigned>((rin_[a] * p.D + dc) * 4) : kConvDrop;
            og[a] = rdy_[a] >= 0 ? static_cast<unsigned>((rdy_[a] * p.D + dc) * 4) : kConvDrop;
        }
        const unsigned od = t.dvalid ? static_cast<unsigned>((t.line_off * p.D + dc) * 4) : kConvDrop;
        // xin[a][c]: input at column j-(K-1)+c of causal row a (0 before
        // column 0). gdy[a][c]: dy at column j+c of anti-causal row a (0 past
        // the line end, where the row offset would land in the next line).
        float xin[KL][K], gdy[KL][K];
#pragma unroll
        for (int a = 0; a < KL; ++a) {
#pragma unroll
            for (int c = 0; c < K - 1; ++c) {
                const int ji = j0 - (K - 1) + c;
                const float vi = F::ld(rin, conv_off(oi[a], ji < 0 ? 0 : ji, rb), 0);
                xin[a][c + 1] = ji >= 0 ? vi : 0.f;
                const int jd = j0 + c;
                const float vd = F::ld(rdy, conv_off(og[a], jd, rb), 0);
                gdy[a][c] = jd < J ? vd : 0.f;
            }
        }
        // The anti-causal row with every leading tap at K-1 is the line itself.
        constexpr int SELF = KL - 1;
        constexpr int CU = conv_chunk(2 * KL);
        static_assert(kStrip % (2 * CU) == 0, "strip is whole chunk pairs");
        float i0[CU][KL], d0[CU][KL], i1[CU][KL], d1[CU][KL];   // chunk buffers
        auto load_chunk = [&](int ch, float (&bi)[CU][KL], float (&bd)[CU][KL]) {
#pragma unroll
            for (int u = 0; u < CU; ++u)
#pragma unroll
                for (int a = 0; a < KL; ++a) {
                    const int j = j0 + ch * CU + u;
                    bi[u][a] = F::ld(rin, conv_off(oi[a], j, rb), 0);
                    bd[u][a] = F::ld(rdy, conv_off(og[a], j + K - 1, rb), 0);
                }
        };
        auto run_chunk = [&](int ch, const float (&bi)[CU][KL], const float (&bd)[CU][KL]) {
#pragma unroll
        for (int u = 0; u < CU; ++u) {
            const int j = j0 + ch * CU + u;
#pragma unroll
            for (int a = 0; a < KL; ++a) {
#pragma unroll
                for (int c = 0; c < K - 1; ++c) xin[a][c] = xin[a][c + 1];
                xin[a][K - 1] = bi[u][a];
                gdy[a][K - 1] = j + K - 1 < J ? bd[u][a] : 0.f;
            }
            const float g = gdy[SELF][0];            // 0 past the line end
            float s = 0.f;
#pragma unroll
            for (int kl = 0; kl < KV; ++kl) {
                const int a = kl / K, k = kl % K;
                s += gdy[a][K - 1 - k] * w[kl];
                acc[kl] = fmaf(g, xin[a][k], acc[kl]);
            }
            acc[KV] += g;
            F::st(rdin, j < J ? conv_off(od, j, rb) : static_cast<int>(kConvDrop), 0, s);
#pragma unroll
            for (int a = 0; a < KL; ++a) {
#pragma unroll
                for (int c = 0; c < K - 1; ++c) gdy[a][c] = gdy[a][c + 1];
            }
        }
        };
        load_chunk(0, i0, d0);
#pragma unroll 1
        for (int ch = 0; ch < kStrip / CU; ch += 2) {
            load_chunk(ch + 1, i1, d1);
            run_chunk(ch, i0, d0);
            load_chunk(ch + 2, i0, d0);
            run_chunk(ch + 1, i1, d1);
        }
        if (!t.dvalid) {
#pragma unroll
            for (int k = 0; k <= KV; ++k) acc[k] = 0.f;
        }
    }
    conv_wg_reduce<KV>(p, red, acc, wave, lane, blk, p.tasks, live && t.dvalid, dc);
}

// Line-group kernels, ND >= 2: a wave covers kConvR consecutive lines along
// axis nd-2 (same coordinates on the axes before it) over one strip of S
// points (S = 64, or 32 / 16 where longer strips would leave fewer than two
// waves per SIMD).
// Those lines share their tap rows: K^(nd-2) x (kConvR + K - 1) distinct rows
// instead of kConvR x K^(nd-1), each loaded once per column and kept as a
// K-wide window.
struct LineTask {
    long batch;
    int j0, i0, d, dc;
    bool dvalid;
    int lc[kConvMaxNd];            // coordinates of axes < nd-2; lc[nd-2] = i0
};

// Task tl of channel group g: tl = ((batch * louter + outer) * ngrp + group)
// * njb_l + strip.
template <int ND, int S>
__device__ __forceinline__ LineTask line_task(const ConvArgs &p, long g, long tl) {
    LineTask t;
    long rest = tl;
    t.j0 = static_cast<int>((rest % p.njb_l) * S);
    rest /= p.njb_l;
    const long lg = rest % (p.louter * p.ngrp);
    t.batch = rest / (p.louter * p.ngrp);
    t.i0 = static_cast<int>((lg % p.ngrp) * kConvR);
    long outer = lg / p.ngrp;
    t.lc[ND - 2] = t.i0;
#pragma unroll
    for (int a = ND - 3; a >= 0; --a) {
        t.lc[a] = static_cast<int>(outer % p.dims[a]);
        outer /= p.dims[a];
    }
    t.d = static_cast<int>(g * 64) + static_cast<int>(threadIdx.x & 63);
    t.dvalid = t.d < p.D;
    t.dc = t.dvalid ? t.d : p.D - 1;
    return t;
}

// Byte offsets of the tap rows of a line group: combination ko of the axes
// < nd-2 (row-major over taps k, coordinate c -/+ (K-1-k)) and s along nd-2,
// coordinate i0 - (K-1) + s (causal) or i0 + s (anti-causal).
template <int ND, int K, bool ANTI>
__device__ __forceinline__ void group_rows(const ConvArgs &p, const LineTask &t,
                                           unsigned (&ro)[ipow(K, ND - 2) * (kConvR + K - 1)]) {
    constexpr int RS = kConvR + K - 1;
#pragma unroll
    for (int ko = 0; ko < ipow(K, ND - 2); ++ko) {
        int rem = ko;
        long off = 0;
        bool ok = true;
#pragma unroll
        for (int a = ND - 3; a >= 0; --a) {
            const int ka = rem % K;
            rem /= K;
            const int c = ANTI ? t.lc[a] + (K - 1 - ka) : t.lc[a] - (K - 1 - ka);
            ok = ok && c >= 0 && c < p.dims[a];
            off += static_cast<long>(c) * p.stride[a];
        }
#pragma unroll
        for (int s = 0; s < RS; ++s) {
            const int c = ANTI ? t.i0 + s : t.i0 - (K - 1) + s;
            const bool okr = ok && c >= 0 && c < p.dims[ND - 2];
            ro[ko * RS + s] =
                okr ? static_cast<unsigned>(((off + static_cast<long>(c) * p.stride[ND - 2]) * p.D + t.dc) * 4)
                    : kConvDrop;
        }
    }
}

// Byte offsets of the kConvR lines of the group themselves, dropped for
// lines past the grid and lanes past D.
template <int ND>
__device__ __forceinline__ void group_lines(const ConvArgs &p, const LineTask &t, unsigned (&oo)[kConvR]) {
    long off = 0;
#pragma unroll
    for (int a = 0; a < ND - 2; ++a) off += static_cast<long>(t.lc[a]) * p.stride[a];
#pragma unroll
    for (int r = 0; r < kConvR; ++r) {
        const bool ok = t.dvalid && t.i0 + r < p.dims[ND - 2];
        oo[r] = ok ? static_cast<unsigned>(((off + static_cast<long>(t.i0 + r) * p.stride[ND - 2]) * p.D + t.dc) * 4)
                   : kConvDrop;
    }
}

// dkernel[k, d] (k < KV) or dbias[d] (k = KV) of channel group g: the sum of
// the nslot per-workgroup slots that convnd_dw_lines stored. Wave w of the
// workgroup adds slots w, w + 4, ... (32 independent loads per round), then
// wave 0 adds the four partials: a fixed order, so the result does not
// depend on timing.
__device__ __forceinline__ void dw_finalize(const ConvArgs &p, const float *part, int nslot, int k, long g,
                                            int wave, int lane, float (&red)[kConvWaves][64]) {
    using F = bio<f32_t>;
    const int KV = p.KV;
    const long per_slot = static_cast<long>(KV + 1) * 64;
    const auto rp = make_rsrc(part + g * nslot * per_slot, nslot * per_slot * 4);
    float s = 0.f;
#pragma unroll 1
    for (int b0 = 0; b0 < nslot; b0 += 32 * kConvWaves) {
        float v[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const int b = b0 + i * kConvWaves + wave;
            v[i] = F::ld(rp, b < nslot ? static_cast<int>(((b * (KV + 1) + k) * 64 + lane) * 4)
                                       : static_cast<int>(kConvDrop), 0);
        }
#pragma unroll
        for (int i = 0; i < 32; ++i) s += v[i];
    }
    red[wave][lane] = s;
    __syncthreads();
    if (wave != 0) return;
    float sum = 0.f;
#pragma unroll
    for (int v = 0; v < kConvWaves; ++v) sum += red[v][lane];
    const long d = g * 64 + lane;
    if (d >= p.D) return;
    if (k < KV) p.dW[k * static_cast<long>(p.D) + d] = sum;
    else if (p.db) p.db[d] = sum;
}

// ANTI = false: the forward, out = bias + causal taps of in.
// ANTI = true: dinput = anti-causal taps of dy (no bias). With part set, the
// first (KV + 1) * groups workgroups instead finish dkernel / dbias from the
// slots of convnd_dw_lines (launched before on the stream), alongside.
// Taps are summed per output in row-major kernel order, as the reference.
// The causal window holds columns j-(K-1)..j (0 before column 0); the
// anti-causal one columns j..j+K-1 (0 past the line end, where the offset
// would land in the next line).
template <int ND, int K, bool ANTI, int S>
__global__ void __launch_bounds__(64 * kConvWaves) convnd_lines(ConvArgs p, const float *part, int nslot) {
    constexpr int R = kConvR;
    constexpr int KO = ipow(K, ND - 2);
    constexpr int RS = R + K - 1;
    constexpr int NR = KO * RS;
    constexpr int KV = ipow(K, ND);
    constexpr int CU = NR <= 6 ? 4 : (NR <= 12 ? 2 : 1);   // columns per load chunk
    constexpr int NCH = S / CU;                      // chunks per strip
    static_assert(NCH >= 2 && NCH % 2 == 0, "strip is whole chunk pairs");
    using F = bio<f32_t>;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    long blk = blockIdx.x, nblk = gridDim.x;
    if (ANTI && part) {
        const long nfin = static_cast<long>(KV + 1) * p.groups;
        if (blk < nfin) {
            __shared__ float red[kConvWaves][64];
            dw_finalize(p, part, nslot, static_cast<int>(blk % (KV + 1)), blk / (KV + 1), wave,
                        threadIdx.x & 63, red);
            return;
        }
        blk -= nfin;
        nblk -= nfin;
    }
    const long task = xcd_block(blk, nblk) * kConvWaves + wave;
    if (task >= p.tasks_l) return;
    const LineTask t = line_task<ND, S>(p, task % p.groups, task / p.groups);
    const int J = p.dims[ND - 1];
    const long bbase = t.batch * p.P;
    const auto rin = make_rsrc((ANTI ? p.dy : p.in) + bbase * p.D, p.P * p.D * 4);
    const auto rout = make_rsrc((ANTI ? p.din : p.out) + bbase * p.D, p.P * p.D * 4);
    const int rb = p.D * 4;
    const int j0 = t.j0;

    float w[KV];
#pragma unroll
    for (int k = 0; k < KV; ++k) w[k] = p.W[static_cast<long>(k) * p.D + t.dc];
    const float b0 = (!ANTI && p.bias) ? p.bias[t.dc] : 0.f;
    unsigned ro[NR], oo[R];
    group_rows<ND, K, ANTI>(p, t, ro);
    group_lines<ND>(p, t, oo);
    // Column loaded at step j, and the one the window starts with.
    constexpr int LEAD = ANTI ? K - 1 : 0;
    float win[NR][K];
#pragma unroll
    for (int q = 0; q < NR; ++q) {
#pragma unroll
        for (int c = 0; c < K - 1; ++c) {
            const int j = j0 - (K - 1) + LEAD + c;
            const float v = F::ld(rin, conv_off(ro[q], j < 0 ? 0 : j, rb), 0);
            win[q][c + 1] = (j >= 0 && j < J) ? v : 0.f;
        }
    }
    float n0[CU][NR], n1[CU][NR];
    auto load_chunk = [&](int ch, float (&bx)[CU][NR]) {
#pragma unroll
        for (int u = 0; u < CU; ++u)
#pragma unroll
            for (int q = 0; q < NR; ++q) bx[u][q] = F::ld(rin, conv_off(ro[q], j0 + ch * CU + u + LEAD, rb), 0);
    };
    auto run_chunk = [&](int ch, const float (&bx)[CU][NR]) {
#pragma unroll
        for (int u = 0; u < CU; ++u) {
            const int j = j0 + ch * CU + u;
            const bool in_line = !ANTI || j + LEAD < J;
#pragma unroll
            for (int q = 0; q < NR; ++q) {
#pragma unroll
                for (int c = 0; c < K - 1; ++c) win[q][c] = win[q][c + 1];
                win[q][K - 1] = in_line ? bx[u][q] : 0.f;
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float s = b0;
#pragma unroll
                for (int ko = 0; ko < KO; ++ko)
#pragma unroll
                    for (int ka = 0; ka < K; ++ka)
#pragma unroll
                        for (int kc = 0; kc < K; ++kc) {
                            const float x = ANTI ? win[ko * RS + r + (K - 1 - ka)][K - 1 - kc]
                                                 : win[ko * RS + r + ka][kc];
                            s += x * w[(ko * K + ka) * K + kc];
                        }
                F::st(rout, j < J ? conv_off(oo[r], j, rb) : static_cast<int>(kConvDrop), 0, s);
            }
        }
    };
    load_chunk(0, n0);
#pragma unroll 1
    for (int ch = 0; ch < NCH - 2; ch += 2) {
        load_chunk(ch + 1, n1);
        run_chunk(ch, n0);
        load_chunk(ch + 2, n0);
        run_chunk(ch + 1, n1);
    }
    load_chunk(NCH - 1, n1);
    run_chunk(NCH - 2, n0);
    run_chunk(NCH - 1, n1);
}

// dkernel / dbias over line groups: acc[k] += dy[line r, j] * in[causal tap
// k of (r, j)], acc[KV] += dy. blockIdx.y is the channel group; workgroup x
// of it takes the tasks quads [x * per, (x + 1) * per) of that group (wave w
// the task 4q + w of quad q), sums its waves' partials in LDS and stores them
// to its slot part[(y * gridDim.x + x) * (KV + 1) * 64 ...]: no atomics, and
// dw_finalize adds the slots in a fixed order.
template <int ND, int K, int S>
__global__ void __launch_bounds__(64 * kConvWaves) convnd_dw_lines(ConvArgs p, float *part, long per) {
    constexpr int R = kConvR;
    constexpr int KO = ipow(K, ND - 2);
    constexpr int RS = R + K - 1;
    constexpr int NR = KO * RS;
    constexpr int KV = ipow(K, ND);
    constexpr int CU = NR + R <= 8 ? 4 : (NR + R <= 14 ? 2 : 1);
    constexpr int NCH = S / CU;                      // chunks per strip
    static_assert(NCH >= 2 && NCH % 2 == 0, "strip is whole chunk pairs");
    using F = bio<f32_t>;
    __shared__ float red[kConvWaves][KV + 1][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const long g = blockIdx.y;
    const long T = p.tasks_l / p.groups;             // tasks per channel group
    const long q0 = xcd_block(blockIdx.x, gridDim.x) * per;   // neighbours on one XCD
    float acc[KV + 1];
#pragma unroll
    for (int k = 0; k <= KV; ++k) acc[k] = 0.f;
#pragma unroll 1
    for (long q = q0; q < q0 + per; ++q) {
        const long tl = q * kConvWaves + wave;
        if (tl >= T) break;
        const LineTask t = line_task<ND, S>(p, g, tl);
        const int J = p.dims[ND - 1];
        const long bbase = t.batch * p.P;
        const auto rin = make_rsrc(p.in + bbase * p.D, p.P * p.D * 4);
        const auto rdy = make_rsrc(p.dy + bbase * p.D, p.P * p.D * 4);
        const int rb = p.D * 4;
        const int j0 = t.j0;
        unsigned ro[NR], og[R];
        group_rows<ND, K, false>(p, t, ro);
        group_lines<ND>(p, t, og);        // dy of lanes past D and lines past the grid: 0
        float win[NR][K];
#pragma unroll
        for (int qq = 0; qq < NR; ++qq) {
#pragma unroll
            for (int c = 0; c < K - 1; ++c) {
                const int j = j0 - (K - 1) + c;
                const float v = F::ld(rin, conv_off(ro[qq], j < 0 ? 0 : j, rb), 0);
                win[qq][c + 1] = j >= 0 ? v : 0.f;
            }
        }
        float x0[CU][NR], g0[CU][R], x1[CU][NR], g1[CU][R];
        auto load_chunk = [&](int ch, float (&bx)[CU][NR], float (&bg)[CU][R]) {
#pragma unroll
            for (int u = 0; u < CU; ++u) {
                const int j = j0 + ch * CU + u;
#pragma unroll
                for (int qq = 0; qq < NR; ++qq) bx[u][qq] = F::ld(rin, conv_off(ro[qq], j, rb), 0);
#pragma unroll
                for (int r = 0; r < R; ++r) bg[u][r] = F::ld(rdy, conv_off(og[r], j, rb), 0);
            }
        };
        auto run_chunk = [&](int ch, const float (&bx)[CU][NR], const float (&bg)[CU][R]) {
#pragma unroll
            for (int u = 0; u < CU; ++u) {
                const int j = j0 + ch * CU + u;
#pragma unroll
                for (int qq = 0; qq < NR; ++qq) {
#pragma unroll
                    for (int c = 0; c < K - 1; ++c) win[qq][c] = win[qq][c + 1];
                    win[qq][K - 1] = bx[u][qq];
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float gy = j < J ? bg[u][r] : 0.f;
#pragma unroll
                    for (int ko = 0; ko < KO; ++ko)
#pragma unroll
                        for (int ka = 0; ka < K; ++ka)
#pragma unroll
                            for (int kc = 0; kc < K; ++kc) {
                                const int k = (ko * K + ka) * K + kc;
                                acc[k] = fmaf(gy, win[ko * RS + r + ka][kc], acc[k]);
                            }
                    acc[KV] += gy;
                }
            }
        };
        load_chunk(0, x0, g0);
#pragma unroll 1
        for (int ch = 0; ch < NCH - 2; ch += 2) {
            load_chunk(ch + 1, x1, g1);
            run_chunk(ch, x0, g0);
            load_chunk(ch + 2, x0, g0);
            run_chunk(ch + 1, x1, g1);
        }
        load_chunk(NCH - 1, x1, g1);
        run_chunk(NCH - 2, x0, g0);
        run_chunk(NCH - 1, x1, g1);
    }
#pragma unroll
    for (int k = 0; k <= KV; ++k) red[wave][k][lane] = acc[k];
    __syncthreads();
    float *slot = part + (g * gridDim.x + blockIdx.x) * static_cast<long>(KV + 1) * 64;
    for (int i = threadIdx.x; i < (KV + 1) * 64; i += 64 * kConvWaves) {
        float sum = 0.f;
#pragma unroll
        for (int v = 0; v < kConvWaves; ++v) sum += red[v][i / 64][i % 64];
        slot[i] = sum;
    }
}

// The backward of a line group in one pass (2D, and 3D with K = 2, where
// both windows fit the registers): dinput of the group's lines from the
// anti-causal window of dy, and the dkernel / dbias terms from the causal
// window of the input times dy of the lines themselves, which that dy
// window already holds (its column j, rows at offset 0 on every axis): dy
// is read once instead of once per kernel. Tasks, slots and the fixed-order
// workgroup sum are those of convnd_dw_lines; convnd_dw_finish adds the
// slots.
template <int ND, int K, int S>
__global__ void __launch_bounds__(64 * kConvWaves) convnd_bwd_lines(ConvArgs p, float *part, long per) {
    constexpr int R = kConvR;
    constexpr int KO = ipow(K, ND - 2);
    constexpr int RS = R + K - 1;
    constexpr int NR = KO * RS;
    constexpr int KV = ipow(K, ND);
    constexpr int CU = 2 * NR <= 12 ? 2 : 1;         // columns per load chunk
    constexpr int NCH = S / CU;
    constexpr int QO = (KO - 1) * RS;                // dy window rows of the lines themselves: QO + r
    static_assert(NCH >= 2 && NCH % 2 == 0, "strip is whole chunk pairs");
    using F = bio<f32_t>;
    __shared__ float red[kConvWaves][KV + 1][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const long g = blockIdx.y;
    const long T = p.tasks_l / p.groups;
    const long q0 = xcd_block(blockIdx.x, gridDim.x) * per;
    float acc[KV + 1];
#pragma unroll
    for (int k = 0; k <= KV; ++k) acc[k] = 0.f;
#pragma unroll 1
    for (long q = q0; q < q0 + per; ++q) {
        const long tl = q * kConvWaves + wave;
        if (tl >= T) break;
        const LineTask t = line_task<ND, S>(p, g, tl);
        const int J = p.dims[ND - 1];
        const long bbase = t.batch * p.P;
        const auto rin = make_rsrc(p.in + bbase * p.D, p.P * p.D * 4);
        const auto rdy = make_rsrc(p.dy + bbase * p.D, p.P * p.D * 4);
        const auto rdin = make_rsrc(p.din + bbase * p.D, p.P * p.D * 4);
        const int rb = p.D * 4;
        const int j0 = t.j0;
        float w[KV];
#pragma unroll
        for (int k = 0; k < KV; ++k) w[k] = p.W[static_cast<long>(k) * p.D + t.dc];
        unsigned rd[NR], ri[NR], oo[R];
        group_rows<ND, K, true>(p, t, rd);
        group_rows<ND, K, false>(p, t, ri);
        group_lines<ND>(p, t, oo);
        // dy window: columns j..j+K-1 (0 past the line end); input window:
        // columns j-(K-1)..j (0 before column 0).
        float wd[NR][K], wi[NR][K];
#pragma unroll
        for (int qq = 0; qq < NR; ++qq) {
#pragma unroll
            for (int c = 0; c < K - 1; ++c) {
                const int jd = j0 + c;
                const float vd = F::ld(rdy, conv_off(rd[qq], jd, rb), 0);
                wd[qq][c + 1] = jd < J ? vd : 0.f;
                const int ji = j0 - (K - 1) + c;
                const float vi = F::ld(rin, conv_off(ri[qq], ji < 0 ? 0 : ji, rb), 0);
                wi[qq][c + 1] = ji >= 0 ? vi : 0.f;
            }
        }
        float d0[CU][NR], i0[CU][NR], d1[CU][NR], i1[CU][NR];
        auto load_chunk = [&](int ch, float (&bd)[CU][NR], float (&bi)[CU][NR]) {
#pragma unroll
            for (int u = 0; u < CU; ++u) {
                const int j = j0 + ch * CU + u;
#pragma unroll
                for (int qq = 0; qq < NR; ++qq) {
                    bd[u][qq] = F::ld(rdy, conv_off(rd[qq], j + K - 1, rb), 0);
                    bi[u][qq] = F::ld(rin, conv_off(ri[qq], j, rb), 0);
                }
            }
        };
        auto run_chunk = [&](int ch, const float (&bd)[CU][NR], const float (&bi)[CU][NR]) {
#pragma unroll
            for (int u = 0; u < CU; ++u) {
                const int j = j0 + ch * CU + u;
                const bool dy_in = j + K - 1 < J;
#pragma unroll
                for (int qq = 0; qq < NR; ++qq) {
#pragma unroll
                    for (int c = 0; c < K - 1; ++c) {
                        wd[qq][c] = wd[qq][c + 1];
                        wi[qq][c] = wi[qq][c + 1];
                    }
                    wd[qq][K - 1] = dy_in ? bd[u][qq] : 0.f;
                    wi[qq][K - 1] = bi[u][qq];
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float sdin = 0.f;
                    const float gy = j < J ? wd[QO + r][0] : 0.f;
#pragma unroll
                    for (int ko = 0; ko < KO; ++ko)
#pragma unroll
                        for (int ka = 0; ka < K; ++ka)
#pragma unroll
                            for (int kc = 0; kc < K; ++kc) {
                                const int k = (ko * K + ka) * K + kc;
                                sdin += wd[ko * RS + r + (K - 1 - ka)][K - 1 - kc] * w[k];
                                acc[k] = fmaf(gy, wi[ko * RS + r + ka][kc], acc[k]);
                            }
                    acc[KV] += gy;
                    F::st(rdin, j < J ? conv_off(oo[r], j, rb) : static_cast<int>(kConvDrop), 0, sdin);
                }
            }
        };
        load_chunk(0, d0, i0);
#pragma unroll 1
        for (int ch = 0; ch < NCH - 2; ch += 2) {
            load_chunk(ch + 1, d1, i1);
            run_chunk(ch, d0, i0);
            load_chunk(ch + 2, d0, i0);
            run_chunk(ch + 1, d1, i1);
        }
        load_chunk(NCH - 1, d1, i1);
        run_chunk(NCH - 2, d0, i0);
        run_chunk(NCH - 1, d1, i1);
    }
#pragma unroll
    for (int k = 0; k <= KV; ++k) red[wave][k][lane] = acc[k];
    __syncthreads();
    float *slot = part + (g * gridDim.x + blockIdx.x) * static_cast<long>(KV + 1) * 64;
    for (int i = threadIdx.x; i < (KV + 1) * 64; i += 64 * kConvWaves) {
        float sum = 0.f;
#pragma unroll
        for (int v = 0; v < kConvWaves; ++v) sum += red[v][i / 64][i % 64];
        slot[i] = sum;
    }
}

// dkernel / dbias from the slots of convnd_bwd_lines: workgroup (k, g)
// finishes tap k (k = KV: the bias) of channel group g.
__global__ void __launch_bounds__(64 * kConvWaves) convnd_dw_finish(ConvArgs p, const float *part, int nslot) {
    __shared__ float red[kConvWaves][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    dw_finalize(p, part, nslot, static_cast<int>(blockIdx.x % (p.KV + 1)), blockIdx.x / (p.KV + 1), wave,
                threadIdx.x & 63, red);
}

// Any ND <= 8 and K: one thread per (point, channel), taps from memory.
__global__ void __launch_bounds__(256) convnd_fwd_generic(ConvArgs p) {
    const long gid = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= p.batch * p.P * p.D) return;
    const long d = gid % p.D, pt = (gid / p.D) % p.P, b = gid / (p.D * p.P);
    int oc[kConvMaxNd];
    long rem = pt;
    for (int a = p.nd - 1; a >= 0; --a) {
        oc[a] = static_cast<int>(rem % p.dims[a]);
        rem /= p.dims[a];
    }
    const float *in = p.in + b * p.P * p.D;
    float s = p.bias ? p.bias[d] : 0.f;
    for (int kl = 0; kl < p.KV; ++kl) {
        int tmp = kl;
        long src = 0;
        bool ok = true;
        for (int a = p.nd - 1; a >= 0; --a) {
            const int ka = tmp % p.K;
            tmp /= p.K;
            const int c = oc[a] - (p.K - 1 - ka);
            ok = ok && c >= 0;
            src += static_cast<long>(c) * p.stride[a];
        }
        if (ok) s += in[src * p.D + d] * p.W[static_cast<long>(kl) * p.D + d];
    }
    p.out[gid] = s;
}

__global__ void __launch_bounds__(256) convnd_bwd_input_generic(ConvArgs p) {
    const long gid = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= p.batch * p.P * p.D) return;
    const long d = gid % p.D, pt = (gid / p.D) % p.P, b = gid / (p.D * p.P);
    int sc[kConvMaxNd];
    long rem = pt;
    for (int a = p.nd - 1; a >= 0; --a) {
        sc[a] = static_cast<int>(rem % p.dims[a]);
        rem /= p.dims[a];
    }
    const float *dy = p.dy + b * p.P * p.D;
    float s = 0.f;
    for (int kl = 0; kl < p.KV; ++kl) {
        int tmp = kl;
        long o = 0;
        bool ok = true;
        for (int a = p.nd - 1; a >= 0; --a) {
            const int ka = tmp % p.K;
            tmp /= p.K;
            const int c = sc[a] + (p.K - 1 - ka);
            ok = ok && c < p.dims[a];
            o += static_cast<long>(c) * p.stride[a];
        }
        if (ok) s += dy[o * p.D + d] * p.W[static_cast<long>(kl) * p.D + d];
    }
    p.din[gid] = s;
}

// dkernel / dbias for any shape: block (tap, 64 channels, slice of points).
__global__ void __launch_bounds__(256) convnd_bwd_kernel_generic(ConvArgs p, long pts_per_block) {
    __shared__ float part[4][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int kl = blockIdx.y;              // KV = bias row
    const long d = static_cast<long>(blockIdx.z) * 64 + lane;
    const long total = p.batch * p.P;
    const long lo = static_cast<long>(blockIdx.x) * pts_per_block;
    const long hi = std::min(lo + pts_per_block, total);
    float s = 0.f;
    if (d < p.D) {
        int kc[kConvMaxNd];
        int tmp = kl;
        for (int a = p.nd - 1; a >= 0; --a) {
            kc[a] = tmp % p.K;
            tmp /= p.K;
        }
        for (long n = lo + wv; n < hi; n += 4) {
            const long pt = n % p.P, b = n / p.P;
            const float g = p.dy[n * p.D + d];
            if (kl == p.KV) { s += g; continue; }
            long rem = pt, src = 0;
            bool ok = true;
            for (int a = p.nd - 1; a >= 0; --a) {
                const int c = static_cast<int>(rem % p.dims[a]) - (p.K - 1 - kc[a]);
                rem /= p.dims[a];
                ok = ok && c >= 0;
                src += static_cast<long>(c) * p.stride[a];
            }
            if (ok) s += g * p.in[(b * p.P + src) * p.D + d];
        }
    }
    part[wv][lane] = s;
    __syncthreads();
    if (wv == 0 && d < p.D) {
        const float t = part[0][lane] + part[1][lane] + part[2][lane] + part[3][lane];
        if (kl < p.KV) unsafeAtomicAdd(p.dW + static_cast<long>(kl) * p.D + d, t);
        else if (p.db) unsafeAtomicAdd(p.db + d, t);
    }
}

__global__ void __launch_bounds__(256) conv_zero(float *p, long n) {
    for (long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<long>(gridDim.x) * blockDim.x)
        p[i] = 0.f;
}

static int zero_dev(float *p, long n, hipStream_t s) {
    if (!p || n <= 0) return 0;
    hipLaunchKernelGGL(conv_zero, dim3(std::min<long>((n + 255) / 256, 4096)), dim3(256), 0, s, p, n);
    KM_HIP_TRY(hipGetLastError());
    return 0;
}

static bool conv_args(const ConvNDParams *p, long batch, bool bwd, ConvArgs &a, const char *who) {
    if (!p || !p->dims || p->ndims <= 0 || p->ndims > kConvMaxNd || p->D <= 0 || p->K <= 0 ||
        !p->input || !p->kernel || batch <= 0) {
        set_error("%s: invalid parameters", who);
        return false;
    }
    if (bwd ? (!p->dy || !p->dinput || !p->dkernel) : !p->output) {
        set_error("%s: missing %s buffers", who, bwd ? "backward" : "output");
        return false;
    }
    if (!wavefront_nd_validate_dims(p->dims, p->ndims)) {
        set_error("%s: invalid dims", who);
        return false;
    }
    const long KV = convnd_kernel_volume(p->ndims, p->K);
    if (KV <= 0 || KV > 65534 || p->D > 0x7fffffffL) {
        set_error("%s: kernel volume %ld out of range", who, KV);
        return false;
    }
    a = ConvArgs{};
    a.in = p->input; a.W = p->kernel; a.bias = p->bias; a.out = p->output;
    a.dy = p->dy; a.din = p->dinput; a.dW = p->dkernel; a.db = p->dbias;
    a.nd = static_cast<int>(p->ndims); a.D = static_cast<int>(p->D);
    a.K = static_cast<int>(p->K); a.KV = static_cast<int>(KV);
    a.batch = batch;
    long s = 1;
    for (int ax = a.nd - 1; ax >= 0; --ax) {
        if (p->dims[ax] > 0x7fffffffL) {
            set_error("%s: dimension too large", who);
            return false;
        }
        a.dims[ax] = static_cast<int>(p->dims[ax]);
        a.stride[ax] = s;
        s *= p->dims[ax];
    }
    a.P = s;
    a.lines = s / a.dims[a.nd - 1];
    a.njb = (a.dims[a.nd - 1] + kStrip - 1) / kStrip;
    a.groups = (a.D + 63) / 64;
    a.tasks = batch * a.lines * a.njb * a.groups;
    if (a.nd >= 2) {
        a.louter = a.lines / a.dims[a.nd - 2];
        a.ngrp = (a.dims[a.nd - 2] + kConvR - 1) / kConvR;
        // Longest strip that still gives two waves per SIMD (256 CUs).
        const int J = a.dims[a.nd - 1];
        for (a.strip_l = 64; a.strip_l > 16; a.strip_l /= 2) {
            const long njb = (J + a.strip_l - 1) / a.strip_l;
            if (batch * a.louter * a.ngrp * njb * a.groups >= 2048) break;
        }
        a.njb_l = (J + a.strip_l - 1) / a.strip_l;
        a.tasks_l = batch * a.louter * a.ngrp * a.njb_l * a.groups;
    }
    return true;
}

// The strip kernels' 32-bit offsets: one batch element, plus a strip's
// overhang past the line end (kStrip + K rows), must stay below 2^31 bytes.
static bool strip_fits(const ConvArgs &a) {
    return (a.P + kStrip + a.K) * static_cast<long>(a.D) * 4 < 0x7fffffffL;
}

#define KM_CONV_SHAPES(X) X(1, 2) X(1, 3) X(1, 4) X(2, 2) X(2, 3) X(2, 4) X(3, 2) X(3, 3)

// Shapes with line-group kernels (the KM_CONV_FWDL / KM_CONV_BWDL lists).
static bool line_shape(const ConvArgs &a) {
    return (a.nd == 2 && a.K >= 2 && a.K <= 4) || (a.nd == 3 && (a.K == 2 || a.K == 3));
}

static int conv_fwd_launch(const ConvArgs &a, hipStream_t s) {
    bool done = false;
    const long lblocks = (a.tasks_l + kConvWaves - 1) / kConvWaves;
    if (line_shape(a) && lblocks > 0 && lblocks <= 0x7fffffffL && strip_fits(a)) {
#define KM_CONV_FWDL(ND, KK)                                                                 \
        if (!done && a.nd == ND && a.K == KK) {                                              \
            const auto kern = a.strip_l == 64 ? convnd_lines<ND, KK, false, 64>                 \
                              : a.strip_l == 32 ? convnd_lines<ND, KK, false, 32>               \
                                                : convnd_lines<ND, KK, false, 16>;              \
            hipLaunchKernelGGL(kern, dim3(lblocks), dim3(64 * kConvWaves), 0, s, a,          \
                               static_cast<const float *>(nullptr), 0);                      \
            done = true;                                                                     \
        }
        KM_CONV_FWDL(2, 2) KM_CONV_FWDL(2, 3) KM_CONV_FWDL(2, 4) KM_CONV_FWDL(3, 2) KM_CONV_FWDL(3, 3)
#undef KM_CONV_FWDL
    }
    const long blocks = (a.tasks + kConvWaves - 1) / kConvWaves;
    if (!done && blocks <= 0x7fffffffL && strip_fits(a)) {
#define KM_CONV_FWD(ND, KK)                                                                  \
        if (!done && a.nd == ND && a.K == KK) {                                              \
            hipLaunchKernelGGL((convnd_fwd_strip<ND, KK>), dim3(blocks), dim3(64 * kConvWaves), \
                               0, s, a);                                                     \
            done = true;                                                                     \
        }
        KM_CONV_SHAPES(KM_CONV_FWD)
#undef KM_CONV_FWD
    }
    if (!done) {
        const long n = a.batch * a.P * a.D;
        hipLaunchKernelGGL(convnd_fwd_generic, dim3((n + 255) / 256), dim3(256), 0, s, a);
    }
    KM_HIP_TRY(hipGetLastError());
    return 0;
}

static int conv_bwd_launch(const ConvArgs &a, hipStream_t s) {
    bool done = false;
    const long lblocks = (a.tasks_l + kConvWaves - 1) / kConvWaves;
    // dkernel slots: about two workgroups per CU over all channel groups.
    const long quads = (a.tasks_l / std::max(a.groups, 1L) + kConvWaves - 1) / kConvWaves;
    const long nslot = std::max(1L, std::min(quads, 512L / std::max(a.groups, 1L)));
    const long per = (quads + nslot - 1) / std::max(nslot, 1L);
    float *part = nullptr;
    if (line_shape(a) && lblocks > 0 && lblocks + (a.KV + 1) * a.groups <= 0x7fffffffL && a.groups <= 65535 &&
        strip_fits(a)) {
        part = static_cast<float *>(
            Workspace::reserve(sizeof(float) * a.groups * nslot * (a.KV + 1) * 64, s, WsUse::ConvBwd));
        if (!part) return -1;
    }
    if (part) {
#define KM_CONV_BWDL(ND, KK)                                                                 \
        if (!done && a.nd == ND && a.K == KK) {                                              \
            const auto kdin = a.strip_l == 64 ? convnd_lines<ND, KK, true, 64>                 \
                              : a.strip_l == 32 ? convnd_lines<ND, KK, true, 32>               \
                                                : convnd_lines<ND, KK, true, 16>;              \
            const auto kdw = a.strip_l == 64 ? convnd_dw_lines<ND, KK, 64>                      \
                             : a.strip_l == 32 ? convnd_dw_lines<ND, KK, 32>                    \
                                               : convnd_dw_lines<ND, KK, 16>;                   \
            hipLaunchKernelGGL(kdw, dim3(nslot, a.groups), dim3(64 * kConvWaves), 0, s, a, part, per); \
            hipLaunchKernelGGL(kdin, dim3(lblocks + (a.KV + 1) * a.groups), dim3(64 * kConvWaves), 0, \
                               s, a, static_cast<const float *>(part), static_cast<int>(nslot)); \
            done = true;                                                                     \
        }
#define KM_CONV_BWDF(ND, KK)                                                                 \
        if (!done && a.nd == ND && a.K == KK) {                                              \
            const auto kf = a.strip_l == 64 ? convnd_bwd_lines<ND, KK, 64>                      \
                            : a.strip_l == 32 ? convnd_bwd_lines<ND, KK, 32>                    \
                                              : convnd_bwd_lines<ND, KK, 16>;                   \
            hipLaunchKernelGGL(kf, dim3(nslot, a.groups), dim3(64 * kConvWaves), 0, s, a, part, per); \
            hipLaunchKernelGGL(convnd_dw_finish, dim3((a.KV + 1) * a.groups), dim3(64 * kConvWaves), 0, \
                               s, a, static_cast<const float *>(part), static_cast<int>(nslot)); \
            done = true;                                                                     \
        }
        // One pass where both windows fit the registers, else dkernel and
        // dinput as two line-group launches (3D with K = 3: the fused form
        // in passes of two lines, to fit, measured 81 against 56 us).
        KM_CONV_BWDF(2, 2) KM_CONV_BWDF(2, 3) KM_CONV_BWDF(2, 4) KM_CONV_BWDF(3, 2)
        KM_CONV_BWDL(3, 3)
#undef KM_CONV_BWDF
#undef KM_CONV_BWDL
    }
    if (!done && (zero_dev(a.dW, static_cast<long>(a.KV) * a.D, s) != 0 || zero_dev(a.db, a.D, s) != 0))
        return -1;
    const long blocks = (a.tasks + kConvWaves - 1) / kConvWaves;
    if (!done && blocks <= 0x7fffffffL && strip_fits(a)) {
#define KM_CONV_BWD(ND, KK)                                                                  \
        if (!done && a.nd == ND && a.K == KK) {                                              \
            hipLaunchKernelGGL((convnd_bwd_strip<ND, KK>), dim3(blocks), dim3(64 * kConvWaves), \
                               0, s, a);                                                     \
            done = true;                                                                     \
        }
        KM_CONV_SHAPES(KM_CONV_BWD)
#undef KM_CONV_BWD
    }
    if (!done) {
        const long n = a.batch * a.P * a.D;
        hipLaunchKernelGGL(convnd_bwd_input_generic, dim3((n + 255) / 256), dim3(256), 0, s, a);
        const long per = 4096;
        const long nb = (a.batch * a.P + per - 1) / per;
        dim3 g(static_cast<unsigned>(nb), static_cast<unsigned>(a.KV + 1),
               static_cast<unsigned>((a.D + 63) / 64));
        hipLaunchKernelGGL(convnd_bwd_kernel_generic, g, dim3(256), 0, s, a, per);
    }
    KM_HIP_TRY(hipGetLastError());
    return 0;
}

int convnd_device(const ConvNDParams *p, long batch, bool fwd, bool bwd, hipStream_t s,
                  const char *who) {
    if (!gpu_ready()) return -1;
    ConvArgs a;
    if (fwd) {
        if (!conv_args(p, batch, false, a, who)) return -1;
        if (conv_fwd_launch(a, s) != 0) return -1;
    }
    if (bwd) {
        if (!conv_args(p, batch, true, a, who)) return -1;
        if (conv_bwd_launch(a, s) != 0) return -1;
    }
    return 0;
}

// Host-pointer path: stage every buffer the mode touches, run, copy back.
static int convnd_host(ConvNDParams *p, bool fwd, bool bwd, const char *who) {
    if (!gpu_ready()) return -1;
    const long P = wavefront_nd_total_points(p->dims, p->ndims);
    const long KV = convnd_kernel_volume(p->ndims, p->K);
    if (P <= 0 || KV <= 0) {
        set_error("%s: invalid dims", who);
        return -1;
    }
    const size_t PD = sizeof(float) * P * p->D, KD = sizeof(float) * KV * p->D,
                 D4 = sizeof(float) * p->D;
    struct B { void *user; size_t bytes; bool in, out; void *dev; };
    B bufs[] = {
        {p->input, PD, true, false, nullptr},
        {const_cast<float *>(p->kernel), KD, true, false, nullptr},
        {const_cast<float *>(p->bias), D4, true, false, nullptr},
        {fwd ? p->output : nullptr, PD, false, true, nullptr},
        {bwd ? p->dy : nullptr, PD, true, false, nullptr},
        {bwd ? p->dinput : nullptr, PD, false, true, nullptr},
        {bwd ? p->dkernel : nullptr, KD, false, true, nullptr},
        {bwd ? p->dbias : nullptr, D4, false, true, nullptr},
    };
    constexpr int NB = sizeof(bufs) / sizeof(bufs[0]);
    bool all_dev = true;
    for (auto &b : bufs)
        if (b.user && !is_device_ptr(b.user)) all_dev = false;
    ConvNDParams q = *p;
    int rc = -1;
    Staging::lock();
    do {
        if (!all_dev) {
            size_t total = 0;
            for (auto &b : bufs)
                if (b.user) total += align_up(b.bytes, 256);
            void *base = Staging::reserve(total);
            if (!base) break;
            Carver c(base);
            bool ok = true;
            for (auto &b : bufs) {
                if (!b.user) continue;
                b.dev = c.take<char>(b.bytes);
                if (b.in && km::copy_h2d(b.dev, b.user, b.bytes) != hipSuccess) ok = false;
            }
            if (!ok) {
                set_error("%s: host-to-device copy failed", who);
                break;
            }
        } else {
            for (auto &b : bufs) b.dev = b.user;
        }
        q.input = static_cast<float *>(bufs[0].dev);
        q.kernel = static_cast<const float *>(bufs[1].dev);
        q.bias = static_cast<const float *>(bufs[2].dev);
        q.output = static_cast<float *>(bufs[3].dev);
        q.dy = static_cast<float *>(bufs[4].dev);
        q.dinput = static_cast<float *>(bufs[5].dev);
        q.dkernel = static_cast<float *>(bufs[6].dev);
        q.dbias = static_cast<float *>(bufs[7].dev);
        if (convnd_device(&q, 1, fwd, bwd, nullptr, who) != 0) break;
        if (hipStreamSynchronize(nullptr) != hipSuccess) {
            set_error("%s: %s", who, hipGetErrorString(hipGetLastError()));
            break;
        }
        bool ok = true;
        if (!all_dev) {
            for (int i = 0; i < NB; ++i) {
                if (!bufs[i].user || !bufs[i].out) continue;
                if (km::copy_d2h(bufs[i].user, bufs[i].dev, bufs[i].bytes) != hipSuccess)
                    ok = false;
            }
        }
        if (!ok) {
            set_error("%s: device-to-host copy failed", who);
            break;
        }
        rc = 0;
    } while (false);
    Staging::unlock();
    return rc;
}

}  // namespace km

extern "C" {

long convnd_kernel_volume(long ndims, long K) {
    if (ndims <= 0 || K <= 0) return 0;
    long v = 1;
    for (long i = 0; i < ndims; ++i) {
        if (v > 0x7fffffffffffffffL / K) return 0;
        v *= K;
    }
    return v;
}

// Reference src/convnd.c:67-129: silently returns on invalid parameters or a
// plan that does not match dims; host or device pointers.
void convnd_forward_wavefront(ConvNDParams *p, const KMWavefrontPlan *plan) {
    km::clear_error();
    if (!p || !p->input || !p->kernel || !p->output || !p->dims || p->ndims <= 0 || p->D <= 0 ||
        p->K <= 0) {
        km::set_error("convnd_forward_wavefront: invalid parameters");
        return;
    }
    if (!km_wavefront_plan_matches_dims(plan, p->dims, p->ndims)) {
        km::set_error("convnd_forward_wavefront: plan does not match dims");
        return;
    }
    km::convnd_host(p, true, false, "convnd_forward_wavefront");
}

// Reference src/convnd.c:135-202: dinput, dkernel, dbias overwritten.
void convnd_backward_wavefront(ConvNDParams *p, const KMWavefrontPlan *plan) {
    km::clear_error();
    if (!p || !p->input || !p->kernel || !p->dy || !p->dinput || !p->dkernel || !p->dims ||
        p->ndims <= 0 || p->D <= 0 || p->K <= 0) {
        km::set_error("convnd_backward_wavefront: invalid parameters");
        return;
    }
    if (!km_wavefront_plan_matches_dims(plan, p->dims, p->ndims)) {
        km::set_error("convnd_backward_wavefront: plan does not match dims");
        return;
    }
    km::convnd_host(p, false, true, "convnd_backward_wavefront");
}

// Reference src/convnd.c:208-244 (mode bits: 1 forward, 2 backward).
void convnd(ConvNDParams *p, ConvNDMode mode) {
    km::clear_error();
    if (!p || !p->dims || p->ndims <= 0) {
        km::set_error("convnd: invalid parameters");
        return;
    }
    const bool fwd = (mode & CONVND_FORWARD) != 0, bwd = (mode & CONVND_BACKWARD) != 0;
    if (fwd && (!p->input || !p->kernel || !p->output || p->D <= 0 || p->K <= 0)) {
        km::set_error("convnd: invalid forward parameters");
        return;
    }
    if (bwd && (!p->input || !p->kernel || !p->dy || !p->dinput || !p->dkernel || p->D <= 0 ||
                p->K <= 0)) {
        km::set_error("convnd: invalid backward parameters");
        return;
    }
    if (!wavefront_nd_validate_dims(p->dims, p->ndims)) {
        km::set_error("convnd: invalid dims");
        return;
    }
    if (fwd || bwd) km::convnd_host(p, fwd, bwd, "convnd");
}

// Reference cuda/convnd.cu:258-436: device pointers (dims on the host),
// synchronous, 0 ok / -1 error.
int om_convnd_forward(ConvNDParams *p) {
    km::clear_error();
    if (km::convnd_device(p, 1, true, false, nullptr, "om_convnd_forward") != 0) return -1;
    if (hipStreamSynchronize(nullptr) != hipSuccess) {
        km::set_error("om_convnd_forward: %s", hipGetErrorString(hipGetLastError()));
        return -1;
    }
    return 0;
}

int om_convnd_backward(ConvNDParams *p) {
    km::clear_error();
    if (km::convnd_device(p, 1, false, true, nullptr, "om_convnd_backward") != 0) return -1;
    if (hipStreamSynchronize(nullptr) != hipSuccess) {
        km::set_error("om_convnd_backward: %s", hipGetErrorString(hipGetLastError()));
        return -1;
    }
    return 0;
}

int km_convnd_fwd(const ConvNDParams *p, long batch, void *stream) {
    km::clear_error();
    return km::convnd_device(p, batch, true, false, static_cast<hipStream_t>(stream), "km_convnd_fwd");
}

int km_convnd_bwd(const ConvNDParams *p, long batch, void *stream) {
    km::clear_error();
    return km::convnd_device(p, batch, false, true, static_cast<hipStream_t>(stream), "km_convnd_bwd");
}

}  // extern "C"

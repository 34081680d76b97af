// scannd_bwd.hip - ScanND backward (km_scannd_bwd): the adjoint of the
// ScanND forward (reference src/scan_nd.c:74-192, non-lambda branch) for
// L = sum dy . y. The reference has no ScanND backward; the oracle's C
// restatement (orc_scannd_backward) is pinned by float64 finite differences
// and, in 1D, by the reference's scan1d_backward.
//
// Launches, no atomics:
//  0. Neighbour flags of every point (successor / predecessor per axis), so
//     the sweeps below do no index division.
//  1. The adjoint state g[p] = dy[p] C[p] + sum_a e_a[p+s_a] g[p+s_a] flows
//     against the forward's wavefront, g kept in dB's memory (no P x D x M
//     scratch): 2D and 3D grids with D*M a multiple of 64 by tile bands (one
//     launch per band, last first), other grids one launch per anti-diagonal
//     level, last level first, one thread per (point, channel-state).
//  2. Gradients, parallel over points, writing dC, dx, ddelta and dB (over
//     g, in place) and per-workgroup dA partials. With M a power of two
//     <= 64, lanes own consecutive channel-states (coalesced) and sum over
//     a channel's states with xor shuffles; otherwise a thread owns one
//     channel, loops over its states and keeps its dA terms in its own LDS
//     slots.
//  3. dA = the workgroups' partials summed in workgroup order.
#include <algorithm>
#include <vector>
#include <cstdint>
#include <cstdlib>
#include <cstring>

#include "km_device.hpp"
#include "scannd_flow.hpp"
#include "../km_runtime.hpp"
#include "kmamba_km.h"
#include "scan_nd.h"
#include "wavefront_nd.h"
#include "wavefront_plan.h"

namespace km {

constexpr int kNdBwdMaxAcc = 64;   // ndims * M: per-thread dA slots in LDS (64 KB)
constexpr int kAdj3P = 4, kAdj3R = 4, kAdj3W = 8;   // 3D adjoint tiles (axis 0, 1, 2)
constexpr int kAdjTR = 16, kAdjTW = 8;              // 2D adjoint tiles (rows, points)
constexpr int kAdjRB = 4;                           // 2D adjoint rows loaded per batch

struct NdBwdArgs {
    const float *x, *A, *B, *C, *delta, *h, *dy;
    float *dx, *ddelta, *dB, *dC;
    float *part;            // [nbx][nd][D][M] dA partials
    const long *offs;       // level offsets of the wavefront plan (device)
    const uint16_t *nbr;    // per point: bit a = has a successor on axis a, bit 8 + a = a predecessor
    long P, D, M;
    long dims[8], strides[8];
};

// Neighbour flags of every point: bit a = a successor on axis a, bit 8 + a
// = a predecessor.
__global__ void __launch_bounds__(256) nd_adjoint_flags(NdBwdArgs a, long nd, uint16_t *nbr) {
    const long q = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (q >= a.P) return;
    unsigned f = 0;
    for (long ax = 0; ax < nd; ++ax) {
        const long i = (q / a.strides[ax]) % a.dims[ax];
        if (i + 1 < a.dims[ax]) f |= 1u << ax;
        if (i > 0) f |= 1u << (8 + ax);
    }
    nbr[q] = static_cast<uint16_t>(f);
}

// One level of the adjoint state: workgroup (x, y) = channel-states
// [256 x, +256) of the level's point s0 + y.
template <int ND>
__global__ void __launch_bounds__(256) nd_adjoint_level(NdBwdArgs a, long s0) {
    const long DM = a.D * a.M;
    const long c = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (c >= DM) return;
    const long d = c / a.M;
    const long q = a.offs[s0 + blockIdx.y];
    const unsigned nb = a.nbr[q];
    float g = a.dy[q * a.D + d] * a.C[q * DM + c];
#pragma unroll
    for (int ax = 0; ax < ND; ++ax) {
        if (nb & (1u << ax)) {
            const long nx = q + a.strides[ax];
            const float e = exp2_fast(a.delta[(ax * a.P + nx) * a.D + d] * a.A[ax * DM + c] * kLog2e);
            g = fmaf(e, a.dB[nx * DM + c], g);
        }
    }
    a.dB[q * DM + c] = g;
}

// Buffer windows of one adjoint tile: every tensor's resource starts at the
// tile's first point qb, so offsets are 32-bit, the point's wave-uniform
// (SGPR offset) and the lane's in the VGPR offset. Windows run to the end of
// the tile's successor row (2D) or plane (3D); delta's covers all axes from
// qb on. The host keeps each window below 2 GiB.
struct AdjWin {
    __amdgpu_buffer_rsrc_t dy, C, dl, g;
    unsigned sD, sDM, sAx;   // bytes per point of [P, D] and [P, D*M]; bytes per delta axis
    int vd, vc;
};
template <int ND>
__device__ __forceinline__ AdjWin adj_window(const NdBwdArgs &a, long qb, long qe, long c, long d) {
    const long DM = a.D * a.M, n = qe - qb;
    AdjWin w;
    w.sD = static_cast<unsigned>(a.D * 4);
    w.sDM = static_cast<unsigned>(DM * 4);
    w.sAx = static_cast<unsigned>(a.P * a.D * 4);
    w.vd = static_cast<int>(d * 4);
    w.vc = static_cast<int>(c * 4);
    w.dy = make_rsrc(a.dy + qb * a.D, n * a.D * 4);
    w.C = make_rsrc(a.C + qb * DM, n * DM * 4);
    w.dl = make_rsrc(a.delta + qb * a.D, ((ND - 1) * a.P + n) * a.D * 4);
    w.g = make_rsrc(a.dB + qb * DM, n * DM * 4);
    return w;
}
__device__ __forceinline__ int adj_oD(const AdjWin &w, long r) { return static_cast<int>(static_cast<unsigned>(r) * w.sD); }
__device__ __forceinline__ int adj_oDM(const AdjWin &w, long r) { return static_cast<int>(static_cast<unsigned>(r) * w.sDM); }
// dy * C, the state g and the delta of axis ax at point qb + r.
__device__ __forceinline__ float adj_dyc(const AdjWin &w, long r) {
    return bio<f32_t>::ld(w.dy, w.vd, adj_oD(w, r)) * bio<f32_t>::ld(w.C, w.vc, adj_oDM(w, r));
}
// A successor's state; COH: written by another workgroup of the same launch
// (the dataflow schedule), read past the CU's L1.
template <bool COH = false>
__device__ __forceinline__ float adj_g(const AdjWin &w, long r) {
    return COH ? bio<f32_t>::ld_agent(w.g, w.vc, adj_oDM(w, r)) : bio<f32_t>::ld(w.g, w.vc, adj_oDM(w, r));
}
__device__ __forceinline__ float adj_dl(const AdjWin &w, int ax, long r) {
    return bio<f32_t>::ld(w.dl, w.vd, static_cast<int>(ax * w.sAx) + adj_oD(w, r));
}
__device__ __forceinline__ void adj_store(const AdjWin &w, long r, float g) {
    bio<f32_t>::st(w.g, w.vc, adj_oDM(w, r), g);
}

// 2D grids with D*M a multiple of 64: the adjoint state by tile bands. The
// grid is cut into TR x TW tiles; tiles with equal tile-index sum (a band)
// are independent, and bands run last to first, one launch each. One wave
// per (tile, group of 64 channel-states) walks its tile's rows bottom-up,
// each row right to left, keeping the row below (its g and axis-0 delta) in
// registers and the right neighbour from the previous step; successors
// across the tile's bottom and right edges were written by the previous
// launch (the next band). Workgroups are numbered XCD-major (xcd_remap):
// the channel groups of a tile, which share the dy / delta row lines (four
// channels, 16 bytes, each), run on one XCD's L2.
//
// adj_tile2d runs one (tile (ti0, ti1), channel group cg); wait() runs before
// any state written by another tile is read (false: nothing is computed).
template <int TR, int TW, int RB, bool COH, typename Wait>
__device__ __forceinline__ bool adj_tile2d(const NdBwdArgs &a, int ti0, int ti1, int cg, Wait &&wait) {
    const int lane = threadIdx.x & 63;
    const long n0 = a.dims[0], n1 = a.dims[1];
    const long r0 = static_cast<long>(ti0) * TR, r1 = std::min<long>(n0, r0 + TR);
    const long j0 = static_cast<long>(ti1) * TW, j1 = std::min<long>(n1, j0 + TW);
    const long DM = a.D * a.M;
    const long c = static_cast<long>(cg) * 64 + lane;
    const long d = c / a.M;
    const float A0 = a.A[c] * kLog2e, A1 = a.A[DM + c] * kLog2e;
    // Window: the tile's rows and the successor row below them.
    const long qb = r0 * n1;
    const AdjWin w = adj_window<2>(a, qb, (std::min<long>(r1, n0 - 1) + 1) * n1, c, d);
    // A row's operands (dy . C, both deltas) and right-edge successor,
    // loaded before the row computes (its g stores would otherwise order
    // every later load); columns past j1 load column j1 - 1 and go unused.
    struct Row {
        float dyc[TW], d0[TW], d1[TW];
        float gr, dr1;
    };
    // The operands no other tile writes (ops) and the right successor's
    // state (succ).
    auto load_ops = [&](long r, Row &rw) __attribute__((always_inline)) {
        const long rq = r * n1 - qb;
#pragma unroll
        for (int jj = 0; jj < TW; ++jj) {
            const long q = rq + std::min<long>(j0 + jj, j1 - 1);
            rw.dyc[jj] = adj_dyc(w, q);
            rw.d0[jj] = adj_dl(w, 0, q);
            rw.d1[jj] = adj_dl(w, 1, q);
        }
        rw.dr1 = adj_dl(w, 1, rq + std::min<long>(j1, n1 - 1));
    };
    auto load_succ = [&](long r, Row &rw) __attribute__((always_inline)) {
        rw.gr = adj_g<COH>(w, r * n1 - qb + std::min<long>(j1, n1 - 1));
    };
    auto load_row = [&](long r, Row &rw) __attribute__((always_inline)) {
        load_ops(r, rw);
        load_succ(r, rw);
    };
    // The first batch's operands go out before the wait on the successors.
    Row ba[RB], bb[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) load_ops(std::max<long>(r1 - 1 - i, r0), ba[i]);
    if (!wait()) return false;
#pragma unroll
    for (int i = 0; i < RB; ++i) load_succ(std::max<long>(r1 - 1 - i, r0), ba[i]);
    float gb[TW], db0[TW];
#pragma unroll
    for (int jj = 0; jj < TW; ++jj) {
        const long q = std::min<long>(r1, n0 - 1) * n1 + std::min<long>(j0 + jj, j1 - 1) - qb;
        gb[jj] = adj_g<COH>(w, q);
        db0[jj] = adj_dl(w, 0, q);
    }
    // Rows go in batches of RB, the next batch's loads issued before the
    // current batch computes: one memory latency per batch, not per row.
    auto load_batch = [&](long rtop, Row (&bt)[RB]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < RB; ++i) load_row(std::max<long>(rtop - i, r0), bt[i]);   // past r0: reload r0
    };
    auto compute_batch = [&](long rtop, const Row (&bt)[RB]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const long r = rtop - i;
            if (r >= r0) {
                const Row &cur = bt[i];
                const bool below = r + 1 < n0;
                float gr = cur.gr, dr1 = cur.dr1;
                bool right = j1 < n1;
#pragma unroll
                for (int jj = TW - 1; jj >= 0; --jj) {
                    if (j0 + jj < j1) {
                        float g = cur.dyc[jj];
                        if (below) g = fmaf(exp2_fast(db0[jj] * A0), gb[jj], g);
                        if (right) g = fmaf(exp2_fast(dr1 * A1), gr, g);
                        adj_store(w, r * n1 + j0 + jj - qb, g);
                        gb[jj] = g;
                        db0[jj] = cur.d0[jj];
                        gr = g;
                        dr1 = cur.d1[jj];
                        right = true;
                    }
                }
            }
        }
    };
    for (long rt = r1 - 1; rt >= r0; rt -= 2 * RB) {
        load_batch(rt - RB, bb);
        compute_batch(rt, ba);
        if (rt - RB >= r0) {
            load_batch(rt - 2 * RB, ba);
            compute_batch(rt - RB, bb);
        }
    }
    return true;
}

template <int TR, int TW, int RB>
__global__ void __launch_bounds__(64) nd_adjoint_tile2d(NdBwdArgs a, int band, int nt1, int ncg) {
    const int lb = static_cast<int>(xcd_remap(blockIdx.x, gridDim.x));
    const int o = lb / ncg, cg = lb - o * ncg;
    const int ti0 = (band > nt1 - 1 ? band - (nt1 - 1) : 0) + o;
    adj_tile2d<TR, TW, RB, false>(a, ti0, band - ti0, cg, [] { return true; });
}

// 3D grids with D*M a multiple of 64: the same by TP x TR x TW tiles (axis
// 0, 1, 2). tiles[] lists each band's tiles (host-built, bands contiguous);
// a wave walks its tile's planes, rows and points in reverse, keeping the
// plane below (g and axis-0 delta of every (row, column) of the tile) and
// the row below in registers (loops fully unrolled: no dynamic indexing).
template <int TP, int TR, int TW, bool COH, typename Wait>
__device__ __forceinline__ bool adj_tile3d(const NdBwdArgs &a, int tp, int tr, int tw, int cg, Wait &&wait) {
    static_assert(TR >= 3, "a ring of TR rows holds the current row and two prefetched ones");
    const int lane = threadIdx.x & 63;
    const long n0 = a.dims[0], n1 = a.dims[1], n2 = a.dims[2];
    const long p0 = static_cast<long>(tp) * TP, p1 = std::min<long>(n0, p0 + TP);
    const long r0 = static_cast<long>(tr) * TR, r1 = std::min<long>(n1, r0 + TR);
    const long j0 = static_cast<long>(tw) * TW, j1 = std::min<long>(n2, j0 + TW);
    const long DM = a.D * a.M, s0 = n1 * n2;
    const long c = static_cast<long>(cg) * 64 + lane;
    const long d = c / a.M;
    const float A0 = a.A[c] * kLog2e, A1 = a.A[DM + c] * kLog2e, A2 = a.A[2 * DM + c] * kLog2e;
    // Window: the tile's planes and the successor plane below them.
    const long qb = p0 * s0;
    const AdjWin w = adj_window<3>(a, qb, (std::min<long>(p1, n0 - 1) + 1) * s0, c, d);
    struct Row {
        float dyc[TW], d0[TW], d1[TW], d2[TW];
        float gr, dr2;
    };
    auto qof = [&](long pp, long rr, long jj) { return pp * s0 + rr * n2 + jj - qb; };
    // Rows in walk order: k = 0, 1, ... is plane p1 - 1 - k / TR, row
    // r0 + TR - 1 - k % TR (rows past r1 and k past the tile load the last
    // row again, unused). Operands no other tile writes (ops) and the right
    // successor's state (succ) load apart.
    const int nk = static_cast<int>(p1 - p0) * TR;
    auto row_at = [&](int k, long &pp, long &rr) __attribute__((always_inline)) {
        k = min(k, nk - 1);
        pp = p1 - 1 - k / TR;
        rr = std::min<long>(r0 + TR - 1 - k % TR, r1 - 1);
    };
    auto load_ops = [&](int k, Row &rw) __attribute__((always_inline)) {
        long pp, rr;
        row_at(k, pp, rr);
#pragma unroll
        for (int jj = 0; jj < TW; ++jj) {
            const long q = qof(pp, rr, std::min<long>(j0 + jj, j1 - 1));
            rw.dyc[jj] = adj_dyc(w, q);
            rw.d0[jj] = adj_dl(w, 0, q);
            rw.d1[jj] = adj_dl(w, 1, q);
            rw.d2[jj] = adj_dl(w, 2, q);
        }
        rw.dr2 = adj_dl(w, 2, qof(pp, rr, std::min<long>(j1, n2 - 1)));
    };
    auto load_succ = [&](int k, Row &rw) __attribute__((always_inline)) {
        long pp, rr;
        row_at(k, pp, rr);
        rw.gr = adj_g<COH>(w, qof(pp, rr, std::min<long>(j1, n2 - 1)));
    };
    // Row below the tile's last row of plane pp: successors along axis 1.
    auto load_below = [&](long pp, float (&gbx)[TW], float (&dbx)[TW]) __attribute__((always_inline)) {
#pragma unroll
        for (int jj = 0; jj < TW; ++jj) {
            const long q = qof(pp, std::min<long>(r1, n1 - 1), std::min<long>(j0 + jj, j1 - 1));
            gbx[jj] = adj_g<COH>(w, q);
            dbx[jj] = adj_dl(w, 1, q);
        }
    };
    // A ring of TR rows (slot = row's index within its plane): row k + 2 is
    // loaded before row k computes (and before its g stores, which would
    // otherwise order every later load). The first two rows' operands go out
    // before the wait on the successors.
    Row R[TR];
    load_ops(0, R[TR - 1]);
    load_ops(1, R[TR - 2]);
    if (!wait()) return false;
    load_succ(0, R[TR - 1]);
    load_succ(1, R[TR - 2]);
    // Plane below: successors along axis 0 of every (row, column).
    float gp[TR][TW], dp0[TR][TW];
#pragma unroll
    for (int ri = 0; ri < TR; ++ri)
#pragma unroll
        for (int jj = 0; jj < TW; ++jj) {
            const long q = qof(std::min<long>(p1, n0 - 1), std::min<long>(r0 + ri, r1 - 1),
                               std::min<long>(j0 + jj, j1 - 1));
            gp[ri][jj] = adj_g<COH>(w, q);
            dp0[ri][jj] = adj_dl(w, 0, q);
        }
    float gbn[TW], dbn[TW];
    load_below(p1 - 1, gbn, dbn);
    for (int kb = 0; kb < nk; kb += TR) {
        const long pp = p1 - 1 - kb / TR;
        const bool pbelow = pp + 1 < n0;
        float gb[TW], db1[TW];
#pragma unroll
        for (int jj = 0; jj < TW; ++jj) {
            gb[jj] = gbn[jj];
            db1[jj] = dbn[jj];
        }
#pragma unroll
        for (int i = 0; i < TR; ++i) {
            const int ri = TR - 1 - i;
            {
                Row &nx = R[(ri + TR - 2) % TR];
                load_ops(kb + i + 2, nx);
                load_succ(kb + i + 2, nx);
            }
            if (i == TR - 2) load_below(std::max<long>(pp - 1, p0), gbn, dbn);   // the next plane's
            const long r = r0 + ri;
            if (r < r1) {
                const Row &cur = R[ri];
                const bool rbelow = r + 1 < n1;
                float gr = cur.gr, dr2 = cur.dr2;
                bool right = j1 < n2;
#pragma unroll
                for (int jj = TW - 1; jj >= 0; --jj) {
                    if (j0 + jj < j1) {
                        float g = cur.dyc[jj];
                        if (pbelow) g = fmaf(exp2_fast(dp0[ri][jj] * A0), gp[ri][jj], g);
                        if (rbelow) g = fmaf(exp2_fast(db1[jj] * A1), gb[jj], g);
                        if (right) g = fmaf(exp2_fast(dr2 * A2), gr, g);
                        adj_store(w, qof(pp, r, j0 + jj), g);
                        gp[ri][jj] = g;
                        dp0[ri][jj] = cur.d0[jj];
                        gb[jj] = g;
                        db1[jj] = cur.d1[jj];
                        gr = g;
                        dr2 = cur.d2[jj];
                        right = true;
                    }
                }
            }
        }
    }
    return true;
}

template <int TP, int TR, int TW>
__global__ void __launch_bounds__(64) nd_adjoint_tile3d(NdBwdArgs a, const int *tiles, int ncg) {
    const int lb = static_cast<int>(xcd_remap(blockIdx.x, gridDim.x));
    const int o = lb / ncg, cg = lb - o * ncg;
    adj_tile3d<TP, TR, TW, false>(a, tiles[3 * o], tiles[3 * o + 1], tiles[3 * o + 2], cg, [] { return true; });
}

// The adjoint sweep on the dataflow schedule (scannd_flow.hpp), one launch:
// items in reverse band order (a tile's successors come first), a tile
// waiting on its successor along each axis; channel groups pinned to XCDs,
// workgroups of flow_q waves, one group per wave. 2D tiles are 8 rows x 4
// points (the critical path runs through nt0 + nt1 - 1 of them), 3D tiles
// those of the band schedule.
constexpr int kAdjFTR = 8, kAdjFTW = 4;   // 2D dataflow tiles (rows, points)
constexpr int kF3S = 2, kF3R = 4, kF3W = 4;   // fused 3D pencils: planes per sub-tile, rows, points

// NaN into the states of one (tile, channel group) whose wait gave up, so
// every tile that depends on it, and every gradient, turns NaN too.
template <int ND>
__device__ void adj_tile_poison(const NdBwdArgs &a, const int *ti, const int *text, int cg) {
    const long DM = a.D * a.M;
    const long c = static_cast<long>(cg) * 64 + (threadIdx.x & 63);
    long lo[ND], ext[ND], npts = 1;
#pragma unroll
    for (int ax = 0; ax < ND; ++ax) {
        lo[ax] = static_cast<long>(ti[ax]) * text[ax];
        ext[ax] = std::min<long>(text[ax], a.dims[ax] - lo[ax]);
        npts *= ext[ax];
    }
    for (long q = 0; q < npts; ++q) {
        long rem = q, off = 0;
#pragma unroll
        for (int ax = ND - 1; ax >= 0; --ax) {
            const long ia = rem % ext[ax];
            rem /= ext[ax];
            off += (lo[ax] + ia) * a.strides[ax];
        }
        a.dB[off * DM + c] = __builtin_nanf("");
    }
}

template <int ND>
__global__ void __launch_bounds__(64 * kFlowQ, 2) nd_adjoint_flow(NdBwdArgs a, FlowArgs f, int nt0, int nt1,
                                                                  int nt2, int ncg) {
    const int xcd = flow_xcd();
    const int cg0 = f.cg_lo[xcd], ncx = f.cg_lo[xcd + 1] - cg0;
    if (ncx <= 0) return;
    const int Q = static_cast<int>(blockDim.x / 64);
    const int nq = ncx / Q;                             // runs of groups per tile
    const int w = static_cast<int>(threadIdx.x / 64);
    const int ntiles = f.band_start[f.nbands];
    const unsigned nitems = static_cast<unsigned>(ntiles) * static_cast<unsigned>(nq);
    const unsigned epoch = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(f.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const int ntile[3] = {nt0, nt1, nt2};
    const int text[3] = {ND == 2 ? kAdjFTR : kAdj3P, ND == 2 ? kAdjFTW : kAdj3R, kAdj3W};
    int tstride[3];
    tstride[ND - 1] = 1;
#pragma unroll
    for (int ax = ND - 2; ax >= 0; --ax) tstride[ax] = tstride[ax + 1] * ntile[ax + 1];
    __shared__ unsigned s_item[2];
    for (int it = 0;; ++it) {
        // One fetch per workgroup, handed to every wave through LDS (two
        // alternating slots: the barrier of the next fetch orders them).
        if (threadIdx.x == 0) s_item[it & 1] = atomicAdd(&f.counter[xcd], 1u);
        __syncthreads();
        const unsigned item = __builtin_amdgcn_readfirstlane(s_item[it & 1]);
        if (item >= nitems) break;
        const int tb = ntiles - 1 - static_cast<int>(item / nq);   // reverse band order
        const int cg = cg0 + static_cast<int>(item % nq) * Q + w;
        const int band = flow_band(f, tb);
        int ti[3] = {0, 0, 0};
        band_tile_n(ND, ntile, band, tb - f.band_start[band], ti);
        int tl = 0;
#pragma unroll
        for (int ax = 0; ax < ND; ++ax) tl += ti[ax] * tstride[ax];
        auto successors_done = [&]() {
            bool ready = true;
#pragma unroll
            for (int ax = 0; ax < ND; ++ax)
                if (ti[ax] + 1 < ntile[ax])
                    ready = flow_wait(f.flags + static_cast<long>(tl + tstride[ax]) * ncg + cg, epoch,
                                      f.spin) && ready;
            return ready;
        };
        bool ok;
        if constexpr (ND == 2)
            ok = adj_tile2d<kAdjFTR, kAdjFTW, 4, true>(a, ti[0], ti[1], cg, successors_done);
        else
            ok = adj_tile3d<kAdj3P, kAdj3R, kAdj3W, true>(a, ti[0], ti[1], ti[2], cg, successors_done);
        if (!ok) {
            adj_tile_poison<ND>(a, ti, text, cg);
            if ((threadIdx.x & 63) == 0)
                __hip_atomic_store(f.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0);   // this wave's g stores acknowledged by L2
        if ((threadIdx.x & 63) == 0)
            __hip_atomic_store(f.flags + static_cast<long>(tl) * ncg + cg, epoch, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Block: 256 threads = qlanes point lanes x db channels (db a power of two);
// the workgroup covers channels [blockIdx.y * db, +db) and points
// [blockIdx.x * qc, +qc).
template <int ND>
__global__ void __launch_bounds__(256) nd_adjoint_grads(NdBwdArgs a, long qc, int db) {
    extern __shared__ float acc[];                 // [ND * M][256]
    const int tid = threadIdx.x;
    const int qlanes = 256 / db;
    const int ql = tid / db, dl = tid - ql * db;
    const long d = static_cast<long>(blockIdx.y) * db + dl;
    const long q0 = static_cast<long>(blockIdx.x) * qc;
    const long q1 = std::min<long>(a.P, q0 + qc);
    const long M = a.M, DM = a.D * M;
    const int nacc = ND * static_cast<int>(M);
    for (int k = 0; k < nacc; ++k) acc[k * 256 + tid] = 0.f;
    if (d < a.D) {
        for (long q = q0 + ql; q < q1; q += qlanes) {
            const float xv = a.x[q * a.D + d], dyv = a.dy[q * a.D + d];
            float dl_[ND];
            long prev[ND];
            bool has[ND];
            float dtb = 0.f;
#pragma unroll
            for (int ax = 0; ax < ND; ++ax) {
                dl_[ax] = a.delta[(ax * a.P + q) * a.D + d];
                dtb += dl_[ax];
                has[ax] = (a.nbr[q] >> (8 + ax)) & 1u;
                prev[ax] = has[ax] ? q - a.strides[ax] : q;
            }
            dtb /= static_cast<float>(ND);
            float sx = 0.f, sbx = 0.f, sdel[ND];
#pragma unroll
            for (int ax = 0; ax < ND; ++ax) sdel[ax] = 0.f;
            const long base = q * DM + d * M;
            for (long m = 0; m < M; ++m) {
                const float gv = a.dB[base + m], bv = a.B[base + m];
                a.dC[base + m] = dyv * a.h[base + m];
                sx += gv * dtb * bv;
                sbx += gv * bv * xv;
#pragma unroll
                for (int ax = 0; ax < ND; ++ax) {
                    if (has[ax]) {
                        const float av = a.A[(ax * a.D + d) * M + m];
                        const float e = exp2_fast(dl_[ax] * av * kLog2e);
                        const float gh = gv * e * a.h[prev[ax] * DM + d * M + m];
                        sdel[ax] += gh * av;
                        acc[(ax * M + m) * 256 + tid] += gh * dl_[ax];
                    }
                }
                a.dB[base + m] = gv * dtb * xv;
            }
            a.dx[q * a.D + d] = sx;
#pragma unroll
            for (int ax = 0; ax < ND; ++ax)
                a.ddelta[(ax * a.P + q) * a.D + d] = sbx / static_cast<float>(ND) + sdel[ax];
        }
    }
    __syncthreads();
    if (ql == 0 && d < a.D) {
        for (int k = 0; k < nacc; ++k) {
            float s = 0.f;
            for (int l = 0; l < qlanes; ++l) s += acc[k * 256 + l * db + dl];
            const long ax = k / M, m = k - ax * M;
            a.part[((static_cast<long>(blockIdx.x) * ND + ax) * a.D + d) * M + m] = s;
        }
    }
}

// Gradients with M a power of two <= 64: lane order follows memory (thread
// t of workgroup (x, y) owns channel-state c = 256 y + t, so every load and
// store of a point is one contiguous run), the M lanes of a channel sum
// their dx / ddelta terms with xor shuffles (groups of M lanes are aligned
// since M divides 64), and each lane keeps its own dA terms in registers
// over the workgroup's points. Workgroup x covers points [x qc, +qc).
template <int ND>
__global__ void __launch_bounds__(256) nd_adjoint_grads_lanes(NdBwdArgs a, long qc) {
    const long M = a.M, DM = a.D * M;
    const long c0 = static_cast<long>(blockIdx.y) * 256 + threadIdx.x;
    const bool active = c0 < DM;
    const long c = active ? c0 : 0;                 // idle lanes still join the shuffles
    const long d = c / M;
    const int m = static_cast<int>(c - d * M);
    const long q0 = static_cast<long>(blockIdx.x) * qc;
    const long q1 = std::min<long>(a.P, q0 + qc);
    float av[ND], dAacc[ND];
#pragma unroll
    for (int ax = 0; ax < ND; ++ax) {
        av[ax] = a.A[ax * DM + c];
        dAacc[ax] = 0.f;
    }
    for (long q = q0; q < q1; ++q) {
        const float xv = a.x[q * a.D + d], dyv = a.dy[q * a.D + d];
        float dl_[ND];
        float dtb = 0.f;
#pragma unroll
        for (int ax = 0; ax < ND; ++ax) {
            dl_[ax] = a.delta[(ax * a.P + q) * a.D + d];
            dtb += dl_[ax];
        }
        dtb /= static_cast<float>(ND);
        const long pc = q * DM + c;
        const unsigned nb = a.nbr[q];
        const float gv = a.dB[pc], bv = a.B[pc];
        float tx = gv * dtb * bv, tbx = gv * bv * xv, td[ND];
#pragma unroll
        for (int ax = 0; ax < ND; ++ax) {
            td[ax] = 0.f;
            if ((nb >> (8 + ax)) & 1u) {
                const float e = exp2_fast(dl_[ax] * av[ax] * kLog2e);
                const float gh = gv * e * a.h[pc - a.strides[ax] * DM];
                td[ax] = gh * av[ax];
                dAacc[ax] += gh * dl_[ax];
            }
        }
        for (int k = 1; k < M; k <<= 1) {
            tx += __shfl_xor(tx, k);
            tbx += __shfl_xor(tbx, k);
#pragma unroll
            for (int ax = 0; ax < ND; ++ax) td[ax] += __shfl_xor(td[ax], k);
        }
        if (active) {
            a.dC[pc] = dyv * a.h[pc];
            a.dB[pc] = gv * dtb * xv;
            if (m == 0) {
                a.dx[q * a.D + d] = tx;
#pragma unroll
                for (int ax = 0; ax < ND; ++ax)
                    a.ddelta[(ax * a.P + q) * a.D + d] = tbx / static_cast<float>(ND) + td[ax];
            }
        }
    }
    if (active) {
#pragma unroll
        for (int ax = 0; ax < ND; ++ax) a.part[(static_cast<long>(blockIdx.x) * ND + ax) * DM + c] = dAacc[ax];
    }
}

// One point of the gradient pass in the lanes layout of
// nd_adjoint_grads_lanes, split in two so that a tile walk can issue the
// loads of a group of points before the arithmetic and stores of the first:
// the compiler does not move a load above a store through pointers it
// cannot tell apart (dB is read as g and written in place).
//
// The tile walks address memory through buffer windows that start at the
// tile's first accessed point qb (the start of the row, or plane, before
// the tile), so every offset is 32-bit: the lane's (channel d or
// channel-state c) in the VGPR offset and the point's, wave-uniform, in the
// SGPR offset. Lanes that own no output store at an offset with bit 31 set,
// past the window, which the range check drops.
template <int ND>
struct GradIn {
    float xv, dyv, dl[ND], gv, bv, hv;
};

struct GradWin {
    __amdgpu_buffer_rsrc_t x, dy, dl, g, B, h, dC, dx, ddl;
    unsigned sD, sDM, sAx;   // bytes per point of [P, D] and [P, D*M]; bytes per delta axis
    int vd, vc;              // the lane's byte offsets in a [P, D] and a [P, D*M] row
    int vcs, vds;            // store offsets: vc / vd, or dropped (inactive lane; dx, ddelta: m != 0)
};

// Windows over the points [qb, qe) of every tensor (delta and ddelta: all
// axes from qb on). The host keeps each window below 2 GiB.
template <int ND>
__device__ __forceinline__ GradWin grad_window(const NdBwdArgs &a, long qb, long qe, long c, long d, int m,
                                               bool active) {
    constexpr unsigned kDrop = 0x80000000u;
    const long DM = a.D * a.M, n = qe - qb;
    GradWin w;
    w.sD = static_cast<unsigned>(a.D * 4);
    w.sDM = static_cast<unsigned>(DM * 4);
    w.sAx = static_cast<unsigned>(a.P * a.D * 4);
    w.vd = static_cast<int>(d * 4);
    w.vc = static_cast<int>(c * 4);
    w.vcs = active ? w.vc : static_cast<int>(kDrop);
    w.vds = (active && m == 0) ? w.vd : static_cast<int>(kDrop);
    w.x = make_rsrc(a.x + qb * a.D, n * a.D * 4);
    w.dy = make_rsrc(a.dy + qb * a.D, n * a.D * 4);
    w.dx = make_rsrc(a.dx + qb * a.D, n * a.D * 4);
    w.dl = make_rsrc(a.delta + qb * a.D, ((ND - 1) * a.P + n) * a.D * 4);
    w.ddl = make_rsrc(a.ddelta + qb * a.D, ((ND - 1) * a.P + n) * a.D * 4);
    w.g = make_rsrc(a.dB + qb * DM, n * DM * 4);
    w.B = make_rsrc(a.B + qb * DM, n * DM * 4);
    w.h = make_rsrc(a.h + qb * DM, n * DM * 4);
    w.dC = make_rsrc(a.dC + qb * DM, n * DM * 4);
    return w;
}

// The state of point qb + r (a predecessor the walk does not carry).
__device__ __forceinline__ float grad_h(const GradWin &w, long r) {
    return bio<f32_t>::ld(w.h, w.vc, static_cast<int>(static_cast<unsigned>(r) * w.sDM));
}

template <int ND>
__device__ __forceinline__ GradIn<ND> grad_load(const GradWin &w, long r) {
    const int oD = static_cast<int>(static_cast<unsigned>(r) * w.sD);
    const int oDM = static_cast<int>(static_cast<unsigned>(r) * w.sDM);
    GradIn<ND> v;
    v.xv = bio<f32_t>::ld(w.x, w.vd, oD);
    v.dyv = bio<f32_t>::ld(w.dy, w.vd, oD);
#pragma unroll
    for (int ax = 0; ax < ND; ++ax) v.dl[ax] = bio<f32_t>::ld(w.dl, w.vd, static_cast<int>(ax * w.sAx) + oD);
    v.gv = bio<f32_t>::ld(w.g, w.vc, oDM);
    v.bv = bio<f32_t>::ld(w.B, w.vc, oDM);
    v.hv = bio<f32_t>::ld(w.h, w.vc, oDM);
    return v;
}

// Sum over the MM lanes of a channel (aligned groups of a power of two up
// to 64), every lane getting the total: xor 1 and xor 2 by quad_perm, the
// half-row mirror (l ^ 7, which pairs the two quads of 8 lanes), row_ror:8
// (l ^ 8), then the 16- and 32-lane swaps, all on the VALU.
template <int MM>
__device__ __forceinline__ float channel_sum(float v) {
    if constexpr (MM >= 2) v += dpp<0xB1>(v);
    if constexpr (MM >= 4) v += dpp<0x4E>(v);
    if constexpr (MM >= 8) v += dpp<0x141>(v);
    if constexpr (MM >= 16) v += dpp<0x128>(v);
    if constexpr (MM >= 32) v = sum_xor16(v);
    if constexpr (MM >= 64) v = sum_xor32(v);
    return v;
}

// The arithmetic and stores of point qb + r, with the states of its axis
// predecessors hp[ax] (used where has[ax]). avl[ax] = A * log2(e).
// Per-channel outputs (dx, ddelta) of the MM lanes of a channel: a wave
// holds 64 / MM channels, so a direct store writes 64 / MM * 4 bytes per
// point. With PTS > 0 (4 <= MM <= 32) lane m = 0 of each channel puts them
// into the workgroup's LDS stage instead, at slot `slot` of PTS points, and
// grad_flush writes a group of points with every lane busy.
template <int MM>
constexpr bool kStageOut = MM >= 4 && MM <= 32;
constexpr int kGradPts = 32;   // points per staged group

template <int ND, int MM, int PTS>
__device__ __forceinline__ void grad_finish(const GradWin &w, const GradIn<ND> &v, long r,
                                            const float (&av)[ND], const float (&avl)[ND], float (&dAacc)[ND],
                                            const float (&hp)[ND], const bool (&has)[ND], float *stage,
                                            int slot) {
    constexpr float kInvNd = 1.0f / ND;
    float dtb = v.dl[0];
#pragma unroll
    for (int ax = 1; ax < ND; ++ax) dtb += v.dl[ax];
    dtb *= kInvNd;
    const float gb = v.gv * v.bv;
    const float tx = channel_sum<MM>(gb * dtb);
    const float tb = gb * v.xv * kInvNd;
    float td[ND];
#pragma unroll
    for (int ax = 0; ax < ND; ++ax) {
        float t = tb;
        if (has[ax]) {
            const float gh = v.gv * exp2_fast(v.dl[ax] * avl[ax]) * hp[ax];
            t = fmaf(gh, av[ax], tb);
            dAacc[ax] = fmaf(gh, v.dl[ax], dAacc[ax]);
        }
        td[ax] = channel_sum<MM>(t);
    }
    const int oD = static_cast<int>(static_cast<unsigned>(r) * w.sD);
    const int oDM = static_cast<int>(static_cast<unsigned>(r) * w.sDM);
    bio<f32_t>::st(w.dC, w.vcs, oDM, v.dyv * v.hv);
    bio<f32_t>::st(w.g, w.vcs, oDM, v.gv * dtb * v.xv);
    if constexpr (PTS > 0) {
        if (w.vds >= 0) {
            constexpr int CPW = 256 / MM;
            const int lc = static_cast<int>(threadIdx.x) / MM;
            stage[slot * CPW + lc] = tx;
#pragma unroll
            for (int ax = 0; ax < ND; ++ax) stage[((ax + 1) * PTS + slot) * CPW + lc] = td[ax];
        }
    } else {
        bio<f32_t>::st(w.dx, w.vds, oD, tx);
#pragma unroll
        for (int ax = 0; ax < ND; ++ax) bio<f32_t>::st(w.ddl, w.vds, static_cast<int>(ax * w.sAx) + oD, td[ax]);
    }
}

// Writes a staged group of PTS points: dx and the ND ddelta planes of the
// workgroup's 256 / MM channels (from channel d0), point slot -> window
// offset point_of(slot) (negative: no point). Consecutive threads take
// consecutive channels of a point, so each point's run is one contiguous
// store per tensor.
template <int ND, int MM, int PTS, typename PointOf>
__device__ __forceinline__ void grad_flush(const GradWin &w, const float *stage, long d0, long D,
                                           PointOf point_of) {
    constexpr int CPW = 256 / MM;
    static_assert((CPW * PTS) % 256 == 0, "one tensor per pass of the workgroup");
    constexpr int NE = (ND + 1) * PTS * CPW;
#pragma unroll
    for (int e0 = 0; e0 < NE; e0 += 256) {
        const int e = e0 + static_cast<int>(threadIdx.x);
        const int k = e0 / (CPW * PTS);   // workgroup-uniform: dx, then the ddelta axes
        const int lc = e % CPW, slot = (e / CPW) % PTS;
        const long r = point_of(slot);
        const long d = d0 + lc;
        if (r >= 0 && d < D) {
            const unsigned off = static_cast<unsigned>(d * 4) + static_cast<unsigned>(r) * w.sD;
            if (k == 0) bio<f32_t>::st(w.dx, static_cast<int>(off), 0, stage[e]);
            else bio<f32_t>::st(w.ddl, static_cast<int>(off + (k - 1) * w.sAx), 0, stage[e]);
        }
    }
}

// The gradient pass over tiles of a 2D grid: workgroup x takes tile x (TR
// rows x TW points) and walks it column by column, down each column, so the
// state of the point above is the previous step's and the one to the left
// is the previous column's (kept per row): only the tile's first row and
// first column read a predecessor's state from memory. A column's TR points
// load one column ahead of the arithmetic.
template <int TR, int TW, int MM>
__global__ void __launch_bounds__(256) nd_adjoint_grads_tile2d(NdBwdArgs a) {
    const long DM = a.D * MM;
    // Tile and channel block, numbered XCD-major: the channel blocks of a
    // tile, which share the x / dy / delta row lines, run on one XCD.
    long tile, cbx;
    xcd_tile(tile, cbx);
    const long c0 = cbx * 256 + threadIdx.x;
    const bool active = c0 < DM;
    const long c = active ? c0 : 0;
    const long d = c / MM;
    const int m = static_cast<int>(c - d * MM);
    const long d1 = a.dims[1];
    const long nt1 = (d1 + TW - 1) / TW;
    const long i0 = (tile / nt1) * TR, j0 = (tile % nt1) * TW;
    const long ie = std::min<long>(TR, a.dims[0] - i0), je = std::min<long>(TW, d1 - j0);
    // Window: from the start of the row above the tile to the end of its last row.
    const long qb = (i0 > 0 ? i0 - 1 : 0) * d1, qe = (i0 + ie) * d1;
    const GradWin w = grad_window<2>(a, qb, qe, c, d, m, active);
    float av[2], avl[2], dAacc[2];
#pragma unroll
    for (int ax = 0; ax < 2; ++ax) {
        av[ax] = a.A[ax * DM + c];
        avl[ax] = av[ax] * kLog2e;
        dAacc[ax] = 0.f;
    }
    float left[TR];
#pragma unroll
    for (int ii = 0; ii < TR; ++ii) {
        const long i = i0 + (ii < ie ? ii : 0);
        left[ii] = j0 > 0 ? grad_h(w, i * d1 + j0 - 1 - qb) : 0.f;
    }
    auto load_col = [&](long jj, GradIn<2> (&v)[TR], float &up0) {
        const long j = j0 + (jj < je ? jj : 0);           // past the tile: reload column j0
#pragma unroll
        for (int ii = 0; ii < TR; ++ii) {
            const long i = i0 + (ii < ie ? ii : 0);       // rows past the grid reload row i0
            v[ii] = grad_load<2>(w, i * d1 + j - qb);
        }
        up0 = i0 > 0 ? grad_h(w, (i0 - 1) * d1 + j - qb) : 0.f;
    };
    // dx / ddelta of kGradPts / TR columns at a time through LDS (double
    // buffered: one barrier per group).
    constexpr int PTS = kStageOut<MM> ? kGradPts : 0;
    constexpr int CPG = kGradPts / TR;   // columns per staged group
    static_assert(kGradPts % TR == 0, "whole columns per staged group");
    __shared__ float stage[kStageOut<MM> ? 2 * 3 * kGradPts * (256 / MM) : 1];
    const long d0 = cbx * (256 / MM);
    auto finish_col = [&](long jj, const GradIn<2> (&v)[TR], float up) {
        const long j = j0 + jj;
        float *st = stage + ((jj / CPG) & 1) * (3 * kGradPts * (256 / MM));
#pragma unroll
        for (int ii = 0; ii < TR; ++ii) {
            if (ii < ie) {
                const long i = i0 + ii;
                const bool has[2] = {i > 0, j > 0};
                const float hp[2] = {up, left[ii]};
                grad_finish<2, MM, PTS>(w, v[ii], i * d1 + j - qb, av, avl, dAacc, hp, has, st,
                                        static_cast<int>((jj % CPG) * TR + ii));
                up = v[ii].hv;
                left[ii] = v[ii].hv;
            }
        }
        if constexpr (PTS > 0) {
            if (jj % CPG == CPG - 1 || jj == je - 1) {
                __syncthreads();
                const long c0j = jj - jj % CPG;   // first column of the group
                grad_flush<2, MM, PTS>(w, st, d0, a.D, [&](int sl) -> long {
                    const long col = c0j + sl / TR, ii = sl % TR;
                    return (col < je && ii < ie) ? (i0 + ii) * d1 + j0 + col - qb : -1;
                });
            }
        }
    };
    GradIn<2> va[TR], vb[TR];
    float ua = 0.f, ub = 0.f;
    load_col(0, va, ua);
    for (long jj = 0; jj < je; jj += 2) {
        load_col(jj + 1, vb, ub);
        finish_col(jj, va, ua);
        if (jj + 1 < je) {
            load_col(jj + 2, va, ua);
            finish_col(jj + 1, vb, ub);
        }
    }
    if (active) {
#pragma unroll
        for (int ax = 0; ax < 2; ++ax) a.part[(tile * 2 + ax) * DM + c] = dAacc[ax];
    }
}

// The same over tiles of a 3D grid (TP planes x TR rows x TW points), TPW
// consecutive tiles per workgroup (fewer dA partials to add afterwards): the
// walk goes row by row, point by point, through the tile's planes at each
// (row, point), so the plane predecessor is the previous step's state, the
// point to the left the previous point's (per plane) and the row above the
// previous row's (per point and plane, TW x TP registers). The TP points of
// a (row, point) load one group ahead of the arithmetic.
template <int TP, int TR, int TW, int TPW, int MM>
__global__ void __launch_bounds__(256) nd_adjoint_grads_tile3d(NdBwdArgs a) {
    const long DM = a.D * MM;
    long blk, cbx;                  // tiles [blk * TPW, +TPW), channel block (XCD-major)
    xcd_tile(blk, cbx);
    const long c0 = cbx * 256 + threadIdx.x;
    const bool active = c0 < DM;
    const long c = active ? c0 : 0;
    const long d = c / MM;
    const int m = static_cast<int>(c - d * MM);
    const long d1 = a.dims[1], d2 = a.dims[2];
    const long nt1 = (d1 + TR - 1) / TR, nt2 = (d2 + TW - 1) / TW;
    const long ntiles = ((a.dims[0] + TP - 1) / TP) * nt1 * nt2;
    const long s0 = d1 * d2;
    float av[3], avl[3], dAacc[3];
#pragma unroll
    for (int ax = 0; ax < 3; ++ax) {
        av[ax] = a.A[ax * DM + c];
        avl[ax] = av[ax] * kLog2e;
        dAacc[ax] = 0.f;
    }
    const long t1 = std::min<long>(ntiles, (blk + 1) * TPW);
#pragma unroll 1
    for (long t = blk * TPW; t < t1; ++t) {
    const long p0 = (t / (nt1 * nt2)) * TP, i0 = ((t / nt2) % nt1) * TR, j0 = (t % nt2) * TW;
    const long pe = std::min<long>(TP, a.dims[0] - p0), ie = std::min<long>(TR, d1 - i0),
               je = std::min<long>(TW, d2 - j0);
    // Window: from the start of the plane before the tile to the end of its last plane.
    const long qb = (p0 > 0 ? p0 - 1 : 0) * s0, qe = (p0 + pe) * s0;
    const GradWin w = grad_window<3>(a, qb, qe, c, d, m, active);
    float above[TW][TP];
    // The TP points of (row ii, point jj) with the states the walk does not
    // carry (the plane before the tile; the row above the tile on its first
    // row; the point left of the tile on its first point), loaded one group
    // ahead of the group being computed.
    struct Group {
        GradIn<3> v[TP];
        float prev0, up[TP], left[TP];
    };
    auto load_grp = [&](long ii, int jj, Group &g) {
        const long i = i0 + (ii < ie ? ii : 0);           // past the tile: reload row i0
        const long j = j0 + (jj < je ? jj : 0);
#pragma unroll
        for (int pp = 0; pp < TP; ++pp) {
            const long pl = p0 + (pp < pe ? pp : 0);      // planes past the grid reload plane p0
            const long r = pl * s0 + i * d2 + j - qb;
            g.v[pp] = grad_load<3>(w, r);
            g.up[pp] = (ii == 0 && i > 0) ? grad_h(w, r - d2) : 0.f;
            g.left[pp] = (jj == 0 && j > 0) ? grad_h(w, r - 1) : 0.f;
        }
        g.prev0 = p0 > 0 ? grad_h(w, (p0 - 1) * s0 + i * d2 + j - qb) : 0.f;
    };
    // dx / ddelta of each row's TW x TP points through LDS (double buffered
    // by row: one barrier per row).
    constexpr int PTS = (kStageOut<MM> && TW * TP == kGradPts) ? kGradPts : 0;
    __shared__ float stage[PTS > 0 ? 2 * 4 * kGradPts * (256 / MM) : 1];
    const long d0 = cbx * (256 / MM);
    Group ga, gb;
    load_grp(0, 0, ga);
    for (long ii = 0; ii < ie; ++ii) {
        const long i = i0 + ii;
        float *st = stage + (ii & 1) * (4 * kGradPts * (256 / MM));
        float left[TP];
#pragma unroll
        for (int jj = 0; jj < TW; ++jj) {
            Group &cur = (jj % 2 == 0) ? ga : gb;
            Group &nxt = (jj % 2 == 0) ? gb : ga;
            if (jj + 1 < TW) load_grp(ii, jj + 1, nxt);
            else load_grp(ii + 1, 0, nxt);
            if (jj < je) {
                const long j = j0 + jj;
                float prev = cur.prev0;
#pragma unroll
                for (int pp = 0; pp < TP; ++pp) {
                    if (pp < pe) {
                        const long pl = p0 + pp;
                        const bool has[3] = {pl > 0, i > 0, j > 0};
                        const float hp[3] = {prev, ii == 0 ? cur.up[pp] : above[jj][pp],
                                             jj == 0 ? cur.left[pp] : left[pp]};
                        grad_finish<3, MM, PTS>(w, cur.v[pp], pl * s0 + i * d2 + j - qb, av, avl, dAacc, hp,
                                                has, st, jj * TP + pp);
                        prev = cur.v[pp].hv;
                        left[pp] = cur.v[pp].hv;
                        above[jj][pp] = cur.v[pp].hv;
                    }
                }
            }
        }
        if constexpr (PTS > 0) {
            __syncthreads();
            grad_flush<3, MM, PTS>(w, st, d0, a.D, [&](int sl) -> long {
                const long jj = sl / TP, pp = sl % TP;
                return (jj < je && pp < pe) ? (p0 + pp) * s0 + i * d2 + j0 + jj - qb : -1;
            });
        }
    }
    }
    if (active) {
#pragma unroll
        for (int ax = 0; ax < 3; ++ax) a.part[(blk * 3 + ax) * DM + c] = dAacc[ax];
    }
}

// The 2D backward fused on the dataflow schedule: an item is a pencil (a
// column strip of TW points through every row, run of kFlowQ channel
// groups), taken right to left. Each wave walks its group's pencil
// bottom-up in sub-tiles of TR rows (a completion flag after each), each
// row right to left as adj_tile2d does, and at each point forms every
// gradient from the adjoint state it just computed, in grad_finish's
// arithmetic. The adjoint state is never stored whole: the row below stays
// in registers across sub-tiles and only the pencil's first column goes to
// the boundary buffer gC, which the pencil to the left reads (a sub-tile
// waits only on the same sub-tile of the pencil to its right). A point's
// own decays exp2(delta_a A_a), which its gradient terms need, are the ones
// its predecessors' adjoint steps need, so each is formed once. dx / ddelta
// go through the workgroup's LDS stage (grad_flush) per sub-tile; dA is
// summed per (pencil, group) in walk order, so every output is identical
// run to run.
struct Fused2PArgs {
    float *gC;   // [n0][nt1][D*M]: the states of each pencil's first column
    int nt1, nsub;
};

template <int TR, int TW, int RB, int MM>
__global__ void __launch_bounds__(64 * kFlowQ, 2) nd_fused2p(NdBwdArgs a, FlowArgs f, Fused2PArgs u) {
    constexpr int PTS = TR * TW;                  // a sub-tile is one staged group
    static_assert(kStageOut<MM> && (256 / MM * PTS) % 256 == 0, "staged per-channel outputs");
    static_assert(TR % RB == 0, "whole batches of rows");
    constexpr float kInvNd = 0.5f;
    constexpr int CPW = 256 / MM;
    constexpr int SG = 3 * PTS * CPW;             // one stage buffer: dx, ddelta0, ddelta1
    const int xcd = flow_xcd();
    const int cg0 = f.cg_lo[xcd], ncx = f.cg_lo[xcd + 1] - cg0;
    if (ncx <= 0) return;
    const int nq = ncx / kFlowQ;
    const int w = static_cast<int>(threadIdx.x / 64);
    const int lane = static_cast<int>(threadIdx.x & 63);
    const int npen = u.nt1;
    const unsigned nitems = static_cast<unsigned>(npen) * static_cast<unsigned>(nq);
    const unsigned epoch = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(f.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const int n0 = static_cast<int>(a.dims[0]), n1 = static_cast<int>(a.dims[1]);
    const int DM = static_cast<int>(a.D) * MM;
    const int ncg = DM / 64;
    const int sD = static_cast<int>(a.D) * 4, sDM = DM * 4, sAx = static_cast<int>(a.P * a.D * 4);
    __shared__ unsigned s_item[2];
    __shared__ float stage[2 * SG];
    using F = bio<f32_t>;
    struct Row {
        float dy[TW], x[TW], d0[TW], d1[TW], C[TW], B[TW], h[TW];
        float hl, dr1, gr;   // h left of the pencil, delta_1 and state right of it
    };
    int sub_n = 0;
    for (int it = 0;; ++it) {
        if (threadIdx.x == 0) s_item[it & 1] = atomicAdd(&f.counter[xcd], 1u);
        __syncthreads();
        const unsigned item = __builtin_amdgcn_readfirstlane(s_item[it & 1]);
        if (item >= nitems) break;
        const int t1 = npen - 1 - static_cast<int>(item / nq);      // right to left
        const int cgr = cg0 + static_cast<int>(item % nq) * kFlowQ;
        const int cg = cgr + w;
        const int c = cg * 64 + lane;
        const int d = c / MM;
        const int m = c - d * MM;
        const int j0 = t1 * TW, j1 = min(n1, j0 + TW), je = j1 - j0;
        const bool right_tile = j1 < n1;
        const float A0 = a.A[c] * kLog2e, A1 = a.A[DM + c] * kLog2e;
        const float av[2] = {a.A[c], a.A[DM + c]};
        const int lc = static_cast<int>(threadIdx.x) / MM;
        int voD[TW], voDM[TW];
#pragma unroll
        for (int jj = 0; jj < TW; ++jj) {
            const int cc = min(jj, je - 1);
            voD[jj] = d * 4 + cc * sD;
            voDM[jj] = c * 4 + cc * sDM;
        }
        // gC (r, t1) at r * nt1 from the pencil's base, the right pencil's at + 1.
        const long gcb = static_cast<long>(t1) * DM;
        const auto rgC = make_rsrc(u.gC + gcb, (static_cast<long>(n0) * u.nt1 * DM - gcb) * 4);
        float gb[TW], eb[TW];             // the row below: state, decay along axis 0
#pragma unroll
        for (int jj = 0; jj < TW; ++jj) gb[jj] = eb[jj] = 0.f;
        float dAacc[2] = {0.f, 0.f};
        bool ok = true;
        for (int s = u.nsub - 1; s >= 0; --s, ++sub_n) {
            const int r0 = s * TR, r1 = min(n0, r0 + TR);
            const int qb = (r0 > 0 ? r0 - 1 : 0) * n1, qe = r1 * n1;
            const long nqp = qe - qb;
            const auto rx = make_rsrc(a.x + static_cast<long>(qb) * a.D, nqp * a.D * 4);
            const auto rdy = make_rsrc(a.dy + static_cast<long>(qb) * a.D, nqp * a.D * 4);
            const auto rdl = make_rsrc(a.delta + static_cast<long>(qb) * a.D, (a.P + nqp) * a.D * 4);
            const auto rg = make_rsrc(a.dB + static_cast<long>(qb) * DM, nqp * DM * 4);
            const auto rB = make_rsrc(a.B + static_cast<long>(qb) * DM, nqp * DM * 4);
            const auto rC = make_rsrc(a.C + static_cast<long>(qb) * DM, nqp * DM * 4);
            const auto rh = make_rsrc(a.h + static_cast<long>(qb) * DM, nqp * DM * 4);
            const auto rdC = make_rsrc(a.dC + static_cast<long>(qb) * DM, nqp * DM * 4);
            float *st = stage + (sub_n & 1) * SG;
            auto rowq = [&](int r) { return r * n1 + j0 - qb; };
            auto ld_ops = [&](int r, Row &rw) __attribute__((always_inline)) {
                const int oD = rowq(r) * sD, oDM = rowq(r) * sDM;
#pragma unroll
                for (int jj = 0; jj < TW; ++jj) {
                    rw.dy[jj] = F::ld(rdy, voD[jj], oD);
                    rw.x[jj] = F::ld(rx, voD[jj], oD);
                    rw.d0[jj] = F::ld(rdl, voD[jj], oD);
                    rw.d1[jj] = F::ld(rdl, voD[jj], sAx + oD);
                    rw.C[jj] = F::ld(rC, voDM[jj], oDM);
                    rw.B[jj] = F::ld(rB, voDM[jj], oDM);
                    rw.h[jj] = F::ld(rh, voDM[jj], oDM);
                }
                rw.hl = j0 > 0 ? F::ld(rh, c * 4, oDM - sDM) : 0.f;
                rw.dr1 = right_tile ? F::ld(rdl, d * 4, sAx + oD + je * sD) : 0.f;
            };
            auto ld_succ = [&](int r, Row &rw) __attribute__((always_inline)) {
                rw.gr = right_tile ? F::ld_agent(rgC, c * 4, (r * u.nt1 + 1) * sDM) : 0.f;
            };
            Row ba[RB], bb[RB];
#pragma unroll
            for (int i = 0; i < RB; ++i) ld_ops(max(r1 - 1 - i, r0), ba[i]);
            float htop[TW];
#pragma unroll
            for (int jj = 0; jj < TW; ++jj) htop[jj] = r0 > 0 ? F::ld(rh, voDM[jj], rowq(r0 - 1) * sDM) : 0.f;
            const long fb = static_cast<long>(s) * npen + t1;
            if (ok && right_tile) ok = flow_wait(f.flags + (fb + 1) * ncg + cg, epoch, f.spin);
            if (ok) {
#pragma unroll
                for (int i = 0; i < RB; ++i) ld_succ(max(r1 - 1 - i, r0), ba[i]);
                auto ld_batch = [&](int rtop, Row (&bt)[RB]) __attribute__((always_inline)) {
#pragma unroll
                    for (int i = 0; i < RB; ++i) {
                        const int r = max(rtop - i, r0);
                        ld_ops(r, bt[i]);
                        ld_succ(r, bt[i]);
                    }
                };
                auto do_batch = [&](int rtop, const Row (&bt)[RB], const Row (&nx)[RB]) __attribute__((always_inline)) {
#pragma unroll
                    for (int i = 0; i < RB; ++i) {
                        const int r = rtop - i;
                        if (r >= r0) {
                            const Row &cur = bt[i];
                            const Row &up = (i + 1 < RB) ? bt[i + 1] : nx[0];
                            const bool below = r + 1 < n0;
                            const int oDM = rowq(r) * sDM;
                            const int slot0 = (r - r0) * TW;
                            float gr = cur.gr;
                            float er = right_tile ? exp2_fast(cur.dr1 * A1) : 0.f;
                            bool right = right_tile;
#pragma unroll
                            for (int jj = TW - 1; jj >= 0; --jj) {
                                if (jj < je) {
                                    float g = cur.dy[jj] * cur.C[jj];
                                    if (below) g = fmaf(eb[jj], gb[jj], g);
                                    if (right) g = fmaf(er, gr, g);
                                    const float e0 = exp2_fast(cur.d0[jj] * A0), e1 = exp2_fast(cur.d1[jj] * A1);
                                    const float hp[2] = {r == r0 ? htop[jj] : up.h[jj], jj > 0 ? cur.h[jj - 1] : cur.hl};
                                    const bool has[2] = {r > 0, j0 + jj > 0};
                                    const float ea[2] = {e0, e1}, dl[2] = {cur.d0[jj], cur.d1[jj]};
                                    float dtb = dl[0];
                                    dtb += dl[1];
                                    dtb *= kInvNd;
                                    const float gbv = g * cur.B[jj];
                                    const float tx = channel_sum<MM>(gbv * dtb);
                                    const float tbv = gbv * cur.x[jj] * kInvNd;
                                    float td[2];
#pragma unroll
                                    for (int ax = 0; ax < 2; ++ax) {
                                        float t = tbv;
                                        if (has[ax]) {
                                            const float gh = g * ea[ax] * hp[ax];
                                            t = fmaf(gh, av[ax], tbv);
                                            dAacc[ax] = fmaf(gh, dl[ax], dAacc[ax]);
                                        }
                                        td[ax] = channel_sum<MM>(t);
                                    }
                                    F::st(rdC, voDM[jj], oDM, cur.dy[jj] * cur.h[jj]);
                                    F::st(rg, voDM[jj], oDM, g * dtb * cur.x[jj]);
                                    if (m == 0) {
                                        st[(slot0 + jj) * CPW + lc] = tx;
                                        st[(PTS + slot0 + jj) * CPW + lc] = td[0];
                                        st[(2 * PTS + slot0 + jj) * CPW + lc] = td[1];
                                    }
                                    if (jj == 0) F::st(rgC, c * 4, r * u.nt1 * sDM, g);
                                    gb[jj] = g;
                                    eb[jj] = e0;
                                    gr = g;
                                    er = e1;
                                    right = true;
                                }
                            }
                        }
                    }
                };
                for (int rt = r1 - 1; rt >= r0; rt -= 2 * RB) {
                    ld_batch(rt - RB, bb);
                    do_batch(rt, ba, bb);
                    if (rt - RB >= r0) {
                        ld_batch(rt - 2 * RB, ba);
                        do_batch(rt - RB, bb, ba);
                    }
                }
            } else {
                const float qn = __builtin_nanf("");
                for (int r = r0; r < r1; ++r)
                    for (int jj = 0; jj < je; ++jj) {
                        const int oDM = (rowq(r) + jj) * sDM;
                        F::st(rdC, c * 4, oDM, qn);
                        F::st(rg, c * 4, oDM, qn);
                        if (m == 0)
                            for (int k = 0; k < 3; ++k) st[(k * PTS + (r - r0) * TW + jj) * CPW + lc] = qn;
                        if (jj == 0) F::st(rgC, c * 4, r * u.nt1 * sDM, qn);
                    }
                dAacc[0] = dAacc[1] = qn;
                if (lane == 0) __hip_atomic_store(f.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __builtin_amdgcn_s_waitcnt(0);   // this wave's stores acknowledged by L2
            if (lane == 0)
                __hip_atomic_store(f.flags + fb * ncg + cg, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            const long dch = static_cast<long>(cgr) * 64 / MM;
            const GradWin fw = grad_window<2>(a, qb, qe, c, d, m, true);
            grad_flush<2, MM, PTS>(fw, st, dch, a.D, [&](int sl) -> long {
                const int rr = r0 + sl / TW, jj = sl % TW;
                return (rr < r1 && jj < je) ? static_cast<long>(rowq(rr) + jj) : -1L;
            });
        }
#pragma unroll
        for (int ax = 0; ax < 2; ++ax) a.part[(static_cast<long>(t1) * 2 + ax) * DM + c] = dAacc[ax];
    }
}

// The 3D backward fused, on pencils: an item is a pencil (a TR x TW column
// of axes 1 and 2 through every plane of axis 0, run of kFlowQ channel
// groups), taken in reverse band order of its (t1, t2). Each wave walks its
// group's pencil from the last plane to the first in sub-tiles of SUB planes
// (a completion flag after each), each plane's rows bottom-up and each row
// right to left, and at every point forms the adjoint state and every
// gradient (grad_finish's arithmetic, so dx, ddelta, dB, dC are bit for bit
// those of the two-pass path). The plane below's states and decays stay in
// registers, as does the current plane's h (the plane above's arrives with
// each row, as the axis-0 predecessor, and becomes the next plane's); only
// the pencil's first row and first column of every plane are stored, in gR
// / gC, for the pencils above and to the left (which wait on this pencil's
// flag for the same sub-tile). dx / ddelta go through the workgroup's LDS
// stage per sub-tile; dA to a partial per (pencil, group).
struct Fused3Args {
    float *gR;   // [n0][nt1][n2][D*M]: the states of each pencil's first row
    float *gC;   // [n0][n1][nt2][D*M]: of each pencil's first column
    int nt1, nt2, nsub;
};

template <int SUB, int TR, int TW, int MM>
__global__ void __launch_bounds__(64 * kFlowQ, 2) nd_fused3d(NdBwdArgs a, FlowArgs f, Fused3Args u) {
    constexpr int PTS = SUB * TR * TW;            // a sub-tile is one staged group
    static_assert(kStageOut<MM> && (256 / MM * PTS) % 256 == 0, "staged per-channel outputs");
    static_assert(TR % 2 == 0, "rows alternate between two prefetch slots");
    constexpr float kInvNd = 1.0f / 3;
    constexpr int CPW = 256 / MM;
    constexpr int SG = 4 * PTS * CPW;             // one stage buffer: dx, ddelta 0..2
    const int xcd = flow_xcd();
    const int cg0 = f.cg_lo[xcd], ncx = f.cg_lo[xcd + 1] - cg0;
    if (ncx <= 0) return;
    const int nq = ncx / kFlowQ;
    const int w = static_cast<int>(threadIdx.x / 64);
    const int lane = static_cast<int>(threadIdx.x & 63);
    const int npen = f.band_start[f.nbands];
    const unsigned nitems = static_cast<unsigned>(npen) * static_cast<unsigned>(nq);
    const unsigned epoch = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(f.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const int n0 = static_cast<int>(a.dims[0]), n1 = static_cast<int>(a.dims[1]), n2 = static_cast<int>(a.dims[2]);
    const int s0 = n1 * n2;
    const int DM = static_cast<int>(a.D) * MM;
    const int ncg = DM / 64;
    const int ntile[2] = {u.nt1, u.nt2};
    const int sD = static_cast<int>(a.D) * 4, sDM = DM * 4, sAx = static_cast<int>(a.P * a.D * 4);
    __shared__ unsigned s_item[2];
    __shared__ float stage[2 * SG];
    using F = bio<f32_t>;
    struct Row {
        float dy[TW], x[TW], d0[TW], d1[TW], d2[TW], C[TW], B[TW];
        float hu0[TW];              // h of the plane above (axis-0 predecessor; 0 on plane 0)
        float hu1[TW];              // h of the row above the pencil (first row only)
        float gbx[TW], dbx[TW];     // state and delta_1 of the row below the pencil (last row only)
        float hl, dr2, gr;          // h left of the pencil; delta_2 and state right of it
    };
    int sub_n = 0;                  // sub-tiles done (a stage buffer per sub-tile, alternating)
    for (int it = 0;; ++it) {
        if (threadIdx.x == 0) s_item[it & 1] = atomicAdd(&f.counter[xcd], 1u);
        __syncthreads();
        const unsigned item = __builtin_amdgcn_readfirstlane(s_item[it & 1]);
        if (item >= nitems) break;
        const int tb = npen - 1 - static_cast<int>(item / nq);      // reverse band order
        const int cgr = cg0 + static_cast<int>(item % nq) * kFlowQ;
        const int cg = cgr + w;
        const int band = flow_band(f, tb);
        int ti[2] = {0, 0};
        band_tile_n(2, ntile, band, tb - f.band_start[band], ti);
        const int pen = ti[0] * u.nt2 + ti[1];
        const int c = cg * 64 + lane;
        const int d = c / MM;
        const int m = c - d * MM;
        const int r0 = ti[0] * TR, r1 = min(n1, r0 + TR), re = r1 - r0;
        const int j0 = ti[1] * TW, j1 = min(n2, j0 + TW), je = j1 - j0;
        const bool below_tile = r1 < n1, right_tile = j1 < n2;
        const float Al[3] = {a.A[c] * kLog2e, a.A[DM + c] * kLog2e, a.A[2 * DM + c] * kLog2e};
        const float av[3] = {a.A[c], a.A[DM + c], a.A[2 * DM + c]};
        const int lc = static_cast<int>(threadIdx.x) / MM;
        int voD[TW], voDM[TW];
#pragma unroll
        for (int jj = 0; jj < TW; ++jj) {
            const int cc = min(jj, je - 1);
            voD[jj] = d * 4 + cc * sD;
            voDM[jj] = c * 4 + cc * sDM;
        }
        // Boundary buffers, based at the pencil: gR (pp, t1, j) at
        // pp * nt1 * n2 + (j - j0), the pencil below at + n2; gC (pp, r, t2)
        // at pp * n1 * nt2 + (r - r0) * nt2, the pencil to the right at + 1.
        const long grb = (static_cast<long>(ti[0]) * n2 + j0) * DM;
        const auto rgR = make_rsrc(u.gR + grb, (static_cast<long>(n0) * u.nt1 * n2 * DM - grb) * 4);
        const long gcb = (static_cast<long>(r0) * u.nt2 + ti[1]) * DM;
        const auto rgC = make_rsrc(u.gC + gcb, (static_cast<long>(n0) * n1 * u.nt2 * DM - gcb) * 4);
        float gp[TR][TW], ep[TR][TW], hcur[TR][TW];
#pragma unroll
        for (int ri = 0; ri < TR; ++ri)
#pragma unroll
            for (int jj = 0; jj < TW; ++jj) gp[ri][jj] = ep[ri][jj] = hcur[ri][jj] = 0.f;
        bool ok = true;
        float dAacc[3] = {0.f, 0.f, 0.f};   // over the pencil, in walk order
        for (int s = u.nsub - 1; s >= 0; --s, ++sub_n) {
            const int P0 = s * SUB, P1 = min(n0, P0 + SUB);
            // Windows: the plane above the sub-tile through its last plane.
            const int qb = max(P0 - 1, 0) * s0, qe = P1 * s0;
            const long nq_ = qe - qb;
            const auto rx = make_rsrc(a.x + static_cast<long>(qb) * a.D, nq_ * a.D * 4);
            const auto rdy = make_rsrc(a.dy + static_cast<long>(qb) * a.D, nq_ * a.D * 4);
            const auto rdl = make_rsrc(a.delta + static_cast<long>(qb) * a.D, (2 * a.P + nq_) * a.D * 4);
            const auto rg = make_rsrc(a.dB + static_cast<long>(qb) * DM, nq_ * DM * 4);
            const auto rB = make_rsrc(a.B + static_cast<long>(qb) * DM, nq_ * DM * 4);
            const auto rC = make_rsrc(a.C + static_cast<long>(qb) * DM, nq_ * DM * 4);
            const auto rh = make_rsrc(a.h + static_cast<long>(qb) * DM, nq_ * DM * 4);
            const auto rdC = make_rsrc(a.dC + static_cast<long>(qb) * DM, nq_ * DM * 4);
            auto pq = [&](int pp, int r) { return pp * s0 + r * n2 + j0 - qb; };   // point (pp, r, j0)
            auto ld_ops = [&](int pp, int r, Row &rw) __attribute__((always_inline)) {
                const int q = pq(pp, r), oD = q * sD, oDM = q * sDM;
#pragma unroll
                for (int jj = 0; jj < TW; ++jj) {
                    rw.dy[jj] = F::ld(rdy, voD[jj], oD);
                    rw.x[jj] = F::ld(rx, voD[jj], oD);
                    rw.d0[jj] = F::ld(rdl, voD[jj], oD);
                    rw.d1[jj] = F::ld(rdl, voD[jj], sAx + oD);
                    rw.d2[jj] = F::ld(rdl, voD[jj], 2 * sAx + oD);
                    rw.C[jj] = F::ld(rC, voDM[jj], oDM);
                    rw.B[jj] = F::ld(rB, voDM[jj], oDM);
                    rw.hu0[jj] = pp > 0 ? F::ld(rh, voDM[jj], oDM - s0 * sDM) : 0.f;
                    rw.hu1[jj] = (r == r0 && r0 > 0) ? F::ld(rh, voDM[jj], oDM - n2 * sDM) : 0.f;
                    rw.dbx[jj] = (r == r1 - 1 && below_tile) ? F::ld(rdl, voD[jj], sAx + oD + n2 * sD) : 0.f;
                }
                rw.hl = j0 > 0 ? F::ld(rh, c * 4, oDM - sDM) : 0.f;
                rw.dr2 = right_tile ? F::ld(rdl, d * 4, 2 * sAx + oD + je * sD) : 0.f;
            };
            // States other pencils wrote: the right neighbour, and (last row)
            // the row below.
            auto ld_succ = [&](int pp, int r, Row &rw) __attribute__((always_inline)) {
                rw.gr = right_tile
                            ? F::ld_agent(rgC, c * 4, ((pp * n1 + (r - r0)) * u.nt2 + 1) * sDM)
                            : 0.f;
#pragma unroll
                for (int jj = 0; jj < TW; ++jj)
                    rw.gbx[jj] = (r == r1 - 1 && below_tile)
                                     ? F::ld_agent(rgR, voDM[jj], (pp * u.nt1 * n2 + n2) * sDM)
                                     : 0.f;
            };
            float *st = stage + (sub_n & 1) * SG;
            // The first row's operands (and, on the pencil's first sub-tile,
            // its last plane's h) go out before the waits.
            Row R0, R1;
            ld_ops(P1 - 1, r0 + re - 1, R0);
            if (s == u.nsub - 1) {
#pragma unroll
                for (int ri = 0; ri < TR; ++ri)
#pragma unroll
                    for (int jj = 0; jj < TW; ++jj)
                        hcur[ri][jj] = F::ld(rh, voDM[jj], pq(P1 - 1, r0 + min(ri, re - 1)) * sDM);
            }
            if (ok) {
                const long fb = (static_cast<long>(s) * npen + pen);
                if (below_tile) ok = flow_wait(f.flags + (fb + u.nt2) * ncg + cg, epoch, f.spin) && ok;
                if (right_tile) ok = flow_wait(f.flags + (fb + 1) * ncg + cg, epoch, f.spin) && ok;
            }
            if (ok) {
                ld_succ(P1 - 1, r0 + re - 1, R0);
                float gb[TW], eb[TW];
#pragma unroll
                for (int jj = 0; jj < TW; ++jj) gb[jj] = eb[jj] = 0.f;
                // One row: (pp, r = r0 + ri) from cur; prefetch the next row
                // in walk order into nx.
                auto do_row = [&](int pp, int ri, const Row &cur) __attribute__((always_inline)) {
                    const int r = r0 + ri;
                    const int oD = pq(pp, r) * sD, oDM = pq(pp, r) * sDM;
                    (void)oD;
                    const bool below = r + 1 < n1, pbelow = pp + 1 < n0;
                    if (r == r1 - 1) {
#pragma unroll
                        for (int jj = 0; jj < TW; ++jj) {
                            gb[jj] = cur.gbx[jj];
                            eb[jj] = below_tile ? exp2_fast(cur.dbx[jj] * Al[1]) : 0.f;
                        }
                    }
                    float gr = cur.gr;
                    float er = right_tile ? exp2_fast(cur.dr2 * Al[2]) : 0.f;
                    bool right = right_tile;
                    const int slot0 = ((pp - P0) * TR + ri) * TW;
#pragma unroll
                    for (int jj = TW - 1; jj >= 0; --jj) {
                        if (jj < je) {
                            float g = cur.dy[jj] * cur.C[jj];
                            if (pbelow) g = fmaf(ep[ri][jj], gp[ri][jj], g);
                            if (below) g = fmaf(eb[jj], gb[jj], g);
                            if (right) g = fmaf(er, gr, g);
                            const float dl[3] = {cur.d0[jj], cur.d1[jj], cur.d2[jj]};
                            const float ea[3] = {exp2_fast(dl[0] * Al[0]), exp2_fast(dl[1] * Al[1]),
                                                 exp2_fast(dl[2] * Al[2])};
                            float hup1 = 0.f;
                            if constexpr (TR > 1) hup1 = ri > 0 ? hcur[ri > 0 ? ri - 1 : 0][jj] : cur.hu1[jj];
                            const float hp[3] = {cur.hu0[jj], r == r0 ? cur.hu1[jj] : hup1,
                                                 jj > 0 ? hcur[ri][jj > 0 ? jj - 1 : 0] : cur.hl};
                            const bool has[3] = {pp > 0, r > 0, j0 + jj > 0};
                            float dtb = dl[0];
                            dtb += dl[1];
                            dtb += dl[2];
                            dtb *= kInvNd;
                            const float gbv = g * cur.B[jj];
                            const float tx = channel_sum<MM>(gbv * dtb);
                            const float tbv = gbv * cur.x[jj] * kInvNd;
                            float td[3];
#pragma unroll
                            for (int ax = 0; ax < 3; ++ax) {
                                float t = tbv;
                                if (has[ax]) {
                                    const float gh = g * ea[ax] * hp[ax];
                                    t = fmaf(gh, av[ax], tbv);
                                    dAacc[ax] = fmaf(gh, dl[ax], dAacc[ax]);
                                }
                                td[ax] = channel_sum<MM>(t);
                            }
                            F::st(rdC, voDM[jj], oDM, cur.dy[jj] * hcur[ri][jj]);
                            F::st(rg, voDM[jj], oDM, g * dtb * cur.x[jj]);
                            if (m == 0) {
                                st[(slot0 + jj) * CPW + lc] = tx;
#pragma unroll
                                for (int ax = 0; ax < 3; ++ax) st[((ax + 1) * PTS + slot0 + jj) * CPW + lc] = td[ax];
                            }
                            if (r == r0) F::st(rgR, voDM[jj], pp * u.nt1 * n2 * sDM, g);
                            if (jj == 0) F::st(rgC, c * 4, (pp * n1 + ri) * u.nt2 * sDM, g);
                            gp[ri][jj] = g;
                            ep[ri][jj] = ea[0];
                            gb[jj] = g;
                            eb[jj] = ea[1];
                            gr = g;
                            er = ea[2];
                            right = true;
                        }
                    }
                    // The plane above's h is the next plane's own.
#pragma unroll
                    for (int jj = 0; jj < TW; ++jj) hcur[ri][jj] = cur.hu0[jj];
                };
                for (int pp = P1 - 1; pp >= P0; --pp) {
#pragma unroll
                    for (int ri = TR - 1; ri >= 0; ri -= 2) {
                        // Rows ri (in R0) and ri - 1 (in R1); the row after
                        // ri - 1 in walk order goes into R0.
                        const int rn = ri - 1;
                        ld_ops(pp, r0 + max(min(rn, re - 1), 0), R1);
                        ld_succ(pp, r0 + max(min(rn, re - 1), 0), R1);
                        __builtin_amdgcn_sched_barrier(0);
                        if (ri < re) do_row(pp, ri, R0);
                        const int pn = rn - 1 >= 0 ? pp : max(pp - 1, P0);
                        const int rnn = rn - 1 >= 0 ? rn - 1 : TR - 1;
                        ld_ops(pn, r0 + max(min(rnn, re - 1), 0), R0);
                        ld_succ(pn, r0 + max(min(rnn, re - 1), 0), R0);
                        __builtin_amdgcn_sched_barrier(0);
                        if (rn < re) do_row(pp, rn, R1);
                    }
                }
            } else {
                // A wait ran out (here or before): NaN into this sub-tile's
                // outputs, boundary states and stage slots.
                const float qn = __builtin_nanf("");
                for (int pp = P0; pp < P1; ++pp)
                    for (int ri = 0; ri < re; ++ri)
                        for (int jj = 0; jj < je; ++jj) {
                            const int oDM = (pq(pp, r0 + ri) + jj) * sDM;
                            F::st(rdC, c * 4, oDM, qn);
                            F::st(rg, c * 4, oDM, qn);
                            if (m == 0)
                                for (int k = 0; k < 4; ++k)
                                    st[(k * PTS + ((pp - P0) * TR + ri) * TW + jj) * CPW + lc] = qn;
                            if (ri == 0) F::st(rgR, c * 4, (pp * u.nt1 * n2 + jj) * sDM, qn);
                            if (jj == 0) F::st(rgC, c * 4, (pp * n1 + ri) * u.nt2 * sDM, qn);
                        }
                dAacc[0] = dAacc[1] = dAacc[2] = qn;
                if (lane == 0) __hip_atomic_store(f.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            const long pb = static_cast<long>(s) * npen + pen;
            __builtin_amdgcn_s_waitcnt(0);   // this wave's stores acknowledged by L2
            if (lane == 0)
                __hip_atomic_store(f.flags + pb * ncg + cg, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // dx / ddelta of the run's channels at the sub-tile's points.
            __syncthreads();
            const long dch = static_cast<long>(cgr) * 64 / MM;
            const GradWin fw = grad_window<3>(a, qb, qe, c, d, m, true);
            grad_flush<3, MM, PTS>(fw, st, dch, a.D, [&](int sl) -> long {
                const int pp = P0 + sl / (TR * TW), ri = (sl / TW) % TR, jj = sl % TW;
                return (pp < P1 && ri < re && jj < je) ? static_cast<long>(pq(pp, r0 + ri) + jj) : -1L;
            });
        }
#pragma unroll
        for (int ax = 0; ax < 3; ++ax) a.part[(static_cast<long>(pen) * 3 + ax) * DM + c] = dAacc[ax];
    }
}

// dA[k] = the nbx workgroup partials of k added in a fixed order: workgroup
// x takes outputs [64 x, +64), wave w the partials b = w, w + 4, ... in four
// interleaved running sums, then wave 0 adds the waves' sums in wave order.
// Workgroup row y takes the ch partials from y * ch on and writes row y of
// dA (a first pass over chunks of many partials; then one row, ch = nbx).
__global__ void __launch_bounds__(256) nd_adjoint_dA(const float *part, float *dA, long nbx, long n, long ch) {
    __shared__ float red[4][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const long y0 = static_cast<long>(blockIdx.y) * ch;
    part += y0 * n;
    dA += static_cast<long>(blockIdx.y) * n;
    nbx = std::min(ch, nbx - y0);
    const long k0 = static_cast<long>(blockIdx.x) * 64 + lane;
    const long k = k0 < n ? k0 : n - 1;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    long b = w;
    for (; b + 12 < nbx; b += 16) {
#pragma unroll
        for (int u = 0; u < 4; ++u) s[u] += part[(b + 4 * u) * n + k];
    }
    for (int u = 0; b < nbx; b += 4, ++u) s[u & 3] += part[b * n + k];
    red[w][lane] = (s[0] + s[1]) + (s[2] + s[3]);
    __syncthreads();
    if (w == 0 && k0 < n) dA[k0] = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
}

// dA from nbx partials [nbx][n]: above kDAChunk partials, chunks of
// kDAChunk are summed first (in parallel, into the ceil(nbx / kDAChunk) rows
// after the partials), then the chunks; each step in a fixed order.
constexpr long kDAChunk = 64;
static long dA_chunks(long nbx) { return nbx > 2 * kDAChunk ? (nbx + kDAChunk - 1) / kDAChunk : 0; }
static void sum_dA(float *part, float *dA, long nbx, long n, hipStream_t st) {
    const unsigned gx = static_cast<unsigned>((n + 63) / 64);
    const long nch = dA_chunks(nbx);
    if (nch > 0) {
        float *rows = part + nbx * n;
        hipLaunchKernelGGL(nd_adjoint_dA, dim3(gx, static_cast<unsigned>(nch)), dim3(256), 0, st, part, rows, nbx, n,
                           kDAChunk);
        hipLaunchKernelGGL(nd_adjoint_dA, dim3(gx), dim3(256), 0, st, rows, dA, nch, n, nch);
    } else {
        hipLaunchKernelGGL(nd_adjoint_dA, dim3(gx), dim3(256), 0, st, part, dA, nbx, n, nbx);
    }
}

constexpr int kGradTR2 = 8, kGradTW2 = 64;                  // 2D gradient tiles (rows, points)
constexpr int kGradTP3 = 4, kGradTR3 = 8, kGradTW3 = 8;     // 3D gradient tiles
constexpr int kGradTPW3 = 1;                                 // 3D tiles per workgroup (2 and 4 measured slower)

// The adjoint sweep's dataflow tiles per axis (0 past nd).
static void adj_flow_tiles(const KMScanNDBwd *a, int nd, int nt[3]) {
    nt[0] = nt[1] = nt[2] = 0;
    if (nd == 2) {
        nt[0] = static_cast<int>((a->dims[0] + kAdjFTR - 1) / kAdjFTR);
        nt[1] = static_cast<int>((a->dims[1] + kAdjFTW - 1) / kAdjFTW);
    } else if (nd == 3) {
        nt[0] = static_cast<int>((a->dims[0] + kAdj3P - 1) / kAdj3P);
        nt[1] = static_cast<int>((a->dims[1] + kAdj3R - 1) / kAdj3R);
        nt[2] = static_cast<int>((a->dims[2] + kAdj3W - 1) / kAdj3W);
    }
}

struct NdBwdShape {
    long P, nd, D, M;
    bool lanes;          // M a power of two <= 64: nd_adjoint_grads_lanes
    bool gtiles;         // ... and 2D or 3D: the tile walks
    bool atile2;         // 2D adjoint state by tile bands
    int db;
    long qc, nbx, nby;
    size_t offs_bytes, nbr_bytes, part_bytes, tile_bytes;
    size_t flow_bytes;   // the adjoint dataflow's counters, status, epoch and flags (tiled sweeps)
    bool fused2;         // 2D with staged per-channel outputs: the fused dataflow backward may run
    size_t gbd_bytes;    // the fused backward's boundary states (2D: gC; 3D: gR, gC)
    long fnt0, fnt1;     // its sub-tiles per pencil and pencils
    bool fused3;         // 3D: the fused pencil backward may run (boundary states in gbd_bytes)
    long f3nt1, f3nt2, f3nsub;   // its pencils per axis 1, 2 and sub-tiles per pencil
};

static bool nd_bwd_shape(const KMScanNDBwd *a, NdBwdShape &s) {
    if (!a || !a->dims || a->ndims < 1 || a->ndims > 8 || a->D <= 0 || a->M <= 0) {
        set_error("km_scannd_bwd: invalid ndims / D / M");
        return false;
    }
    if (!wavefront_nd_validate_dims(a->dims, a->ndims)) {
        set_error("km_scannd_bwd: invalid dims");
        return false;
    }
    // The per-channel path keeps ndims * M dA terms per thread in LDS.
    const bool pow2 = a->M <= 64 && (a->M & (a->M - 1)) == 0;
    if (!pow2 && a->ndims * a->M > kNdBwdMaxAcc) {
        set_error("km_scannd_bwd: ndims * M = %ld exceeds %d (M not a power of two <= 64)",
                  a->ndims * a->M, kNdBwdMaxAcc);
        return false;
    }
    s.P = wavefront_nd_total_points(a->dims, a->ndims);
    if (s.P <= 0) {
        set_error("km_scannd_bwd: empty grid");
        return false;
    }
    s.nd = a->ndims;
    s.D = a->D;
    s.M = a->M;
    s.lanes = s.M <= 64 && (s.M & (s.M - 1)) == 0;
    int db = 1;
    while (db < 256 && db < s.D) db *= 2;
    s.db = db;
    if (s.lanes) {
        s.nby = (s.D * s.M + 255) / 256;
        const long want = std::max<long>(1, 2048 / s.nby);    // ~2048 workgroups
        s.qc = std::max<long>(1, (s.P + want - 1) / want);
    } else {
        s.nby = (s.D + db - 1) / db;
        const long want = std::max<long>(1, 1024 / s.nby);    // ~1024 workgroups
        s.qc = std::max<long>(256 / db, (s.P + want - 1) / want);
    }
    s.nbx = (s.P + s.qc - 1) / s.qc;
    // 2D and 3D grids on the lanes path walk tiles (one workgroup column per
    // tile), carrying the predecessors' states in registers.
    s.gtiles = s.lanes && (s.nd == 2 || s.nd == 3);
    if (s.gtiles) {
        // Their buffer windows (a tile's planes / rows plus the one before,
        // and delta's axes before them) must stay below 2 GiB.
        const long lead = s.nd == 2 ? kGradTR2 + 1 : kGradTP3 + 1;
        long row = 1;
        for (long ax = 1; ax < s.nd; ++ax) row *= a->dims[ax];
        const long n = std::min<long>(s.P, lead * row);
        const double win = std::max(static_cast<double>(n) * s.D * s.M * 4,
                                    (static_cast<double>(s.nd - 1) * s.P + n) * s.D * 4);
        s.gtiles = win < 2147483000.0;
    }
    if (s.gtiles) {
        const long t2[2] = {kGradTR2, kGradTW2}, t3[3] = {kGradTP3, kGradTR3, kGradTW3};
        long nt = 1;
        for (long ax = 0; ax < s.nd; ++ax) {
            const long te = s.nd == 2 ? t2[ax] : t3[ax];
            nt *= (a->dims[ax] + te - 1) / te;
        }
        const long nb = s.nd == 2 ? nt : (nt + kGradTPW3 - 1) / kGradTPW3;
        // Tiles go on the grid's y dimension.
        if (nb <= 65535) s.nbx = nb;
        else s.gtiles = false;
    }
    s.offs_bytes = align_up(sizeof(long) * s.P, 256);
    s.nbr_bytes = align_up(sizeof(uint16_t) * s.P, 256);
    s.tile_bytes = 0;
    // The adjoint tile sweeps address a tile's rows (planes) and the
    // successor row (plane) through buffer windows below 2 GiB.
    auto adj_win_ok = [&](long lead_points) {
        const double n = static_cast<double>(std::min<long>(s.P, lead_points));
        return std::max(n * s.D * s.M * 4, (static_cast<double>(s.nd - 1) * s.P + n) * s.D * 4) < 2147483000.0;
    };
    s.atile2 = s.nd == 2 && (s.D * s.M) % 64 == 0 && adj_win_ok((kAdjTR + 1) * a->dims[1]);
    if (s.nd == 3 && (s.D * s.M) % 64 == 0 && adj_win_ok((kAdj3P + 1) * a->dims[1] * a->dims[2])) {
        long nt = 1;
        const long tdim[3] = {kAdj3P, kAdj3R, kAdj3W};
        for (int ax = 0; ax < 3; ++ax) nt *= (a->dims[ax] + tdim[ax] - 1) / tdim[ax];
        s.tile_bytes = align_up(sizeof(int) * 3 * nt, 256);
    }
    s.part_bytes = sizeof(float) * (s.nbx + dA_chunks(s.nbx)) * s.nd * s.D * s.M;
    // The fused 2D backward (nd_fused2p): per-channel outputs staged (4 <= M
    // <= 32), windows of a sub-tile's rows and of the boundary buffer below
    // 2 GiB. It writes the states of every pencil's first column and a dA
    // partial per pencil.
    s.fused2 = false;
    s.gbd_bytes = 0;
    s.fnt0 = s.fnt1 = 0;
    if (s.nd == 2 && s.lanes && s.M >= 4 && s.M <= 32 && (s.D * s.M) % 64 == 0 &&
        adj_win_ok((kAdjFTR + 2) * a->dims[1])) {
        const long DM = s.D * s.M;
        s.fnt0 = (a->dims[0] + kAdjFTR - 1) / kAdjFTR;
        s.fnt1 = (a->dims[1] + kAdjFTW - 1) / kAdjFTW;
        const double wc = static_cast<double>(a->dims[0]) * s.fnt1 * DM * 4;
        if (wc < 2147483000.0) {
            s.fused2 = true;
            s.gbd_bytes = align_up(sizeof(float) * a->dims[0] * s.fnt1 * DM, 256);
            const long nf = s.fnt1;
            s.part_bytes = std::max<size_t>(s.part_bytes, sizeof(float) * (nf + dA_chunks(nf)) * 2 * DM);
        }
    }
    // The fused 3D backward (nd_fused3d): pencils of kF3R x kF3W points
    // through every plane in sub-tiles of kF3S planes, 8 <= M <= 32 (its LDS
    // stage), D*M a multiple of 2048 (workgroups of four channel groups per
    // XCD), every window and boundary buffer below 2 GiB.
    s.fused3 = false;
    s.f3nt1 = s.f3nt2 = s.f3nsub = 0;
    if (s.nd == 3 && s.lanes && s.M >= 8 && s.M <= 32 && (s.D * s.M) % 2048 == 0) {
        const long DM = s.D * s.M, n0 = a->dims[0], n1 = a->dims[1], n2 = a->dims[2];
        const long nt1 = (n1 + kF3R - 1) / kF3R, nt2 = (n2 + kF3W - 1) / kF3W, nsub = (n0 + kF3S - 1) / kF3S;
        const double lim = 2147483000.0;
        const double win = static_cast<double>(kF3S + 1) * n1 * n2 * DM * 4;
        const double dwin = (2.0 * s.P + static_cast<double>(kF3S + 1) * n1 * n2) * s.D * 4;
        const double bR = static_cast<double>(n0) * nt1 * n2 * DM * 4, bC = static_cast<double>(n0) * n1 * nt2 * DM * 4;
        if (win < lim && dwin < lim && bR < lim && bC < lim && nt1 + nt2 - 1 <= kMaxFlowBands) {
            s.fused3 = true;
            s.f3nt1 = nt1;
            s.f3nt2 = nt2;
            s.f3nsub = nsub;
            s.gbd_bytes = std::max<size_t>(s.gbd_bytes, align_up(sizeof(float) * (n0 * nt1 * n2 + n0 * n1 * nt2) * DM, 256));
            const long nf = nt1 * nt2;
            s.part_bytes = std::max<size_t>(s.part_bytes, sizeof(float) * (nf + dA_chunks(nf)) * 3 * DM);
        }
    }
    s.flow_bytes = 0;
    if (s.atile2 || s.tile_bytes) {
        int nt[3];
        adj_flow_tiles(a, static_cast<int>(s.nd), nt);
        const long ntiles = static_cast<long>(nt[0]) * nt[1] * (s.nd == 3 ? nt[2] : 1);
        s.flow_bytes = align_up(4 * (kFlowHead + static_cast<size_t>(ntiles) * (s.D * s.M / 64)), 256);
    }
    if (s.fused3) {
        const size_t nfl = static_cast<size_t>(s.f3nsub * s.f3nt1 * s.f3nt2) * (s.D * s.M / 64);
        s.flow_bytes = std::max<size_t>(s.flow_bytes, align_up(4 * (kFlowHead + nfl), 256));
    }
    if (s.fused2) {   // 2D pencils: a flag per (sub-tile, pencil, channel group)
        const size_t nfl = static_cast<size_t>(s.fnt0 * s.fnt1) * (s.D * s.M / 64);
        s.flow_bytes = std::max<size_t>(s.flow_bytes, align_up(4 * (kFlowHead + nfl), 256));
    }
    return true;
}


// The tiled gradient pass for the M lanes of a channel (a power of two up
// to 64, a compile-time constant of the kernels' lane sums).
template <int ND, int MM>
static void grads_tile_go(const NdBwdArgs &args, const NdBwdShape &s, hipStream_t st) {
    // The channel blocks of a tile are consecutive workgroups: they read the
    // same points' rows (all of each row between them) at about the same
    // time, and with 8 (or 16) blocks, block k runs on XCD k % 8 for every
    // tile, next to the neighbouring tiles' states it reads.
    const dim3 grid(static_cast<unsigned>(s.nby), static_cast<unsigned>(s.nbx));
    if constexpr (ND == 2)
        hipLaunchKernelGGL((nd_adjoint_grads_tile2d<kGradTR2, kGradTW2, MM>), grid, dim3(256), 0, st, args);
    else
        hipLaunchKernelGGL((nd_adjoint_grads_tile3d<kGradTP3, kGradTR3, kGradTW3, kGradTPW3, MM>), grid, dim3(256),
                           0, st, args);
}
template <int ND>
static void grads_tile_launch(const NdBwdArgs &args, const NdBwdShape &s, hipStream_t st) {
    if constexpr (ND == 2 || ND == 3) {
        switch (s.M) {
        case 1: grads_tile_go<ND, 1>(args, s, st); break;
        case 2: grads_tile_go<ND, 2>(args, s, st); break;
        case 4: grads_tile_go<ND, 4>(args, s, st); break;
        case 8: grads_tile_go<ND, 8>(args, s, st); break;
        case 16: grads_tile_go<ND, 16>(args, s, st); break;
        case 32: grads_tile_go<ND, 32>(args, s, st); break;
        default: grads_tile_go<ND, 64>(args, s, st); break;
        }
    }
}

// Binds the adjoint sweep's dataflow state (band table, channel groups per
// XCD) when the tiled sweep applies, the device has 8 XCDs and the bands fit
// the kernel arguments: in the caller's workspace (ext, cleared here, so
// nothing is allocated) or in the stream's dataflow block. Returns 1 when
// bound, 0 for the band schedule, -1 on an error.
static int adj_flow_setup(const KMScanNDBwd *a, const NdBwdShape &s, hipStream_t st, FlowArgs &fa,
                          int nt[3], FlowBuf *ext) {
    const bool tiled = (s.nd == 2 && s.atile2) || (s.nd == 3 && s.tile_bytes);
    if (!tiled || !flow_wanted(s.nd)) return 0;
    adj_flow_tiles(a, static_cast<int>(s.nd), nt);
    const int nb = nt[0] + nt[1] + (s.nd == 3 ? nt[2] : 1) - (s.nd == 3 ? 2 : 1);
    const long ncg = s.D * s.M / 64;
    if (nb > kMaxFlowBands || nb <= 0) return 0;
    fa.nbands = nb;
    for (int x = 0; x <= 8; ++x) fa.cg_lo[x] = static_cast<int>(static_cast<long>(x) * ncg / 8);
    fa.band_start[0] = 0;
    for (int b = 0; b < nb; ++b) {
        long c = 0;
        if (s.nd == 2) {
            const int lo = std::max(0, b - (nt[1] - 1)), hi = std::min(b, nt[0] - 1);
            c = hi >= lo ? hi - lo + 1 : 0;
        } else {
            for (int t0 = 0; t0 < nt[0] && t0 <= b; ++t0) {
                const int r = b - t0, lo = std::max(0, r - (nt[2] - 1)), hi = std::min(r, nt[1] - 1);
                c += hi >= lo ? hi - lo + 1 : 0;
            }
        }
        fa.band_start[b + 1] = fa.band_start[b] + static_cast<int>(c);
    }
    const long ntiles = fa.band_start[nb];
    if (ntiles * ncg >= 0x7fffffffL) return 0;
    if (ext) flow_zero(ext->buf, ext->cap, st);
    int kind = 0;
    const int bound = flow_bind(st, static_cast<size_t>(ntiles * ncg), ext, fa, &kind);
    note_flow(st, kind, kind == 2 ? fa.counter : nullptr);
    return bound;
}

// The fused 3D backward's dataflow state: bands of the (nt1, nt2) pencil
// grid, a flag per (sub-tile, pencil, channel group). Returns as
// flow_bind (1 bound, 0 not available, -1 error).
static int fused3_flow_setup(const NdBwdShape &s, hipStream_t st, FlowArgs &fa, FlowBuf *ext) {
    const int n1 = static_cast<int>(s.f3nt1), n2 = static_cast<int>(s.f3nt2);
    const long ncg = s.D * s.M / 64;
    const int nb = n1 + n2 - 1;
    fa.nbands = nb;
    for (int x = 0; x <= 8; ++x) fa.cg_lo[x] = static_cast<int>(static_cast<long>(x) * ncg / 8);
    if (flow_q(fa) != kFlowQ) return 0;
    fa.band_start[0] = 0;
    for (int b = 0; b < nb; ++b) {
        const int lo = std::max(0, b - (n2 - 1)), hi = std::min(b, n1 - 1);
        fa.band_start[b + 1] = fa.band_start[b] + (hi >= lo ? hi - lo + 1 : 0);
    }
    const long nfl = s.f3nsub * s.f3nt1 * s.f3nt2 * ncg;
    if (nfl >= 0x7fffffffL) return 0;
    if (ext) flow_zero(ext->buf, ext->cap, st);
    int kind = 0;
    const int bound = flow_bind(st, static_cast<size_t>(nfl), ext, fa, &kind);
    note_flow(st, kind, kind == 2 ? fa.counter : nullptr);
    return bound;
}

// The fused 2D pencils' dataflow state: pencils are taken right to left
// (the kernel derives a pencil from its item), a flag per (sub-tile, pencil,
// channel group).
static int fused2p_flow_setup(const NdBwdShape &s, hipStream_t st, FlowArgs &fa, FlowBuf *ext) {
    const long ncg = s.D * s.M / 64;
    fa.nbands = 1;
    for (int x = 0; x <= 8; ++x) fa.cg_lo[x] = static_cast<int>(static_cast<long>(x) * ncg / 8);
    if (flow_q(fa) != kFlowQ) return 0;
    fa.band_start[0] = 0;
    fa.band_start[1] = static_cast<int>(s.fnt1);
    const long nfl = s.fnt0 * s.fnt1 * ncg;
    if (nfl >= 0x7fffffffL) return 0;
    if (ext) flow_zero(ext->buf, ext->cap, st);
    int kind = 0;
    const int bound = flow_bind(st, static_cast<size_t>(nfl), ext, fa, &kind);
    note_flow(st, kind, kind == 2 ? fa.counter : nullptr);
    return bound;
}

template <int ND>
static void nd_bwd_launch(const NdBwdArgs &args, const NdBwdShape &s, const KMWavefrontPlan *plan,
                          float *dA, const int *dtiles, const std::vector<long> &bstart, hipStream_t st,
                          const FlowArgs *flow, const int *nt) {
    const long DM = s.D * s.M;
    const unsigned bx = static_cast<unsigned>((DM + 255) / 256);
    if ((ND == 2 || ND == 3) && flow) {
        // One dataflow launch: 8k workgroups of Q waves (k <= 256 / Q, two
        // waves per SIMD), k = the largest per-XCD item count.
        const int q = flow_q(*flow);
        const long ntiles = flow->band_start[flow->nbands];
        long per_xcd = 0;
        for (int x = 0; x < 8; ++x)
            per_xcd = std::max<long>(per_xcd, ntiles * ((flow->cg_lo[x + 1] - flow->cg_lo[x]) / q));
        const long grid = 8 * std::min<long>(per_xcd, 256 / q);
        if (grid > 0)
            hipLaunchKernelGGL((nd_adjoint_flow<ND == 2 ? 2 : 3>), dim3(static_cast<unsigned>(grid)),
                               dim3(64 * q), 0, st, args, *flow, nt[0], nt[1], nt[2],
                               static_cast<int>(DM / 64));
    } else if (ND == 3 && s.tile_bytes) {
        const int ncg = static_cast<int>(DM / 64);
        for (long b = static_cast<long>(bstart.size()) - 2; b >= 0; --b) {
            const long n = bstart[b + 1] - bstart[b];
            if (n > 0)
                hipLaunchKernelGGL((nd_adjoint_tile3d<kAdj3P, kAdj3R, kAdj3W>),
                                   dim3(static_cast<unsigned>(n * ncg)), dim3(64), 0, st, args,
                                   dtiles + 3 * bstart[b], ncg);
        }
    } else if (ND == 2 && s.atile2) {
        const int nt0 = static_cast<int>((args.dims[0] + kAdjTR - 1) / kAdjTR);
        const int nt1 = static_cast<int>((args.dims[1] + kAdjTW - 1) / kAdjTW);
        const int ncg = static_cast<int>(DM / 64);
        for (int band = nt0 + nt1 - 2; band >= 0; --band) {
            const int lo = band > nt1 - 1 ? band - (nt1 - 1) : 0;
            const int hi = band < nt0 - 1 ? band : nt0 - 1;
            const long tiles = hi - lo + 1;
            hipLaunchKernelGGL((nd_adjoint_tile2d<kAdjTR, kAdjTW, kAdjRB>),
                               dim3(static_cast<unsigned>(tiles * ncg)), dim3(64), 0, st, args, band, nt1, ncg);
        }
    } else {
    for (long lvl = plan->max_level; lvl >= 0; --lvl) {
        // Levels of more than 65535 points go in several launches.
        for (long s0 = plan->level_starts[lvl]; s0 < plan->level_starts[lvl + 1]; s0 += 65535) {
            const long n = std::min<long>(65535, plan->level_starts[lvl + 1] - s0);
            hipLaunchKernelGGL(nd_adjoint_level<ND>, dim3(bx, static_cast<unsigned>(n)), dim3(256), 0, st,
                               args, s0);
        }
    }
    }
    if (s.gtiles && (ND == 2 || ND == 3)) {
        grads_tile_launch<ND>(args, s, st);
    } else if (s.lanes) {
        hipLaunchKernelGGL(nd_adjoint_grads_lanes<ND>,
                           dim3(static_cast<unsigned>(s.nbx), static_cast<unsigned>(s.nby)), dim3(256), 0, st,
                           args, s.qc);
    } else {
        const size_t lds = sizeof(float) * ND * s.M * 256;
        hipLaunchKernelGGL(nd_adjoint_grads<ND>,
                           dim3(static_cast<unsigned>(s.nbx), static_cast<unsigned>(s.nby)), dim3(256), lds, st,
                           args, s.qc, s.db);
    }
    sum_dA(args.part, dA, s.nbx, s.nd * DM, st);
}

}  // namespace km

extern "C" {

size_t km_scannd_bwd_workspace_bytes(const KMScanNDBwd *a) {
    km::clear_error();
    km::NdBwdShape s;
    if (!km::nd_bwd_shape(a, s)) return 0;
    return s.offs_bytes + s.nbr_bytes + s.part_bytes + s.tile_bytes + s.flow_bytes + s.gbd_bytes;
}

int km_scannd_bwd(const KMScanNDBwd *a, void *stream) {
    km::clear_error();
    km::NdBwdShape s;
    if (!km::nd_bwd_shape(a, s)) return -1;
    if (!a->x || !a->A || !a->B || !a->C || !a->delta || !a->h || !a->dy || !a->dx || !a->ddelta ||
        !a->dA || !a->dB || !a->dC) {
        km::set_error("km_scannd_bwd: NULL tensor pointer");
        return -1;
    }
    if (s.nbx > 0x7fffffffL || s.nby > 65535 || s.nd * s.D * s.M > 0x7fffffffL * 256L) {
        km::set_error("km_scannd_bwd: grid out of range");
        return -1;
    }
    if (!km::gpu_ready()) return -1;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t need = s.offs_bytes + s.nbr_bytes + s.part_bytes + s.tile_bytes + s.flow_bytes + s.gbd_bytes;
    char *ws = static_cast<char *>(a->workspace);
    if (ws) {
        if (a->workspace_bytes < need) {
            km::set_error("km_scannd_bwd: workspace of %zu bytes, %zu needed", a->workspace_bytes, need);
            return -1;
        }
    } else {
        ws = static_cast<char *>(km::Workspace::reserve(need, st, km::WsUse::ScanNDBwd));
        if (!ws) return -1;
    }
    // The per-level path reads the plan's level offsets; the tile-band paths
    // (2D and 3D with D*M a multiple of 64) need no plan.
    const bool tiles2d = s.atile2;
    const bool levels = !tiles2d && !s.tile_bytes;
    KMWavefrontPlan *plan = nullptr;
    if (levels && !(plan = km_wavefront_plan_create(a->dims, a->ndims))) {
        km::set_error("km_scannd_bwd: wavefront plan could not be built");
        return -1;
    }
    km::NdBwdArgs args{};
    args.x = a->x; args.A = a->A; args.B = a->B; args.C = a->C; args.delta = a->delta;
    args.h = a->h; args.dy = a->dy; args.dx = a->dx; args.ddelta = a->ddelta; args.dB = a->dB;
    args.dC = a->dC;
    args.offs = reinterpret_cast<const long *>(ws);
    args.nbr = reinterpret_cast<const uint16_t *>(ws + s.offs_bytes);
    args.part = reinterpret_cast<float *>(ws + s.offs_bytes + s.nbr_bytes);
    args.P = s.P; args.D = s.D; args.M = s.M;
    long stride = 1;
    for (long ax = s.nd - 1; ax >= 0; --ax) {
        args.dims[ax] = a->dims[ax];
        args.strides[ax] = stride;
        stride *= a->dims[ax];
    }
    // The adjoint sweep on the dataflow schedule where it applies (no tile
    // list to upload), else by tile bands.
    static thread_local km::FlowArgs fa;
    int nt[3] = {0, 0, 0};
    // 2D on the dataflow schedule: the fused backward on pencils
    // (KM_SCANND_BWD_FUSED=0: the adjoint sweep, then the gradient pass).
    {
        const char *fe = std::getenv("KM_SCANND_BWD_FUSED");
        if (s.fused2 && km::flow_wanted(2) && !(fe && std::strcmp(fe, "0") == 0)) {
            km::FlowBuf wf{reinterpret_cast<unsigned *>(ws + s.offs_bytes + s.nbr_bytes + s.part_bytes + s.tile_bytes),
                           s.flow_bytes / 4, 8};
            const int fbp = km::fused2p_flow_setup(s, st, fa, (a->workspace && s.flow_bytes) ? &wf : nullptr);
            if (fbp < 0) return -1;
            if (fbp > 0) {
                float *gbd = reinterpret_cast<float *>(ws + s.offs_bytes + s.nbr_bytes + s.part_bytes + s.tile_bytes +
                                                       s.flow_bytes);
                const long DM = s.D * s.M;
                km::Fused2PArgs u{gbd, static_cast<int>(s.fnt1), static_cast<int>(s.fnt0)};
                long per_xcd = 0;
                for (int x = 0; x < 8; ++x)
                    per_xcd = std::max<long>(per_xcd, s.fnt1 * ((fa.cg_lo[x + 1] - fa.cg_lo[x]) / km::kFlowQ));
                const dim3 grid(static_cast<unsigned>(8 * std::min<long>(per_xcd, 256 / km::kFlowQ)));
                const dim3 blk(64 * km::kFlowQ);
                switch (s.M) {
                case 4: hipLaunchKernelGGL((km::nd_fused2p<km::kAdjFTR, km::kAdjFTW, 2, 4>), grid, blk, 0, st, args, fa, u); break;
                case 8: hipLaunchKernelGGL((km::nd_fused2p<km::kAdjFTR, km::kAdjFTW, 2, 8>), grid, blk, 0, st, args, fa, u); break;
                case 16: hipLaunchKernelGGL((km::nd_fused2p<km::kAdjFTR, km::kAdjFTW, 2, 16>), grid, blk, 0, st, args, fa, u); break;
                default: hipLaunchKernelGGL((km::nd_fused2p<km::kAdjFTR, km::kAdjFTW, 2, 32>), grid, blk, 0, st, args, fa, u); break;
                }
                km::sum_dA(args.part, a->dA, s.fnt1, 2 * DM, st);
                if (plan) km_wavefront_plan_free(plan);
                const hipError_t e = hipGetLastError();
                if (e != hipSuccess) {
                    km::set_error("km_scannd_bwd: launch failed: %s", hipGetErrorString(e));
                    return -1;
                }
                return 0;
            }
        }
    }
    // 3D on the dataflow schedule: the fused pencil backward (adjoint state
    // and gradients in one launch; KM_SCANND_BWD_FUSED=0: two passes).
    const char *fe3 = std::getenv("KM_SCANND_BWD_FUSED");
    if (s.fused3 && km::flow_wanted(3) && !(fe3 && std::strcmp(fe3, "0") == 0)) {
        km::FlowBuf wf{reinterpret_cast<unsigned *>(ws + s.offs_bytes + s.nbr_bytes + s.part_bytes + s.tile_bytes),
                       s.flow_bytes / 4, 8};
        const int fb3 = km::fused3_flow_setup(s, st, fa, (a->workspace && s.flow_bytes) ? &wf : nullptr);
        if (fb3 < 0) return -1;
        if (fb3 > 0) {
            float *gbd = reinterpret_cast<float *>(ws + s.offs_bytes + s.nbr_bytes + s.part_bytes + s.tile_bytes +
                                                   s.flow_bytes);
            const long DM = s.D * s.M;
            km::Fused3Args u{gbd, gbd + a->dims[0] * s.f3nt1 * a->dims[2] * DM, static_cast<int>(s.f3nt1),
                             static_cast<int>(s.f3nt2), static_cast<int>(s.f3nsub)};
            const long npen = s.f3nt1 * s.f3nt2;
            long per_xcd = 0;
            for (int x = 0; x < 8; ++x)
                per_xcd = std::max<long>(per_xcd, npen * ((fa.cg_lo[x + 1] - fa.cg_lo[x]) / km::kFlowQ));
            const dim3 grid(static_cast<unsigned>(8 * std::min<long>(per_xcd, 256 / km::kFlowQ)));
            const dim3 blk(64 * km::kFlowQ);
            switch (s.M) {
            case 8: hipLaunchKernelGGL((km::nd_fused3d<km::kF3S, km::kF3R, km::kF3W, 8>), grid, blk, 0, st, args, fa, u); break;
            case 16: hipLaunchKernelGGL((km::nd_fused3d<km::kF3S, km::kF3R, km::kF3W, 16>), grid, blk, 0, st, args, fa, u); break;
            default: hipLaunchKernelGGL((km::nd_fused3d<km::kF3S, km::kF3R, km::kF3W, 32>), grid, blk, 0, st, args, fa, u); break;
            }
            km::sum_dA(args.part, a->dA, npen, 3 * DM, st);
            if (plan) km_wavefront_plan_free(plan);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) {
                km::set_error("km_scannd_bwd: launch failed: %s", hipGetErrorString(e));
                return -1;
            }
            return 0;
        }
    }
    // With the caller's workspace the flags live in it (cleared per call);
    // otherwise in the stream's dataflow block.
    km::FlowBuf wflow{reinterpret_cast<unsigned *>(ws + s.offs_bytes + s.nbr_bytes + s.part_bytes + s.tile_bytes),
                      s.flow_bytes / 4, 8};
    const int fb = km::adj_flow_setup(a, s, st, fa, nt, (a->workspace && s.flow_bytes) ? &wflow : nullptr);
    if (fb < 0) {
        if (plan) km_wavefront_plan_free(plan);
        return -1;
    }
    if (fb == 0) km::note_flow(st, 0);
    const km::FlowArgs *flow = fb > 0 ? &fa : nullptr;

    // 3D tile bands: each band's tiles (tile-index sum b), bands contiguous.
    std::vector<int> tl;
    std::vector<long> bstart;
    if (s.tile_bytes && !flow) {
        const long nt0 = (a->dims[0] + km::kAdj3P - 1) / km::kAdj3P;
        const long nt1 = (a->dims[1] + km::kAdj3R - 1) / km::kAdj3R;
        const long nt2 = (a->dims[2] + km::kAdj3W - 1) / km::kAdj3W;
        for (long b = 0; b <= nt0 + nt1 + nt2 - 3; ++b) {
            bstart.push_back(static_cast<long>(tl.size() / 3));
            for (long t0 = 0; t0 < nt0; ++t0)
                for (long t1 = 0; t1 < nt1; ++t1) {
                    const long t2 = b - t0 - t1;
                    if (t2 >= 0 && t2 < nt2) {
                        tl.push_back(static_cast<int>(t0));
                        tl.push_back(static_cast<int>(t1));
                        tl.push_back(static_cast<int>(t2));
                    }
                }
        }
        bstart.push_back(static_cast<long>(tl.size() / 3));
    }
    char *tile_ws = ws + s.offs_bytes + s.nbr_bytes + s.part_bytes;
    int rc = 0;
    hipLaunchKernelGGL(km::nd_adjoint_flags, dim3(static_cast<unsigned>((s.P + 255) / 256)), dim3(256), 0, st,
                       args, s.nd, reinterpret_cast<uint16_t *>(ws + s.offs_bytes));
    // The host tables must outlive their copies: wait for them.
    if ((plan && hipMemcpyAsync(ws, plan->level_offsets, sizeof(long) * s.P, hipMemcpyHostToDevice, st) !=
                     hipSuccess) ||
        (!tl.empty() && hipMemcpyAsync(tile_ws, tl.data(), sizeof(int) * tl.size(), hipMemcpyHostToDevice,
                                       st) != hipSuccess) ||
        ((plan || !tl.empty()) && hipStreamSynchronize(st) != hipSuccess)) {
        km::set_error("km_scannd_bwd: plan upload failed");
        rc = -1;
    } else {
        const int *dtiles = reinterpret_cast<const int *>(tile_ws);
        switch (s.nd) {
        case 1: km::nd_bwd_launch<1>(args, s, plan, a->dA, dtiles, bstart, st, flow, nt); break;
        case 2: km::nd_bwd_launch<2>(args, s, plan, a->dA, dtiles, bstart, st, flow, nt); break;
        case 3: km::nd_bwd_launch<3>(args, s, plan, a->dA, dtiles, bstart, st, flow, nt); break;
        case 4: km::nd_bwd_launch<4>(args, s, plan, a->dA, dtiles, bstart, st, flow, nt); break;
        case 5: km::nd_bwd_launch<5>(args, s, plan, a->dA, dtiles, bstart, st, flow, nt); break;
        case 6: km::nd_bwd_launch<6>(args, s, plan, a->dA, dtiles, bstart, st, flow, nt); break;
        case 7: km::nd_bwd_launch<7>(args, s, plan, a->dA, dtiles, bstart, st, flow, nt); break;
        default: km::nd_bwd_launch<8>(args, s, plan, a->dA, dtiles, bstart, st, flow, nt); break;
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) {
            km::set_error("km_scannd_bwd: launch failed: %s", hipGetErrorString(e));
            rc = -1;
        }
    }
    if (plan) km_wavefront_plan_free(plan);
    return rc;
}

}  // extern "C"

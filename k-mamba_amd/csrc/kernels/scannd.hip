// scannd.hip - ScanND / Scan2D selective-scan forward for gfx950.
//
// Recurrence (reference src/scan_nd.c:95-192, lambda == NULL branch):
//   dt_bar(p,d) = (sum_axis delta(axis,p,d)) / ndims
//   h(p,d,m)    = dt_bar * (B(p,d,m) * x(p,d))
//               + sum_axis[idx_axis > 0] exp(delta(axis,p,d) * A(axis,d,m)) * h(p - e_axis, d, m)
//   y(p,d)      = sum_m C(p,d,m) * h(p,d,m)
// Scan2D (cpu/scan2d.asm:66-275) is the ndims = 2 case with separate A/delta
// pointers per axis; it differs from scannd_ref only in the association of
// the same products and sums.
//
// Layout and schedule (instead of one launch per wavefront level):
//  * lanes: 64 consecutive flattened (d, m) pairs, so B, C and h rows are
//    256-byte coalesced accesses and y is a reduction over the M lanes of a
//    channel;
//  * the grid is cut into tiles; tiles with equal tile-index sum (a tile
//    band) are independent. 2D grids run one launch per tile band (47 for a
//    256x256 grid with 16x8 tiles instead of 511 per-level launches); the
//    kernel boundary publishes every tile's h to the next band. Grids of 3
//    or more dims run one dataflow launch per step, in which a tile waits
//    only for its own axis predecessors (completion flags, each channel
//    group kept on one XCD so producer and consumer share an L2);
//  * one wave per (tile, channel group) walks its tile row by row (rows
//    along the last axis), keeping the row above in registers and taking
//    the left neighbour from the previous column; neighbours across the
//    tile's boundary and along leading axes are read back from h.
#include <cstdlib>
#include <mutex>
#include <cstring>

#include <cstdio>

#include "km_device.hpp"
#include "scannd_flow.hpp"
#include "../km_runtime.hpp"
#include "kmamba_km.h"
#include "scan.h"
#include "scan_nd.h"
#include "mamba_scan.h"
#include "mamba_scan_cuda.h"

namespace km {

int scan1d_fwd_launch(const KMScan1DFwd *k, hipStream_t stream, bool allow_split);

constexpr int kMaxNd = 8;

struct ScanNDArgs {
    const float *x;
    const float *A[kMaxNd];      // per axis [D, M]
    const float *dt[kMaxNd];     // per axis [P, D]
    const float *B, *C;
    float *h, *y;
    int nd;
    int dims[kMaxNd];
    long pstride[kMaxNd];        // row-major point strides
    int tile[kMaxNd];            // tile extent per axis
    int ntile[kMaxNd];           // tiles per axis
    int band;                    // tile band (sum of tile indices)
    int sub;                     // pencil tiles (3D dataflow): planes per flag along axis 0
    int D, M, DM;
    int ncg;                     // channel groups of 64 (d, m) lanes
};

// Tile band b, ordinal o of the grid's tiles (band_tile_n).
__device__ inline bool band_tile(const ScanNDArgs &p, int band, int ordinal, int *ti) {
    return band_tile_n(p.nd, p.ntile, band, ordinal, ti);
}

// Sum over the M consecutive lanes of a channel (M a power of two <= 64);
// every lane of the group receives the sum. Within a 16-lane row the steps
// are DPP VALU ops (no LDS round trip).
template <int MM>
__device__ __forceinline__ float sum_m_lanes(float v) {
    if constexpr (MM == 2) {
        v += dpp<0xB1>(v);                       // quad_perm [1,0,3,2]
    } else if constexpr (MM == 4) {
        v += dpp<0x4E>(v);                       // quad_perm [2,3,0,1]
        v += dpp<0xB1>(v);
    } else if constexpr (MM == 8) {
        v += dpp<0x141>(v);                      // row_half_mirror
        v += dpp<0x4E>(v);
        v += dpp<0xB1>(v);
    } else if constexpr (MM >= 16) {
        v += dpp<0x128>(v);                      // row_ror:8
        v += dpp<0x124>(v);                      // row_ror:4
        v += dpp<0x122>(v);                      // row_ror:2
        v += dpp<0x121>(v);                      // row_ror:1
        if constexpr (MM >= 32) v = sum_xor16(v);
        if constexpr (MM >= 64) v = sum_xor32(v);
    }
    return v;
}

// One wave per (tile, channel group). The wave walks its tile row by row
// (rows along axis ND-2, leading axes outermost), each row along the last
// axis, prefetching the next row's operands while the current row computes.
// The row above is kept in registers; leading-axis neighbours and the tile's
// top/left boundary are read from h (written earlier by this wave or by a
// previous band's launch).
template <int ND, int TW>
struct NDRow {
    float x[TW], b[TW], c[TW], dt[ND][TW], hn[ND - 1][TW];
    float hleft;
    int gi[ND];
    int base;                   // row offset from the B / C / h origin, in points
    int xbase;                  // row offset from the x / delta / y origin
};

// PL > 0 (3D, tiles of PL rows along axis 1): the wave also keeps the
// previous plane's PL rows in registers, so only the tile's first plane reads
// its axis-0 neighbours from h. COH: states written by other workgroups of
// the same launch (the dataflow schedule) are read with agent-coherent loads
// that bypass the CU's L1.
//
// wait(0) runs once the operands of the tile's first rows (which no other
// tile writes) are in flight and before any state written by another tile
// is read; when it returns false nothing is computed and the function
// returns 0, else 1.
//
// PEN (3D ring tiles spanning all of axis 0, the dataflow schedule): the
// tile is a pencil of sub-tiles of p.sub planes. Before sub-tile s the wave
// runs wait(s) (its axis-1 / axis-2 neighbours), after it publish(s); the
// axis-0 neighbour of every plane is the ring, so no axis-0 state is read
// back from h. B, C and h are addressed from the sub-tile's origin (their
// resources move with it, keeping offsets 32-bit), x, delta and y from the
// pencil's. Returns the number of sub-tiles computed and published.
template <int ND, int TW, int MM, int PL, bool COH = false, bool PEN = false, typename Wait,
          typename Publish>
__device__ __forceinline__ int scannd_tile(const ScanNDArgs &p, const int (&ti)[kMaxNd], int cg,
                                           Wait &&wait, Publish &&publish) {
    constexpr bool RING = (ND == 3 && PL > 0);
    static_assert(!PEN || RING, "pencils are 3D ring tiles");
    static_assert(PL % 2 == 0, "planes of whole row pairs");
    const int lane = threadIdx.x & 63;

    constexpr int ar = ND - 2, ac = ND - 1;       // row / column axes
    const int f = cg * 64 + lane;                 // flattened (d, m)
    const int d = f / MM;
    const int DM = p.DM;
    const int D = p.D;
    const bool y_lane = (lane % MM) == 0;

    float Ap[ND];
#pragma unroll
    for (int a = 0; a < ND; ++a) Ap[a] = p.A[a][f] * kLog2e;

    int lo[ND], ext[ND];
#pragma unroll
    for (int a = 0; a < ND; ++a) {
        lo[a] = ti[a] * p.tile[a];
        ext[a] = min(p.tile[a], p.dims[a] - lo[a]);
    }
    const int TC = ext[ac];
    int nrows = 1;
#pragma unroll
    for (int a = 0; a < ac; ++a) nrows *= ext[a];

    // Addressing: buffer resources based at the tile origin (h one axis-0
    // stride earlier, for the neighbours before the tile), so every offset
    // below is a small non-negative 32-bit value. A point's lane offset
    // within its row is fixed per tile (voffX / voffB, VGPRs); a row adds one
    // scalar offset per array. Columns past the tile's edge repeat the last
    // column's offsets and are never computed or stored.
    long origin = lo[ac];
#pragma unroll
    for (int a = 0; a < ac; ++a) origin += static_cast<long>(lo[a]) * p.pstride[a];
    const long P = static_cast<long>(p.dims[0]) * p.pstride[0];
    auto win = [](long bytes) { return bytes < 0x7fffffffL ? bytes : 0x7fffffffL; };
    const auto rx = make_rsrc(p.x + origin * D, win((P - origin) * D * 4));
    __amdgpu_buffer_rsrc_t rdt[ND];
#pragma unroll
    for (int a = 0; a < ND; ++a) rdt[a] = make_rsrc(p.dt[a] + origin * D, win((P - origin) * D * 4));
    const auto ry = make_rsrc(p.y + origin * D, win((P - origin) * D * 4));
    // B / C / h from the origin of the (sub-)tile starting `plane` planes
    // into the tile; h one axis-0 stride earlier (or from the array's
    // start), for the neighbours before it. rh / hback serve the neighbour
    // loads, rh_st / hback_st the state stores: a pencil moves the loads'
    // resources to the next sub-tile while its last row still computes.
    __amdgpu_buffer_rsrc_t rB, rC, rh, rh_st;
    long hback = 0, hback_st = 0;
    auto rebase_ops = [&](int plane) {
        const long o = origin + static_cast<long>(plane) * p.pstride[0];
        rB = make_rsrc(p.B + o * DM, win((P - o) * DM * 4));
        rC = make_rsrc(p.C + o * DM, win((P - o) * DM * 4));
    };
    auto rebase_h = [&](int plane) {
        const long o = origin + static_cast<long>(plane) * p.pstride[0];
        hback = min(o, p.pstride[0]);
        rh = make_rsrc(p.h + (o - hback) * DM, win((P - o + hback) * DM * 4));
        rh_st = rh;
        hback_st = hback;
    };
    rebase_ops(0);
    rebase_h(0);
    int voffX[TW], voffB[TW];
#pragma unroll
    for (int c = 0; c < TW; ++c) {
        const int cc = (c < TC) ? c : TC - 1;
        voffX[c] = (cc * D + d) * 4;
        voffB[c] = (cc * DM + f) * 4;
    }
    using F = bio<f32_t>;
    // Neighbour states: L1-bypassing loads when other workgroups of this
    // launch may have written them.
    auto hld = [](__amdgpu_buffer_rsrc_t r, int voff, int soff) {
        return COH ? F::ld_agent(r, voff, soff) : F::ld(r, voff, soff);
    };

    // Operands of one row (tile-relative row offset in points: r.base).
    // The operand loads are unconditional; only the neighbour-state loads
    // sit under wave-uniform branches (measured: skipping the unneeded ones
    // is 5 % faster in 3D than loading B again in their place).
    // plane0: planes between the x origin and the B origin (pencils).
    auto load_ops = [&](int row, NDRow<ND, TW> &r, int plane0 = 0) {
        int rem = row;
        int roff = 0;
#pragma unroll
        for (int a = ac - 1; a >= 0; --a) {
            const int ia = rem % ext[a];
            rem /= ext[a];
            r.gi[a] = lo[a] + ia;
            roff += ia * static_cast<int>(p.pstride[a]);
        }
        r.gi[ac] = lo[ac];
        r.base = roff;
        r.xbase = roff;
        if constexpr (PEN) {
            r.gi[0] += plane0;
            r.xbase += plane0 * static_cast<int>(p.pstride[0]);
        }
        const int sx = r.xbase * D * 4, sb = roff * DM * 4;
#pragma unroll
        for (int c = 0; c < TW; ++c) {
            r.x[c] = F::ld(rx, voffX[c], sx);
            r.b[c] = F::ld(rB, voffB[c], sb);
            r.c[c] = F::ld(rC, voffB[c], sb);
#pragma unroll
            for (int a = 0; a < ND; ++a) r.dt[a][c] = F::ld(rdt[a], voffX[c], sx);
        }
    };
    auto load_nbr = [&](NDRow<ND, TW> &r) {
        // Neighbours along leading axes, and along the row axis on the tile's
        // first row of a plane (tile boundary). An unneeded neighbour is not
        // loaded (0; compute_row skips its term). Rows are prefetched one
        // row ahead, so a leading-axis
        // neighbour inside the tile must lie at least two rows back: the
        // launcher never builds a tile with a single row per plane below an
        // in-tile leading axis. In 2D the only such neighbour is the row above
        // the tile, which the wave loads into `top` before its first row.
        const int sh = (r.base + static_cast<int>(hback)) * DM * 4;
#pragma unroll
        for (int a = 0; a < (ND == 2 ? 0 : ND - 1); ++a) {
            // Wave-uniform (readfirstlane): a scalar branch around the loads.
            const bool need = __builtin_amdgcn_readfirstlane(
                                  (a < ar && !(RING && a == 0)) ? (r.gi[a] > 0) : (r.gi[a] > 0 && r.gi[a] == lo[a])) != 0;
            const int sn = sh - static_cast<int>(p.pstride[a]) * DM * 4;
#pragma unroll
            for (int c = 0; c < TW; ++c) r.hn[a][c] = need ? hld(rh, voffB[c], sn) : 0.f;
        }
        const bool left = __builtin_amdgcn_readfirstlane(lo[ac] > 0) != 0;
        r.hleft = left ? hld(rh, voffB[0], sh - DM * 4) : 0.f;
    };
    auto load_row = [&](int row, NDRow<ND, TW> &r, int plane0 = 0) {
        load_ops(row, r, plane0);
        load_nbr(r);
    };

    float top[TW];
#pragma unroll
    for (int c = 0; c < TW; ++c) top[c] = 0.f;
    // 2D: the row above the tile (from an earlier band), or 0 on the grid's
    // first row; h at the tile origin minus one row is the start of rh's
    // window whenever that row exists.
    auto load_top = [&]() {
        if constexpr (ND == 2) {
            const bool up = __builtin_amdgcn_readfirstlane(lo[0] > 0) != 0;
#pragma unroll
            for (int c = 0; c < TW; ++c) top[c] = up ? hld(rh, voffB[c], 0) : 0.f;
        }
    };
    // dt_bar = sum / ndims: 1/ndims is exact for ndims 2 and 4; for 3 the
    // product differs from the reference's division by at most one ulp.
    const float inv_nd = 1.0f / static_cast<float>(ND);

    // Stores of columns past the tile's edge (c >= TC, computed on repeated
    // operands) and of lanes that own no output go to an offset with bit 31
    // set, past the window, and are dropped: no branch around any store.
    constexpr unsigned kDrop = 0x80000000u;
    int hoff[TW];
#pragma unroll
    for (int c = 0; c < TW; ++c) hoff[c] = static_cast<int>(c < TC ? static_cast<unsigned>(voffB[c]) : kDrop);
    // M = 16 and TW | 16: the row's TW readouts are reduce-scattered over
    // the 16 state lanes of a channel, leaving lane l with column
    // (l % 16) / (16 / TW), and stored with one instruction per row.
    constexpr bool kRowY = (MM == 16) && (16 % TW == 0);
    constexpr int YG = kRowY ? 16 / TW : 1;
    int yoff = 0;
    if constexpr (kRowY) {
        const int yc = (lane % 16) / YG;
        yoff = static_cast<int>((lane % YG == 0 && yc < TC) ? static_cast<unsigned>((yc * D + d) * 4) : kDrop);
    }

    // ring0 / from_ring: the axis-0 neighbour row kept in registers (PL > 0,
    // rows past the tile's first plane) instead of r.hn[0].
    auto compute_row = [&](const NDRow<ND, TW> &r, bool live, const float (&ring0)[TW], bool from_ring) {
        const bool first_row_of_plane = (r.gi[ar] == lo[ar]);
        const int sh = (r.base + static_cast<int>(hback_st)) * DM * 4;
        const int sx = r.xbase * D * 4;
        float hleft = r.hleft;
        float yr[TW];
#pragma unroll
        for (int c = 0; c < TW; ++c) {
            float dsum = 0.f;
#pragma unroll
            for (int a = 0; a < ND; ++a) dsum += r.dt[a][c];
            float acc = (dsum * inv_nd) * (r.b[c] * r.x[c]);
#pragma unroll
            for (int a = 0; a < ar; ++a) {
                const float hn = (RING && a == 0 && from_ring) ? ring0[c] : r.hn[a][c];
                if (r.gi[a] > 0) acc = fmaf(exp2_fast(r.dt[a][c] * Ap[a]), hn, acc);
            }
            if (r.gi[ar] > 0) {
                float hu = top[c];
                if constexpr (ND > 2) hu = first_row_of_plane ? r.hn[ar][c] : top[c];
                acc = fmaf(exp2_fast(r.dt[ar][c] * Ap[ar]), hu, acc);
            }
            if (lo[ac] + c > 0) acc = fmaf(exp2_fast(r.dt[ac][c] * Ap[ac]), hleft, acc);
            F::st(rh_st, live ? hoff[c] : static_cast<int>(kDrop), sh, acc);
            top[c] = acc;
            hleft = acc;
            if constexpr (kRowY) {
                yr[c] = r.c[c] * acc;
            } else {
                const float yv = sum_m_lanes<MM>(r.c[c] * acc);
                F::st(ry, static_cast<int>(live && y_lane && c < TC ? static_cast<unsigned>(voffX[c]) : kDrop),
                      sx, yv);
            }
        }
        if constexpr (kRowY) F::st(ry, live ? yoff : static_cast<int>(kDrop), sx, row_readout<TW>(yr));
    };

    // Rows are prefetched ahead and processed in groups with no branch in
    // the loop: past the last row the last row is reloaded (in bounds) and
    // computed with its stores dropped. The scheduling barriers keep a row's
    // prefetch ahead of the previous row's arithmetic, so a row's first wait
    // covers only older loads. 2D tiles hold one wave per SIMD in a band, so
    // their rows are prefetched two ahead through a ring of four; deeper
    // tiles have more waves per SIMD and prefetch one ahead.
    float none[TW];
#pragma unroll
    for (int c = 0; c < TW; ++c) none[c] = 0.f;
    if constexpr (ND == 2) {
        NDRow<ND, TW> R0, R1, R2, R3;
        load_ops(0, R0);
        load_ops(min(1, nrows - 1), R1);
        if (!wait(0)) return 0;
        load_top();
        load_nbr(R0);
        load_nbr(R1);
        for (int row = 0; row < nrows; row += 4) {
            load_row(min(row + 2, nrows - 1), R2);
            __builtin_amdgcn_sched_barrier(0);
            compute_row(R0, true, none, false);
            load_row(min(row + 3, nrows - 1), R3);
            __builtin_amdgcn_sched_barrier(0);
            compute_row(R1, row + 1 < nrows, none, false);
            load_row(min(row + 4, nrows - 1), R0);
            __builtin_amdgcn_sched_barrier(0);
            compute_row(R2, row + 2 < nrows, none, false);
            load_row(min(row + 5, nrows - 1), R1);
            __builtin_amdgcn_sched_barrier(0);
            compute_row(R3, row + 3 < nrows, none, false);
        }
    } else if constexpr (PEN) {
        // The ring branch below over sub-tiles of p.sub planes. The first
        // row of sub-tile s + 1 is prefetched (operands only, from its own
        // origin) during the last row of sub-tile s; its neighbour loads
        // wait for wait(s + 1). Past the pencil's last plane the last row
        // of the last sub-tile is reloaded and nothing more is computed.
        const int e0 = ext[0], e1 = ext[1], SUB = p.sub;
        const int nsub = (e0 + SUB - 1) / SUB;
        auto row_in = [&](int i0l, int i1) { return i0l * e1 + min(i1, e1 - 1); };
        float ring[PL][TW];
#pragma unroll
        for (int i = 0; i < PL; ++i)
#pragma unroll
            for (int c = 0; c < TW; ++c) ring[i][c] = 0.f;
        NDRow<ND, TW> R0, R1;
        load_ops(row_in(0, 0), R0, 0);
        if (!wait(0)) return 0;
        load_nbr(R0);
        for (int s = 0; s < nsub; ++s) {
            const int p0 = s * SUB, np = min(SUB, e0 - p0);
            const bool more = s + 1 < nsub;
            for (int i0l = 0; i0l < np; ++i0l) {
                const bool inner = p0 + i0l > 0;
                const bool last_plane = i0l + 1 == np;
#pragma unroll
                for (int i1 = 0; i1 < PL; i1 += 2) {
                    load_row(row_in(i0l, i1 + 1), R1, p0);
                    __builtin_amdgcn_sched_barrier(0);
                    compute_row(R0, i1 < e1, ring[i1], inner);
#pragma unroll
                    for (int c = 0; c < TW; ++c) ring[i1][c] = top[c];
                    if (i1 + 2 < PL) {
                        load_row(row_in(i0l, i1 + 2), R0, p0);
                    } else if (!last_plane) {
                        load_row(row_in(i0l + 1, 0), R0, p0);
                    } else if (more) {
                        rebase_ops(p0 + SUB);
                        load_ops(row_in(0, 0), R0, p0 + SUB);
                    } else {
                        load_ops(row_in(i0l, 0), R0, p0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    compute_row(R1, i1 + 1 < e1, ring[i1 + 1], inner);
#pragma unroll
                    for (int c = 0; c < TW; ++c) ring[i1 + 1][c] = top[c];
                }
            }
            publish(s);
            if (!more) break;
            rebase_h(p0 + SUB);
            if (!wait(s + 1)) return s + 1;
            load_nbr(R0);
        }
        return nsub;
    } else if constexpr (RING) {
        // Planes of PL rows (i1 = 0..PL-1; rows past ext[1] are recomputed
        // on the last row's operands with their stores dropped), row pairs
        // prefetched one row ahead. ring[i1] holds h of row (i0 - 1, i1).
        const int e0 = ext[0], e1 = ext[1];
        auto row_at = [&](int i0, int i1) { return min(i0, e0 - 1) * e1 + min(i1, e1 - 1); };
        float ring[PL][TW];
#pragma unroll
        for (int i = 0; i < PL; ++i)
#pragma unroll
            for (int c = 0; c < TW; ++c) ring[i][c] = 0.f;
        NDRow<ND, TW> R0, R1;
        load_ops(0, R0);
        if (!wait(0)) return 0;
        load_nbr(R0);
        for (int i0 = 0; i0 < e0; ++i0) {
            const bool inner = i0 > 0;
#pragma unroll
            for (int i1 = 0; i1 < PL; i1 += 2) {
                load_row(row_at(i0, i1 + 1), R1);
                __builtin_amdgcn_sched_barrier(0);
                compute_row(R0, i1 < e1, ring[i1], inner);
#pragma unroll
                for (int c = 0; c < TW; ++c) ring[i1][c] = top[c];
                load_row(i1 + 2 < PL ? row_at(i0, i1 + 2) : row_at(i0 + 1, 0), R0);
                __builtin_amdgcn_sched_barrier(0);
                compute_row(R1, i1 + 1 < e1, ring[i1 + 1], inner);
#pragma unroll
                for (int c = 0; c < TW; ++c) ring[i1 + 1][c] = top[c];
            }
        }
    } else {
        NDRow<ND, TW> R0, R1;
        load_ops(0, R0);
        if (!wait(0)) return 0;
        load_nbr(R0);
        for (int row = 0; row < nrows; row += 2) {
            load_row(min(row + 1, nrows - 1), R1);
            __builtin_amdgcn_sched_barrier(0);
            compute_row(R0, true, none, false);
            load_row(min(row + 2, nrows - 1), R0);
            __builtin_amdgcn_sched_barrier(0);
            compute_row(R1, row + 1 < nrows, none, false);
        }
    }
    return 1;
}

// One launch per tile band: workgroup = (tile of band p.band, channel group).
// Workgroups are dealt to the 8 XCDs round-robin; they are renumbered so
// that consecutive channel groups of a tile, which share x / delta cache
// lines (4 channels = 16 bytes of a row each), run on one XCD's L2.
template <int ND, int TW, int MM, int PL>
__global__ void __launch_bounds__(64) scannd_tile_kernel(ScanNDArgs p) {
    const int nb = gridDim.x, q = nb / 8, r = nb % 8, xcd = blockIdx.x % 8;
    const int lb = xcd * q + min(xcd, r) + static_cast<int>(blockIdx.x / 8);
    const int cg = lb % p.ncg;
    const int ordinal = lb / p.ncg;
    int ti[kMaxNd];
    if (!band_tile(p, p.band, ordinal, ti)) return;
    scannd_tile<ND, TW, MM, PL>(p, ti, cg, [](int) { return true; }, [](int) {});
}

// Dataflow schedule (scannd_flow.hpp), one launch per step: a tile waits
// only for its own axis predecessors. A wait that runs out writes NaN into
// the tile's states and outputs and sets the launch's status word, which the
// synchronous entry points read to re-run the call on the band schedule.
// NaN into the states and outputs of one (tile, channel group): the wave's
// 64 (channel, state) lanes at every point of the tile, or of its planes
// [plane_lo, plane_hi) along axis 0 when plane_hi > 0.
template <int ND>
__device__ void scannd_tile_poison(const ScanNDArgs &p, const int (&ti)[kMaxNd], int cg,
                                   int plane_lo = 0, int plane_hi = 0) {
    const int lane = threadIdx.x & 63;
    const int f = cg * 64 + lane;
    const int MM = p.M;
    const int d = f / MM;
    const float qnan = __builtin_nanf("");
    int lo[ND], ext[ND];
    long npts = 1;
#pragma unroll
    for (int a = 0; a < ND; ++a) {
        lo[a] = ti[a] * p.tile[a];
        ext[a] = min(p.tile[a], p.dims[a] - lo[a]);
    }
    if (plane_hi > 0) {
        lo[0] += plane_lo;
        ext[0] = min(plane_hi, ext[0]) - plane_lo;
    }
#pragma unroll
    for (int a = 0; a < ND; ++a) npts *= ext[a];
    for (long q = 0; q < npts; ++q) {
        long rem = q, off = 0;
#pragma unroll
        for (int a = ND - 1; a >= 0; --a) {
            const long ia = rem % ext[a];
            rem /= ext[a];
            off += (lo[a] + ia) * p.pstride[a];
        }
        p.h[off * p.DM + f] = qnan;
        if (lane % MM == 0) p.y[off * p.D + d] = qnan;
    }
}

// Workgroups of Q waves (flow_q): an item is (tile, run of Q consecutive
// channel groups of the XCD), one group per wave, so no wave idles. The
// waves of a workgroup share a CU, start an item together and read the
// same x / delta lines (the groups of four consecutive channels are 16
// bytes apart), so those lines come from the CU's L1 or one L2 fill
// instead of up to Q fills spread over the time the groups' waves happen
// to run.
//
// PEN: an item is a pencil (3D tiles spanning all of axis 0) whose
// sub-tiles of p.sub planes carry the flags: flag (s, t1, t2) after
// sub-tile s, waits on sub-tile s of the axis-1 and axis-2 neighbours. A
// pencil only waits on pencils of earlier bands, taken before it.
template <int ND, int TW, int MM, int PL, bool PEN>
__device__ __forceinline__ void scannd_flow_body(const ScanNDArgs &p, const FlowArgs &f) {
    const int xcd = flow_xcd();
    const int cg0 = f.cg_lo[xcd], ncx = f.cg_lo[xcd + 1] - cg0;
    if (ncx <= 0) return;
    const int Q = static_cast<int>(blockDim.x / 64);
    const int nq = ncx / Q;                             // runs of groups per tile
    const int w = static_cast<int>(threadIdx.x / 64);
    const int ntiles = f.band_start[f.nbands];
    const unsigned nitems = static_cast<unsigned>(ntiles) * static_cast<unsigned>(nq);
    // The epoch lives in device memory (flow_reset advances it), so a
    // launch replayed from a captured graph gets a new one each time.
    const unsigned epoch = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(f.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    int tstride[kMaxNd];                 // row-major tile index strides
    tstride[ND - 1] = 1;
#pragma unroll
    for (int a = ND - 2; a >= 0; --a) tstride[a] = tstride[a + 1] * p.ntile[a + 1];
    __shared__ unsigned s_item[2];
    for (int it = 0;; ++it) {
        // One fetch per workgroup, handed to every wave through LDS; the
        // two slots alternate, and the barrier ending the previous item
        // keeps a slot from being rewritten while a wave still reads it.
        if (threadIdx.x == 0) s_item[it & 1] = atomicAdd(&f.counter[xcd], 1u);
        __syncthreads();
        const unsigned item = __builtin_amdgcn_readfirstlane(s_item[it & 1]);
        if (item >= nitems) break;
        const int tb = static_cast<int>(item / nq);
        const int cg = cg0 + static_cast<int>(item % nq) * Q + w;
        const int band = flow_band(f, tb);
        int ti[kMaxNd];
        band_tile(p, band, tb - f.band_start[band], ti);
        if constexpr (PEN) {
            // Flags of sub-tile s: row-major over (s, t1, t2).
            auto flag_of = [&](int sub, int t1, int t2) {
                return f.flags + ((static_cast<long>(sub) * p.ntile[1] + t1) * p.ntile[2] + t2) * p.ncg + cg;
            };
            auto wait_sub = [&](int sub) {
                bool ready = true;
                if (ti[1] > 0) ready = flow_wait(flag_of(sub, ti[1] - 1, ti[2]), epoch, f.spin) && ready;
                if (ti[2] > 0) ready = flow_wait(flag_of(sub, ti[1], ti[2] - 1), epoch, f.spin) && ready;
                return ready;
            };
            auto publish_sub = [&](int sub) {
                __builtin_amdgcn_s_waitcnt(0);   // this wave's h stores acknowledged by L2
                if ((threadIdx.x & 63) == 0)
                    __hip_atomic_store(flag_of(sub, ti[1], ti[2]), epoch, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            };
            const int nsub = (p.dims[0] + p.sub - 1) / p.sub;
            const int done = scannd_tile<ND, TW, MM, PL, true, true>(p, ti, cg, wait_sub, publish_sub);
            if (done < nsub) {
                scannd_tile_poison<ND>(p, ti, cg, done * p.sub, p.dims[0]);
                if ((threadIdx.x & 63) == 0)
                    __hip_atomic_store(f.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                for (int sub = done; sub < nsub; ++sub) publish_sub(sub);
            }
            continue;
        }
        int tl = 0;
#pragma unroll
        for (int a = 0; a < ND; ++a) tl += ti[a] * tstride[a];
        // The tile's first operand loads are issued before the waits on its
        // upstream neighbours, so their latency overlaps the wait.
        auto upstream_done = [&](int) {
            bool ready = true;
#pragma unroll
            for (int a = 0; a < ND; ++a)
                if (ti[a] > 0)
                    ready = flow_wait(f.flags + static_cast<long>(tl - tstride[a]) * p.ncg + cg, epoch,
                                      f.spin) && ready;
            return ready;
        };
        if (!scannd_tile<ND, TW, MM, PL, true>(p, ti, cg, upstream_done, [](int) {})) {
            scannd_tile_poison<ND>(p, ti, cg);
            if ((threadIdx.x & 63) == 0)
                __hip_atomic_store(f.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0);   // this wave's h stores acknowledged by L2
        if ((threadIdx.x & 63) == 0)
            __hip_atomic_store(f.flags + static_cast<long>(tl) * p.ncg + cg, epoch, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int ND, int TW, int MM, int PL>
__global__ void __launch_bounds__(64 * kFlowQ, 2) scannd_flow_kernel(ScanNDArgs p, FlowArgs f) {
    scannd_flow_body<ND, TW, MM, PL, false>(p, f);
}

// Pencils: the 3D launch runs one wave per SIMD (its grid cap), so the
// kernel may hold up to 512 VGPRs.
template <int TW, int MM>
__global__ void __launch_bounds__(64 * kFlowQ, 1) scannd_pencil_kernel(ScanNDArgs p, FlowArgs f) {
    scannd_flow_body<3, TW, MM, 4, true>(p, f);
}

// Before each dataflow launch: zeroes the item counters and the status
// word and advances the epoch. When the epoch wraps, every one of the
// nflags flags is cleared first, so no flag holds the new epoch. One
// workgroup of 256 threads.
__global__ void __launch_bounds__(256) flow_reset(unsigned *head, long nflags) {
    __shared__ unsigned s_next;
    if (threadIdx.x == 0) s_next = head[kFlowEpoch] + 1u;
    __syncthreads();
    const unsigned next = s_next;
    if (next == 0u)
        for (long i = threadIdx.x; i < nflags; i += 256) head[kFlowHead + i] = 0u;
    if (threadIdx.x < 8) head[threadIdx.x] = 0u;
    if (threadIdx.x == kFlowStatus) head[kFlowStatus] = 0u;
    if (threadIdx.x == kFlowEpoch) head[kFlowEpoch] = next == 0u ? 1u : next;
}

// General fallback (any D, M): one launch per wavefront level of the point
// grid, one thread per (point, channel), reading the level's offsets from
// the device copy of the plan.
__global__ void __launch_bounds__(256) scannd_level_kernel(ScanNDArgs p, const long *offsets,
                                                           long start, long count) {
    const long gid = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= count * p.D) return;
    const long off = offsets[start + gid / p.D];
    const int d = static_cast<int>(gid % p.D);
    int idx[kMaxNd];
    {
        long rem = off;
        for (int a = p.nd - 1; a >= 0; --a) {
            idx[a] = static_cast<int>(rem % p.dims[a]);
            rem /= p.dims[a];
        }
    }
    float dsum = 0.f;
    for (int a = 0; a < p.nd; ++a) dsum += p.dt[a][off * p.D + d];
    const float dtb = dsum / static_cast<float>(p.nd);
    const float xv = p.x[off * p.D + d];
    float y = 0.f;
    for (int m = 0; m < p.M; ++m) {
        const long q = off * p.DM + static_cast<long>(d) * p.M + m;
        float acc = dtb * (p.B[q] * xv);
        for (int a = 0; a < p.nd; ++a) {
            if (idx[a] > 0) {
                const float e = exp2_fast(p.dt[a][off * p.D + d] * p.A[a][d * p.M + m] * kLog2e);
                acc = fmaf(e, p.h[q - p.pstride[a] * p.DM], acc);
            }
        }
        p.h[q] = acc;
        y = fmaf(p.C[q], acc, y);
    }
    p.y[off * p.D + d] = y;
}

// Mamba-3 branch (lambda != NULL) of the reference scannd_ref_with_plan
// (src/scan_nd.c:59-210), per wavefront level, one thread per (point,
// channel pair): the pair's states at every m, the readouts y, and the
// pair's rotated states R(theta) h, which the point's successors read (the
// state itself when theta is NULL; an odd last channel is never rotated).
// The reference keeps the rotated states in a [D, M] buffer indexed with
// point offsets (out of bounds, and unread-before-write when theta is NULL);
// hrot here is the [P, D, M] buffer that indexing implies. Per (d, m):
//   bu = B x;  over the axes with a predecessor: sum of B[prev] x[prev] and
//   of alpha_a = exp(delta_a min(A_a, -1e-5));  their averages bpa, aavg;
//   h = bpa * ((1 - lambda) dt_bar aavg) + bu * (lambda dt_bar)
//       + sum_a alpha_a hrot[prev_a]
struct ScanM3Args {
    const float *x, *B, *C, *theta, *lambda;
    const float *A[kMaxNd];      // per axis [D, M]
    const float *dt[kMaxNd];     // per axis [P, D]
    float *h, *y, *hrot;
    int nd;
    int dims[kMaxNd];
    long pstride[kMaxNd];
    int D, M;
    long DM;
};

__global__ void __launch_bounds__(256) scannd_m3_level_kernel(ScanM3Args p, const long *offsets,
                                                              long start, long count) {
    const int npair = (p.D + 1) / 2;
    const long gid = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= count * npair) return;
    const long off = offsets[start + gid / npair];
    const int d0 = 2 * static_cast<int>(gid % npair);
    const int nc = (d0 + 1 < p.D) ? 2 : 1;       // channels of this pair
    int idx[kMaxNd];
    {
        long rem = off;
        for (int a = p.nd - 1; a >= 0; --a) {
            idx[a] = static_cast<int>(rem % p.dims[a]);
            rem /= p.dims[a];
        }
    }
    const float lam = p.lambda[off];
    float dtb[2], xv[2], yacc[2] = {0.f, 0.f};
    for (int c = 0; c < nc; ++c) {
        float dsum = 0.f;
        for (int a = 0; a < p.nd; ++a) dsum += p.dt[a][off * p.D + d0 + c];
        dtb[c] = dsum / static_cast<float>(p.nd);
        xv[c] = p.x[off * p.D + d0 + c];
    }
    float cs = 1.f, sn = 0.f;
    const bool rot = p.theta && nc == 2;
    if (rot) {
        const float th = p.theta[d0 >> 1];
        cs = cosf(th);
        sn = sinf(th);
    }
    for (int m = 0; m < p.M; ++m) {
        float hv[2] = {0.f, 0.f};
        for (int c = 0; c < nc; ++c) {
            const long dm = static_cast<long>(d0 + c) * p.M + m;
            const long q = off * p.DM + dm;
            const float bu = p.B[q] * xv[c];
            float bpa = 0.f, aacc = 0.f, hs = 0.f;
            int npred = 0;
            for (int a = 0; a < p.nd; ++a) {
                if (idx[a] > 0) {
                    const long prev = off - p.pstride[a];
                    const float ar = p.A[a][dm];
                    const float av = (ar > -1e-5f) ? -1e-5f : ar;   // the branch's clamp (:129)
                    const float al = exp2_fast(p.dt[a][off * p.D + d0 + c] * av * kLog2e);
                    bpa += p.B[prev * p.DM + dm] * p.x[prev * p.D + d0 + c];
                    aacc += al;
                    hs = fmaf(al, p.hrot[prev * p.DM + dm], hs);
                    ++npred;
                }
            }
            float hn = bu * (lam * dtb[c]);
            if (npred > 0) {
                const float inv = 1.f / static_cast<float>(npred);
                hn = fmaf(bpa * inv, (1.f - lam) * dtb[c] * (aacc * inv), hn) + hs;
            }
            p.h[q] = hn;
            yacc[c] = fmaf(p.C[q], hn, yacc[c]);
            hv[c] = hn;
        }
        const long q0 = off * p.DM + static_cast<long>(d0) * p.M + m;
        if (rot) {
            p.hrot[q0] = cs * hv[0] - sn * hv[1];
            p.hrot[q0 + p.M] = sn * hv[0] + cs * hv[1];
        } else {
            for (int c = 0; c < nc; ++c) p.hrot[q0 + c * p.M] = hv[c];
        }
    }
    for (int c = 0; c < nc; ++c) p.y[off * p.D + d0 + c] = yacc[c];
}

// Tuning knob (read once): KM_SCANND_T2 / KM_SCANND_T3 = "TW,TL" sets the
// 2D / 3D tile to TW points along the last axis (4, 8 or 16 in 2D; 4 or 8 in
// 3D) and TL along each leading axis.
static void scannd_tile_shape(int nd, int &tw, int &tl) {
    static int t2w = 0, t2l = 0, t3w = 0, t3l = 0;
    static bool once = [] {
        auto parse = [](const char *e, int &w, int &l) {
            if (e && std::sscanf(e, "%d,%d", &w, &l) != 2) w = l = 0;
        };
        parse(std::getenv("KM_SCANND_T2"), t2w, t2l);
        parse(std::getenv("KM_SCANND_T3"), t3w, t3l);
        return true;
    }();
    (void)once;
    if (nd == 2 && (t2w == 4 || t2w == 8 || t2w == 16) && t2l > 0 && t2l <= 64) { tw = t2w; tl = t2l; }
    if (nd == 3 && (t3w == 4 || t3w == 8) && t3l > 0 && t3l <= 64) { tw = t3w; tl = t3l; }
}

template <int ND, int TW, int MM, int PL>
static void launch_tile_pl(dim3 g, const ScanNDArgs &a, const FlowArgs *flow, hipStream_t s) {
    const dim3 blk(64 * (flow ? flow_q(*flow) : 1));
    if constexpr (ND == 3 && PL > 0) {
        if (flow && a.sub > 0) {
            static_assert(PL == 4, "pencils are ring tiles of 4 rows");
            hipLaunchKernelGGL((scannd_pencil_kernel<TW, MM>), g, blk, 0, s, a, *flow);
            return;
        }
    }
    if (flow) hipLaunchKernelGGL((scannd_flow_kernel<ND, TW, MM, PL>), g, blk, 0, s, a, *flow);
    else      hipLaunchKernelGGL((scannd_tile_kernel<ND, TW, MM, PL>), g, blk, 0, s, a);
}

template <int ND, int TW, int MM>
static void launch_tile(dim3 g, const ScanNDArgs &a, bool ring, const FlowArgs *flow, hipStream_t s) {
    if constexpr (ND == 3) {
        if (ring) {
            launch_tile_pl<ND, TW, MM, 4>(g, a, flow, s);
            return;
        }
    }
    launch_tile_pl<ND, TW, MM, 0>(g, a, flow, s);
}

// The dataflow schedule's state lives in the stream's ScanNDFlow workspace
// block (header as above, then the flags): launches on one stream run in
// order, so they may share it; launches on different streams use
// different blocks. A new block is cleared once; afterwards flags only
// ever hold epochs of earlier launches.

// XCD count of a device (-1 until looked up).
static int device_xcds(int dev) {
    static std::mutex mu;
    static int nx[64];
    static bool init = [] {
        for (int &v : nx) v = -1;
        return true;
    }();
    (void)init;
    if (dev < 0 || dev >= 64) return 0;
    std::lock_guard<std::mutex> guard(mu);
    if (nx[dev] < 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess) n = 0;
        nx[dev] = n;
    }
    return nx[dev];
}

// Polls per dataflow wait (KM_SCANND_FLOW_SPIN, read once): the safety
// budget after which a wait gives up (see scannd_flow_kernel).
static unsigned flow_spin() {
    static unsigned spin = [] {
        const char *e = std::getenv("KM_SCANND_FLOW_SPIN");
        if (!e || !*e) return kFlowSpinDefault;
        return static_cast<unsigned>(std::strtoul(e, nullptr, 10));
    }();
    return spin;
}

// Which status word the latest ScanND forward or backward on a (device,
// stream) left: 0 none (band or level schedule), 1 the stream's ScanNDFlow
// block, 2 a buffer given to the call (the allocation-free scratch of the
// device, or the backward's workspace), whose header address is kept.
struct LastFlow {
    int dev;
    hipStream_t stream;
    int kind;
    const unsigned *word;
    unsigned long long tick;
};
constexpr int kMaxLastFlow = 64;
static LastFlow g_last_flow[kMaxLastFlow];
static int g_last_flow_n = 0;
static unsigned long long g_last_flow_tick = 0;
static std::mutex g_last_flow_mu;

void note_flow(hipStream_t s, int kind, const unsigned *word) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return;
    std::lock_guard<std::mutex> guard(g_last_flow_mu);
    int idx = -1;
    for (int i = 0; i < g_last_flow_n; ++i)
        if (g_last_flow[i].dev == dev && g_last_flow[i].stream == s) idx = i;
    if (idx < 0) {
        if (g_last_flow_n < kMaxLastFlow) {
            idx = g_last_flow_n++;
        } else {
            idx = 0;   // the least recently noted stream
            for (int i = 1; i < g_last_flow_n; ++i)
                if (g_last_flow[i].tick < g_last_flow[idx].tick) idx = i;
        }
    }
    g_last_flow[idx] = LastFlow{dev, s, kind, kind == 2 ? word : nullptr, ++g_last_flow_tick};
}

static int last_flow_kind(hipStream_t s, const unsigned **word) {
    *word = nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> guard(g_last_flow_mu);
    for (int i = 0; i < g_last_flow_n; ++i)
        if (g_last_flow[i].dev == dev && g_last_flow[i].stream == s) {
            *word = g_last_flow[i].word;
            return g_last_flow[i].kind;
        }
    return 0;
}

// The dataflow schedule runs grids of 2 or more dims on a device with the 8
// XCDs the kernel reads from the hardware (XCC_ID 0-7);
// KM_SCANND_SCHED=band keeps one launch per band.
bool flow_wanted(int nd) {
    const char *e = std::getenv("KM_SCANND_SCHED");
    if (nd < 2 || (e && std::strcmp(e, "band") == 0)) return false;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return false;
    return device_xcds(dev) == 8;
}

__global__ void __launch_bounds__(256) flow_clear(unsigned *p, long n) {
    for (long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<long>(gridDim.x) * 256)
        p[i] = 0u;
}

void flow_zero(unsigned *p, size_t words, hipStream_t s) {
    hipLaunchKernelGGL(flow_clear, dim3(256), dim3(256), 0, s, p, static_cast<long>(words));
}

int flow_bind(hipStream_t s, size_t nflags_needed, FlowBuf *ext, FlowArgs &fa, int *kind) {
    *kind = 0;
    const size_t words = kFlowHead + nflags_needed;
    unsigned *fbuf = nullptr;
    long nflags = 0;   // flag words the state holds (cleared when the epoch wraps)
    if (ext) {
        if (ext->nxcc != 8) return 0;
        if (words > ext->cap) {
            set_error("scannd: the dataflow schedule needs %zu flag words, the scratch holds %zu",
                      words, ext->cap);
            return -1;
        }
        fbuf = ext->buf;
        nflags = static_cast<long>(ext->cap - kFlowHead);
        *kind = 2;
    } else {
        bool fresh = false;
        size_t got = 0;
        fbuf = static_cast<unsigned *>(Workspace::reserve(words * 4, s, WsUse::ScanNDFlow, &fresh, &got));
        if (!fbuf) {
            clear_error();   // no block: another schedule instead
            return 0;
        }
        nflags = static_cast<long>(got / 4 - kFlowHead);
        *kind = 1;
        if (fresh)
            hipLaunchKernelGGL(flow_clear, dim3(256), dim3(256), 0, s, fbuf, static_cast<long>(got / 4));
    }
    fa.counter = fbuf;
    fa.status = fbuf + kFlowStatus;
    fa.epoch = fbuf + kFlowEpoch;
    fa.flags = fbuf + kFlowHead;
    fa.spin = flow_spin();
    hipLaunchKernelGGL(flow_reset, dim3(1), dim3(256), 0, s, fbuf, nflags);
    return 1;
}

// Launches the forward on stream s. With allow_flow, grids of 3+ dims may
// use the dataflow schedule; *status then points at that launch's status
// word (device memory; nonzero after the launch when a wait gave up), else
// it is null. With ext, the dataflow state lives in ext's buffer and
// nothing is allocated: shapes that need the per-level fallback's plan
// buffer, or more flags than ext holds, fail with an error.
static int scannd_launch(ScanNDArgs &a, long P, hipStream_t s, bool allow_flow,
                         const unsigned **status, FlowBuf *ext = nullptr) {
    if (status) *status = nullptr;
    bool fast = (a.DM % 64 == 0) && (64 % a.M == 0) && a.nd >= 2 && a.nd <= 4;
    // Tiles: rows of TWc points along the last axis, Tlead along each
    // leading axis. One wave per (tile, channel group); one dataflow launch,
    // or one launch per tile band. Defaults measured fastest on MI355X at
    // 2D rows of 8 points x 16 rows per band launch (4 x 8 under
    // the dataflow schedule); 3D rows of 8 points x 4 per leading axis; 4D
    // rows of 4 x 4.
    const bool flow_pref = allow_flow && flow_wanted(a.nd);
    int TWc = (a.nd <= 3) ? 8 : 4;
    int Tlead = (a.nd == 2) ? 16 : 4;
    if (a.nd == 2 && flow_pref) {
        // 2D under the dataflow schedule: the critical path runs through
        // ntile0 + ntile1 - 1 tiles, so smaller tiles than the band
        // schedule's (measured fastest: 8 rows of 4 points).
        TWc = 4;
        Tlead = 8;
    }
    int nbands = 1;
    if (fast) {
        scannd_tile_shape(a.nd, TWc, Tlead);
        // Rows are prefetched one ahead, so every tile needs at least two
        // rows per plane below an in-tile leading axis: grow the row-axis
        // tile while its last tile would hold one row, and use tiles of 1
        // along the leading axes when the row axis has length 1.
        const int rax = a.nd - 2;
        int trow = (a.dims[rax] < Tlead) ? a.dims[rax] : Tlead;
        while (trow < a.dims[rax] && a.dims[rax] % trow == 1) ++trow;
        for (int ax = 0; ax < a.nd; ++ax) {
            int t = (ax == a.nd - 1) ? TWc : (ax == rax ? trow : Tlead);
            if (ax < rax && a.dims[rax] == 1) t = 1;
            a.tile[ax] = (a.dims[ax] < t) ? a.dims[ax] : t;
            a.ntile[ax] = (a.dims[ax] + a.tile[ax] - 1) / a.tile[ax];
            nbands += a.ntile[ax] - 1;
        }
        a.ncg = a.DM / 64;
        // The tile kernel addresses a tile (and the axis-0 plane before it)
        // with 32-bit byte offsets.
        long span = a.tile[a.nd - 1] + a.pstride[0];
        for (int ax = 0; ax + 1 < a.nd; ++ax) span += static_cast<long>(a.tile[ax] - 1) * a.pstride[ax];
        if (span * static_cast<long>(a.DM) * 4 >= 0x7fffffffL) fast = false;
    }
    if (fast) {
        if (nbands > 4096) {
            set_error("scannd: too many tile bands");
            return -1;
        }
        // Tiles per band: distribution of tile-index sums.
        static thread_local long cnt[4096], nxt[4096];
        auto count_bands = [&]() {
            nbands = 1;
            for (int ax = 0; ax < a.nd; ++ax) nbands += a.ntile[ax] - 1;
            for (int i = 0; i < nbands; ++i) cnt[i] = 0;
            cnt[0] = 1;
            int reach = 0;
            for (int ax = 0; ax < a.nd; ++ax) {
                for (int i = 0; i <= reach + a.ntile[ax] - 1; ++i) nxt[i] = 0;
                for (int sidx = 0; sidx <= reach; ++sidx)
                    for (int v = 0; v < a.ntile[ax]; ++v) nxt[sidx + v] += cnt[sidx];
                reach += a.ntile[ax] - 1;
                for (int sidx = 0; sidx <= reach; ++sidx) cnt[sidx] = nxt[sidx];
            }
            long n = 0;
            for (int b = 0; b < nbands; ++b) n += cnt[b];
            return n;
        };
        long ntiles = count_bands();
        // 3D tiles of 4 rows along axis 1 keep the previous plane in registers.
        const bool ring = a.nd == 3 && a.tile[1] == 4;
        // Under the dataflow schedule 3D ring tiles become pencils along
        // axis 0 with a flag per a.sub planes (the tile's depth): the ring
        // carries the axis-0 neighbour from one sub-tile to the next instead
        // of reading it back from h. x / delta / y are then addressed from
        // the pencil's origin with 32-bit offsets. KM_SCANND_PENCIL=0 keeps
        // separate tiles.
        a.sub = 0;
        const char *pe = std::getenv("KM_SCANND_PENCIL");
        const bool pencil = flow_pref && ring && !(pe && std::strcmp(pe, "0") == 0) && a.ntile[0] > 1 &&
                            P * static_cast<long>(a.D) * 4 < 0x7fffffffL;
        const int tile0 = a.tile[0], ntile0 = a.ntile[0];
        long nflags = ntiles * a.ncg;
        if (pencil) {
            a.sub = tile0;
            a.tile[0] = a.dims[0];
            a.ntile[0] = 1;
            ntiles = count_bands();
            nflags = static_cast<long>(ntile0) * ntiles * a.ncg;
        }
        static thread_local FlowArgs fa;
        int kind = 0, bound = 0;
        if (flow_pref && nbands <= kMaxFlowBands && nflags < 0x7fffffffL) {
            fa.nbands = nbands;
            for (int x = 0; x <= 8; ++x) fa.cg_lo[x] = static_cast<int>(static_cast<long>(x) * a.ncg / 8);
            fa.band_start[0] = 0;
            for (int b = 0; b < nbands; ++b) fa.band_start[b + 1] = fa.band_start[b] + static_cast<int>(cnt[b]);
            bound = flow_bind(s, static_cast<size_t>(nflags), ext, fa, &kind);
            if (bound < 0) return -1;
        }
        if (pencil && bound == 0) {
            // No dataflow state: one launch per band of separate tiles.
            a.sub = 0;
            a.tile[0] = tile0;
            a.ntile[0] = ntile0;
            ntiles = count_bands();
        }
        note_flow(s, kind, kind == 2 ? fa.counter : nullptr);
        const FlowArgs *flow = nullptr;
        if (bound > 0) {
            flow = &fa;
            if (status) *status = fa.status;
        }
        // Dataflow: one launch of 8k workgroups of Q waves that take items
        // until their XCD's queue is empty. The hardware deals workgroups to
        // the XCDs round-robin, so each XCD runs k of them, k = the largest
        // per-XCD item count up to kcap / Q: two waves per SIMD in 2D, one in
        // 3D and 4D (measured at configs[2]: 3D 1.864 ms with one wave per
        // SIMD against 1.967 ms with two, whose larger set of tiles in
        // flight thrashed the L2: 7.13 -> 6.55 GB read; 2D 1.10 against
        // 0.96 ms the other way).
        const long kcap = a.nd == 2 ? 256 : 128;
        long per_xcd = 0;
        const int fq = flow ? flow_q(fa) : 1;
        if (flow)
            for (int x = 0; x < 8; ++x)
                per_xcd = std::max<long>(per_xcd, ntiles * ((fa.cg_lo[x + 1] - fa.cg_lo[x]) / fq));
        const int nlaunch = flow ? 1 : nbands;
        for (int b = 0; b < nlaunch; ++b) {
            a.band = b;
            const long grid = flow ? 8 * std::min<long>(per_xcd, kcap / fq) : cnt[b] * a.ncg;
            if (grid <= 0) continue;
            const dim3 g(static_cast<unsigned>(grid));
#define KM_ND_LAUNCH(NDv, TWv, MMv) launch_tile<NDv, TWv, MMv>(g, a, ring, flow, s)
#define KM_ND_BY_M(NDv, TWv)                                  \
            switch (a.M) {                                    \
            case 1: KM_ND_LAUNCH(NDv, TWv, 1); break;         \
            case 2: KM_ND_LAUNCH(NDv, TWv, 2); break;         \
            case 4: KM_ND_LAUNCH(NDv, TWv, 4); break;         \
            case 8: KM_ND_LAUNCH(NDv, TWv, 8); break;         \
            case 16: KM_ND_LAUNCH(NDv, TWv, 16); break;       \
            case 32: KM_ND_LAUNCH(NDv, TWv, 32); break;       \
            default: KM_ND_LAUNCH(NDv, TWv, 64); break;       \
            }
            if (a.nd == 2) {
                if (TWc == 4) { KM_ND_BY_M(2, 4) }
                else if (TWc == 8) { KM_ND_BY_M(2, 8) }
                else { KM_ND_BY_M(2, 16) }
            } else if (a.nd == 3) {
                if (TWc == 4) { KM_ND_BY_M(3, 4) }
                else { KM_ND_BY_M(3, 8) }
            } else {
                if (TWc == 4) { KM_ND_BY_M(4, 4) }
                else { KM_ND_BY_M(4, 8) }
            }
#undef KM_ND_BY_M
#undef KM_ND_LAUNCH
            KM_HIP_TRY(hipGetLastError());
        }
        return 0;
    }
    // Fallback: per-level launches over the plan.
    note_flow(s, 0);
    if (ext) {
        set_error("scannd: this shape needs the per-level schedule, whose plan buffer is "
                  "allocated; use km_scannd_fwd");
        return -1;
    }
    long dims[kMaxNd];
    for (int ax = 0; ax < a.nd; ++ax) dims[ax] = a.dims[ax];
    KMWavefrontPlan *plan = km_wavefront_plan_create(dims, a.nd);
    if (!plan) {
        set_error("scannd: plan creation failed");
        return -1;
    }
    const size_t bytes = sizeof(long) * P;
    long *offs = static_cast<long *>(Workspace::reserve(bytes, s, WsUse::ScanNDPlan));
    if (!offs) {
        km_wavefront_plan_free(plan);
        return -1;
    }
    // The plan is host memory that is freed below: a synchronous copy.
    if (hipMemcpyAsync(offs, plan->level_offsets, bytes, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        km_wavefront_plan_free(plan);
        set_error("scannd: plan upload failed");
        return -1;
    }
    for (long lvl = 0; lvl <= plan->max_level; ++lvl) {
        const long start = plan->level_starts[lvl];
        const long count = plan->level_starts[lvl + 1] - start;
        const long threads = count * a.D;
        hipLaunchKernelGGL(scannd_level_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)),
                           dim3(256), 0, s, a, offs, start, count);
    }
    km_wavefront_plan_free(plan);
    KM_HIP_TRY(hipGetLastError());
    return 0;
}

// Mamba-3 branch on device pointers: per-level launches over the wavefront
// plan; the level offsets and the rotated states live in the stream's
// library workspace.
static int scannd_m3_device(const ScanNDParams *p, hipStream_t s, bool sync) {
    if (!is_device_ptr(p->lambda) || (p->theta && !is_device_ptr(p->theta))) {
        set_error("scannd: theta and lambda must be device memory on the device-pointer path");
        return -1;
    }
    if (p->ndims > kMaxNd) {
        set_error("scannd: the Mamba-3 branch supports up to %d dimensions", kMaxNd);
        return -1;
    }
    const long P = wavefront_nd_total_points(p->dims, p->ndims);
    if (P <= 0 || P > 0x7fffffffL || p->D > 0x7fffffffL || p->M > 0x7fffffffL) {
        set_error("scannd: sizes out of range for the Mamba-3 branch");
        return -1;
    }
    KMWavefrontPlan *plan = km_wavefront_plan_create(p->dims, p->ndims);
    if (!plan) {
        set_error("scannd: plan creation failed");
        return -1;
    }
    note_flow(s, 0);
    const size_t off_bytes = align_up(sizeof(long) * P, 256);
    const size_t rot_bytes = sizeof(float) * static_cast<size_t>(P) * p->D * p->M;
    char *ws = static_cast<char *>(Workspace::reserve(off_bytes + rot_bytes, s, WsUse::ScanNDM3));
    if (!ws) {
        km_wavefront_plan_free(plan);
        return -1;
    }
    long *offs = reinterpret_cast<long *>(ws);
    ScanM3Args a{};
    a.x = p->x; a.B = p->B; a.C = p->C; a.theta = p->theta; a.lambda = p->lambda;
    a.h = p->h; a.y = p->y; a.hrot = reinterpret_cast<float *>(ws + off_bytes);
    a.nd = static_cast<int>(p->ndims);
    a.D = static_cast<int>(p->D);
    a.M = static_cast<int>(p->M);
    a.DM = p->D * p->M;
    long stride = 1;
    for (int ax = a.nd - 1; ax >= 0; --ax) {
        a.dims[ax] = static_cast<int>(p->dims[ax]);
        a.pstride[ax] = stride;
        stride *= p->dims[ax];
    }
    for (int ax = 0; ax < a.nd; ++ax) {
        a.A[ax] = p->A + ax * p->D * p->M;
        a.dt[ax] = p->delta + ax * P * p->D;
    }
    // The plan is host memory that is freed below: a synchronous copy.
    if (hipMemcpyAsync(offs, plan->level_offsets, sizeof(long) * P, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        km_wavefront_plan_free(plan);
        set_error("scannd: plan upload failed");
        return -1;
    }
    const long npair = (p->D + 1) / 2;
    for (long lvl = 0; lvl <= plan->max_level; ++lvl) {
        const long start = plan->level_starts[lvl];
        const long count = plan->level_starts[lvl + 1] - start;
        const long threads = count * npair;
        hipLaunchKernelGGL(scannd_m3_level_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)),
                           dim3(256), 0, s, a, offs, start, count);
    }
    km_wavefront_plan_free(plan);
    KM_HIP_TRY(hipGetLastError());
    if (sync && hipStreamSynchronize(s) != hipSuccess) {
        set_error("scannd: %s", hipGetErrorString(hipGetLastError()));
        return -1;
    }
    return 0;
}

// Shared front end: device pointers, scannd_ref semantics for ndims >= 2.
// sync: wait for the result; if a dataflow wait gave up, run the call again
// on the band schedule, so the synchronous entry points always return the
// exact result.
static int scannd_device(const float *x, const float *const *A, const float *const *dt,
                         const float *B, const float *C, float *h, float *y, const long *dims,
                         long nd, long D, long M, hipStream_t s, bool sync,
                         FlowBuf *ext = nullptr) {
    if (nd < 2 || nd > kMaxNd) {
        set_error("scannd: ndims %ld outside [2, %d] for the band kernel", nd, kMaxNd);
        return -1;
    }
    ScanNDArgs a{};
    a.x = x;
    a.B = B;
    a.C = C;
    a.h = h;
    a.y = y;
    a.nd = static_cast<int>(nd);
    a.D = static_cast<int>(D);
    a.M = static_cast<int>(M);
    a.DM = static_cast<int>(D * M);
    long P = 1;
    for (int ax = 0; ax < nd; ++ax) {
        if (dims[ax] <= 0 || dims[ax] > 0x7fffffff) {
            set_error("scannd: invalid dims[%d] = %ld", ax, dims[ax]);
            return -1;
        }
        a.dims[ax] = static_cast<int>(dims[ax]);
        a.A[ax] = A[ax];
        a.dt[ax] = dt[ax];
        P *= dims[ax];
    }
    long st = 1;
    for (int ax = static_cast<int>(nd) - 1; ax >= 0; --ax) {
        a.pstride[ax] = st;
        st *= dims[ax];
    }
    if (D * M > 0x7fffffffL || P * D * M > (1L << 46)) {
        set_error("scannd: problem too large");
        return -1;
    }
    const unsigned *status = nullptr;
    if (scannd_launch(a, P, s, true, sync ? &status : nullptr, ext) != 0) return -1;
    if (!sync) return 0;
    if (hipStreamSynchronize(s) != hipSuccess) {
        set_error("scannd: %s", hipGetErrorString(hipGetLastError()));
        return -1;
    }
    if (!status) return 0;
    unsigned failed = 0;
    if (km::copy_d2h(&failed, status, sizeof failed) != hipSuccess) {
        set_error("scannd: status read failed");
        return -1;
    }
    if (!failed) return 0;
    // A dataflow wait ran out of budget (its tiles hold NaN): once more on
    // the band schedule, whose launches order the tiles.
    if (scannd_launch(a, P, s, false, nullptr) != 0) return -1;
    if (hipStreamSynchronize(s) != hipSuccess) {
        set_error("scannd: %s", hipGetErrorString(hipGetLastError()));
        return -1;
    }
    return 0;
}

static bool scannd_params_ok(const ScanNDParams *p) {
    if (!scannd_validate(p)) {
        set_error("scannd: invalid parameters");
        return false;
    }
    return true;
}

int scannd_device_params(const ScanNDParams *p, hipStream_t s, bool sync, FlowBuf *ext = nullptr) {
    if (!scannd_params_ok(p)) return -1;
    if (!gpu_ready()) return -1;
    // Mamba-3 branch (lambda given); theta alone changes nothing, as in the
    // reference, where the rotation belongs to the lambda branch.
    if (p->lambda) {
        if (ext) {
            set_error("km_scannd_fwd_noalloc: the Mamba-3 (lambda) branch needs the library "
                      "workspace; use km_scannd_fwd");
            return -1;
        }
        return scannd_m3_device(p, s, sync);
    }
    const long P = wavefront_nd_total_points(p->dims, p->ndims);
    const float *A[kMaxNd], *dt[kMaxNd];
    for (long ax = 0; ax < p->ndims && ax < kMaxNd; ++ax) {
        A[ax] = p->A + ax * p->D * p->M;
        dt[ax] = p->delta + ax * P * p->D;
    }
    if (p->ndims == 1) {
        // ndims == 1: the 1D recurrence with the full state written, no clamp.
        KMScan1DFwd k{};
        k.x = p->x; k.delta = p->delta; k.A = p->A; k.Bm = p->B; k.Cm = p->C; k.y = p->y;
        k.h_hist = p->h;
        k.B = 1; k.L = P; k.D = p->D; k.N = p->M;
        k.bc_sb = P * p->D * p->M; k.bc_st = p->D * p->M; k.bc_sd = p->M;
        k.dtype = KM_F32; k.clamp = 0;
        note_flow(s, 0);
        // Without allocation (ext given): kernels that need no workspace.
        if (scan1d_fwd_launch(&k, s, ext == nullptr) != 0) return -1;
        if (sync && hipStreamSynchronize(s) != hipSuccess) {
            set_error("scannd: %s", hipGetErrorString(hipGetLastError()));
            return -1;
        }
        return 0;
    }
    return scannd_device(p->x, A, dt, p->B, p->C, p->h, p->y, p->dims, p->ndims, p->D, p->M, s, sync,
                         ext);
}

// The allocation-free variant's dataflow state: a file-scope device array
// (each GPU holds its own copy for the life of the process), 16 words of
// counters and status and then the completion flags of up to
// kScratchWords - 16 (tile, channel group) items. Its device address is
// looked up once per device with hipGetSymbolAddress; host code uses that
// address, never the array's name (which on the host is only a stand-in).
constexpr size_t kScratchWords = size_t(1) << 18;   // 1 MiB
static __device__ __align__(256) unsigned scratch[kScratchWords];

struct NoAllocDevice {
    bool ready = false;
    unsigned *ptr = nullptr;
    int nxcc = 0;
};
constexpr int kMaxDevices = 64;
static NoAllocDevice g_noalloc[kMaxDevices];
static std::mutex g_noalloc_mu;

int scannd_fwd_noalloc(const ScanNDParams *p, hipStream_t s) {
    if (!scannd_params_ok(p)) return -1;
    if (!gpu_ready()) return -1;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error("km_scannd_fwd_noalloc: no current HIP device below %d", kMaxDevices);
        return -1;
    }
    std::lock_guard<std::mutex> guard(g_noalloc_mu);
    NoAllocDevice &nd = g_noalloc[dev];
    if (!nd.ready) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            set_error("km_scannd_fwd_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
            return -1;
        }
        nd.ptr = static_cast<unsigned *>(ptr);
        nd.nxcc = device_xcds(dev);
        nd.ready = true;
    }
    FlowBuf fb{nd.ptr, kScratchWords, nd.nxcc};
    return scannd_device_params(p, s, false, &fb);
}

// Status of the latest ScanND forward enqueued on stream s (see
// km_scannd_status).
int scannd_status(hipStream_t s) {
    if (!gpu_ready()) return -1;
    const unsigned *word = nullptr;
    const int kind = last_flow_kind(s, &word);
    if (kind == 1) word = static_cast<const unsigned *>(Workspace::find(s, WsUse::ScanNDFlow));
    if (hipStreamSynchronize(s) != hipSuccess) {
        set_error("km_scannd_status: %s", hipGetErrorString(hipGetLastError()));
        return -1;
    }
    if (!word) return 0;
    unsigned failed = 0;
    if (hipMemcpy(&failed, word + kFlowStatus, sizeof failed, hipMemcpyDeviceToHost) != hipSuccess) {
        set_error("km_scannd_status: status read failed");
        return -1;
    }
    return failed ? 1 : 0;
}

// Host-pointer staging for the reference's host API: copies inputs to the
// device (or uses them in place when they already are device memory), runs,
// and copies h and y back.
struct NDStage {
    float *x, *A, *B, *C, *dt, *h, *y;
};

static int scannd_host(const ScanNDParams *p, bool scan1d_semantics) {
    if (!scannd_params_ok(p)) return -1;
    if (!gpu_ready()) return -1;
    const long P = wavefront_nd_total_points(p->dims, p->ndims);
    const long nd = p->ndims, D = p->D, M = p->M;
    const size_t nx = P * D, nA = nd * D * M, nB = P * D * M, ndt = nd * P * D;
    const size_t nh = scan1d_semantics ? static_cast<size_t>(D * M) : nB;
    const bool dev = is_device_ptr(p->x) && is_device_ptr(p->A) && is_device_ptr(p->B) &&
                     is_device_ptr(p->C) && is_device_ptr(p->delta) && is_device_ptr(p->h) &&
                     is_device_ptr(p->y) && (!p->lambda || is_device_ptr(p->lambda)) &&
                     (!p->lambda || !p->theta || is_device_ptr(p->theta));
    int rc = 0;
    if (dev) {
        if (scan1d_semantics) {
            ScanParams sp{const_cast<float *>(p->x), const_cast<float *>(p->A), const_cast<float *>(p->B),
                          const_cast<float *>(p->C), const_cast<float *>(p->delta), p->h, p->y,
                          P, D, M};
            scan1d(&sp);
            return km_last_error()[0] ? -1 : 0;
        }
        return scannd_device_params(p, nullptr, true);
    }
    if (scan1d_semantics) {
        ScanParams sp{const_cast<float *>(p->x), const_cast<float *>(p->A), const_cast<float *>(p->B),
                      const_cast<float *>(p->C), const_cast<float *>(p->delta), p->h, p->y, P, D, M};
        scan1d(&sp);
        return km_last_error()[0] ? -1 : 0;
    }
    Staging::lock();
    // Mamba-3 operands: theta [D/2] (rotation pairs) and lambda [P].
    const size_t nth = p->lambda && p->theta ? static_cast<size_t>(D / 2 > 0 ? D / 2 : 1) : 0;
    const size_t nlam = p->lambda ? static_cast<size_t>(P) : 0;
    const size_t bytes = sizeof(float) * (2 * nx + nA + 3 * nB + ndt + nth + nlam) + 10 * 256;
    void *base = Staging::reserve(bytes);
    if (!base) {
        Staging::unlock();
        return -1;
    }
    Carver c(base);
    NDStage st{c.take<float>(nx), c.take<float>(nA), c.take<float>(nB), c.take<float>(nB),
               c.take<float>(ndt), c.take<float>(nh), c.take<float>(nx)};
    float *th = nth ? c.take<float>(nth) : nullptr;
    float *lam = nlam ? c.take<float>(nlam) : nullptr;
    const bool ok = km::copy_h2d(st.x, p->x, nx * 4) == hipSuccess &&
                    km::copy_h2d(st.A, p->A, nA * 4) == hipSuccess &&
                    km::copy_h2d(st.B, p->B, nB * 4) == hipSuccess &&
                    km::copy_h2d(st.C, p->C, nB * 4) == hipSuccess &&
                    km::copy_h2d(st.dt, p->delta, ndt * 4) == hipSuccess &&
                    (!th || D / 2 == 0 || hipMemcpy(th, p->theta, (D / 2) * 4, hipMemcpyDefault) == hipSuccess) &&
                    (!lam || hipMemcpy(lam, p->lambda, nlam * 4, hipMemcpyDefault) == hipSuccess);
    if (!ok) {
        set_error("scannd: host-to-device copy failed");
        rc = -1;
    } else {
        ScanNDParams q = *p;
        q.x = st.x; q.A = st.A; q.B = st.B; q.C = st.C; q.delta = st.dt; q.h = st.h; q.y = st.y;
        q.theta = th; q.lambda = lam;
        rc = scannd_device_params(&q, nullptr, true);
        if (rc == 0 && (km::copy_d2h(p->h, st.h, nh * 4) != hipSuccess ||
                        km::copy_d2h(p->y, st.y, nx * 4) != hipSuccess)) {
            set_error("scannd: device-to-host copy failed");
            rc = -1;
        }
    }
    Staging::unlock();
    return rc;
}

}  // namespace km

extern "C" {

int scannd_validate(const ScanNDParams *p) {
    if (!p || !p->dims) return 0;
    if (p->ndims <= 0 || p->D <= 0 || p->M <= 0) return 0;
    if (!p->x || !p->A || !p->B || !p->C || !p->delta || !p->h || !p->y) return 0;
    if (!wavefront_nd_validate_dims(p->dims, p->ndims)) return 0;
    if (wavefront_nd_total_points(p->dims, p->ndims) <= 0) return 0;
    return 1;
}

int km_scannd_fwd(const ScanNDParams *p, void *stream) {
    km::clear_error();
    return km::scannd_device_params(p, static_cast<hipStream_t>(stream), false);
}

// No counterpart in the reference: km_scannd_fwd for callers that cannot
// allocate (see kmamba_km.h).
int km_scannd_fwd_noalloc(const ScanNDParams *p, void *stream) {
    km::clear_error();
    return km::scannd_fwd_noalloc(p, static_cast<hipStream_t>(stream));
}

int km_scannd_status(void *stream) {
    km::clear_error();
    return km::scannd_status(static_cast<hipStream_t>(stream));
}

int om_scannd_forward(ScanNDParams *p) {
    km::clear_error();
    return km::scannd_device_params(p, nullptr, true);
}

int mamba_scannd_cuda_forward(ScanNDParams *p) { return om_scannd_forward(p); }

int scannd_ref(ScanNDParams *p) {
    km::clear_error();
    return km::scannd_host(p, false);
}

int scannd_ref_with_plan(ScanNDParams *p, const KMWavefrontPlan *plan) {
    km::clear_error();
    if (!p || !km_wavefront_plan_matches_dims(plan, p->dims, p->ndims)) {
        km::set_error("scannd_ref_with_plan: plan does not match dims");
        return -1;
    }
    return km::scannd_host(p, false);
}

int scannd(ScanNDParams *p) {
    km::clear_error();
    if (!scannd_validate(p)) {
        km::set_error("scannd: invalid parameters");
        return -1;
    }
    // Ranks 1 and 2 take the reference's scan1d / scan2d paths, which have
    // no Mamba-3 operands (src/scan_nd.c:265-305): theta and lambda are
    // ignored there, and honoured by the scannd_ref path of rank >= 3.
    if (p->ndims <= 2 && (p->theta || p->lambda)) {
        ScanNDParams q = *p;
        q.theta = nullptr;
        q.lambda = nullptr;
        return km::scannd_host(&q, q.ndims == 1);
    }
    return km::scannd_host(p, p->ndims == 1);
}

void scan2d(Scan2DParams *p) {
    km::clear_error();
    if (!p || !p->x || !p->A1 || !p->A2 || !p->B || !p->C || !p->delta1 || !p->delta2 || !p->h ||
        !p->y || p->d1 <= 0 || p->d2 <= 0 || p->D <= 0 || p->M <= 0) {
        km::set_error("scan2d: invalid parameters");
        return;
    }
    if (!km::gpu_ready()) return;
    const long dims[2] = {p->d1, p->d2};
    const long P = p->d1 * p->d2, D = p->D, M = p->M;
    const size_t nx = P * D, nA = D * M, nB = P * D * M;
    const bool dev = km::is_device_ptr(p->x) && km::is_device_ptr(p->A1) && km::is_device_ptr(p->A2) &&
                     km::is_device_ptr(p->B) && km::is_device_ptr(p->C) &&
                     km::is_device_ptr(p->delta1) && km::is_device_ptr(p->delta2) &&
                     km::is_device_ptr(p->h) && km::is_device_ptr(p->y);
    if (dev) {
        const float *A[2] = {p->A1, p->A2}, *dt[2] = {p->delta1, p->delta2};
        (void)km::scannd_device(p->x, A, dt, p->B, p->C, p->h, p->y, dims, 2, D, M, nullptr, true);
        return;
    }
    km::Staging::lock();
    void *base = km::Staging::reserve(sizeof(float) * (4 * nx + 2 * nA + 3 * nB) + 10 * 256);
    if (base) {
        km::Carver c(base);
        float *x = c.take<float>(nx), *A1 = c.take<float>(nA), *A2 = c.take<float>(nA);
        float *B = c.take<float>(nB), *C = c.take<float>(nB), *d1 = c.take<float>(nx);
        float *d2 = c.take<float>(nx), *h = c.take<float>(nB), *y = c.take<float>(nx);
        const bool ok = km::copy_h2d(x, p->x, nx * 4) == hipSuccess &&
                        km::copy_h2d(A1, p->A1, nA * 4) == hipSuccess &&
                        km::copy_h2d(A2, p->A2, nA * 4) == hipSuccess &&
                        km::copy_h2d(B, p->B, nB * 4) == hipSuccess &&
                        km::copy_h2d(C, p->C, nB * 4) == hipSuccess &&
                        km::copy_h2d(d1, p->delta1, nx * 4) == hipSuccess &&
                        km::copy_h2d(d2, p->delta2, nx * 4) == hipSuccess;
        if (!ok) {
            km::set_error("scan2d: host-to-device copy failed");
        } else {
            const float *A[2] = {A1, A2}, *dt[2] = {d1, d2};
            if (km::scannd_device(x, A, dt, B, C, h, y, dims, 2, D, M, nullptr, true) == 0) {
                if (km::copy_d2h(p->h, h, nB * 4) != hipSuccess ||
                    km::copy_d2h(p->y, y, nx * 4) != hipSuccess)
                    km::set_error("scan2d: device-to-host copy failed");
            }
        }
    }
    km::Staging::unlock();
}

void mamba_scan2d_forward(MambaScan2DParams *p) { scan2d(p); }

}  // extern "C"

// scan1d_fwd.hip - Scan1D selective-scan forward for gfx950.
//
// Recurrence (reference cpu/scan1d.asm:53-169, per batch element):
//   e = exp(delta*A[d,n]);  h = e*h + B*(delta*x);  y = sum_n C*h
//
// Design (one kernel, no scratch memory):
//  * A wave covers DL = 64/NS channels; its lanes split the N states into NS
//    groups of NPL states kept in registers (N=16: 32 channels x 2 halves), so
//    x/delta/y rows are read and written as whole 128-byte lines and the
//    B/C operand a lane needs is one LDS broadcast row.
//  * A workgroup of W waves owns one (batch, channel group) for the whole
//    sequence and walks it in super-chunks of W*TC steps. Wave w runs a local
//    pass over its TC steps from a zero state, keeping every exp in registers,
//    and publishes its chunk map h -> P*h + h_loc (P = exp2(A*log2e*sum
//    delta)) through LDS. After one barrier each wave folds the carry and the
//    maps of the waves before it, then replays its steps from the exact
//    incoming state with the stored exps, writing y (and the state history
//    when asked). The last wave's state is the next super-chunk's carry.
//  * Shared B/C ([B, L, N], stride over channels 0) are staged per
//    super-chunk into LDS, double-buffered and prefetched one super-chunk
//    ahead; per-channel B/C (the reference [L, D, M] layout) are read
//    straight from memory. x/delta of the next super-chunk are prefetched into
//    registers.
//  * The reference clamps the state to +-1000 after every step
//    (cpu/scan1d.asm:136-140), which is not associative. The chunked pass runs
//    unclamped and tracks max|h| and NaN; a workgroup that saw either re-runs
//    its whole sequence with the sequential clamped recurrence, so results
//    follow the per-step clamp exactly.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "km_device.hpp"
#include "../km_runtime.hpp"
#include "kmamba_km.h"
#include "scan.h"
#include "mamba_scan.h"
#include "mamba_scan_cuda.h"

namespace km {

struct Scan1DFwdArgs {
    const void *x, *dt;
    const float *A;
    const void *Bm, *Cm;
    void *y;
    const float *h0;
    float *hfin;
    float *hist;
    float *ckpt;     // [B, nck, D, N] state after every kCkptSteps steps, or null
    long nck;
    const void *z;        // [B, L, D] gate: y *= SiLU(z), or null
    const float *Dskip;   // [D] skip: y += Dskip * x, or null
    long B, L, D, N;
    long sb, st, sd;
    int clamp;
    // Segmented launches (the sequence split over workgroups): a workgroup
    // whose states leave [-1000, 1000] sets clamp_flag[b / nseg * groups +
    // group] and leaves the sequential re-run to scan1d_clamp_repair, or
    // null for the workgroup's own fallback.
    int *clamp_flag;
    long nseg;
    // [B, D] sum of delta over the sequence (kernels built with DSUM).
    float *dsum_out;
};

// Output of one step: the readout, plus Dskip*x and times SiLU(z) when
// given (the Mamba gating, applied after the readout sum).
template <typename T>
__device__ __forceinline__ float gated(const Scan1DFwdArgs &p, float y, float xv, float dsk,
                                       float zv) {
    if (p.Dskip) y = fmaf(dsk, xv, y);
    if (p.z) y *= silu_fast(zv);
    return y;
}

// Sequential clamped recurrence for the lanes of one wave (the clamp
// fallback): the reference's step order, one (batch, channel, state group)
// per lane.
template <typename T, int NPL, int NS, bool SHARED, bool HIST>
__device__ void scan1d_serial_wave(const Scan1DFwdArgs &p, long b, long d, bool dvalid,
                                   int n0, const float *Ap) {
    using IO = io<T>;
    const long dc = dvalid ? d : p.D - 1;
    const long N = p.N;
    float hs[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) hs[j] = p.h0 ? p.h0[(b * p.D + dc) * N + n0 + j] : 0.f;
    for (long t = 0; t < p.L; ++t) {
        const long xi = (b * p.L + t) * p.D + dc;
        const float xv = IO::ld(p.x, xi), dv = IO::ld(p.dt, xi);
        const long bc = b * p.sb + t * p.st + (SHARED ? 0 : dc * p.sd) + n0;
        float yp = 0.f;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            const float e = exp2_fast(dv * Ap[j]);
            const float dB = __fmul_rn(IO::ld(p.Bm, bc + j), dv);
            float hn = __fadd_rn(__fmul_rn(e, hs[j]), __fmul_rn(dB, xv));
            hn = (hn < 1000.f) ? hn : 1000.f;
            hn = (hn > -1000.f) ? hn : -1000.f;
            hs[j] = hn;
            yp = __fadd_rn(yp, __fmul_rn(IO::ld(p.Cm, bc + j), hn));
        }
        if (NS >= 4) yp += __shfl_xor(yp, 16);
        if (NS >= 2) yp += __shfl_xor(yp, 32);
        if (dvalid) {
            if (n0 == 0 && p.y) {
                const float zv = p.z ? IO::ld(p.z, xi) : 0.f;
                IO::st(p.y, xi, gated<T>(p, yp, xv, p.Dskip ? p.Dskip[dc] : 0.f, zv));
            }
            if (p.ckpt && ((t + 1) % kCkptSteps == 0 || t == p.L - 1)) {
#pragma unroll
                for (int j = 0; j < NPL; ++j)
                    p.ckpt[((b * p.nck + t / kCkptSteps) * p.D + d) * N + n0 + j] = hs[j];
            }
            if (HIST) {
#pragma unroll
                for (int j = 0; j < NPL; ++j) p.hist[xi * N + n0 + j] = hs[j];
            }
        }
    }
    if (p.hfin && dvalid) {
#pragma unroll
        for (int j = 0; j < NPL; ++j) p.hfin[(b * p.D + d) * N + n0 + j] = hs[j];
    }
}

// Decays of a lane's states n = NS*j + ns (states interleaved over the NS
// lane groups of a channel) when A[d, n] = (n+1) A[d, 0]: e1^(n+1) =
// e1^(ns+1) * (e1^NS)^j, one multiply per state after the base.
template <int NPL, int NS>
__device__ __forceinline__ void pow_chain_il(float e1, int ns, float (&e)[NPL]) {
    float pw[NS];
    pw[0] = e1;
#pragma unroll
    for (int i = 1; i < NS; ++i) pw[i] = pw[i - 1] * e1;
    float base = pw[0];
#pragma unroll
    for (int i = 1; i < NS; ++i) base = (ns == i) ? pw[i] : base;
    const float step = pw[NS - 1];
    e[0] = base;
#pragma unroll
    for (int j = 1; j < NPL; ++j) e[j] = e[j - 1] * step;
}

// OCC: waves per SIMD the register allocation must allow (2 workgroups of
// 8 waves per CU need 4).
template <typename T, int NPL, int NS, int W, int TC, bool SHARED, bool HIST, bool STORE_BU, int OCC,
          bool GATE, bool DSUM = false>
__global__ void __launch_bounds__(64 * W, OCC) scan1d_fwd_chunked(Scan1DFwdArgs p) {
    using IO = bio<T>;
    constexpr int DL = 64 / NS;      // channels per wave
    constexpr int N = NPL * NS;      // states per channel
    constexpr int SC = W * TC;       // steps per super-chunk
    constexpr int TILE = SC * N;     // B (or C) values per super-chunk
    constexpr int NT = 64 * W;
    constexpr int TPT = (TILE + NT - 1) / NT;
    constexpr int TS = IO::size;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index, kept in an SGPR
    const int dl = lane % DL;
    const int ns = lane / DL;
    const int n0 = ns * NPL;
    const long ngroups = (p.D + DL - 1) / DL;
    // Workgroups numbered XCD-major: the channel groups of a batch element
    // run on as few XCDs as possible, so its shared B/C rows and (bf16: a
    // group's 32 channels are half of a 128-byte line) its x / delta lines
    // are fetched into one L2.
    const long wg = xcd_remap(blockIdx.x, gridDim.x);
    const long b = wg / ngroups;
    const long grp = wg - b * ngroups;
    const long d = grp * DL + dl;
    const bool dvalid = d < p.D;
    const int dc = static_cast<int>(dvalid ? d : p.D - 1);
    const int L = static_cast<int>(p.L);
    const int Dm = static_cast<int>(p.D);
    const int nit = (L + SC - 1) / SC;
    const bool store_y = dvalid && ns == 0;
    const float dsk = (GATE && p.Dskip) ? p.Dskip[dvalid ? d : p.D - 1] : 0.f;
    // Two state halves per channel (NS = 2): the readouts of steps 2i and
    // 2i + 1 are summed over the halves by one lane swap, which leaves step
    // 2i's sum in the lower half and step 2i + 1's in the upper half; each
    // half then stores (and gates, loading only its own steps' z) its step:
    // one swap, one add, one SiLU and one 64-lane store per step pair.
    constexpr bool PAIR = NS == 2 && TC % 2 == 0;
    constexpr bool PAIRG = GATE && PAIR;
    constexpr int ZC = GATE ? (PAIRG ? TC / 2 : TC) : 1;

    // Per-batch-element windows addressed with 32-bit byte offsets (the
    // launcher keeps every window and offset below 1 GiB). Every variable
    // offset goes in the VGPR offset so the hardware range check applies:
    // rows past L load as 0 and their stores are dropped.
    const long xoff = b * p.L * p.D;
    const auto rx = make_rsrc(static_cast<const char *>(p.x) + xoff * TS, p.L * p.D * TS);
    const auto rdt = make_rsrc(static_cast<const char *>(p.dt) + xoff * TS, p.L * p.D * TS);
    // y may be null (checkpoint-only forward): a zero-sized window drops the stores.
    const auto ry = make_rsrc(p.y ? static_cast<char *>(p.y) + xoff * TS : nullptr,
                              p.y ? p.L * p.D * TS : 0);
    const auto rz = make_rsrc(GATE && p.z ? static_cast<const char *>(p.z) + xoff * TS : nullptr,
                              GATE && p.z ? p.L * p.D * TS : 0);
    const auto rB = make_rsrc(static_cast<const char *>(p.Bm) + b * p.sb * TS, p.L * p.st * TS);
    const auto rC = make_rsrc(static_cast<const char *>(p.Cm) + b * p.sb * TS, p.L * p.st * TS);
    const auto rh = make_rsrc(p.hist ? p.hist + xoff * p.N : nullptr, HIST ? p.L * p.D * p.N * 4 : 0);
    const int vx = dc * TS;                             // lane byte offset in an x row
    const int rowx = Dm * TS;                           // bytes per x row
    const int rowbc = static_cast<int>(p.st) * TS;      // bytes per B/C row
    const int vbc = SHARED ? 0 : (dc * static_cast<int>(p.sd) + ns) * TS;
    const int vh = (dc * N + ns) * 4;
    // Lanes that own no output store at an offset with bit 31 set, past every
    // window, which the range check drops: the stores need no branch.
    constexpr unsigned kDrop = 0x80000000u;
    const unsigned vy = store_y ? static_cast<unsigned>(vx) : kDrop;
    const unsigned vy2 = dvalid ? static_cast<unsigned>(vx + ns * Dm * TS) : kDrop;   // paired steps
    // Row t of a window with rb bytes per row at lane offset v, all in the
    // range-checked VGPR offset: rows past L load 0 and their stores drop.
    // (Wave-uniform row offsets in the SGPR offset measured slower on gfx950:
    // the clamp and multiply they need per access cost issue slots of the
    // wave, which issue rate limits this kernel more than VALU throughput.
    // With whole super-chunks and the step's row in a loop-invariant SGPR
    // offset, one add per chunk, the kernel still ran 146.3 us against
    // 143.2 us at configs[1], with 2 % fewer VALU instructions.)
    auto ld_row = [&](__amdgpu_buffer_rsrc_t r, int v, int t, int rb) -> float {
        return IO::ld(r, v + t * rb, 0);
    };
    auto st_row = [&](__amdgpu_buffer_rsrc_t r, unsigned v, int t, int rb, float val) {
        IO::st(r, static_cast<int>(v + static_cast<unsigned>(t * rb)), 0, val);
    };
    const unsigned vhs = dvalid ? static_cast<unsigned>(vh) : kDrop;

    __shared__ float sB[SHARED ? 3 : 1][SHARED ? TILE : 1];
    __shared__ float sC[SHARED ? 3 : 1][SHARED ? TILE : 1];
    // Chunk maps and incoming states are written between two barriers and
    // read before the next write can start, so one buffer each suffices; the
    // carry is read and rewritten in the same phase and keeps two.
    __shared__ float aggP[W][NPL][64];
    __shared__ float aggH[W][NPL][64];
    __shared__ float carry[2][NPL][64];
    __shared__ float pin[W][NPL][64];       // incoming state of each wave

    // A lane holds the states n = NS*j + ns of its channel (interleaved over
    // the lane groups), so the structured decays below form one chain.
    float Ap[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) Ap[j] = p.A[dc * N + NS * j + ns] * kLog2e;
    const float A0p = p.A[dc * N] * kLog2e;
    // Structured decays (A[d,n] == (n+1)*A[d,0] for every state of every
    // channel of the workgroup) switch exp per state for a power chain.
    bool structured = true;
#pragma unroll
    for (int j = 0; j < NPL; ++j)
        structured = structured &&
                     (p.A[dc * N + NS * j + ns] == static_cast<float>(NS * j + ns + 1) * p.A[dc * N]);
    const bool fast = __builtin_amdgcn_readfirstlane(__syncthreads_and(structured)) != 0;

    if (w == 0) {
#pragma unroll
        for (int j = 0; j < NPL; ++j)
            carry[0][j][lane] = p.h0 ? p.h0[(b * Dm + dc) * N + NS * j + ns] : 0.f;
    }

    // B/C tile of super-chunk s: element e = (step, state) at row s*SC + e/N.
    float rb[TPT], rc[TPT];
    auto load_tile = [&](int s) {
#pragma unroll
        for (int i = 0; i < TPT; ++i) {
            const int e = tid + i * NT;
            const int t = s * SC + e / N;
            const int off = (e % N) * TS;
            const int so = t * rowbc;
            rb[i] = IO::ld(rB, off + so, 0);   // e >= TILE: a row the store skips
            rc[i] = IO::ld(rC, off + so, 0);
        }
    };
    // Tile element e = (step e/N, state n = e%N) is stored at
    // step*N + (n%NS)*NPL + n/NS: a lane's interleaved states are contiguous.
    auto store_tile = [&](int slot) {
#pragma unroll
        for (int i = 0; i < TPT; ++i) {
            const int e = tid + i * NT;
            if (e < TILE) {
                const int n = e % N;
                const int o = (e / N) * N + (n % NS) * NPL + n / NS;
                sB[slot][o] = rb[i];
                sC[slot][o] = rc[i];
            }
        }
    };
    auto load_xd = [&](int s, float (&xo)[TC], float (&dto)[TC], float (&zo)[ZC]) {
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const int t = s * SC + w * TC + k;   // rows past L read as 0
            xo[k] = ld_row(rx, vx, t, rowx);
            dto[k] = ld_row(rdt, vx, t, rowx);
            // z is 0 when null; with paired gating, step 2i + ns of this half.
            if constexpr (PAIRG) {
                if (k % 2 == 0) zo[k / 2] = ld_row(rz, vx + ns * rowx, t, rowx);
            } else if constexpr (GATE) {
                zo[k] = ld_row(rz, vx, t, rowx);
            }
        }
    };
    auto bc_row = [&](const float (*tile)[SHARED ? TILE : 1], __amdgpu_buffer_rsrc_t r, int slot,
                      int s, int k, float (&out)[NPL]) {
        if constexpr (SHARED) {
            const float *row = &tile[slot][(w * TC + k) * N + n0];
#pragma unroll
            for (int j = 0; j < NPL; ++j) out[j] = row[j];
        } else {
            const int t = s * SC + w * TC + k;
#pragma unroll
            for (int j = 0; j < NPL; ++j) out[j] = ld_row(r, vbc + j * NS * TS, t, rowbc);
        }
    };

    // Prefetches are issued unconditionally: rows past L read as 0 through
    // the range check. A load under a branch would make the compiler's
    // wait-count merge at the join wait for it before the current data is
    // used, exposing one HBM latency per super-chunk.
    if constexpr (SHARED) {
        load_tile(0);
        store_tile(0);
        load_tile(1);
    }
    float X0[TC], D0[TC], X1[TC], D1[TC];
    float Z0[ZC], Z1[ZC];
    load_xd(0, X0, D0, Z0);
    __syncthreads();

    float h[NPL];
    float hmax = 0.f;
    bool nan_seen = false;
    float dtot = 0.f;      // DSUM: this wave's sum of delta over the sequence

    // FASTC selects the structured-decay form at compile time, so each body
    // is straight-line code the scheduler can interleave across steps.
    auto body = [&](auto fastc, int s, float (&xs)[TC], float (&ds)[TC], float (&zs)[ZC],
                    float (&xn)[TC], float (&dn)[TC], float (&zn)[ZC]) __attribute__((always_inline)) {
        constexpr bool FAST = decltype(fastc)::value;
        const int cur = s & 1;
        const int slot = s % 3;
        if constexpr (SHARED) {
            store_tile((s + 1) % 3);     // tile s+1 -> LDS (slot last read in s-2)
            load_tile(s + 2);
        }
        load_xd(s + 1, xn, dn, zn);

        // Local pass from a zero state; decays (and optionally B*u) kept for
        // the replay.
        float e[TC][NPL];
        float bus[STORE_BU ? TC : 1][NPL];
        // The first step starts from zero: hl = B*u and dsum = delta, with no
        // fma(e, 0, .) (which the compiler may not fold: e*0 is NaN for e
        // inf or NaN).
        float hl[NPL];
        float dsum = 0.f;
        float bln[NPL];
        bc_row(sB, rB, slot, s, 0, bln);
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            float bv[NPL];
#pragma unroll
            for (int j = 0; j < NPL; ++j) bv[j] = bln[j];
            if (k + 1 < TC) bc_row(sB, rB, slot, s, k + 1, bln);
            const float u = ds[k] * xs[k];
            dsum = (k == 0) ? ds[0] : dsum + ds[k];
            if constexpr (FAST) {
                pow_chain_il<NPL, NS>(exp2_fast(ds[k] * A0p), ns, e[k]);
            } else {
#pragma unroll
                for (int j = 0; j < NPL; ++j) e[k][j] = exp2_fast(ds[k] * Ap[j]);
            }
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
                const float bu = bv[j] * u;
                if constexpr (STORE_BU) bus[k][j] = bu;
                hl[j] = (k == 0) ? bu : fmaf(e[k][j], hl[j], bu);
            }
        }
        if constexpr (DSUM) dtot += dsum;
        float P[NPL];
        if constexpr (FAST) {
            pow_chain_il<NPL, NS>(exp2_fast(dsum * A0p), ns, P);
        } else {
#pragma unroll
            for (int j = 0; j < NPL; ++j) P[j] = exp2_fast(Ap[j] * dsum);
        }
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            aggP[w][j][lane] = P[j];
            aggH[w][j][lane] = hl[j];
        }
        __syncthreads();

        // Balanced prefix over the W chunk maps: thread (w, lane) scans the
        // states j = w, w+W, ... of its lane across all waves, writing each
        // wave's incoming state and the super-chunk's outgoing carry.
        for (int j = w; j < NPL; j += W) {
            float pv[W], hv[W];
#pragma unroll
            for (int v = 0; v < W; ++v) {
                pv[v] = aggP[v][j][lane];
                hv[v] = aggH[v][j][lane];
            }
            float run = carry[cur][j][lane];
#pragma unroll
            for (int v = 0; v < W; ++v) {
                pin[v][j][lane] = run;
                run = fmaf(pv[v], run, hv[v]);
                // Checkpoint after every kCkptSteps-th step (rows past L are
                // identity steps, so a checkpoint past the end holds the
                // final state). Launches with checkpoints use super-chunks
                // that are multiples of kCkptSteps.
                if (((v + 1) * TC) % kCkptSteps == 0) {   // folded after unrolling
                    const long c = (static_cast<long>(s) * SC + (v + 1) * TC) / kCkptSteps - 1;
                    if (p.ckpt && dvalid && c < p.nck)
                        p.ckpt[((b * p.nck + c) * Dm + d) * N + NS * j + ns] = run;
                }
            }
            carry[cur ^ 1][j][lane] = run;
        }
        __syncthreads();
        // The segment-map pass (DSUM) needs only the outgoing carry: no replay.
        if constexpr (DSUM) return;
#pragma unroll
        for (int j = 0; j < NPL; ++j) h[j] = pin[w][j][lane];

        // Replay from the exact incoming state; B/C rows of step k+1 are read
        // while step k computes.
        float bvn[NPL], cvn[NPL];
        float yprev = 0.f;
        if constexpr (!STORE_BU) bc_row(sB, rB, slot, s, 0, bvn);
        bc_row(sC, rC, slot, s, 0, cvn);
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const int t = s * SC + w * TC + k;
            float bv[NPL], cv[NPL];
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
                bv[j] = bvn[j];
                cv[j] = cvn[j];
            }
            if (k + 1 < TC) {
                if constexpr (!STORE_BU) bc_row(sB, rB, slot, s, k + 1, bvn);
                bc_row(sC, rC, slot, s, k + 1, cvn);
            }
            const float u = ds[k] * xs[k];
            float yp = 0.f;
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
                const float bu = STORE_BU ? bus[k][j] : bv[j] * u;
                h[j] = fmaf(e[k][j], h[j], bu);
                yp = fmaf(cv[j], h[j], yp);
                hmax = fmaxf(hmax, fabsf(h[j]));
            }
            // Sum the state groups of this channel (lanes dl + DL*ns). Rows
            // past L and lanes without output are dropped by the range check.
            if constexpr (NS >= 4) yp = sum_xor16(yp);
            if constexpr (PAIR) {
                if (k % 2 == 0) {
                    yprev = yp;
                } else {
                    // One swap trades the upper half of step k-1's partial
                    // sums for the lower half of step k's: the sum is step
                    // k-1's readout in the lower half and step k's in the
                    // upper half, each added in the order of sum_xor32.
                    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(yprev), __float_as_uint(yp),
                                                                    false, false);
                    const float yv = __uint_as_float(r[0]) + __uint_as_float(r[1]);
                    if constexpr (GATE) {
                        const float xv = ns ? xs[k] : xs[k - 1];
                        st_row(ry, vy2, t - 1, rowx, gated<T>(p, yv, xv, dsk, zs[k / 2]));
                    } else {
                        st_row(ry, vy2, t - 1, rowx, yv);
                    }
                }
            } else {
                if constexpr (NS >= 2) yp = sum_xor32(yp);
                if constexpr (GATE) st_row(ry, vy, t, rowx, gated<T>(p, yp, xs[k], dsk, zs[k]));
                else st_row(ry, vy, t, rowx, yp);
            }
            if constexpr (HIST) {
#pragma unroll
                for (int j = 0; j < NPL; ++j)
                    bio<f32_t>::st(rh, static_cast<int>(vhs + static_cast<unsigned>(j * NS * 4 + t * Dm * N * 4)),
                                   0, h[j]);
            }
        }
    };

    auto run = [&](auto fastc) __attribute__((always_inline)) {
        for (int s = 0; s < nit; s += 2) {
            body(fastc, s, X0, D0, Z0, X1, D1, Z1);
            if (s + 1 < nit) body(fastc, s + 1, X1, D1, Z1, X0, D0, Z0);
        }
    };
    if (fast) run(std::true_type{});
    else run(std::false_type{});

    if constexpr (DSUM) {
        // Sum of delta over the sequence: the waves' partial sums in wave
        // order (aggP is free once every wave is past the last super-chunk).
        if constexpr (W > 1) {
            __syncthreads();
            aggP[w][0][lane] = dtot;
            __syncthreads();
            if (w == 0) {
                dtot = aggP[0][0][lane];
#pragma unroll
                for (int i = 1; i < W; ++i) dtot += aggP[i][0][lane];
            }
        }
        if (w == 0 && dvalid && ns == 0) p.dsum_out[b * Dm + d] = dtot;
    }

    if constexpr (DSUM) {
        // The segment's local end state is the last super-chunk's outgoing
        // carry (the segment-map pass runs without the clamp).
        if (w == W - 1 && p.hfin && dvalid) {
#pragma unroll
            for (int j = 0; j < NPL; ++j) p.hfin[(b * Dm + d) * N + NS * j + ns] = carry[nit & 1][j][lane];
        }
        return;
    }
    // A NaN state stays NaN through every later step (e * NaN + bu), so a
    // NaN anywhere in the sequence shows in the final state of the wave that
    // ran the last steps; finite excursions past 1000 are in hmax.
#pragma unroll
    for (int j = 0; j < NPL; ++j) nan_seen |= !(fabsf(h[j]) <= 1000.f);
    const int bad = p.clamp && (nan_seen || hmax > 1000.f);
    if (__syncthreads_or(bad)) {
        if (p.clamp_flag) {
            // A segment of a split sequence: states entering later segments
            // are also off, so the whole sequence is re-run by the repair.
            if (tid == 0) p.clamp_flag[(b / p.nseg) * ngroups + grp] = 1;
            return;
        }
        // The sequential pass keeps each lane's states contiguous
        // (n = n0 + j) and writes every output itself.
        if (w == 0) {
            float Apc[NPL];
#pragma unroll
            for (int j = 0; j < NPL; ++j) Apc[j] = p.A[dc * N + n0 + j] * kLog2e;
            scan1d_serial_wave<T, NPL, NS, SHARED, HIST>(p, b, d, dvalid, n0, Apc);
        }
        return;
    }
    if (w == W - 1 && p.hfin && dvalid) {
#pragma unroll
        for (int j = 0; j < NPL; ++j) p.hfin[(b * Dm + d) * N + NS * j + ns] = h[j];
    }
}

// Fallback for state sizes without a register-blocked instantiation
// (N not in {1, 2, 4, 8, 16}, N <= 64): one thread per (batch, channel), the
// reference's sequential step order with the per-step clamp.
template <typename T, bool HIST>
__global__ void __launch_bounds__(256) scan1d_fwd_serial(Scan1DFwdArgs p) {
    using IO = io<T>;
    const long gid = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= p.B * p.D) return;
    const long b = gid / p.D, d = gid % p.D;
    const long N = p.N;
    float st[64];
    for (long m = 0; m < N; ++m) st[m] = p.h0 ? p.h0[(b * p.D + d) * N + m] : 0.f;
    for (long t = 0; t < p.L; ++t) {
        const long xi = (b * p.L + t) * p.D + d;
        const float xv = IO::ld(p.x, xi), dv = IO::ld(p.dt, xi);
        const long bc = b * p.sb + t * p.st + d * p.sd;
        float y = 0.f;
        for (long m = 0; m < N; ++m) {
            const float e = exp2_fast(dv * p.A[d * N + m] * kLog2e);
            const float dB = __fmul_rn(IO::ld(p.Bm, bc + m), dv);
            float hn = __fadd_rn(__fmul_rn(e, st[m]), __fmul_rn(dB, xv));
            if (p.clamp) {
                hn = (hn < 1000.f) ? hn : 1000.f;
                hn = (hn > -1000.f) ? hn : -1000.f;
            }
            st[m] = hn;
            if (HIST) p.hist[xi * N + m] = hn;
            if (p.ckpt && ((t + 1) % kCkptSteps == 0 || t == p.L - 1))
                p.ckpt[((b * p.nck + t / kCkptSteps) * p.D + d) * N + m] = hn;
            y = __fadd_rn(y, __fmul_rn(IO::ld(p.Cm, bc + m), hn));
        }
        if (p.y) {
            const float zv = p.z ? IO::ld(p.z, xi) : 0.f;
            IO::st(p.y, xi, gated<T>(p, y, xv, p.Dskip ? p.Dskip[d] : 0.f, zv));
        }
    }
    if (p.hfin)
        for (long m = 0; m < N; ++m) p.hfin[(b * p.D + d) * N + m] = st[m];
}

template <typename T, int NPL, int NS, int W, int TC, bool SBU = false, int OCC = 2>
static int launch_chunked(const Scan1DFwdArgs &a, bool shared, bool hist, hipStream_t s) {
    const long DL = 64 / NS;
    const long grid = a.B * ((a.D + DL - 1) / DL);
    if (grid <= 0 || grid > 0x7fffffffL) {
        set_error("km_scan1d_fwd: grid of %ld workgroups out of range", grid);
        return -1;
    }
    dim3 g(static_cast<unsigned>(grid)), blk(64 * W);
    const bool gate = a.z || a.Dskip;
    // B*u is kept in registers only without history stores or gating, whose
    // extra registers would otherwise spill.
#define KM_CH(SH, HI, GA) \
    hipLaunchKernelGGL((scan1d_fwd_chunked<T, NPL, NS, W, TC, SH, HI, SBU && !HI && !GA, OCC, GA>), \
                       g, blk, 0, s, a)
    if (shared) {
        if (hist) { if (gate) KM_CH(true, true, true); else KM_CH(true, true, false); }
        else      { if (gate) KM_CH(true, false, true); else KM_CH(true, false, false); }
    } else {
        if (hist) { if (gate) KM_CH(false, true, true); else KM_CH(false, true, false); }
        else      { if (gate) KM_CH(false, false, true); else KM_CH(false, false, false); }
    }
#undef KM_CH
    KM_HIP_TRY(hipGetLastError());
    return 0;
}

// Tuning knob for N = 16 (KM_SCAN1D_CFG, read once): 0 = 32 channels x 2
// state halves, 8 waves, 8 steps per wave, B*u recomputed in the replay;
// any other value (default) = the same with B*u kept in registers.
static int scan1d_cfg16() {
    static int cfg = [] {
        const char *e = std::getenv("KM_SCAN1D_CFG");
        return e ? std::atoi(e) : 6;
    }();
    return cfg;
}

template <typename T>
static int launch_n16(const Scan1DFwdArgs &a, bool shared, bool hist, hipStream_t s) {
    // Checkpoints are written at 32-step boundaries inside 64-step super-chunks.
    if (!a.ckpt && scan1d_cfg16() == 0) return launch_chunked<T, 8, 2, 8, 8>(a, shared, hist, s);
    return launch_chunked<T, 8, 2, 8, 8, true>(a, shared, hist, s);
}

// ---------------------------------------------------------------------------
// Sequences split over workgroups (few (batch, channel group) pairs, long L):
// segment s of batch element b is "batch element" b*S + s of a [B*S, Ls, .]
// view of the same buffers. (1) the chunked kernel runs every segment from a
// zero state, writing its local end state hl and its sum of delta; (2)
// scan1d_segment_fold forms each segment's incoming state
// h_in[s+1] = exp(A * sum delta over s) h_in[s] + hl[s] (and the final
// state); (3) the chunked kernel replays every segment from its incoming
// state, writing y. With the per-step clamp, a
// segment whose states leave [-1000, 1000] flags its (batch, group) and
// scan1d_clamp_repair re-runs that whole sequence with the sequential
// clamped recurrence.
// ---------------------------------------------------------------------------

// One thread per (batch, channel, state) of N = 16 states: the fold over
// at most kMaxSegments segments, h_in[s+1] = exp(A * dsum[s]) h_in[s] + hl[s].
// Every segment's operands are loaded before the arithmetic (they do not
// depend on the state), so the kernel waits for memory once, not once per
// segment. Also zeroes the clamp flags.
constexpr int kMaxSegments = 64;
__global__ void __launch_bounds__(256) scan1d_segment_fold(const float *A, const float *h0,
                                                           const float *hl, const float *dsum,
                                                           float *hin, float *hfin, int *flags,
                                                           long nflags, long B, long D, int nseg) {
    constexpr int N = 16;
    const long gid = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid < nflags) flags[gid] = 0;
    if (gid >= B * D * N) return;
    const long bd = gid / N, n = gid - bd * N;
    const long b = bd / D, d = bd - b * D;
    const long base = b * nseg;                      // segment sg is row base + sg of [B*S, D, N]
    float ds[kMaxSegments], hv[kMaxSegments];
#pragma unroll
    for (int sg = 0; sg < kMaxSegments; ++sg) {
        if (sg < nseg) {
            ds[sg] = dsum[(base + sg) * D + d];
            hv[sg] = hl[((base + sg) * D + d) * N + n];
        }
    }
    const float a2 = A[d * N + n] * kLog2e;
    float h = h0 ? h0[gid] : 0.f;                    // h0 is [B, D, N]: index gid
#pragma unroll
    for (int sg = 0; sg < kMaxSegments; ++sg) {
        if (sg < nseg) {
            hin[((base + sg) * D + d) * N + n] = h;
            h = fmaf(exp2_fast(ds[sg] * a2), h, hv[sg]);
        }
    }
    if (hfin) hfin[gid] = h;
}

// Re-runs every flagged (batch, channel group) sequence from its start with
// the sequential clamped recurrence (wave 0 of a one-wave workgroup per
// pair), writing y, the history and the final state over the segmented
// results; unflagged pairs exit at once.
template <typename T, int NPL, int NS, bool SHARED, bool HIST>
__global__ void __launch_bounds__(64) scan1d_clamp_repair(Scan1DFwdArgs p, const int *flags) {
    constexpr int DL = 64 / NS;
    const long ngroups = (p.D + DL - 1) / DL;
    if (flags[blockIdx.x] == 0) return;
    const int lane = threadIdx.x & 63;
    const long b = blockIdx.x / ngroups;
    const long d = (blockIdx.x - b * ngroups) * DL + lane % DL;
    const bool dvalid = d < p.D;
    const int n0 = (lane / DL) * NPL;
    const long dc = dvalid ? d : p.D - 1;
    float Apc[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) Apc[j] = p.A[dc * p.N + n0 + j] * kLog2e;
    scan1d_serial_wave<T, NPL, NS, SHARED, HIST>(p, b, d, dvalid, n0, Apc);
}

// Segment length override (KM_SCAN1D_SPLIT, read once): 0 never splits, a
// multiple of 64 that divides L is used as the segment length, unset (or any
// other value) leaves the choice to segment_length's cost model.
static long scan1d_split_override() {
    static const long v = [] {
        const char *e = std::getenv("KM_SCAN1D_SPLIT");
        return e ? std::atol(e) : -1L;
    }();
    return v;
}

// Segment length for a split launch, or 0 to run unsplit. Only N = 16 and
// layouts whose batch stride is the sequence's (the [B*S, Ls, .] view),
// without checkpoints, when the unsplit grid leaves CUs idle. The model,
// from gfx950 timings of the 8-wave kernel with one workgroup per CU: a
// launch of n workgroups over Ls steps takes (4 + 2.1 ceil(Ls/64))
// ceil(n/256) us; a split runs two such launches over S = L/Ls segments of
// B*groups*S workgroups, plus ~6 us for the fold and the clamp check. The
// split is taken when the best segment length beats the unsplit launch by
// 15 %.
static long segment_length(const KMScan1DFwd *k, long groups_total) {
    if (k->N != 16 || k->h_ckpt || groups_total >= 128 || k->L % 64 != 0 || k->L < 128) return 0;
    if (k->B > 1 && k->bc_sb != k->L * k->bc_st) return 0;
    const long ov = scan1d_split_override();
    if (ov == 0) return 0;
    if (ov > 0)
        return (ov % 64 == 0 && ov < k->L && k->L % ov == 0 && k->L / ov <= kMaxSegments) ? ov : 0;
    auto launch_us = [](long steps, long wgs) {
        return (4.0 + 2.1 * static_cast<double>((steps + 63) / 64)) *
               static_cast<double>((wgs + 255) / 256);
    };
    const double unsplit = launch_us(k->L, groups_total);
    double best_t = 0.85 * unsplit;
    long best = 0;
    for (long ls = 64; ls < k->L; ls += 64) {
        if (k->L % ls != 0 || k->L / ls > kMaxSegments) continue;
        const double t = 2.0 * launch_us(ls, groups_total * (k->L / ls)) + 6.0;
        if (t < best_t) {
            best_t = t;
            best = ls;
        }
    }
    return best;
}

// Segment workgroups have the unsplit kernel's shape: 8 waves of 8 steps
// (64-step super-chunks).
template <typename T>
static int launch_segmented(const KMScan1DFwd *k, long Ls, hipStream_t s) {
    constexpr int NPL = 8, NS = 2, DL = 32, WS = 8;
    const long S = k->L / Ls;
    const long groups = (k->D + DL - 1) / DL;
    const long BS = k->B * S;
    const size_t st = align_up(sizeof(float) * BS * k->D * k->N, 256);
    const size_t sd = align_up(sizeof(float) * BS * k->D, 256);
    char *ws = static_cast<char *>(Workspace::reserve(2 * st + sd + align_up(4 * k->B * groups, 256), s, WsUse::Scan1DSplit));
    if (!ws) return -1;
    float *hl = reinterpret_cast<float *>(ws);
    float *hin = reinterpret_cast<float *>(ws + st);
    float *dsum = reinterpret_cast<float *>(ws + 2 * st);
    int *flags = reinterpret_cast<int *>(ws + 2 * st + sd);
    const long grid = BS * groups;
    if (grid > 0x7fffffffL) {
        set_error("km_scan1d_fwd: grid of %ld workgroups out of range", grid);
        return -1;
    }
    const bool shared = (k->bc_sd == 0), hist = (k->h_hist != nullptr);
    const bool gate = k->z || k->Dskip;
    // (1) local end states and delta sums of every segment, from zero
    Scan1DFwdArgs a{k->x, k->delta, k->A, k->Bm, k->Cm, nullptr, nullptr, hl, nullptr, nullptr, 1,
                    nullptr, nullptr, BS, Ls, k->D, k->N, Ls * k->bc_st, k->bc_st, k->bc_sd, 0,
                    nullptr, S, dsum};
#define KM_SEG(SH, HI, GA, BU) \
    hipLaunchKernelGGL((scan1d_fwd_chunked<T, NPL, NS, WS, 8, SH, HI, BU, 2, GA, true>), dim3(grid), dim3(64 * WS), 0, s, a)
    if (shared) KM_SEG(true, false, false, true); else KM_SEG(false, false, false, true);
    KM_HIP_TRY(hipGetLastError());
    // (2) incoming state of every segment, the final state, flags cleared
    const long nth = k->B * k->D * k->N;      // >= B * groups flags
    hipLaunchKernelGGL(scan1d_segment_fold, dim3((nth + 255) / 256), dim3(256), 0, s, k->A, k->h0,
                       static_cast<const float *>(hl), static_cast<const float *>(dsum), hin,
                       k->h_final, flags, k->B * groups, k->B, k->D, static_cast<int>(S));
    KM_HIP_TRY(hipGetLastError());
    // (3) replay every segment from its incoming state
    Scan1DFwdArgs r{k->x, k->delta, k->A, k->Bm, k->Cm, k->y, hin, nullptr, k->h_hist, nullptr, 1,
                    k->z, k->Dskip, BS, Ls, k->D, k->N, Ls * k->bc_st, k->bc_st, k->bc_sd, k->clamp,
                    k->clamp ? flags : nullptr, S};
#define KM_SEGR(SH, HI, GA) \
    hipLaunchKernelGGL((scan1d_fwd_chunked<T, NPL, NS, WS, 8, SH, HI, !HI && !GA, 2, GA>), dim3(grid), dim3(64 * WS), 0, s, r)
    if (shared) {
        if (hist) { if (gate) KM_SEGR(true, true, true); else KM_SEGR(true, true, false); }
        else      { if (gate) KM_SEGR(true, false, true); else KM_SEGR(true, false, false); }
    } else {
        if (hist) { if (gate) KM_SEGR(false, true, true); else KM_SEGR(false, true, false); }
        else      { if (gate) KM_SEGR(false, false, true); else KM_SEGR(false, false, false); }
    }
#undef KM_SEGR
#undef KM_SEG
    KM_HIP_TRY(hipGetLastError());
    if (k->clamp) {
        // (4) flagged sequences again, sequentially with the clamp
        Scan1DFwdArgs q{k->x, k->delta, k->A, k->Bm, k->Cm, k->y, k->h0, k->h_final, k->h_hist, nullptr,
                        1, k->z, k->Dskip, k->B, k->L, k->D, k->N, k->bc_sb, k->bc_st, k->bc_sd, 1,
                        nullptr, 1};
        const dim3 g2(static_cast<unsigned>(k->B * groups));
        if (shared) {
            if (hist) hipLaunchKernelGGL((scan1d_clamp_repair<T, NPL, NS, true, true>), g2, dim3(64), 0, s, q, flags);
            else      hipLaunchKernelGGL((scan1d_clamp_repair<T, NPL, NS, true, false>), g2, dim3(64), 0, s, q, flags);
        } else {
            if (hist) hipLaunchKernelGGL((scan1d_clamp_repair<T, NPL, NS, false, true>), g2, dim3(64), 0, s, q, flags);
            else      hipLaunchKernelGGL((scan1d_clamp_repair<T, NPL, NS, false, false>), g2, dim3(64), 0, s, q, flags);
        }
        KM_HIP_TRY(hipGetLastError());
    }
    return 0;
}

template <typename T>
static int launch_serial(const Scan1DFwdArgs &a, bool hist, hipStream_t s) {
    const long threads = a.B * a.D;
    const long grid = (threads + 255) / 256;
    if (grid > 0x7fffffffL) {
        set_error("km_scan1d_fwd: grid out of range");
        return -1;
    }
    if (hist) hipLaunchKernelGGL((scan1d_fwd_serial<T, true>), dim3(grid), dim3(256), 0, s, a);
    else      hipLaunchKernelGGL((scan1d_fwd_serial<T, false>), dim3(grid), dim3(256), 0, s, a);
    KM_HIP_TRY(hipGetLastError());
    return 0;
}

// allow_split = false keeps every shape on kernels that use no workspace
// (the allocation-free ScanND entry point's 1D grids).
int scan1d_fwd_launch(const KMScan1DFwd *k, hipStream_t stream, bool allow_split) {
    if (!k) { set_error("km_scan1d_fwd: NULL arguments"); return -1; }
    // With no steps (L = 0) only A, h0 and h_final take part.
    if (!k->A || (k->L > 0 && (!k->x || !k->delta || !k->Bm || !k->Cm))) {
        set_error("km_scan1d_fwd: NULL tensor pointer");
        return -1;
    }
    if (!k->y && !k->h_final && !k->h_hist && !k->h_ckpt) {
        set_error("km_scan1d_fwd: no output requested");
        return -1;
    }
    if (k->B <= 0 || k->L < 0 || k->D <= 0 || k->N <= 0 || k->N > 64) {
        set_error("km_scan1d_fwd: invalid sizes B=%ld L=%ld D=%ld N=%ld (need N <= 64)",
                  k->B, k->L, k->D, k->N);
        return -1;
    }
    if (k->dtype != KM_F32 && k->dtype != KM_BF16) {
        set_error("km_scan1d_fwd: unknown dtype %d", k->dtype);
        return -1;
    }
    if (!gpu_ready()) return -1;
    if (k->L == 0) {   // no steps: the final state is the initial state (no checkpoints)
        if (k->h_final && k->h_final != k->h0) {
            const size_t bytes = sizeof(float) * k->B * k->D * k->N;
            if (k->h0) KM_HIP_TRY(hipMemcpyAsync(k->h_final, k->h0, bytes, hipMemcpyDeviceToDevice, stream));
            else       KM_HIP_TRY(hipMemsetAsync(k->h_final, 0, bytes, stream));
        }
        return 0;
    }
    Scan1DFwdArgs a{k->x, k->delta, k->A, k->Bm, k->Cm, k->y, k->h0, k->h_final, k->h_hist,
                    k->h_ckpt, (k->L + kCkptSteps - 1) / kCkptSteps, k->z, k->Dskip,
                    k->B, k->L, k->D, k->N, k->bc_sb, k->bc_st, k->bc_sd, k->clamp, nullptr, 1};
    // The register-blocked kernel addresses each batch element's windows with
    // 32-bit byte offsets; larger problems take the sequential kernel.
    const long es = (k->dtype == KM_BF16) ? 2 : 4;
    const long lim = 0x3fffffffL;   // offsets reach (L + W*TC) rows
    const bool small_windows = k->L * k->D * es < lim && k->L * k->bc_st * es < lim &&
                               (!k->h_hist || k->L * k->D * k->N * 4 < lim) &&
                               k->bc_st >= 0 && k->bc_sd >= 0 && k->bc_sb >= 0;
    const bool shared = (k->bc_sd == 0);
    const bool hist = (k->h_hist != nullptr);
    const bool bf = (k->dtype == KM_BF16);
    if (!small_windows)
        return bf ? launch_serial<bf16_t>(a, hist, stream) : launch_serial<f32_t>(a, hist, stream);
    // Few (batch, channel group) pairs and a long sequence: split the
    // sequence over workgroups.
    if (const long Ls = allow_split ? segment_length(k, k->B * ((k->D + 31) / 32)) : 0)
        return bf ? launch_segmented<bf16_t>(k, Ls, stream) : launch_segmented<f32_t>(k, Ls, stream);
    switch (k->N) {
    case 16:
        return bf ? launch_n16<bf16_t>(a, shared, hist, stream)
                  : launch_n16<f32_t>(a, shared, hist, stream);
    case 8:
        if (!bf) return launch_chunked<f32_t, 8, 1, 8, 8>(a, shared, hist, stream);
        break;
    case 4:
        if (!bf) return launch_chunked<f32_t, 4, 1, 8, 8>(a, shared, hist, stream);
        break;
    case 2:
        if (!bf) return k->h_ckpt ? launch_chunked<f32_t, 2, 1, 8, 8>(a, shared, hist, stream)
                                  : launch_chunked<f32_t, 2, 1, 8, 16>(a, shared, hist, stream);
        break;
    case 1:
        if (!bf) return k->h_ckpt ? launch_chunked<f32_t, 1, 1, 8, 8>(a, shared, hist, stream)
                                  : launch_chunked<f32_t, 1, 1, 8, 16>(a, shared, hist, stream);
        break;
    default:
        break;
    }
    return bf ? launch_serial<bf16_t>(a, hist, stream) : launch_serial<f32_t>(a, hist, stream);
}

}  // namespace km

extern "C" {

int km_scan1d_fwd(const KMScan1DFwd *a, void *stream) {
    km::clear_error();
    return km::scan1d_fwd_launch(a, static_cast<hipStream_t>(stream), true);
}

// Reference cuda/scan1d.cu:258-310: B, C, h are [L, D, M]; h receives the
// whole state history; zero initial state; per-step clamp as on the CPU.
void om_scan1d_forward(const float *d_x, const float *d_A, const float *d_B, const float *d_C,
                       const float *d_dt, float *d_y, float *d_h, int L, int D, int M) {
    km::clear_error();
    if (L < 0 || D <= 0 || M <= 0) {
        km::set_error("om_scan1d_forward: invalid sizes L=%d D=%d M=%d", L, D, M);
        return;
    }
    KMScan1DFwd a{};
    a.x = d_x; a.delta = d_dt; a.A = d_A; a.Bm = d_B; a.Cm = d_C; a.y = d_y;
    a.h0 = nullptr; a.h_final = nullptr; a.h_hist = d_h;
    a.B = 1; a.L = L; a.D = D; a.N = M;
    a.bc_sb = static_cast<long>(L) * D * M; a.bc_st = static_cast<long>(D) * M; a.bc_sd = M;
    a.dtype = KM_F32; a.clamp = 1;
    if (km::scan1d_fwd_launch(&a, nullptr, true) != 0) return;
    if (hipStreamSynchronize(nullptr) != hipSuccess)
        km::set_error("om_scan1d_forward: %s", hipGetErrorString(hipGetLastError()));
}

void mamba_scan1d_cuda_forward(const float *d_x, const float *d_A, const float *d_B,
                               const float *d_C, const float *d_dt, float *d_y, float *d_h,
                               int L, int D, int M) {
    om_scan1d_forward(d_x, d_A, d_B, d_C, d_dt, d_y, d_h, L, D, M);
}

// Reference scan1d (cpu/scan1d.asm:40-179): host or device pointers; h is
// the running [D, M] state (read, then overwritten with the final state).
void scan1d(ScanParams *p) {
    km::clear_error();
    if (!p || !p->x || !p->A || !p->B || !p->C || !p->delta || !p->h || !p->y ||
        p->L < 0 || p->D <= 0 || p->M <= 0) {
        km::set_error("scan1d: invalid parameters");
        return;
    }
    if (!km::gpu_ready()) return;
    const long L = p->L, D = p->D, M = p->M;
    const size_t nLD = L * D, nDM = D * M, nLDM = L * D * M;
    KMScan1DFwd a{};
    a.B = 1; a.L = L; a.D = D; a.N = M;
    a.bc_sb = nLDM; a.bc_st = D * M; a.bc_sd = M;
    a.dtype = KM_F32; a.clamp = 1;
    const bool dev = km::is_device_ptr(p->x) && km::is_device_ptr(p->y) &&
                     km::is_device_ptr(p->B) && km::is_device_ptr(p->C) &&
                     km::is_device_ptr(p->delta) && km::is_device_ptr(p->A) &&
                     km::is_device_ptr(p->h);
    if (dev) {
        a.x = p->x; a.delta = p->delta; a.A = p->A; a.Bm = p->B; a.Cm = p->C; a.y = p->y;
        a.h0 = p->h; a.h_final = p->h;
        if (km::scan1d_fwd_launch(&a, nullptr, true) == 0 && hipStreamSynchronize(nullptr) != hipSuccess)
            km::set_error("scan1d: %s", hipGetErrorString(hipGetLastError()));
        return;
    }
    km::Staging::lock();
    const size_t bytes = sizeof(float) * (3 * nLD + nDM * 2 + 2 * nLDM) + 8 * 256;
    void *base = km::Staging::reserve(bytes);
    if (base) {
        km::Carver c(base);
        float *x = c.take<float>(nLD), *dt = c.take<float>(nLD), *y = c.take<float>(nLD);
        float *A = c.take<float>(nDM), *h = c.take<float>(nDM);
        float *Bm = c.take<float>(nLDM), *Cm = c.take<float>(nLDM);
        bool ok = km::copy_h2d(x, p->x, nLD * 4) == hipSuccess &&
                  km::copy_h2d(dt, p->delta, nLD * 4) == hipSuccess &&
                  km::copy_h2d(A, p->A, nDM * 4) == hipSuccess &&
                  km::copy_h2d(h, p->h, nDM * 4) == hipSuccess &&
                  km::copy_h2d(Bm, p->B, nLDM * 4) == hipSuccess &&
                  km::copy_h2d(Cm, p->C, nLDM * 4) == hipSuccess;
        if (!ok) {
            km::set_error("scan1d: host-to-device copy failed");
        } else {
            a.x = x; a.delta = dt; a.A = A; a.Bm = Bm; a.Cm = Cm; a.y = y; a.h0 = h; a.h_final = h;
            if (km::scan1d_fwd_launch(&a, nullptr, true) == 0) {
                if (km::copy_d2h(p->y, y, nLD * 4) != hipSuccess ||
                    km::copy_d2h(p->h, h, nDM * 4) != hipSuccess)
                    km::set_error("scan1d: device-to-host copy failed");
            }
        }
    }
    km::Staging::unlock();
}

void mamba_scan1d_forward(MambaScan1DParams *p) { scan1d(p); }

}  // extern "C"

// scan1d_bwd.hip - Scan1D selective-scan backward for gfx950.
//
// Adjoint of the forward recurrence in reverse time (reference
// cpu/scan1d_backward.c:248-295, per batch element):
//   e  = exp(delta*A[d,n]);  hp = state before step t;  ht = state after it
//   ah = adj + dy*C                         (dL/dh_t)
//   dC = dy*ht;  dB = ah*delta*x;  dA += ah*delta*e*hp
//   dx = sum_n ah*delta*B;  ddelta = sum_n ah*(A*e*hp + B*x)
//   adj = ah*e                              (handed to step t-1)
// The per-step clamp of the forward is not differentiated (as in the
// reference, which consumes the clamped states).
//
// Design (same lane layout as the forward kernel):
//  * A wave covers DL = 64/NS channels x NS groups of NPL states; a workgroup
//    of W waves owns one (batch, channel group) and walks the sequence
//    backwards in super-chunks of W*TC = 32 steps, one wave per TC steps.
//  * Forward states of a super-chunk are either read from the history or
//    recomputed from the 32-step checkpoint the forward wrote: local pass
//    from zero, chunk maps through LDS, fold, replay (as the forward).
//  * The adjoint is the same linear recurrence run backwards with the same
//    decays: g -> P*g + a over a wave's steps, so the chunk maps fold in
//    reverse order and each wave replays its steps from the exact incoming
//    adjoint, producing every gradient term in registers.
//  * dx and ddelta reduce over the states of a channel across lanes; dA
//    accumulates per lane over the sequence and the waves of a workgroup add
//    their sums in wave order. Shared B/C ([B, L, N], stride 0 over
//    channels) need dB, dC summed over channels: a per-wave LDS block of
//    rows and columns (N = 16) or a reduce-scatter over the wave's lanes
//    gives the wave's channel-group sum, stored to the workgroup's own
//    partial slot; a finalize kernel adds the slots of every channel group
//    (and dA's per-batch partials) in a fixed order. With N = 16, on grids
//    large enough to give every CU a workgroup, a workgroup runs two such
//    8-wave halves on 16 channels each and adds their sums in LDS, so its
//    slot covers 32 channels (half the slots to write and to sum). No
//    atomics: every output is identical run to run.
//  * States recomputed from checkpoints run unclamped; if any leaves
//    [-1000, 1000] the workgroup re-runs every super-chunk with the
//    sequential clamped recurrence, which matches the forward's clamp
//    fallback.
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "km_device.hpp"
#include "../km_runtime.hpp"
#include "kmamba_km.h"
#include "scan.h"
#include "mamba_scan.h"
#include "mamba_scan_cuda.h"

namespace km {

int scan1d_fwd_launch(const KMScan1DFwd *k, hipStream_t stream, bool allow_split);

struct Scan1DBwdArgs {
    const void *x, *dt, *dy;
    const float *A;
    const void *Bm, *Cm;
    const float *h0;       // [B, D, N] or null
    const float *hist;     // [B, L, D, N] state after each step, or null
    const float *ckpt;     // [B, nck, D, N] state after each 32-step block, or null
    long nck;
    void *dx, *ddt;        // [B, L, D]
    float *dApart;         // [B, D, N] per-batch dA partials (every element written)
    float *slot;           // shared B/C: [B, G, L, 2, N] per-channel-group partials (dB, dC)
    long G;                // channel groups per batch element (shared B/C slots)
    void *dB, *dC;         // per-channel B/C: written at the B/C strides
    long B, L, D, N, sb, st, sd;
    int clamp;
};

// v from the lane whose id differs in bit MASK: ds_swizzle inside 32-lane
// halves, ds_bpermute across them.
template <int MASK>
__device__ __forceinline__ float xor_lane(float v) {
    if constexpr (MASK >= 32) return __shfl_xor(v, 32);
    else return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (MASK << 10)));
}

// One exchange of the reduce-scatter below: while CNT values remain, keep
// half of them and add the partner's copy of that half; then butterfly.
template <int MASK, int CNT, int NV>
__device__ __forceinline__ void rs_step(float (&cur)[NV], int lane) {
    if constexpr (MASK >= 1) {
        if constexpr (CNT > 1) {
            constexpr int H = CNT / 2;
            const bool hi = (lane & MASK) != 0;
#pragma unroll
            for (int i = 0; i < H; ++i) {
                const float keep = hi ? cur[H + i] : cur[i];
                const float send = hi ? cur[i] : cur[H + i];
                cur[i] = keep + xor_lane<MASK>(send);
            }
            rs_step<MASK / 2, H>(cur, lane);
        } else {
            cur[0] += xor_lane<MASK>(cur[0]);
            rs_step<MASK / 2, 1>(cur, lane);
        }
    }
}

// Sums v[0..NV) over the DLN lanes of a lane's group (lanes sharing
// lane / DLN). Lane l ends with the total of value index (l % DLN) / (DLN / NV).
template <int NV, int DLN>
__device__ __forceinline__ float reduce_scatter(const float (&v)[NV], int lane) {
    static_assert(NV <= DLN && DLN <= 64, "reduce over at most 64 lanes");
    if constexpr (DLN == 16 && NV == 4) return row_readout<4>(v);   // DPP, no LDS swizzles
    float cur[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) cur[i] = v[i];
    rs_step<DLN / 2, NV>(cur, lane);
    return cur[0];
}

template <int NPL, int NS>
__device__ __forceinline__ void pow_chain_b(float e1, int n0, float (&e)[NPL]) {
    float pw = e1;
    if constexpr (NS > 1) {
        float sq = e1;
#pragma unroll
        for (int k = 1; k < NPL; k <<= 1) sq *= sq;
#pragma unroll
        for (int bit = NPL; bit < NPL * NS; bit <<= 1) {
            pw *= (n0 & bit) ? sq : 1.0f;
            sq *= sq;
        }
    }
    e[0] = pw;
#pragma unroll
    for (int j = 1; j < NPL; ++j) e[j] = e[j - 1] * e1;
}

// Register-blocked backward. A workgroup of W = 8 waves owns one (batch,
// channel group) and walks the sequence backwards in super-chunks of
// W * TC = 32 steps (the forward's checkpoint spacing), one wave per TC = 4
// steps. The launch bound keeps a wave within 128 VGPRs, so two workgroups
// share a CU and one's barriers and folds overlap the other's arithmetic.
// Per super-chunk, between two barriers:
//   A  decays, the forward local pass from a zero state and the adjoint
//      local pass (reverse) from a zero adjoint; their chunk maps (shared P)
//      go to LDS;
//   F  the forward fold from the checkpoint (waves 0..NPL-1, one state
//      each) and the adjoint fold from the carried adjoint (waves
//      NPL..2*NPL-1), writing each wave's incoming state and adjoint over
//      its own map in LDS; the folds also bound |h| over the super-chunk
//      for the clamp check;
//   R  the forward replay from the exact incoming state, then the adjoint
//      replay forming every gradient term.
// With N = 16 the shared dB / dC channel sums go through a per-wave LDS
// block: each step's products are written as rows, and every two steps
// each lane adds one (step, gradient, state) column over the wave's 16
// channels in channel order. Other N use the in-wave reduce-scatter.
// With HWT = 2 the workgroup is 16 waves, two halves of W = 8 on channels
// [32 g, +16) and [32 g + 16, +16) of the same steps: they share the
// staged B / C tiles and the barriers, keep their maps, folds and carries
// in their own halves of the LDS arrays (lane index lane + 64 * half), and
// leave their column sums in comb; after the next barrier each half adds
// the two halves' sums of one round of every wave's steps (half 0's first)
// and stores them to the slot. The LDS then holds one workgroup per CU
// (16 waves, as two 8-wave workgroups did).
template <typename T, int NPL, int NS, bool SHARED, bool HIN, int HWT>
__global__ void __launch_bounds__(HWT == 2 ? 1024 : 512, 4) scan1d_bwd_chunked(Scan1DBwdArgs p) {
    using IO = bio<T>;
    constexpr int W = 8, TC = 4;
    constexpr int DL = 64 / NS;
    constexpr int N = NPL * NS;
    constexpr int SC = W * TC;
    static_assert(SC == kCkptSteps, "backward super-chunks follow the forward checkpoints");
    static_assert(2 * NPL <= W, "one fold per wave");
    constexpr int TILE = SC * N;
    // HWT = 2 (LDS channel sums: N = 16, shared B/C): two halves of 8 waves
    // in one workgroup, each half on its own 16 channels; the halves' sums
    // are added in LDS, so a workgroup's slot covers 32 channels.
    constexpr int HW = HWT;
    static_assert(HW == 1 || (HW == 2 && SHARED && N == 16 && NS == 4), "two halves: LDS channel sums");
    constexpr int NT = 64 * W * HW;
    constexpr int TPT = (TILE + NT - 1) / NT;
    constexpr int TS = IO::size;
    // LDS channel sums (N = 16): RS = 2 steps per round, 2 gradients, 16
    // states: 64 sums, one per lane, each over the DL = 16 channels. A
    // (step, gradient) block holds, per state group ns, the NPL states of
    // every channel contiguously ([ns][dl][NPL], groups padded by 4 floats):
    // a wave's 128-bit row writes cover consecutive 16-byte words, and the
    // column reads of 16 lanes (states n) fall in 16 distinct banks, the
    // next 16 lanes' block 16 banks further (block size = 16 mod 32).
    // The rows hold the factors that vary with the state, ah for dB and h
    // for dC; the per-channel factors u = delta*x and dy of each step go to
    // a vector block RVEC ([step][gradient][channel]; the NS lanes of a
    // channel store the same value), and the column reader forms
    // sum_c row[c] * vec[c] with one fma per channel.
    constexpr bool LRED = SHARED && N == 16 && NS == 4;
    constexpr int RS = 2;
    constexpr int RGRP = DL * NPL + 4;
    constexpr int RBLK = NS * RGRP;
    constexpr int RVEC = RS * 2 * RBLK;                // vector block offset
    constexpr int RWAVE = LRED ? RVEC + RS * 2 * DL : 1;
    static_assert(!LRED || RBLK % 32 == 16, "block offset of the second gradient");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane((tid >> 6) & (W - 1));   // wave of the half
    const int hh = HW > 1 ? __builtin_amdgcn_readfirstlane(tid >> 9) : 0; // half
    // Lane index into the per-half LDS arrays ([..][64 * HW]): one address
    // register serves every array, as the lane alone does with one half.
    const int lh = lane + 64 * hh;
    const int dl = lane % DL;
    const int ns = lane / DL;
    const int n0 = ns * NPL;
    const long ngroups = (p.D + DL * HW - 1) / (DL * HW);
    // Workgroups numbered so that consecutive channel groups run on one
    // XCD: a group's DL channels are only part of each 128-byte row line
    // of x / delta / dy, and the neighbours that read the rest of the line
    // then find it in the same L2 instead of fetching it again.
    const long wg = xcd_remap(blockIdx.x, gridDim.x);
    const long b = wg / ngroups;
    const long grp = wg - b * ngroups;
    const long d = grp * DL * HW + hh * DL + dl;
    const bool dvalid = d < p.D;
    const int dc = static_cast<int>(dvalid ? d : p.D - 1);
    const int L = static_cast<int>(p.L);
    const int Dm = static_cast<int>(p.D);
    const int nit = (L + SC - 1) / SC;
    const bool own_x = dvalid && ns == 0;

    // Per-batch-element windows, 32-bit byte offsets in the VGPR offset (the
    // launcher keeps them below 1 GiB): rows past L load 0, stores drop.
    const long xoff = b * p.L * p.D;
    const long xbytes = p.L * p.D * TS;
    const auto rx = make_rsrc(static_cast<const char *>(p.x) + xoff * TS, xbytes);
    const auto rdt = make_rsrc(static_cast<const char *>(p.dt) + xoff * TS, xbytes);
    const auto rdy = make_rsrc(static_cast<const char *>(p.dy) + xoff * TS, xbytes);
    const auto rdx = make_rsrc(static_cast<char *>(p.dx) + xoff * TS, xbytes);
    const auto rdd = make_rsrc(static_cast<char *>(p.ddt) + xoff * TS, xbytes);
    const long bcbytes = p.L * p.st * TS;
    const auto rB = make_rsrc(static_cast<const char *>(p.Bm) + b * p.sb * TS, bcbytes);
    const auto rC = make_rsrc(static_cast<const char *>(p.Cm) + b * p.sb * TS, bcbytes);
    const auto rdB = make_rsrc(SHARED ? nullptr : static_cast<char *>(p.dB) + b * p.sb * TS,
                               SHARED ? 0 : bcbytes);
    const auto rdC = make_rsrc(SHARED ? nullptr : static_cast<char *>(p.dC) + b * p.sb * TS,
                               SHARED ? 0 : bcbytes);
    const auto rh = make_rsrc(HIN ? p.hist + xoff * p.N : nullptr, HIN ? p.L * p.D * p.N * 4 : 0);
    const int vx = dc * TS;
    const int rowx = Dm * TS;
    const int rowbc = static_cast<int>(p.st) * TS;
    const int vbc = SHARED ? 0 : (dc * static_cast<int>(p.sd) + n0) * TS;
    const int vh = (dc * N + n0) * 4;
    const int rowh = Dm * N * 4;
    // Output offsets of lanes that own no output get bit 31 set: past every
    // window, so the range check drops those stores without a branch.
    constexpr unsigned kDrop = 0x80000000u;
    constexpr int GRP = DL / NPL;   // lanes per reduced B/C gradient value (reduce-scatter)
    const unsigned vxs = own_x ? static_cast<unsigned>(vx) : kDrop;
    // x and dy of lanes past D load as 0: their dB / dC terms (ah*delta*x,
    // dy*h) vanish without a select, and every other output of such a lane
    // is dropped.
    const int vxz = static_cast<int>(dvalid ? static_cast<unsigned>(vx) : kDrop);
    const unsigned vbcs = dvalid ? static_cast<unsigned>(vbc) : kDrop;
    // This workgroup's partial slot of the shared dB / dC: [L, 2, N] of
    // [B, G, L, 2, N] (dB then dC of each step), one writer per element.
    const auto rslot = make_rsrc(SHARED ? p.slot + (b * p.G + grp) * p.L * 2 * N : nullptr,
                                 SHARED ? p.L * 2 * N * 4 : 0);
    // Reduce-scatter path: lane l holds state n0 + (l % DL) / GRP of step t.
    const unsigned vacc = (dl % GRP) == 0 ? static_cast<unsigned>((n0 + dl / GRP) * 4) : kDrop;
    // LDS path: lane l sums column (step ri, gradient gi, state ni) of a round.
    const int ri = lane >> 5, gi = (lane >> 4) & 1, ni = lane & 15;

    __shared__ float sB[SHARED ? 3 : 1][SHARED ? TILE : 1];
    __shared__ float sC[SHARED ? 3 : 1][SHARED ? TILE : 1];
    __shared__ float aggP[W][NPL][64 * HW];            // chunk decay products
    __shared__ float aggF[HIN ? 1 : W][NPL][64 * HW];  // forward maps, then incoming states
    __shared__ float aggA[W][NPL][64 * HW];            // adjoint maps, then incoming adjoints
    __shared__ float lmx[HIN ? 1 : W][64 * HW];        // max |local state| (inf: no bound)
    __shared__ float acar[2][NPL][64 * HW];            // adjoint carried between super-chunks
    __shared__ __align__(16) float red[LRED ? W * HW : 1][RWAVE];
    __shared__ float comb[HW > 1 ? W : 1][2][64 * HW]; // the halves' channel sums of a super-chunk
    __shared__ int s_bad;                              // some bound failed: clamped re-run

    // Decays exp2((delta * log2 e) * A): the first product once per step.
    float Ar[NPL];
    bool apos = false;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
        Ar[j] = p.A[dc * N + n0 + j];
        apos = apos || !(Ar[j] <= 0.f);
    }
    // Structured decays (A[d,n] == (n+1)*A[d,0], the S4D-real form) need
    // fewer exps: with N <= 8 one exp per step and a power chain where n0
    // is 0 or a power of two; with four state groups (N = 16) a second exp
    // gives each lane its first power e1^(n0+1), and the lane's other
    // states follow by multiplying with e1.
    bool structured = (NS == 4) || (n0 == 0 || (n0 & (n0 - 1)) == 0);
#pragma unroll
    for (int j = 0; j < NPL; ++j)
        structured = structured && (Ar[j] == static_cast<float>(n0 + j + 1) * p.A[dc * N]);
    const float A0p = p.A[dc * N] * kLog2e;
    const float Afp = static_cast<float>(n0 + 1) * A0p;   // log2 of the lane's first power
    const bool fast = __builtin_amdgcn_readfirstlane(__syncthreads_and(structured)) != 0;
    // Decays of one step (or of a sum of steps) of delta dv in the
    // structured form.
    auto decay_chain = [&](float dv, float (&out)[NPL]) __attribute__((always_inline)) {
        if constexpr (NS == 4) {
            const float e1 = exp2_fast(dv * A0p);
            out[0] = exp2_fast(dv * Afp);
#pragma unroll
            for (int j = 1; j < NPL; ++j) out[j] = out[j - 1] * e1;
        } else {
            pow_chain_b<NPL, NS>(exp2_fast(dv * A0p), n0, out);
        }
    };

    if (w == 0) {
#pragma unroll
        for (int j = 0; j < NPL; ++j) acar[0][j][lh] = 0.f;
    }
    if (tid == 0) s_bad = 0;

    float rb[TPT], rc[TPT];
    auto load_tile = [&](int s) {
#pragma unroll
        for (int i = 0; i < TPT; ++i) {
            const int e = tid + i * NT;
            const int t = s * SC + e / N;
            const int off = (e % N) * TS;
            rb[i] = IO::ld(rB, off + t * rowbc, 0);   // e >= TILE: a row the store skips
            rc[i] = IO::ld(rC, off + t * rowbc, 0);
        }
    };
    auto store_tile = [&](int slot) {
#pragma unroll
        for (int i = 0; i < TPT; ++i) {
            const int e = tid + i * NT;
            if (e < TILE) {
                sB[slot][e] = rb[i];
                sC[slot][e] = rc[i];
            }
        }
    };
    auto load_xd = [&](int s, float (&xo)[TC], float (&dto)[TC], float (&go)[TC]) {
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const int so = (s * SC + w * TC + k) * rowx;
            xo[k] = IO::ld(rx, vxz + so, 0);
            dto[k] = IO::ld(rdt, vx + so, 0);
            go[k] = IO::ld(rdy, vxz + so, 0);
        }
    };
    // B or C row of step rr of super-chunk s.
    auto bc_row = [&](const float (*tile)[SHARED ? TILE : 1], __amdgpu_buffer_rsrc_t r, int slot,
                      int s, int rr, float (&out)[NPL]) {
        if constexpr (SHARED) {
            const float *row = &tile[slot][rr * N + n0];
#pragma unroll
            for (int j = 0; j < NPL; ++j) out[j] = row[j];
        } else {
            const int so = (s * SC + rr) * rowbc;
#pragma unroll
            for (int j = 0; j < NPL; ++j) out[j] = IO::ld(r, vbc + j * TS + so, 0);
        }
    };
    // Forward state entering super-chunk s, state j (checkpoint or h0).
    auto h_start = [&](int s, int j) -> float {
        if (s == 0) return p.h0 ? p.h0[(b * Dm + dc) * N + n0 + j] : 0.f;
        return p.ckpt[((b * p.nck + (s - 1)) * Dm + dc) * N + n0 + j];
    };
    // The same for the state this wave folds (wave w < NPL folds state w),
    // as a load prefetched with the super-chunk's x / delta / dy; super-chunk
    // 0 starts from h0 (zero when null).
    const int jf = w < NPL ? w : NPL - 1;
    const float *ck0 = HIN ? nullptr : p.ckpt + (b * p.nck * Dm + dc) * N + n0 + jf;
    const float h0v = p.h0 ? p.h0[(b * Dm + dc) * N + n0 + jf] : 0.f;
    auto load_ck = [&](int s) -> float {
        const float cv = ck0[static_cast<long>(max(s - 1, 0)) * Dm * N];
        return (s == 0) ? h0v : cv;
    };

    // Prefetches are issued unconditionally (clamped to super-chunk 0, or
    // past the end where the range check reads 0): a load under a branch
    // would make the compiler's wait-count merge at the join wait for it
    // before the current data is used.
    if constexpr (SHARED) {
        load_tile(nit - 1);
        store_tile(0);
        load_tile(max(nit - 2, 0));
    }
    float X0[TC], D0[TC], G0[TC], X1[TC], D1[TC], G1[TC];
    float K0 = 0.f, K1 = 0.f;
    load_xd(nit - 1, X0, D0, G0);
    if constexpr (!HIN) K0 = load_ck(nit - 1);
    __syncthreads();

    float dAacc[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) dAacc[j] = 0.f;

    // ---- A: decays, forward local pass (FWD) and adjoint local pass -------
    auto phase_a = [&](auto fwdc, int s, int slot, const float (&xs)[TC], const float (&ds)[TC],
                       const float (&gs)[TC], float (&e)[TC][NPL]) __attribute__((always_inline)) {
        constexpr bool FWD = decltype(fwdc)::value;
        float dsum = 0.f;
        float dmin = ds[0];
        // The decay form is a wave-uniform branch around these few
        // instructions, so one loop body serves both.
        if (fast) {
#pragma unroll
            for (int k = 0; k < TC; ++k) decay_chain(ds[k], e[k]);
        } else {
#pragma unroll
            for (int k = 0; k < TC; ++k) {
                const float dl2 = ds[k] * kLog2e;
#pragma unroll
                for (int j = 0; j < NPL; ++j) e[k][j] = exp2_fast(dl2 * Ar[j]);
            }
        }
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            dsum = (k == 0) ? ds[0] : dsum + ds[k];
            dmin = fminf(dmin, ds[k]);
        }
        float P[NPL];
        if (fast) {
            decay_chain(dsum, P);
        } else {
            const float sl2 = dsum * kLog2e;
#pragma unroll
            for (int j = 0; j < NPL; ++j) P[j] = exp2_fast(sl2 * Ar[j]);
        }
        if constexpr (FWD) {
            float hl[NPL];
            float lm = 0.f;
#pragma unroll
            for (int k = 0; k < TC; ++k) {
                float bv[NPL];
                bc_row(sB, rB, slot, s, w * TC + k, bv);
                const float u = ds[k] * xs[k];
#pragma unroll
                for (int j = 0; j < NPL; ++j) {
                    hl[j] = (k == 0) ? bv[j] * u : fmaf(e[k][j], hl[j], bv[j] * u);
                    lm = fmaxf(lm, fabsf(hl[j]));
                }
            }
#pragma unroll
            for (int j = 0; j < NPL; ++j) aggF[w][j][lh] = hl[j];
            // |h| <= |h_in| + |local state| holds while every decay is <= 1
            // (A <= 0, delta >= 0); otherwise no bound (inf).
            lmx[w][lh] = (apos || !(dmin >= 0.f)) ? __builtin_inff() : lm;
        }
        float g[NPL];
#pragma unroll
        for (int j = 0; j < NPL; ++j) g[j] = 0.f;
#pragma unroll
        for (int k = TC - 1; k >= 0; --k) {
            float cv[NPL];
            bc_row(sC, rC, slot, s, w * TC + k, cv);
#pragma unroll
            for (int j = 0; j < NPL; ++j) g[j] = fmaf(gs[k], cv[j], g[j]) * e[k][j];
        }
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            aggP[w][j][lh] = P[j];
            aggA[w][j][lh] = g[j];
        }
    };

    // ---- F: folds (wave w < NPL: forward state w from the checkpoint ks;
    // NPL <= w < 2 NPL: adjoint state w - NPL). The forward fold also
    // bounds |h| over the super-chunk: a bound above 1000 (or not finite)
    // marks the workgroup for the clamped re-run. ----------------------------
    auto phase_f = [&](auto fwdc, int cur, float ks) __attribute__((always_inline)) {
        constexpr bool FWD = decltype(fwdc)::value;
        if (FWD && w < NPL) {
            const int j = w;
            float pv[W], hv[W], mv[W];
#pragma unroll
            for (int v = 0; v < W; ++v) {
                pv[v] = aggP[v][j][lh];
                hv[v] = aggF[v][j][lh];
                mv[v] = lmx[v][lh];
            }
            float run = ks;
            bool bad = false;
#pragma unroll
            for (int v = 0; v < W; ++v) {
                aggF[v][j][lh] = run;
                bad = bad || !(fabsf(run) + mv[v] <= 1000.f);
                run = fmaf(pv[v], run, hv[v]);
            }
            bad = bad || !(fabsf(run) <= 1000.f);
            if (p.clamp && bad) s_bad = 1;
        } else if (w >= NPL && w < 2 * NPL) {
            const int j = w - NPL;
            float pv[W], gv[W];
#pragma unroll
            for (int v = 0; v < W; ++v) {
                pv[v] = aggP[v][j][lh];
                gv[v] = aggA[v][j][lh];
            }
            float run = acar[cur][j][lh];
#pragma unroll
            for (int v = W - 1; v >= 0; --v) {
                aggA[v][j][lh] = run;
                run = fmaf(pv[v], run, gv[v]);
            }
            acar[cur ^ 1][j][lh] = run;
        }
    };

    // ---- R (second half): adjoint replay from the exact incoming adjoint,
    // forming every gradient term -------------------------------------------
    // hin_lds: the incoming states are still in aggF (main pass, no
    // history): read them at the last step instead of holding registers.
    auto grad_replay = [&](auto hin_ldsc, int s, int slot, const float (&xs)[TC],
                           const float (&ds)[TC], const float (&gs)[TC],
                           const float (&e)[TC][NPL], const float (&hs)[TC][NPL],
                           const float (&hin)[NPL]) __attribute__((always_inline)) {
        constexpr bool HIN_LDS = decltype(hin_ldsc)::value;
        const int t0 = s * SC + w * TC;
        float g[NPL];
#pragma unroll
        for (int j = 0; j < NPL; ++j) g[j] = aggA[w][j][lh];
        float *rw = &red[LRED ? hh * W + w : 0][0];
#pragma unroll
        for (int k = TC - 1; k >= 0; --k) {
            // One step at a time: operand reads of later steps hoisted here
            // would push the wave past its 128 registers.
            __builtin_amdgcn_sched_barrier(0);
            const int t = t0 + k;
            float bv[NPL], cv[NPL];
            bc_row(sB, rB, slot, s, w * TC + k, bv);
            bc_row(sC, rC, slot, s, w * TC + k, cv);
            const float dtk = ds[k], xk = xs[k], gk = gs[k];
            const float u = dtk * xk;
            float sa = 0.f, sbv = 0.f;
            float ahv[NPL];
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
                const float ah = fmaf(gk, cv[j], g[j]);
                const float hp = (k > 0) ? hs[k - 1][j] : HIN_LDS ? aggF[HIN ? 0 : w][j][lh] : hin[j];
                const float ae = ah * e[k][j];
                const float q = ae * hp;
                dAacc[j] = fmaf(dtk, q, dAacc[j]);
                sa = fmaf(Ar[j], q, sa);
                sbv = fmaf(ah, bv[j], sbv);
                ahv[j] = ah;
                g[j] = ae;
            }
            // Sum the state groups of the channel (lanes dl + DL*ns), both
            // values at once: a 32-lane swap of (sa, sbv) leaves partial sums
            // of sa in lanes 0-31 and of sbv in lanes 32-63, a 16-lane swap
            // completes them (NS = 4), and a last 32-lane swap hands every
            // lane both totals.
            if constexpr (NS >= 2) {
                const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(sa), __float_as_uint(sbv),
                                                                false, false);
                float z = __uint_as_float(r[0]) + __uint_as_float(r[1]);
                if constexpr (NS >= 4) z = sum_xor16(z);
                const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(z), __float_as_uint(z),
                                                                false, false);
                sa = __uint_as_float(q[0]);
                sbv = __uint_as_float(q[1]);
            }
            // Rows past L and lanes without output are dropped by the range
            // check, so none of the stores below needs a branch.
            const int xo = static_cast<int>(vxs + static_cast<unsigned>(t * rowx));
            IO::st(rdx, xo, 0, dtk * sbv);
            IO::st(rdd, xo, 0, fmaf(xk, sbv, sa));
            if constexpr (LRED) {
                // This step's rows: lane (dl, ns) writes its NPL states of ah
                // and of h; the state-group-0 lanes write u and dy of their
                // channel. Lanes past D have x = dy = 0 (u = dy = 0): they add
                // nothing to the channel sums.
                const int rk = (TC - 1 - k) % RS;
                float *row = rw + (rk * 2) * RBLK + ns * RGRP + dl * NPL;
#pragma unroll
                for (int j = 0; j < NPL; ++j) {
                    row[j] = ahv[j];
                    row[RBLK + j] = hs[k][j];
                }
                float *vec = rw + RVEC + rk * 2 * DL + dl;   // same value from every state group
                vec[0] = u;
                vec[DL] = gk;
                if (rk == RS - 1) {
                    // Column (ri, gi, ni) against its vector, channel by
                    // channel in order; step ri of the round is
                    // t + RS - 1 - ri.
                    const float *col = rw + (ri * 2 + gi) * RBLK + (ni / NPL) * RGRP + ni % NPL;
                    const float *cvec = rw + RVEC + (ri * 2 + gi) * DL;
                    float acc = col[0] * cvec[0];
#pragma unroll
                    for (int c = 1; c < DL; ++c) acc = fmaf(col[c * NPL], cvec[c], acc);
                    if constexpr (HW > 1) {
                        // Round (TC - RS - k) / RS of the super-chunk's
                        // steps: slotted by comb_flush after the next barrier.
                        comb[w][(TC - RS - k) / RS][lh] = acc;
                    } else {
                        const int tt = t + RS - 1 - ri;
                        bio<f32_t>::st(rslot, ((tt * 2 + gi) * N + ni) * 4, 0, acc);
                    }
                }
            } else if constexpr (SHARED) {
                float dBv[NPL], dCv[NPL];
#pragma unroll
                for (int j = 0; j < NPL; ++j) {
                    dBv[j] = ahv[j] * u;
                    dCv[j] = gk * hs[k][j];
                }
                // Sum over the wave's channels; lane l then holds state
                // n0 + (l % DL) / (DL / NPL) of step t.
                const float rbv = reduce_scatter<NPL, DL>(dBv, lane);
                const float rcv = reduce_scatter<NPL, DL>(dCv, lane);
                const int ao = static_cast<int>(vacc + static_cast<unsigned>(t * 2 * N * 4));
                bio<f32_t>::st(rslot, ao, 0, rbv);
                bio<f32_t>::st(rslot, ao + N * 4, 0, rcv);
            } else {
#pragma unroll
                for (int j = 0; j < NPL; ++j) {
                    const int bo = static_cast<int>(vbcs + static_cast<unsigned>(j * TS + t * rowbc));
                    IO::st(rdB, bo, 0, ahv[j] * u);
                    IO::st(rdC, bo, 0, gk * hs[k][j]);
                }
            }
        }
    };

    // The two halves' channel sums of super-chunk s (written in comb by the
    // replay, read after a barrier): half hh slots round hh of each wave's
    // steps, half 0's sum plus half 1's, in that order.
    auto comb_flush = [&](int s) __attribute__((always_inline)) {
        if constexpr (HW > 1) {
            const int rnd = hh;
            const int tt = s * SC + w * TC + (TC - RS - rnd * RS) + RS - 1 - ri;
            const float v = comb[w][rnd][lane] + comb[w][rnd][lane + 64];
            bio<f32_t>::st(rslot, ((tt * 2 + gi) * N + ni) * 4, 0, v);
        }
    };

    // One super-chunk of the main pass: the forward states come from the
    // history (HIN) or from the checkpoint by local pass, fold and replay,
    // unclamped; the next super-chunk's operands are prefetched.
    auto body = [&](int it, float (&xs)[TC], float (&ds)[TC], float (&gs)[TC],
                    float ks, float (&xn)[TC], float (&dn)[TC], float (&gn)[TC],
                    float &kn) __attribute__((always_inline)) {
        const int s = nit - 1 - it;
        const int cur = it & 1;
        const int slot = it % 3;
        if constexpr (SHARED) {
            store_tile((it + 1) % 3);    // tile s-1 -> LDS (slot last read in it-2)
            load_tile(max(s - 2, 0));
        }
        load_xd(max(s - 1, 0), xn, dn, gn);
        if constexpr (!HIN) kn = load_ck(max(s - 1, 0));
        float e[TC][NPL];
        phase_a(std::integral_constant<bool, !HIN>{}, s, slot, xs, ds, gs, e);
        __syncthreads();
        if (it > 0) comb_flush(s + 1);
        phase_f(std::integral_constant<bool, !HIN>{}, cur, ks);
        __syncthreads();
        const int t0 = s * SC + w * TC;
        float hs[TC][NPL];
        float hin[NPL];
        if constexpr (HIN) {
#pragma unroll
            for (int k = 0; k < TC; ++k) {
#pragma unroll
                for (int j = 0; j < NPL; ++j)
                    hs[k][j] = bio<f32_t>::ld(rh, vh + j * 4 + (t0 + k) * rowh, 0);
            }
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
                if (t0 > 0) hin[j] = bio<f32_t>::ld(rh, vh + j * 4 + (t0 - 1) * rowh, 0);
                else hin[j] = p.h0 ? p.h0[(b * Dm + dc) * N + n0 + j] : 0.f;
            }
        } else {
#pragma unroll
            for (int k = 0; k < TC; ++k) {
                float bv[NPL];
                bc_row(sB, rB, slot, s, w * TC + k, bv);
                const float u = ds[k] * xs[k];
#pragma unroll
                for (int j = 0; j < NPL; ++j)
                    hs[k][j] = fmaf(e[k][j], (k == 0) ? aggF[HIN ? 0 : w][j][lh] : hs[k - 1][j],
                                    bv[j] * u);
            }
        }
        grad_replay(std::integral_constant<bool, !HIN>{}, s, slot, xs, ds, gs, e, hs, hin);
    };

    // One super-chunk of the clamped re-run: operands loaded in place, the
    // tile staged synchronously, and each wave's forward states recomputed
    // from the checkpoint with the sequential clamped recurrence in the
    // forward fallback's arithmetic order.
    auto body_rerun = [&](int it) __attribute__((always_inline)) {
        const int s = nit - 1 - it;
        const int cur = it & 1;
        __syncthreads();                 // the previous super-chunk's tile reads are done
        if (it > 0) comb_flush(s + 1);
        if constexpr (SHARED) {
            load_tile(s);
            store_tile(0);
        }
        float xs[TC], ds[TC], gs[TC];
        load_xd(s, xs, ds, gs);
        __syncthreads();
        float e[TC][NPL];
        phase_a(std::false_type{}, s, 0, xs, ds, gs, e);
        __syncthreads();
        phase_f(std::false_type{}, cur, 0.f);
        __syncthreads();
        float hs[TC][NPL];
        float hin[NPL];
        float h[NPL];
#pragma unroll
        for (int j = 0; j < NPL; ++j) h[j] = h_start(s, j);
        for (int r = 0; r < w * TC; ++r) {
            const int so = (s * SC + r) * rowx;
            const float xv = IO::ld(rx, vx + so, 0), dv = IO::ld(rdt, vx + so, 0);
            float bv[NPL];
            bc_row(sB, rB, 0, s, r, bv);
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
                const float ee = exp2_fast(dv * (Ar[j] * kLog2e));
                float hn = __fadd_rn(__fmul_rn(ee, h[j]), __fmul_rn(__fmul_rn(bv[j], dv), xv));
                hn = (hn < 1000.f) ? hn : 1000.f;
                h[j] = (hn > -1000.f) ? hn : -1000.f;
            }
        }
#pragma unroll
        for (int j = 0; j < NPL; ++j) hin[j] = h[j];
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            float bv[NPL];
            bc_row(sB, rB, 0, s, w * TC + k, bv);
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
                const float ee = exp2_fast(ds[k] * (Ar[j] * kLog2e));
                float hn = __fadd_rn(__fmul_rn(ee, h[j]), __fmul_rn(__fmul_rn(bv[j], ds[k]), xs[k]));
                hn = (hn < 1000.f) ? hn : 1000.f;
                h[j] = (hn > -1000.f) ? hn : -1000.f;
                hs[k][j] = h[j];
            }
        }
        grad_replay(std::false_type{}, s, 0, xs, ds, gs, e, hs, hin);
    };

    for (int it = 0; it < nit; it += 2) {
        body(it, X0, D0, G0, K0, X1, D1, G1, K1);
        if (it + 1 < nit) body(it + 1, X1, D1, G1, K1, X0, D0, G0, K0);
    }
    __syncthreads();
    comb_flush(0);
    if constexpr (!HIN) {
        // Some super-chunk's states may have left [-1000, 1000]: every
        // output of this workgroup again, with the clamped states.
        if (__builtin_amdgcn_readfirstlane(s_bad) != 0) {
#pragma unroll
            for (int j = 0; j < NPL; ++j) dAacc[j] = 0.f;
            if (w == 0) {
#pragma unroll
                for (int j = 0; j < NPL; ++j) acar[0][j][lh] = 0.f;
            }
            for (int it = 0; it < nit; ++it) body_rerun(it);
            __syncthreads();
            comb_flush(0);
        }
    }

    // dA: the waves' sums over their steps, added in wave order, one
    // store per (batch, channel, state).
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NPL; ++j) aggA[w][j][lh] = dAacc[j];
    __syncthreads();
    if (w == 0 && dvalid) {
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            float acc = aggA[0][j][lh];
#pragma unroll
            for (int v = 1; v < W; ++v) acc += aggA[v][j][lh];
            p.dApart[(b * Dm + d) * N + n0 + j] = acc;
        }
    }
}

// Any N <= 64 (and windows too large for 32-bit offsets): one thread per
// (batch, channel), the reference's reverse step order, states from the
// history. A workgroup holds kSerialNB channels of one batch element; with
// shared B/C the channels' dB / dC terms of a step are summed in channel
// order through LDS into the workgroup's partial slot.
constexpr int kSerialNB = 128;

template <typename T>
__global__ void __launch_bounds__(kSerialNB) scan1d_bwd_serial(Scan1DBwdArgs p) {
    using IO = io<T>;
    __shared__ float red[2][64][kSerialNB];
    const int tid = threadIdx.x;
    const long cblocks = (p.D + kSerialNB - 1) / kSerialNB;
    const long b = blockIdx.x / cblocks, g = blockIdx.x - b * cblocks;
    const long d = g * kSerialNB + tid;
    const bool ok = d < p.D;
    const long dc = ok ? d : p.D - 1;
    const long N = p.N;
    const bool shared = (p.sd == 0);
    float adj[64], dAl[64];
    for (long m = 0; m < N; ++m) {
        adj[m] = 0.f;
        dAl[m] = 0.f;
    }
    // Every thread walks every step (uniform barriers); lanes past D compute
    // on channel D-1 and contribute nothing.
    for (long t = p.L - 1; t >= 0; --t) {
        const long td = (b * p.L + t) * p.D + dc;
        const float dt = IO::ld(p.dt, td), xt = IO::ld(p.x, td), gy = IO::ld(p.dy, td);
        const long bc = b * p.sb + t * p.st + dc * p.sd;
        float dxv = 0.f, ddt = 0.f;
        for (long m = 0; m < N; ++m) {
            const float a = p.A[dc * N + m];
            const float bb = IO::ld(p.Bm, bc + m), c = IO::ld(p.Cm, bc + m);
            const float e = exp2_fast(dt * a * kLog2e);
            float hp = 0.f;
            if (t > 0) hp = p.hist[(td - p.D) * N + m];
            else if (p.h0) hp = p.h0[(b * p.D + dc) * N + m];
            const float ah = adj[m] + gy * c;
            const float dCv = gy * p.hist[td * N + m];
            const float dBv = ah * dt * xt;
            dAl[m] += ah * dt * e * hp;
            dxv += ah * dt * bb;
            ddt += ah * (a * e * hp + bb * xt);
            adj[m] = ah * e;
            if (shared) {
                red[0][m][tid] = ok ? dBv : 0.f;
                red[1][m][tid] = ok ? dCv : 0.f;
            } else if (ok) {
                IO::st(p.dB, bc + m, dBv);
                IO::st(p.dC, bc + m, dCv);
            }
        }
        if (ok) {
            IO::st(p.dx, td, dxv);
            IO::st(p.ddt, td, ddt);
        }
        if (shared) {
            __syncthreads();
            const long so = (b * p.G + g) * p.L;   // + t: row of the [L, 2, N] slot
            for (long k = tid; k < 2 * N; k += kSerialNB) {
                const int which = static_cast<int>(k / N);
                const long m = k - which * N;
                float acc = 0.f;
                for (int i = 0; i < kSerialNB; ++i) acc += red[which][m][i];
                p.slot[(so + t) * 2 * N + which * N + m] = acc;
            }
            __syncthreads();
        }
    }
    if (ok)
        for (long m = 0; m < N; ++m) p.dApart[(b * p.D + d) * N + m] = dAl[m];
}

// Zeroes p[0, n) (16-byte stores when p is 16-byte aligned).
__global__ void __launch_bounds__(256) fill_zero_kernel(float *p, long n) {
    const long i0 = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    const long stride = static_cast<long>(gridDim.x) * blockDim.x;
    const long n4 = (reinterpret_cast<uintptr_t>(p) & 15) == 0 ? n / 4 : 0;
    float4 *p4 = reinterpret_cast<float4 *>(p);
    for (long i = i0; i < n4; i += stride) p4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (long i = n4 * 4 + i0; i < n; i += stride) p[i] = 0.f;
}

// Fixed-order sums of the partials: dA[i] = sum over b of dApart[b, i]
// (b ascending); with shared B/C, dB / dC at b*sb + t*st + n = sum over the
// channel groups g (ascending) of slot[b, g, t, 0 / 1, n].
template <typename T>
// With q4 (N a multiple of 4) a thread sums four consecutive states with
// 16-byte loads, four groups' loads in flight before their adds; each
// state's sum still adds the groups in ascending order.
__global__ void __launch_bounds__(256) scan1d_bwd_finalize(const float *slot, long G, void *dB,
                                                           void *dC, long B, long L, long N,
                                                           long sb, long st, const float *dApart,
                                                           float *dA, long DN, int q4) {
    using IO = io<T>;
    const long Q = q4 ? 4 : 1;                 // states per thread
    const long Nq = N / Q;
    const long n_bc = slot ? B * L * Nq : 0;
    const long LNq = L * Nq;
    const long S = 2 * L * N;   // floats per (b, g) slot
    const long stride = static_cast<long>(gridDim.x) * blockDim.x;
    for (long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_bc + DN;
         i += stride) {
        if (i < n_bc) {
            const long b = i / LNq, r = i - b * LNq, t = r / Nq, n = (r - t * Nq) * Q;
            const float *pb = slot + b * G * S + t * 2 * N + n;
            const long o = b * sb + t * st + n;
            if (q4) {
                float4 aB = make_float4(0.f, 0.f, 0.f, 0.f), aC = aB;
                long g = 0;
                for (; g + 4 <= G; g += 4) {
                    float4 vB[4], vC[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        vB[u] = *reinterpret_cast<const float4 *>(pb + (g + u) * S);
                        vC[u] = *reinterpret_cast<const float4 *>(pb + (g + u) * S + N);
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        aB.x += vB[u].x; aB.y += vB[u].y; aB.z += vB[u].z; aB.w += vB[u].w;
                        aC.x += vC[u].x; aC.y += vC[u].y; aC.z += vC[u].z; aC.w += vC[u].w;
                    }
                }
                for (; g < G; ++g) {
                    const float4 vB = *reinterpret_cast<const float4 *>(pb + g * S);
                    const float4 vC = *reinterpret_cast<const float4 *>(pb + g * S + N);
                    aB.x += vB.x; aB.y += vB.y; aB.z += vB.z; aB.w += vB.w;
                    aC.x += vC.x; aC.y += vC.y; aC.z += vC.z; aC.w += vC.w;
                }
                IO::st(dB, o, aB.x); IO::st(dB, o + 1, aB.y); IO::st(dB, o + 2, aB.z); IO::st(dB, o + 3, aB.w);
                IO::st(dC, o, aC.x); IO::st(dC, o + 1, aC.y); IO::st(dC, o + 2, aC.z); IO::st(dC, o + 3, aC.w);
            } else {
                float sB = 0.f, sC = 0.f;
                for (long g = 0; g < G; ++g) {
                    sB += pb[g * S];
                    sC += pb[g * S + N];
                }
                IO::st(dB, o, sB);
                IO::st(dC, o, sC);
            }
        } else {
            const long k = i - n_bc;
            float acc = 0.f;
            for (long b = 0; b < B; ++b) acc += dApart[b * DN + k];
            dA[k] = acc;
        }
    }
}

static int fill_zero(float *p, long n, hipStream_t s) {
    if (n <= 0) return 0;
    const long blocks = std::min<long>((n / 4 + 255) / 256 + 1, 4096);
    hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, s, p, n);
    KM_HIP_TRY(hipGetLastError());
    return 0;
}

struct BwdPlan {
    bool shared, hist_in, need_ckpt, serial, need_hist;
    bool wide;              // N = 16 shared B/C on 32-channel workgroups (two halves)
    long G;                 // channel groups per batch element (partial slots)
    size_t off_slots, off_dA, off_ckpt, off_hist, bytes;
};

// Channels per workgroup of the register-blocked backward for a state size.
static long bwd_group_channels(long N, bool wide) {
    if (N == 16) return wide ? 32 : 16;     // wide: two 16-channel halves
    if (N == 8) return 32;
    return 64;
}

// Shared B/C with N = 16 runs 16-wave workgroups on 32 channels (half the
// dB / dC partial slots) when they still fill the chip, one per CU of the
// 256; fewer would leave CUs idle while each holds twice the waves, so
// smaller grids keep 8-wave workgroups on 16 channels.
// KM_SCAN1D_BWD_WIDE=1 / 0 forces either.
constexpr long kWideMinGroups = 256;
static bool bwd_wide(long B, long D) {
    const char *e = std::getenv("KM_SCAN1D_BWD_WIDE");
    if (e && std::strcmp(e, "1") == 0) return true;
    if (e && std::strcmp(e, "0") == 0) return false;
    return B * ((D + 31) / 32) >= kWideMinGroups;
}

static BwdPlan bwd_plan(const KMScan1DBwd *k) {
    BwdPlan pl{};
    pl.shared = (k->bc_sd == 0);
    const long es = (k->dtype == KM_BF16) ? 2 : 4;
    const long lim = 0x3fffffffL;
    const bool small_windows = k->L * k->D * es < lim && k->L * k->bc_st * es < lim &&
                               (!k->h_hist || k->L * k->D * k->N * 4 < lim);
    const bool chunk_n = (k->N == 16 || k->N == 8 || k->N == 4 || k->N == 2 || k->N == 1);
    pl.serial = !(small_windows && chunk_n);
    pl.hist_in = (k->h_hist != nullptr);
    pl.need_hist = pl.serial && !pl.hist_in;
    pl.need_ckpt = !pl.serial && !pl.hist_in && !k->h_ckpt;
    pl.wide = pl.shared && !pl.serial && k->N == 16 && bwd_wide(k->B, k->D);
    const long gc = pl.serial ? kSerialNB : bwd_group_channels(k->N, pl.wide);
    pl.G = (k->D + gc - 1) / gc;
    size_t off = 0;
    pl.off_slots = off;
    if (pl.shared) off += align_up(sizeof(float) * 2 * k->B * pl.G * k->L * k->N, 256);
    pl.off_dA = off;
    off += align_up(sizeof(float) * k->B * k->D * k->N, 256);
    pl.off_ckpt = off;
    if (pl.need_ckpt)
        off += align_up(sizeof(float) * k->B * ((k->L + kCkptSteps - 1) / kCkptSteps) * k->D * k->N, 256);
    pl.off_hist = off;
    if (pl.need_hist) off += align_up(sizeof(float) * k->B * k->L * k->D * k->N, 256);
    pl.bytes = off;
    return pl;
}

static bool bwd_args_ok(const KMScan1DBwd *k, const char *who) {
    if (!k) { set_error("%s: NULL arguments", who); return false; }
    // With no steps (L = 0) only A and dA (zeroed) take part.
    if (!k->A || !k->dA ||
        (k->L > 0 && (!k->x || !k->delta || !k->Bm || !k->Cm || !k->dy || !k->dx || !k->ddelta ||
                      !k->dB || !k->dC))) {
        set_error("%s: NULL tensor pointer", who);
        return false;
    }
    if (k->B <= 0 || k->L < 0 || k->D <= 0 || k->N <= 0 || k->N > 64) {
        set_error("%s: invalid sizes B=%ld L=%ld D=%ld N=%ld (need N <= 64)", who, k->B, k->L,
                  k->D, k->N);
        return false;
    }
    if (k->dtype != KM_F32 && k->dtype != KM_BF16) {
        set_error("%s: unknown dtype %d", who, k->dtype);
        return false;
    }
    if (k->bc_sb < 0 || k->bc_st < 0 || k->bc_sd < 0 ||
        (k->B > 1 && k->L > 0 && k->bc_sb == 0) || (k->L > 1 && k->bc_st == 0)) {
        set_error("%s: B/C strides must be non-negative and distinct over batch and time "
                  "(sb=%ld st=%ld sd=%ld)", who, k->bc_sb, k->bc_st, k->bc_sd);
        return false;
    }
    return true;
}

static int bwd_chunked_launch(const Scan1DBwdArgs &a, bool shared, bool hin, bool bf, bool wide,
                              hipStream_t s) {
    constexpr int W = 8;
    const long DL = bwd_group_channels(a.N, wide);
    const int HW = wide ? 2 : 1;   // the kernel's two halves (LDS sums)
    const long grid = a.B * ((a.D + DL - 1) / DL);
    if (grid <= 0 || grid > 0x7fffffffL) {
        set_error("km_scan1d_bwd: grid of %ld workgroups out of range", grid);
        return -1;
    }
    dim3 g(static_cast<unsigned>(grid)), blk(64 * W * HW);
#define KM_BWD_GO(TT, NPL, NS)                                                                    \
    do {                                                                                          \
        if (shared) {                                                                             \
            if (hin) hipLaunchKernelGGL((scan1d_bwd_chunked<TT, NPL, NS, true, true, 1>), g, blk, 0, s, a);   \
            else     hipLaunchKernelGGL((scan1d_bwd_chunked<TT, NPL, NS, true, false, 1>), g, blk, 0, s, a);  \
        } else {                                                                                  \
            if (hin) hipLaunchKernelGGL((scan1d_bwd_chunked<TT, NPL, NS, false, true, 1>), g, blk, 0, s, a);  \
            else     hipLaunchKernelGGL((scan1d_bwd_chunked<TT, NPL, NS, false, false, 1>), g, blk, 0, s, a); \
        }                                                                                         \
    } while (0)
#define KM_BWD_WIDE(TT)                                                                           \
    do {                                                                                          \
        if (hin) hipLaunchKernelGGL((scan1d_bwd_chunked<TT, 4, 4, true, true, 2>), g, blk, 0, s, a);      \
        else     hipLaunchKernelGGL((scan1d_bwd_chunked<TT, 4, 4, true, false, 2>), g, blk, 0, s, a);     \
    } while (0)
    if (wide) {
        if (bf) KM_BWD_WIDE(bf16_t);
        else    KM_BWD_WIDE(f32_t);
        KM_HIP_TRY(hipGetLastError());
        return 0;
    }
#undef KM_BWD_WIDE
    switch (a.N) {
    case 16: if (bf) KM_BWD_GO(bf16_t, 4, 4); else KM_BWD_GO(f32_t, 4, 4); break;
    case 8:  if (bf) KM_BWD_GO(bf16_t, 4, 2); else KM_BWD_GO(f32_t, 4, 2); break;
    case 4:  if (bf) KM_BWD_GO(bf16_t, 4, 1); else KM_BWD_GO(f32_t, 4, 1); break;
    case 2:  if (bf) KM_BWD_GO(bf16_t, 2, 1); else KM_BWD_GO(f32_t, 2, 1); break;
    case 1:  if (bf) KM_BWD_GO(bf16_t, 1, 1); else KM_BWD_GO(f32_t, 1, 1); break;
    default:
        set_error("km_scan1d_bwd: no register-blocked kernel for N=%ld", a.N);
        return -1;
    }
#undef KM_BWD_GO
    KM_HIP_TRY(hipGetLastError());
    return 0;
}

static int scan1d_bwd_run(const KMScan1DBwd *k, const BwdPlan &pl, bool bf, hipStream_t stream);

size_t scan1d_bwd_workspace(const KMScan1DBwd *k) {
    if (!bwd_args_ok(k, "km_scan1d_bwd_workspace_bytes")) return 0;
    return bwd_plan(k).bytes;
}

int scan1d_bwd_launch(const KMScan1DBwd *k, hipStream_t stream) {
    if (!bwd_args_ok(k, "km_scan1d_bwd")) return -1;
    if (!gpu_ready()) return -1;
    const BwdPlan pl = bwd_plan(k);
    const bool bf = (k->dtype == KM_BF16);
    if (k->L == 0) return fill_zero(k->dA, k->D * k->N, stream);
    return scan1d_bwd_run(k, pl, bf, stream);
}

static int scan1d_bwd_run(const KMScan1DBwd *k, const BwdPlan &pl, bool bf, hipStream_t stream) {
    char *ws = nullptr;
    if (pl.bytes > 0) {
        if (k->workspace) {
            if (k->workspace_bytes < pl.bytes) {
                set_error("km_scan1d_bwd: workspace of %zu bytes, %zu needed", k->workspace_bytes,
                          pl.bytes);
                return -1;
            }
            ws = static_cast<char *>(k->workspace);
        } else {
            ws = static_cast<char *>(Workspace::reserve(pl.bytes, stream, WsUse::Scan1DBwd));
            if (!ws) return -1;
        }
    }
    Scan1DBwdArgs a{};
    a.x = k->x; a.dt = k->delta; a.dy = k->dy; a.A = k->A; a.Bm = k->Bm; a.Cm = k->Cm;
    a.h0 = k->h0; a.hist = k->h_hist; a.ckpt = k->h_ckpt;
    a.nck = (k->L + kCkptSteps - 1) / kCkptSteps;
    a.dx = k->dx; a.ddt = k->ddelta; a.dB = k->dB; a.dC = k->dC;
    a.B = k->B; a.L = k->L; a.D = k->D; a.N = k->N;
    a.sb = k->bc_sb; a.st = k->bc_st; a.sd = k->bc_sd; a.clamp = k->clamp;
    // Every partial slot is written by exactly one workgroup: nothing is
    // zeroed first.
    a.G = pl.G;
    a.dApart = reinterpret_cast<float *>(ws + pl.off_dA);
    if (pl.shared) a.slot = reinterpret_cast<float *>(ws + pl.off_slots);
    if (pl.need_ckpt || pl.need_hist) {
        // Forward states from the same inputs (y not written).
        KMScan1DFwd f{};
        f.x = k->x; f.delta = k->delta; f.A = k->A; f.Bm = k->Bm; f.Cm = k->Cm; f.y = nullptr;
        f.h0 = k->h0; f.B = k->B; f.L = k->L; f.D = k->D; f.N = k->N;
        f.bc_sb = k->bc_sb; f.bc_st = k->bc_st; f.bc_sd = k->bc_sd;
        f.dtype = k->dtype; f.clamp = k->clamp;
        if (pl.need_ckpt) {
            f.h_ckpt = reinterpret_cast<float *>(ws + pl.off_ckpt);
            a.ckpt = f.h_ckpt;
        } else {
            f.h_hist = reinterpret_cast<float *>(ws + pl.off_hist);
            a.hist = f.h_hist;
        }
        if (scan1d_fwd_launch(&f, stream, true) != 0) return -1;
    }
    if (pl.serial) {
        const long grid = k->B * pl.G;
        if (grid > 0x7fffffffL) {
            set_error("km_scan1d_bwd: grid of %ld workgroups out of range", grid);
            return -1;
        }
        if (bf) hipLaunchKernelGGL(scan1d_bwd_serial<bf16_t>, dim3(grid), dim3(kSerialNB), 0, stream, a);
        else    hipLaunchKernelGGL(scan1d_bwd_serial<f32_t>, dim3(grid), dim3(kSerialNB), 0, stream, a);
        KM_HIP_TRY(hipGetLastError());
    } else if (bwd_chunked_launch(a, pl.shared, a.hist != nullptr, bf, pl.wide, stream) != 0) {
        return -1;
    }
    // Slots hold whole [L, 2, N] rows from the workspace's slot offset: with
    // N % 4 == 0 and that offset 16-byte aligned (a caller's workspace may
    // not be), every thread's four states are.
    const int q4 = (k->N % 4 == 0 && (reinterpret_cast<uintptr_t>(a.slot) & 15) == 0) ? 1 : 0;
    const long n = (pl.shared ? k->B * k->L * k->N / (q4 ? 4 : 1) : 0) + k->D * k->N;
    const long blocks = std::min<long>((n + 255) / 256, 8192);
#define KM_FIN(TT)                                                                                 \
    hipLaunchKernelGGL(scan1d_bwd_finalize<TT>, dim3(blocks), dim3(256), 0, stream, a.slot,       \
                       pl.G, k->dB, k->dC, k->B, k->L, k->N, k->bc_sb, k->bc_st,                  \
                       a.dApart, k->dA, k->D * k->N, q4)
    if (bf) KM_FIN(bf16_t);
    else    KM_FIN(f32_t);
#undef KM_FIN
    KM_HIP_TRY(hipGetLastError());
    return 0;
}

}  // namespace km

namespace km {

struct M1Args {
    const float *x, *A, *Adiag, *B, *C, *delta, *h0, *h, *dy;
    float *dx, *dA, *dB, *dC, *ddelta;
    long L, D;
    float *part;   // [gridDim.x, L] per-workgroup ddelta partials
    int taylor;    // decay without Adiag: 0 exp, 1 / 2 the AVX2 / scalar asm polynomial
};

// Decay of the reference's assembly M = 1 backward routines when A_diag is
// NULL: 1 + x + x^2/2 + x^3/6 of x = delta*A in their instruction order
// (cpu/scan1d_backward_m1_shared_bc.asm:220-231: x^3/6 = (x^3 * 0.5) *
// 0.33333334; _simple.asm:212-225: x^3 * 0.16666667), every operation
// rounded on its own.
__device__ __forceinline__ float m1_asm_taylor(float x, bool scalar_form) {
#pragma clang fp contract(off)
    const float x2 = x * x;
    float acc = x + x2 * 0.5f;
    float x3 = x2 * x;
    x3 = scalar_form ? x3 * 0.16666667f : (x3 * 0.5f) * 0.33333334f;
    acc = acc + x3;
    return acc + 1.0f;
}

// M = 1 with B, C shared over time ([D]) and delta shared over channels
// ([L]) (reference cpu/scan1d_backward.c:23-70): one thread per channel in
// reverse time. ddelta[t] sums the channels' terms: each workgroup sums its
// 256 channels (wave shuffles, then the four waves in order) into its own
// partial slot, and m1_finalize adds the slots in workgroup order.
__global__ void __launch_bounds__(256) scan1d_bwd_m1_shared(M1Args p) {
    __shared__ float part[4];
    const int tid = threadIdx.x;
    const long d = static_cast<long>(blockIdx.x) * 256 + tid;
    const bool ok = d < p.D;
    const long dc = ok ? d : p.D - 1;
    const float a = p.A[dc], bb = p.B[dc], c = p.C[dc];
    float adj = 0.f, dAl = 0.f, dBl = 0.f, dCl = 0.f;
    for (long t = p.L - 1; t >= 0; --t) {
        const long td = t * p.D + dc;
        const float dt = p.delta[t];
        const float xt = p.x[td], gy = p.dy[td];
        const float e = p.Adiag ? p.Adiag[td]
                        : p.taylor ? m1_asm_taylor(dt * a, p.taylor == 2)
                                   : exp2_fast(dt * a * kLog2e);
        const float hp = (t > 0) ? p.h[td - p.D] : (p.h0 ? p.h0[dc] : 0.f);
        const float ah = adj + gy * c;
        dCl += gy * p.h[td];
        dBl += ah * dt * xt;
        dAl += ah * dt * e * hp;
        if (ok) p.dx[td] = ah * dt * bb;
        float term = ok ? ah * (a * e * hp + bb * xt) : 0.f;
        adj = ah * e;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) term += __shfl_xor(term, m);
        if ((tid & 63) == 0) part[tid >> 6] = term;
        __syncthreads();
        if (tid == 0) p.part[blockIdx.x * p.L + t] = ((part[0] + part[1]) + part[2]) + part[3];
        __syncthreads();
    }
    if (ok) {
        p.dA[d] = dAl;
        p.dB[d] = dBl;
        p.dC[d] = dCl;
    }
}

// ddelta[t] = sum over workgroups (ascending) of part[wg, t].
__global__ void __launch_bounds__(256) m1_finalize(const float *part, long nwg, long L,
                                                   float *ddelta) {
    const long t = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (t >= L) return;
    float acc = 0.f;
    for (long g = 0; g < nwg; ++g) acc += part[g * L + t];
    ddelta[t] = acc;
}

static int m1_launch(M1Args a, hipStream_t s) {
    const long grid = (a.D + 255) / 256;
    a.part = static_cast<float *>(Workspace::reserve(sizeof(float) * grid * a.L, s, WsUse::Scan1DM1));
    if (!a.part) return -1;
    hipLaunchKernelGGL(scan1d_bwd_m1_shared, dim3(grid), dim3(256), 0, s, a);
    KM_HIP_TRY(hipGetLastError());
    hipLaunchKernelGGL(m1_finalize, dim3((a.L + 255) / 256), dim3(256), 0, s,
                       static_cast<const float *>(a.part), grid, a.L, a.ddelta);
    KM_HIP_TRY(hipGetLastError());
    return 0;
}

// Host-or-device buffers of one host-pointer call: device pointers pass
// through, host buffers are staged (inputs copied in, outputs copied back).
struct StagedCall {
    struct Buf { const void *user; void *dev; size_t bytes; bool out; };
    Buf bufs[24];
    int n = 0;
    bool all_dev = true;
    void add(const void *user, size_t bytes, bool out) {
        bufs[n++] = Buf{user, const_cast<void *>(user), bytes, out};
        if (user && !is_device_ptr(user)) all_dev = false;
    }
    // Reserves staging and copies inputs; false on failure (error set).
    bool stage_in(const char *who) {
        if (all_dev) return true;
        size_t total = 0;
        for (int i = 0; i < n; ++i) if (bufs[i].user) total += align_up(bufs[i].bytes, 256);
        void *base = Staging::reserve(total);
        if (!base) return false;
        Carver c(base);
        for (int i = 0; i < n; ++i) {
            if (!bufs[i].user) continue;
            bufs[i].dev = c.take<char>(bufs[i].bytes);
            if (!bufs[i].out &&
                km::copy_h2d(bufs[i].dev, bufs[i].user, bufs[i].bytes) != hipSuccess) {
                set_error("%s: host-to-device copy failed", who);
                return false;
            }
        }
        return true;
    }
    bool stage_out(const char *who) {
        if (hipStreamSynchronize(nullptr) != hipSuccess) {
            set_error("%s: %s", who, hipGetErrorString(hipGetLastError()));
            return false;
        }
        if (all_dev) return true;
        for (int i = 0; i < n; ++i) {
            if (!bufs[i].user || !bufs[i].out) continue;
            if (copy_d2h(const_cast<void *>(bufs[i].user), bufs[i].dev, bufs[i].bytes) != hipSuccess) {
                set_error("%s: device-to-host copy failed", who);
                return false;
            }
        }
        return true;
    }
    template <typename P> P *dev(int i) { return static_cast<P *>(bufs[i].dev); }
};

}  // namespace km

extern "C" {

size_t km_scan1d_bwd_workspace_bytes(const KMScan1DBwd *a) {
    km::clear_error();
    return km::scan1d_bwd_workspace(a);
}

int km_scan1d_bwd(const KMScan1DBwd *a, void *stream) {
    km::clear_error();
    return km::scan1d_bwd_launch(a, static_cast<hipStream_t>(stream));
}

// Reference cuda/scan1d_backward.cu:113-137: device pointers, B, C, h
// [L, D, M] (h = forward state history), zero initial state; synchronous.
void om_scan1d_backward(const float *d_dy, const float *d_x, const float *d_A, const float *d_B,
                        const float *d_C, const float *d_dt, const float *d_h, float *d_dx,
                        float *d_dA, float *d_dB, float *d_dC, float *d_ddt, int L, int D, int M) {
    km::clear_error();
    if (L < 0 || D <= 0 || M <= 0) {
        km::set_error("om_scan1d_backward: invalid sizes L=%d D=%d M=%d", L, D, M);
        return;
    }
    KMScan1DBwd a{};
    a.x = d_x; a.delta = d_dt; a.A = d_A; a.Bm = d_B; a.Cm = d_C; a.dy = d_dy;
    a.h_hist = d_h; a.dx = d_dx; a.ddelta = d_ddt; a.dA = d_dA; a.dB = d_dB; a.dC = d_dC;
    a.B = 1; a.L = L; a.D = D; a.N = M;
    a.bc_sb = static_cast<long>(L) * D * M; a.bc_st = static_cast<long>(D) * M; a.bc_sd = M;
    a.dtype = KM_F32; a.clamp = 1;
    if (km::scan1d_bwd_launch(&a, nullptr) != 0) return;
    if (hipStreamSynchronize(nullptr) != hipSuccess)
        km::set_error("om_scan1d_backward: %s", hipGetErrorString(hipGetLastError()));
}

void mamba_scan1d_cuda_backward(const float *d_dy, const float *d_x, const float *d_A,
                                const float *d_B, const float *d_C, const float *d_dt,
                                const float *d_h, float *d_dx, float *d_dA, float *d_dB,
                                float *d_dC, float *d_ddt, int L, int D, int M) {
    om_scan1d_backward(d_dy, d_x, d_A, d_B, d_C, d_dt, d_h, d_dx, d_dA, d_dB, d_dC, d_ddt, L, D, M);
}

// Reference scan1d_backward (cpu/scan1d_backward.c:297-306): host or device
// pointers; B, C, h, dB, dC [L, D, M]; h = forward history; h0 [D, M] or
// NULL; every output is overwritten.
void scan1d_backward(ScanBackwardParams *p) {
    km::clear_error();
    if (!p || !p->x || !p->A || !p->B || !p->C || !p->delta || !p->h || !p->dy || !p->dx ||
        !p->dA || !p->dB || !p->dC || !p->ddelta || p->L <= 0 || p->D <= 0 || p->M <= 0) {
        km::set_error("scan1d_backward: invalid parameters");
        return;
    }
    if (!km::gpu_ready()) return;
    const size_t LD = p->L * p->D * 4, DM = p->D * p->M * 4, LDM = p->L * p->D * p->M * 4;
    km::Staging::lock();
    km::StagedCall sc;
    sc.add(p->x, LD, false);      // 0
    sc.add(p->A, DM, false);      // 1
    sc.add(p->B, LDM, false);     // 2
    sc.add(p->C, LDM, false);     // 3
    sc.add(p->delta, LD, false);  // 4
    sc.add(p->h0, DM, false);     // 5
    sc.add(p->h, LDM, false);     // 6
    sc.add(p->dy, LD, false);     // 7
    sc.add(p->dx, LD, true);      // 8
    sc.add(p->dA, DM, true);      // 9
    sc.add(p->dB, LDM, true);     // 10
    sc.add(p->dC, LDM, true);     // 11
    sc.add(p->ddelta, LD, true);  // 12
    if (sc.stage_in("scan1d_backward")) {
        KMScan1DBwd a{};
        a.x = sc.dev<float>(0); a.A = sc.dev<float>(1); a.Bm = sc.dev<float>(2);
        a.Cm = sc.dev<float>(3); a.delta = sc.dev<float>(4); a.h0 = sc.dev<float>(5);
        a.h_hist = sc.dev<float>(6); a.dy = sc.dev<float>(7); a.dx = sc.dev<float>(8);
        a.dA = sc.dev<float>(9); a.dB = sc.dev<float>(10); a.dC = sc.dev<float>(11);
        a.ddelta = sc.dev<float>(12);
        a.B = 1; a.L = p->L; a.D = p->D; a.N = p->M;
        a.bc_sb = p->L * p->D * p->M; a.bc_st = p->D * p->M; a.bc_sd = p->M;
        a.dtype = KM_F32; a.clamp = 1;
        if (km::scan1d_bwd_launch(&a, nullptr) == 0) sc.stage_out("scan1d_backward");
    }
    km::Staging::unlock();
}

void mamba_scan1d_backward(MambaScan1DBackwardParams *p) { scan1d_backward(p); }

}  // extern "C"

namespace km {

// One host-or-device call of the M = 1 backward (L, D > 0, parameters
// checked by the caller) with the decay form `taylor` (M1Args::taylor).
static void m1_host_call(ScanBackwardSharedParams *p, int taylor, const char *who) {
    const size_t LD = p->L * p->D * 4, D4 = p->D * 4, L4 = p->L * 4;
    Staging::lock();
    StagedCall sc;
    sc.add(p->x, LD, false);       // 0
    sc.add(p->A, D4, false);       // 1
    sc.add(p->A_diag, LD, false);  // 2
    sc.add(p->B, D4, false);       // 3
    sc.add(p->C, D4, false);       // 4
    sc.add(p->delta, L4, false);   // 5
    sc.add(p->h0, D4, false);      // 6
    sc.add(p->h, LD, false);       // 7
    sc.add(p->dy, LD, false);      // 8
    sc.add(p->dx, LD, true);       // 9
    sc.add(p->dA, D4, true);       // 10
    sc.add(p->dB, D4, true);       // 11
    sc.add(p->dC, D4, true);       // 12
    sc.add(p->ddelta, L4, true);   // 13
    if (sc.stage_in(who)) {
        M1Args a{sc.dev<float>(0), sc.dev<float>(1), sc.dev<float>(2), sc.dev<float>(3),
                 sc.dev<float>(4), sc.dev<float>(5), sc.dev<float>(6), sc.dev<float>(7),
                 sc.dev<float>(8), sc.dev<float>(9), sc.dev<float>(10), sc.dev<float>(11),
                 sc.dev<float>(12), sc.dev<float>(13), p->L, p->D, nullptr, taylor};
        if (m1_launch(a, nullptr) == 0) sc.stage_out(who);
    }
    Staging::unlock();
}

// The reference's assembly routines (scan1d_backward_m1_shared_bc_asm and
// _simple_asm) check only p; with L or D zero they still clear the
// outputs of the other size (dA, dB, dC when L = 0; ddelta when D = 0).
// Here every output they write must be present, and a missing buffer or a
// negative size is an error instead of a fault.
static void m1_asm_call(ScanBackwardSharedParams *p, int taylor, const char *who) {
    clear_error();
    if (!p || p->L < 0 || p->D < 0) {
        set_error("%s: invalid parameters", who);
        return;
    }
    const bool work = p->L > 0 && p->D > 0;
    if ((work && (!p->x || !p->A || !p->B || !p->C || !p->delta || !p->h || !p->dy || !p->dx)) ||
        (p->D > 0 && (!p->dA || !p->dB || !p->dC)) || (p->L > 0 && !p->ddelta)) {
        set_error("%s: invalid parameters", who);
        return;
    }
    if (p->L == 0 && p->D == 0) return;
    if (!gpu_ready()) return;
    if (work) {
        m1_host_call(p, taylor, who);
        return;
    }
    // One size is zero: the outputs of the other are cleared on the device.
    Staging::lock();
    StagedCall sc;
    const size_t D4 = p->D * 4, L4 = p->L * 4;
    if (p->D > 0) {
        sc.add(p->dA, D4, true);
        sc.add(p->dB, D4, true);
        sc.add(p->dC, D4, true);
    } else {
        sc.add(p->ddelta, L4, true);
    }
    if (sc.stage_in(who)) {
        bool ok = true;
        for (int i = 0; i < sc.n && ok; ++i)
            ok = hipMemsetAsync(sc.bufs[i].dev, 0, sc.bufs[i].bytes, nullptr) == hipSuccess;
        if (!ok) set_error("%s: %s", who, hipGetErrorString(hipGetLastError()));
        else sc.stage_out(who);
    }
    Staging::unlock();
}

}  // namespace km

extern "C" {

// Reference scan1d_backward_m1_shared_bc (cpu/scan1d_backward.c:17-191):
// M = 1; B, C, dA, dB, dC [D]; delta, ddelta [L]; x, h, dy, dx [L, D];
// A_diag [L, D] precomputed decays or NULL; h0 [D] or NULL.
void scan1d_backward_m1_shared_bc(ScanBackwardSharedParams *p) {
    km::clear_error();
    if (!p || !p->x || !p->A || !p->B || !p->C || !p->delta || !p->h || !p->dy || !p->dx ||
        !p->dA || !p->dB || !p->dC || !p->ddelta || p->L <= 0 || p->D <= 0) {
        km::set_error("scan1d_backward_m1_shared_bc: invalid parameters");
        return;
    }
    if (!km::gpu_ready()) return;
    km::m1_host_call(p, 0, "scan1d_backward_m1_shared_bc");
}

// Reference scan1d_backward_m1_shared_bc_asm (include/scan.h:103,
// cpu/scan1d_backward_m1_shared_bc.asm): the same recurrence; without
// A_diag the decay is the routine's third-order Taylor polynomial.
void scan1d_backward_m1_shared_bc_asm(ScanBackwardSharedParams *p) {
    km::m1_asm_call(p, 1, "scan1d_backward_m1_shared_bc_asm");
}

// Reference scan1d_backward_m1_shared_bc_simple_asm (include/scan.h:104,
// cpu/scan1d_backward_m1_shared_bc_simple.asm): as above, the scalar
// routine's polynomial constants.
void scan1d_backward_m1_shared_bc_simple_asm(ScanBackwardSharedParams *p) {
    km::m1_asm_call(p, 2, "scan1d_backward_m1_shared_bc_simple_asm");
}

void mamba_scan1d_backward_m1_shared_bc(MambaScan1DBackwardM1Params *p) {
    scan1d_backward_m1_shared_bc(p);
}

}  // extern "C"

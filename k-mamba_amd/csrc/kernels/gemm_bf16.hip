// gemm_bf16.hip - bf16 GEMM on the gfx950 matrix cores (MFMA), fp32
// accumulate, for the Mamba block projections:
//   C[M, N] = epi(A[M, K] . B[N, K]^T + bias[N])
// A and B are row-major bf16 with leading dimensions lda, ldb (B holds the
// weights as [out, in], like a linear layer); C is fp32 or bf16 with ldc.
//
// Design: a 256-thread workgroup computes a 128 x 128 tile of C; each of its
// 4 waves owns a 64 x 64 quarter as 2 x 2 v_mfma_f32_32x32x16_bf16 tiles
// (64 fp32 accumulators per lane). K advances in steps of 64: the next
// step's A and B tiles are loaded from global memory into registers while
// the current step runs from LDS (double-buffered), so one barrier per step
// separates the LDS write of step k+1 from the reads of step k. LDS rows are
// 64 bf16 (eight 16-byte chunks) with chunk c of row r stored at c ^ (r & 7),
// so the 32 rows a fragment read touches fall on different banks. Loads go
// through raw buffer resources: rows past M (or N) read as zero, and the K
// tail is masked per 16-byte chunk (K must be a multiple of 8).
#include <algorithm>
#include <cstdlib>

#include "km_device.hpp"
#include "../km_runtime.hpp"
#include "kmamba_km.h"

namespace km {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

struct GemmArgs {
    const uint16_t *A, *B;
    void *C;
    const float *bias;
    long M, N, K, lda, ldb, ldc;
    int c_bf16;
    int epi;
    // Split output (256 x 256 kernel): columns [nsplit, N) go to C2 (same
    // ldc) at column - nsplit; nsplit is a multiple of the tile width.
    void *C2;
    long nsplit;
};

constexpr int kBM = 128, kBN = 128, kBK = 64;

template <int EPI>
__device__ __forceinline__ float epilogue(float v) {
    // softplus: log(1 + e^v) as in reference include/kmamba_kernels.h:47-49
    // (which has no overflow guard: v > 88 gives inf there, v here).
    if constexpr (EPI == KM_EPI_SOFTPLUS) return softplus_fast(v);
    else if constexpr (EPI == KM_EPI_SILU) return silu_fast(v);
    else return v;
}

// Epilogue of one wave's TI x TJ grid of 32 x 32 MFMA tiles at (row0, col0)
// of C: bias, activation and conversion, staged through the wave's 16 KB of
// LDS (row-major, a few row tiles per pass) so that C is written with
// 16-byte stores of whole row segments instead of one scalar store per
// element. The accumulator r of lane l holds row 8*(r/4) + 4*(l/32) + r%4,
// column l%32 of its tile. Chunks that cross the N edge, or a C whose rows
// are not 16-byte aligned, are stored element by element.
template <int EPI, bool CBF16, int TI, int TJ>
__device__ __forceinline__ void store_wave_tile(const GemmArgs &p, const f32x16 (&acc)[TI][TJ],
                                                long row0, long col0, char *lds, int lane) {
    constexpr int ES = CBF16 ? 2 : 4;
    constexpr int ROWB = TJ * 32 * ES;                 // LDS bytes per row
    constexpr int RC = (16384 / ROWB) < TI * 32 ? (16384 / ROWB) : TI * 32;   // rows per pass
    static_assert(RC % 32 == 0 && (TI * 32) % RC == 0, "whole row tiles per pass");
    constexpr int CPR = ROWB / 16;                     // 16-byte chunks per row
    constexpr int EPC = 16 / ES;                       // elements per chunk
    const int fr = lane & 31, fk = lane >> 5;
    const bool vec = ((p.ldc * ES) % 16 == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15) == 0);
    float bv[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const long col = col0 + j * 32 + fr;
        bv[j] = (p.bias && col < p.N) ? p.bias[col] : 0.f;
    }
#pragma unroll
    for (int pass = 0; pass < TI * 32 / RC; ++pass) {
#pragma unroll
        for (int ii = 0; ii < RC / 32; ++ii) {
            const int i = pass * (RC / 32) + ii;
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int rr = ii * 32 + 8 * (r >> 2) + 4 * fk + (r & 3);
                    const float v = epilogue<EPI>(acc[i][j][r] + bv[j]);
                    char *dst = lds + rr * ROWB + (j * 32 + fr) * ES;
                    if constexpr (CBF16) *reinterpret_cast<uint16_t *>(dst) = f32_to_bf16(v);
                    else *reinterpret_cast<float *>(dst) = v;
                }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);            // lgkmcnt(0): this wave's LDS writes done
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int q = 0; q < RC * CPR / 64; ++q) {
            const int idx = q * 64 + lane;
            const int rr = idx / CPR, cb = idx % CPR;
            const long row = row0 + pass * RC + rr;
            const long col = col0 + cb * EPC;
            const u32x4 v = *reinterpret_cast<const u32x4 *>(lds + rr * ROWB + cb * 16);
            if (row >= p.M || col >= p.N) continue;
            char *g = static_cast<char *>(p.C) + (row * p.ldc + col) * ES;
            if (vec && col + EPC <= p.N) {
                *reinterpret_cast<u32x4 *>(g) = v;
            } else {
                const char *src = reinterpret_cast<const char *>(&v);
                for (int e = 0; e < EPC && col + e < p.N; ++e)
                    for (int b = 0; b < ES; ++b) g[e * ES + b] = src[e * ES + b];
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);            // reads done before the next pass writes
        __builtin_amdgcn_wave_barrier();
    }
}

template <int EPI, bool CBF16>
__global__ void __launch_bounds__(256, 2) gemm_bf16_mfma(GemmArgs p) {
    __shared__ u32x4 sA[2][kBM * 8];
    __shared__ u32x4 sB[2][kBN * 8];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = w >> 1, wn = w & 1;
    long mb, nb;
    xcd_tile(mb, nb);                  // tiles of one row block share an XCD's L2
    const long m0 = mb * kBM;
    const long n0 = nb * kBN;

    // Windows over the rows this workgroup reads (offsets stay below 2 GiB:
    // the launcher splits M so that a window fits).
    const long arows = std::min<long>(kBM, p.M - m0), brows = std::min<long>(kBN, p.N - n0);
    const auto rA = make_rsrc(p.A + m0 * p.lda, (arows - 1) * p.lda * 2 + p.K * 2);
    const auto rB = make_rsrc(p.B + n0 * p.ldb, (brows - 1) * p.ldb * 2 + p.K * 2);

    u32x4 ga[4], gb[4];
    auto gload = [&](long k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + i * 256;
            const int row = c >> 3, ch = c & 7;
            const long k = k0 + ch * 8;
            const bool kin = k < p.K;
            const int offa = static_cast<int>((row * p.lda + k) * 2);
            const int offb = static_cast<int>((row * p.ldb + k) * 2);
            // rows past the window lie past the resource end and read 0
            ga[i] = kin && row < arows ? __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rA, offa, 0, 0))
                                       : u32x4{0, 0, 0, 0};
            gb[i] = kin && row < brows ? __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rB, offb, 0, 0))
                                       : u32x4{0, 0, 0, 0};
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + i * 256;
            const int row = c >> 3, ch = c & 7;
            sA[buf][row * 8 + (ch ^ (row & 7))] = ga[i];
            sB[buf][row * 8 + (ch ^ (row & 7))] = gb[i];
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const long nk = (p.K + kBK - 1) / kBK;
    gload(0);
    sstore(0);
    __syncthreads();
    const int fr = lane & 31;        // fragment row (A) / column (B) within a 32-tile
    const int fk = lane >> 5;        // which 8-wide k group of a 16-wide step
    for (long kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * kBK);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int ch = kk * 2 + fk;
            bf16x8 af[2], bfr[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int ra = wm * 64 + i * 32 + fr;
                af[i] = __builtin_bit_cast(bf16x8, sA[buf][ra * 8 + (ch ^ (ra & 7))]);
                const int rb = wn * 64 + i * 32 + fr;
                bfr[i] = __builtin_bit_cast(bf16x8, sB[buf][rb * 8 + (ch ^ (rb & 7))]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) sstore(buf ^ 1);
        __syncthreads();
    }

    // The loop ended with a barrier after every wave's last LDS read: each
    // wave now stages its tile through 16 KB of the operand buffers.
    char *lds = (w < 2 ? reinterpret_cast<char *>(&sA[0][0]) : reinterpret_cast<char *>(&sB[0][0])) +
                (w & 1) * 16384;
    store_wave_tile<EPI, CBF16, 2, 2>(p, acc, m0 + wm * 64, n0 + wn * 64, lds, lane);
}

// Large shapes: a 512-thread workgroup computes a 256 x 256 tile of C
// (gemm_bf16_mfma_pp below), K in stages of 32.
constexpr int kGM = 256, kGN = 256, kGK = 32;   // rows, columns, k per stage

// Shallow shapes (K <= 64: dt_proj): K is one block of 64, so each
// workgroup loads its operands once. A wave computes a 32 x 32*TN block of
// C and the 4 waves of a workgroup take 4 consecutive row blocks (workgroup
// tile 128 x 32*TN), so the B rows (the workgroup's 32*TN columns) are
// shared: they go straight from HBM into LDS (gfx950 buffer_load_dwordx4 ...
// lds, 8 whole 128-byte rows per instruction), each wave's 32 A rows
// straight into registers. Lane l < 32 takes row l's first 32 k and lane
// l + 32 its last 32, four 16-byte chunks each, and MFMA step s takes chunk
// s of both halves: the order of the terms of a dot product is free, and A
// and B use the same one. LDS slot row * 8 + pc holds chunk pc ^ (row & 7)
// of its B row. Chunks past K load as zero (out-of-range offset).
template <int EPI, bool CBF16, int TN>
__global__ void __launch_bounds__(256) gemm_bf16_direct(GemmArgs p) {
    constexpr int ES = CBF16 ? 2 : 4;
    constexpr int CPB = 4;                             // 16-byte chunks per lane
    constexpr int KB = 16 * CPB;                       // k per block
    constexpr int NBI = 32 * TN * 8 / 256;             // B load instructions per wave
    __shared__ __attribute__((aligned(16))) char stage[4][32 * TN * 32 * ES];
    __shared__ u32x4 sB[32 * TN * 8];
    constexpr unsigned kDrop = 0x80000000u;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int fr = lane & 31, fh = lane >> 5;
    long mb, nb;
    xcd_tile(mb, nb);
    const long m0 = mb * 128 + w * 32;
    const long n0 = nb * (32 * TN);
    const long arows = std::min<long>(32, p.M - m0), brows = std::min<long>(32 * TN, p.N - n0);
    const auto rA = make_rsrc(p.A + (arows > 0 ? m0 : 0) * p.lda,
                              arows > 0 ? (arows - 1) * p.lda * 2 + p.K * 2 : 0);
    const auto rB = make_rsrc(p.B + n0 * p.ldb, brows > 0 ? (brows - 1) * p.ldb * 2 + p.K * 2 : 0);
    const int aoff = fr * static_cast<int>(p.lda) * 2;
    bf16x8 a0[CPB];
#pragma unroll
    for (int c = 0; c < CPB; ++c) {
        const long k = (KB / 2) * fh + 8 * c;
        const int off = static_cast<int>(k < p.K ? static_cast<unsigned>(aoff + k * 2) : kDrop);
        a0[c] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rA, off, 0, 0));
    }
    using lds_t = __attribute__((address_space(3))) void *;
#pragma unroll
    for (int i = 0; i < NBI; ++i) {
        const int slot = (w + 4 * i) * 64 + lane;
        const int row = slot >> 3, c = (slot & 7) ^ (row & 7);
        const unsigned off = c * 8 < p.K ? static_cast<unsigned>(row * p.ldb * 2 + c * 16) : kDrop;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_t)(sB + (w + 4 * i) * 64), 16, off, 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);                // vmcnt(0): this wave's loads done
    __syncthreads();                                   // ... and every wave's B rows
    f32x16 acc[1][TN];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[0][j][r] = 0.f;
#pragma unroll
    for (int c = 0; c < CPB; ++c)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int rb = j * 32 + fr, ch = fh * CPB + c;
            const bf16x8 bf = __builtin_bit_cast(bf16x8, sB[rb * 8 + (ch ^ (rb & 7))]);
            acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[c], bf, acc[0][j], 0, 0, 0);
        }
    store_wave_tile<EPI, CBF16, 1, TN>(p, acc, m0, n0, stage[w], lane);
}

// The 256x256 tile on eight waves, two per SIMD, in ping-pong: waves w and
// w + 4 share a SIMD; wave (g, s) = (w / 4, w % 4) owns rows [128 g, +128)
// and columns [64 s, +64) of the tile (4 x 2 MFMA tiles, 128 accumulators).
// Each stage of 32 k is two phases per wave: a memory phase (its 12 fragment
// reads of the stage from LDS, its 4 of the 32 direct-to-LDS loads of the
// stage three ahead, then waits for both) and a compute phase (16 MFMAs on
// the fragments in registers). Group 1 runs one phase behind group 0, every
// phase ends at a workgroup barrier, so on each SIMD one wave computes while
// the other moves data and the matrix core is fed from alternate waves
// (one wave per SIMD issuing both measured 6-9 % slower on the block's
// projection shapes). Operands go straight from HBM into LDS (gfx950
// buffer_load_dwordx4 ... lds, no staging registers) through four stage
// buffers per operand (separate arrays, so the compiler's wait counts track
// each apart): a stage of A (or B) is 256 rows x 4 chunks of 16 B, LDS slot
// row * 4 + pc holding chunk pc ^ ((row >> 2) & 3) of its row, so the 16
// rows a quarter-wave's fragment read touches land on 16 distinct 16-byte
// bank slots. Buffer reuse: the loads of stage k + 3, issued in a memory
// phase of stage k, overwrite stage k - 1's buffer, which both groups
// finished reading (waited) before the phase barriers that precede it.
template <int EPI, bool CBF16>
__global__ void __launch_bounds__(512, 1) gemm_bf16_mfma_pp(GemmArgs p) {
    __shared__ u32x4 sA0[kGM * 4], sA1[kGM * 4], sA2[kGM * 4], sA3[kGM * 4];
    __shared__ u32x4 sB0[kGN * 4], sB1[kGN * 4], sB2[kGN * 4], sB3[kGN * 4];
    constexpr unsigned kDrop = 0x80000000u;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = w >> 2, sg = w & 3;
    long mb, nb;
    xcd_tile(mb, nb);
    const long m0 = mb * kGM;
    const long n0 = nb * kGN;
    const long arows = std::min<long>(kGM, p.M - m0), brows = std::min<long>(kGN, p.N - n0);
    const auto rA = make_rsrc(p.A + m0 * p.lda, (arows - 1) * p.lda * 2 + p.K * 2);
    const auto rB = make_rsrc(p.B + n0 * p.ldb, (brows - 1) * p.ldb * 2 + p.K * 2);
    // Load instruction i (0, 1) of wave w fills LDS slots [64 (2w + i), +64):
    // slot = row * 4 + pc holds chunk pc ^ ((row >> 2) & 3) of its row.
    int arow_off[2], brow_off[2], chk[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int slot = (w * 2 + i) * 64 + lane;
        const int row = slot >> 2, pc = slot & 3;
        chk[i] = pc ^ ((row >> 2) & 3);
        arow_off[i] = static_cast<int>(row * p.lda * 2);
        brow_off[i] = static_cast<int>(row * p.ldb * 2);
    }
    using lds_t = __attribute__((address_space(3))) void *;
    auto dma = [&](long kt, u32x4 *dA, u32x4 *dB) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const long k = kt * kGK + chk[i] * 8;
            const bool kin = k < p.K;
            const unsigned oa = kin ? static_cast<unsigned>(arow_off[i] + k * 2) : kDrop;
            const unsigned ob = kin ? static_cast<unsigned>(brow_off[i] + k * 2) : kDrop;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_t)(dA + (w * 2 + i) * 64), 16, oa, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_t)(dB + (w * 2 + i) * 64), 16, ob, 0, 0, 0);
        }
    };
    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    const int fr = lane & 31, fk = lane >> 5;
    bf16x8 fa[2][4], fb[2][2];          // [k half][tile]
    auto mem = [&](long kt, const u32x4 *bA, const u32x4 *bB, u32x4 *nA, u32x4 *nB)
        __attribute__((always_inline)) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int c = kk * 2 + fk;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ra = g * 128 + i * 32 + fr;
                fa[kk][i] = __builtin_bit_cast(bf16x8, bA[ra * 4 + (c ^ ((ra >> 2) & 3))]);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int rb = sg * 64 + j * 32 + fr;
                fb[kk][j] = __builtin_bit_cast(bf16x8, bB[rb * 4 + (c ^ ((rb >> 2) & 3))]);
            }
        }
        dma(kt + 3, nA, nB);
        __builtin_amdgcn_s_waitcnt(0x0F78);              // vmcnt(8): own loads of stage kt + 1 done
        __builtin_amdgcn_s_waitcnt(0xC07F);              // lgkmcnt(0): own fragment reads done
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        __builtin_amdgcn_sched_barrier(0);
    };
    auto comp = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[kk][i], fb[kk][j], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };
    const long nk = (p.K + kGK - 1) / kGK;
    dma(0, sA0, sB0);
    dma(1, sA1, sB1);
    dma(2, sA2, sB2);
    __builtin_amdgcn_s_waitcnt(0x0F78);                  // vmcnt(8): stage 0 loaded
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if (g == 1) __builtin_amdgcn_s_barrier();            // group 1 runs one phase behind
    __builtin_amdgcn_sched_barrier(0);
    for (long kt = 0; kt < nk; kt += 4) {
        mem(kt, sA0, sB0, sA3, sB3);
        comp();
        mem(kt + 1, sA1, sB1, sA0, sB0);
        comp();
        mem(kt + 2, sA2, sB2, sA1, sB1);
        comp();
        mem(kt + 3, sA3, sB3, sA2, sB2);
        comp();
    }
    if (g == 0) __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    char *lds = reinterpret_cast<char *>(w == 0 ? sA0 : w == 1 ? sA1 : w == 2 ? sA2 : w == 3 ? sA3
                                         : w == 4 ? sB0 : w == 5 ? sB1 : w == 6 ? sB2 : sB3);
    if (p.C2 && n0 >= p.nsplit) {
        GemmArgs q = p;
        q.C = p.C2;
        q.N = p.N - p.nsplit;
        q.bias = p.bias ? p.bias + p.nsplit : nullptr;
        store_wave_tile<EPI, CBF16, 4, 2>(q, acc, m0 + g * 128, n0 - p.nsplit + sg * 64, lds, lane);
    } else {
        if (p.C2) {
            GemmArgs q = p;
            q.N = p.nsplit;
            store_wave_tile<EPI, CBF16, 4, 2>(q, acc, m0 + g * 128, n0 + sg * 64, lds, lane);
        } else {
            store_wave_tile<EPI, CBF16, 4, 2>(p, acc, m0 + g * 128, n0 + sg * 64, lds, lane);
        }
    }
}

// Narrow shapes with a long K (N <= 128, K >= 512: x_proj): a workgroup
// computes 64 rows x 32*TN columns. Operands go straight from HBM into LDS
// (gfx950 buffer_load_dwordx4 ... lds) in stages of 128 k: a load
// instruction fills 4 whole rows of 256 bytes, so both operands stream in
// full cache lines (loading fragments straight into registers, one 16-byte
// piece of 32 rows per instruction, kept the texture unit busy at ~51 L1
// accesses per load). Three stage buffers, loads two stages ahead. Wave w
// takes rows 32 (w & 1) and the 64-k half (w >> 1) of every stage, so the
// B rows of a stage, the larger operand here, serve four waves; the two
// halves' partial sums are added in LDS (fixed order) before the epilogue.
// LDS slot row * 16 + pc holds 16-byte chunk pc ^ (row & 7) of its row: the
// eight rows a quarter of a fragment read touches fall on distinct banks.
template <int EPI, bool CBF16, int TN>
__global__ void __launch_bounds__(256) gemm_bf16_narrow(GemmArgs p) {
    constexpr int RA = 64, RB = 32 * TN, CH = 16;            // rows, 16-byte chunks per row per stage
    constexpr int KS = CH * 8;                                // k per stage
    constexpr int NI = (RA + RB) * CH / 64 / 4;               // load instructions per wave per stage
    static_assert((RA + RB) * CH % 256 == 0, "whole load instructions per wave");
    __shared__ u32x4 sA0[RA * CH], sA1[RA * CH], sA2[RA * CH];
    __shared__ u32x4 sB0[RB * CH], sB1[RB * CH], sB2[RB * CH];
    constexpr unsigned kDrop = 0x80000000u;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int half = w >> 1, rw = w & 1;
    long mb, nb;
    xcd_tile(mb, nb);
    const long m0 = mb * RA, n0 = nb * RB;
    const long arows = std::min<long>(RA, p.M - m0), brows = std::min<long>(RB, p.N - n0);
    const auto rA = make_rsrc(p.A + m0 * p.lda, (arows - 1) * p.lda * 2 + p.K * 2);
    const auto rB = make_rsrc(p.B + n0 * p.ldb, (brows - 1) * p.ldb * 2 + p.K * 2);
    // Load instruction i of wave w: the first NA fill A slots
    // [64 (w + 4 i), +64), the rest B slots [64 (w + 4 (i - NA)), +64).
    constexpr int NA = RA * CH / 256;
    int roff[NI], chk[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int slot = (w + 4 * (i < NA ? i : i - NA)) * 64 + lane;
        const int row = slot / CH, pc = slot % CH;
        chk[i] = pc ^ (row & 7);
        roff[i] = static_cast<int>(row * (i < NA ? p.lda : p.ldb) * 2);
    }
    using lds_t = __attribute__((address_space(3))) void *;
    auto dma = [&](long st, u32x4 *dA, u32x4 *dB) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const long k = st * KS + chk[i] * 8;
            const unsigned off = k < p.K ? static_cast<unsigned>(roff[i] + k * 2) : kDrop;
            if (i < NA)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_t)(dA + (w + 4 * i) * 64), 16, off, 0, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_t)(dB + (w + 4 * (i - NA)) * 64), 16, off, 0,
                                                         0, 0);
        }
    };
    f32x16 acc[1][TN];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[0][j][r] = 0.f;
    const int fr = lane & 31, fk = lane >> 5;
    auto compute = [&](const u32x4 *bA, const u32x4 *bB) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int c = half * 8 + ks * 2 + fk;
            const int ra = rw * 32 + fr;
            const bf16x8 af = __builtin_bit_cast(bf16x8, bA[ra * CH + (c ^ (ra & 7))]);
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int rb = j * 32 + fr;
                const bf16x8 bf = __builtin_bit_cast(bf16x8, bB[rb * CH + (c ^ (rb & 7))]);
                acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf, acc[0][j], 0, 0, 0);
            }
        }
    };
    const long nst = (p.K + KS - 1) / KS;
    dma(0, sA0, sB0);
    dma(1, sA1, sB1);
    // Groups of three stages with no branch inside; stages past K load
    // zeros and add nothing.
    for (long st = 0; st < nst; st += 3) {
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            u32x4 *cA = u == 0 ? sA0 : u == 1 ? sA1 : sA2;
            u32x4 *cB = u == 0 ? sB0 : u == 1 ? sB1 : sB2;
            u32x4 *nA = u == 0 ? sA2 : u == 1 ? sA0 : sA1;
            u32x4 *nB = u == 0 ? sB2 : u == 1 ? sB0 : sB1;
            __builtin_amdgcn_s_waitcnt(0x0F70 | NI);             // vmcnt(NI): own loads of stage st + u done
            __builtin_amdgcn_s_barrier();                        // ... and every wave's; stage st + u - 1 read
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            __builtin_amdgcn_sched_barrier(0);
            dma(st + u + 2, nA, nB);
            compute(cA, cB);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // The second k half's partials, added by the first half's waves.
    float *red = reinterpret_cast<float *>(sB0);              // [2 waves][TN * 16][64]: TN * 8 KB
    if (half == 1) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) red[(rw * TN * 16 + j * 16 + r) * 64 + lane] = acc[0][j][r];
    }
    __syncthreads();
    if (half == 1) return;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[0][j][r] += red[(rw * TN * 16 + j * 16 + r) * 64 + lane];
    char *lds = reinterpret_cast<char *>(rw == 0 ? sA1 : sA2);
    store_wave_tile<EPI, CBF16, 1, TN>(p, acc, m0 + rw * 32, n0, lds, lane);
}

template <int EPI>
static void gemm_go(const GemmArgs &a, dim3 g, bool big, hipStream_t s) {
    if (big) {
        if (a.c_bf16) hipLaunchKernelGGL((gemm_bf16_mfma_pp<EPI, true>), g, dim3(512), 0, s, a);
        else          hipLaunchKernelGGL((gemm_bf16_mfma_pp<EPI, false>), g, dim3(512), 0, s, a);
    } else {
        if (a.c_bf16) hipLaunchKernelGGL((gemm_bf16_mfma<EPI, true>), g, dim3(256), 0, s, a);
        else          hipLaunchKernelGGL((gemm_bf16_mfma<EPI, false>), g, dim3(256), 0, s, a);
    }
}

template <int EPI>
static void direct_go(const GemmArgs &a, dim3 g, hipStream_t s) {
    if (a.c_bf16) hipLaunchKernelGGL((gemm_bf16_direct<EPI, true, 4>), g, dim3(256), 0, s, a);
    else          hipLaunchKernelGGL((gemm_bf16_direct<EPI, false, 4>), g, dim3(256), 0, s, a);
}

template <int EPI, int TN>
static void narrow_go(const GemmArgs &a, dim3 g, hipStream_t s) {
    if (a.c_bf16) hipLaunchKernelGGL((gemm_bf16_narrow<EPI, true, TN>), g, dim3(256), 0, s, a);
    else          hipLaunchKernelGGL((gemm_bf16_narrow<EPI, false, TN>), g, dim3(256), 0, s, a);
}

template <int EPI>
static void narrow_by_tn(const GemmArgs &a, dim3 g, int tn, hipStream_t s) {
    switch (tn) {
    case 1: narrow_go<EPI, 1>(a, g, s); break;
    case 2: narrow_go<EPI, 2>(a, g, s); break;
    case 3: narrow_go<EPI, 3>(a, g, s); break;
    default: narrow_go<EPI, 4>(a, g, s); break;
    }
}

// Skinny shapes: N <= 128 with K >= 512 on gemm_bf16_narrow, K <= 64 on
// gemm_bf16_direct. Returns 1 when launched, 0 when the shape is neither,
// -1 on a launch error.
static int direct_launch(const KMGemm *g, hipStream_t s) {
    const bool narrow = g->N <= 128 && g->K >= 512;
    const bool shallow = g->K <= 64;
    if (!narrow && !shallow) return 0;
    const int tn = narrow ? static_cast<int>((g->N + 31) / 32) : 4;
    const long TM = narrow ? 64 : 128, TN = 32L * tn;
    if (g->ldb * 2 * (TN + 1) > 0x7fffffffL || g->lda * 2 * (TM + 1) > 0x7fffffffL) return 0;
    const long nbn = (g->N + TN - 1) / TN, nbm = (g->M + TM - 1) / TM;
    if (nbn > 0x7fffffffL) return 0;
    const long chunk = 65535;
    for (long mb = 0; mb < nbm; mb += chunk) {
        const long nb = std::min(chunk, nbm - mb);
        GemmArgs a{};
        a.A = static_cast<const uint16_t *>(g->A) + mb * TM * g->lda;
        a.B = static_cast<const uint16_t *>(g->B);
        a.c_bf16 = (g->c_dtype == KM_BF16);
        a.C = static_cast<char *>(g->C) + mb * TM * g->ldc * (a.c_bf16 ? 2 : 4);
        a.bias = g->bias;
        a.M = std::min(g->M - mb * TM, nb * TM);
        a.N = g->N; a.K = g->K; a.lda = g->lda; a.ldb = g->ldb; a.ldc = g->ldc;
        a.epi = g->epilogue;
        const dim3 grid(static_cast<unsigned>(nbn), static_cast<unsigned>(nb));
        if (narrow) {
            switch (g->epilogue) {
            case KM_EPI_SOFTPLUS: narrow_by_tn<KM_EPI_SOFTPLUS>(a, grid, tn, s); break;
            case KM_EPI_SILU:     narrow_by_tn<KM_EPI_SILU>(a, grid, tn, s); break;
            default:              narrow_by_tn<KM_EPI_NONE>(a, grid, tn, s); break;
            }
        } else {
            switch (g->epilogue) {
            case KM_EPI_SOFTPLUS: direct_go<KM_EPI_SOFTPLUS>(a, grid, s); break;
            case KM_EPI_SILU:     direct_go<KM_EPI_SILU>(a, grid, s); break;
            default:              direct_go<KM_EPI_NONE>(a, grid, s); break;
            }
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) {
            set_error("km_gemm_bf16: launch failed: %s", hipGetErrorString(e));
            return -1;
        }
    }
    return 1;
}

static int gemm_launch_impl(const KMGemm *g, void *C2, long nsplit, hipStream_t s);

int gemm_bf16_launch(const KMGemm *g, hipStream_t s) { return gemm_launch_impl(g, nullptr, 0, s); }

// One launch for C[:, :nsplit] and C2[:, :N - nsplit] = the two column
// ranges of one product (the Mamba block's in_proj x and z halves), both
// with g->ldc; two launches when the 256 x 256 kernel does not take the
// shape or nsplit is not a multiple of its tile width.
int gemm_bf16_launch_split(const KMGemm *g, void *C2, long nsplit, hipStream_t s) {
    if (!g || !C2 || nsplit <= 0 || nsplit >= g->N) {
        set_error("km_gemm_bf16: invalid split");
        return -1;
    }
    const bool big = g->M >= kGM && g->N >= kGN && g->K >= 4 * kGK && nsplit % kGN == 0 &&
                     g->ldb * 2 * (kGN + 1) <= 0x7fffffffL && g->lda * 2 * (kGM + 1) <= 0x7fffffffL &&
                     g->ldc >= nsplit && g->ldc >= g->N - nsplit;
    if (big) return gemm_launch_impl(g, C2, nsplit, s);
    KMGemm h = *g;
    h.N = nsplit;
    if (gemm_launch_impl(&h, nullptr, 0, s) != 0) return -1;
    h.B = static_cast<const uint16_t *>(g->B) + nsplit * g->ldb;
    h.C = C2;
    h.N = g->N - nsplit;
    if (g->bias) h.bias = g->bias + nsplit;
    return gemm_launch_impl(&h, nullptr, 0, s);
}

static int gemm_launch_impl(const KMGemm *g, void *C2, long nsplit, hipStream_t s) {
    if (!g || !g->A || !g->B || !g->C) { set_error("km_gemm_bf16: NULL pointer"); return -1; }
    if (g->M < 0 || g->N < 0 || g->K <= 0 || g->K % 8 != 0 || g->lda < g->K || g->ldb < g->K ||
        (!C2 && g->ldc < g->N) || g->lda % 8 != 0 || g->ldb % 8 != 0) {
        set_error("km_gemm_bf16: invalid shape M=%ld N=%ld K=%ld lda=%ld ldb=%ld ldc=%ld "
                  "(K, lda, ldb must be multiples of 8)", g->M, g->N, g->K, g->lda, g->ldb, g->ldc);
        return -1;
    }
    if (g->c_dtype != KM_F32 && g->c_dtype != KM_BF16) {
        set_error("km_gemm_bf16: unknown C dtype %d", g->c_dtype);
        return -1;
    }
    if (g->epilogue != KM_EPI_NONE && g->epilogue != KM_EPI_SOFTPLUS && g->epilogue != KM_EPI_SILU) {
        set_error("km_gemm_bf16: unknown epilogue %d", g->epilogue);
        return -1;
    }
    if (g->M == 0 || g->N == 0) return 0;
    if (!gpu_ready()) return -1;
    if (!C2)
        if (const int d = direct_launch(g, s)) return d > 0 ? 0 : -1;
    // 256 x 256 tiles when both output dimensions fill them (and K spans
    // at least a few stages); 128 x 128 otherwise.
    const bool big = g->M >= kGM && g->N >= kGN && g->K >= 4 * kGK &&
                     g->ldb * 2 * (kGN + 1) <= 0x7fffffffL && g->lda * 2 * (kGM + 1) <= 0x7fffffffL;
    if (C2 && !big) {
        set_error("km_gemm_bf16: split output needs the 256 x 256 kernel");
        return -1;
    }
    const long TM = big ? kGM : kBM, TN = big ? kGN : kBN;
    if (g->ldb * 2 * (TN + 1) > 0x7fffffffL || g->lda * 2 * (TM + 1) > 0x7fffffffL) {
        set_error("km_gemm_bf16: leading dimension too large");
        return -1;
    }
    const long nbn = (g->N + TN - 1) / TN;
    const long nbm = (g->M + TM - 1) / TM;
    if (nbn > 0x7fffffffL) { set_error("km_gemm_bf16: N too large"); return -1; }
    // Row blocks per launch stay within the 65535 grid-y limit.
    const long chunk = 65535;
    for (long mb = 0; mb < nbm; mb += chunk) {
        const long nb = std::min(chunk, nbm - mb);
        GemmArgs a{};
        a.A = static_cast<const uint16_t *>(g->A) + mb * TM * g->lda;
        a.B = static_cast<const uint16_t *>(g->B);
        a.c_bf16 = (g->c_dtype == KM_BF16);
        a.C = static_cast<char *>(g->C) + mb * TM * g->ldc * (a.c_bf16 ? 2 : 4);
        a.bias = g->bias;
        a.M = std::min(g->M - mb * TM, nb * TM);
        a.N = g->N; a.K = g->K; a.lda = g->lda; a.ldb = g->ldb; a.ldc = g->ldc;
        a.epi = g->epilogue;
        if (C2) {
            a.C2 = static_cast<char *>(C2) + mb * TM * g->ldc * (a.c_bf16 ? 2 : 4);
            a.nsplit = nsplit;
        }
        dim3 grid(static_cast<unsigned>(nbn), static_cast<unsigned>(nb));
        switch (g->epilogue) {
        case KM_EPI_SOFTPLUS: gemm_go<KM_EPI_SOFTPLUS>(a, grid, big, s); break;
        case KM_EPI_SILU:     gemm_go<KM_EPI_SILU>(a, grid, big, s); break;
        default:              gemm_go<KM_EPI_NONE>(a, grid, big, s); break;
        }
        KM_HIP_TRY(hipGetLastError());
    }
    return 0;
}

}  // namespace km

extern "C" int km_gemm_bf16(const KMGemm *g, void *stream) {
    km::clear_error();
    return km::gemm_bf16_launch(g, static_cast<hipStream_t>(stream));
}

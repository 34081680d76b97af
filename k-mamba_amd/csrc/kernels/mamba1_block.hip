// mamba1_block.hip - Mamba-1 block forward on gfx950.
//
// No single reference function: the block composes the reference pieces
// (kernels/gemm_f32.c:13-31 projections, the causal convnd of
// src/convnd.c:83-126 in 1D, SiLU / softplus of include/kmamba_kernels.h:35-49
// and the scan1d recurrence of cpu/scan1d.asm:53-169):
//   xi = x W_in[0:di]^T              z = x W_in[di:2di]^T        (MFMA GEMMs)
//   u  = SiLU(conv1d_causal(xi) + conv_b)                        (fused kernel)
//   xdbl = u W_x^T = [dt_low | B | C]                            (MFMA GEMM)
//   delta = softplus(dt_low W_dt^T + dt_bias)                    (MFMA GEMM, epilogue)
//   y  = (scan(u, delta, A, B, C) + Dskip*u) * SiLU(z)           (scan, gated store)
//   out = y W_out^T                                              (MFMA GEMM)
// Activations are bf16 between kernels, state and accumulation fp32. B and C
// are read by the scan straight out of xdbl through its B/C strides.
#include <algorithm>

#include "km_device.hpp"
#include "../km_runtime.hpp"
#include "kmamba_km.h"

namespace km {

int scan1d_fwd_launch(const KMScan1DFwd *k, hipStream_t stream, bool allow_split);
int gemm_bf16_launch(const KMGemm *g, hipStream_t s);
int gemm_bf16_launch_split(const KMGemm *g, void *C2, long nsplit, hipStream_t s);

constexpr int kConvStrip = 64;

// u[b,t,d] = SiLU(bias[d] + sum_k x[b, t-(KC-1-k), d] * w[k, d]), taps before
// t = 0 skipped (the causal convnd in 1D). One thread per channel pair and
// strip of kConvStrip steps; 64 lanes read 256 contiguous bytes per step.
// The strip's inputs are all loaded before the arithmetic (one memory
// latency per strip); rows past L read 0 and their stores are dropped by the
// buffer range check.
template <int KC>
__global__ void __launch_bounds__(256) conv1d_silu_bf16(const uint32_t *x, const float *w,
                                                        const float *bias, uint32_t *u, long L,
                                                        long D, int kc_rt) {
    const int K = KC > 0 ? KC : kc_rt;
    const long c = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;   // channel pair
    const long D2 = D / 2;
    if (c >= D2) return;
    const long b = blockIdx.z;
    const int t0 = static_cast<int>(blockIdx.y) * kConvStrip;
    const auto rx = make_rsrc(x + b * L * D2, L * D2 * 4);
    const auto ru = make_rsrc(u + b * L * D2, L * D2 * 4);
    const int row = static_cast<int>(D2) * 4, lane_off = static_cast<int>(c) * 4;
    uint32_t xv[kConvStrip];
#pragma unroll
    for (int i = 0; i < kConvStrip; ++i)
        xv[i] = __builtin_amdgcn_raw_buffer_load_b32(rx, lane_off + (t0 + i) * row, 0, 0);
    float w0[8], w1[8];
    for (int k = 0; k < K; ++k) {
        w0[k] = w[k * D + 2 * c];
        w1[k] = w[k * D + 2 * c + 1];
    }
    const float b0 = bias ? bias[2 * c] : 0.f, b1 = bias ? bias[2 * c + 1] : 0.f;
    float h0[8], h1[8];                      // inputs at t-(K-1) .. t
    for (int k = 0; k < K - 1; ++k) {
        const int t = t0 - (K - 1) + k;
        const uint32_t v = t >= 0 ? __builtin_amdgcn_raw_buffer_load_b32(rx, lane_off + t * row, 0, 0) : 0u;
        h0[k + 1] = bf16_to_f32(static_cast<uint16_t>(v & 0xffff));
        h1[k + 1] = bf16_to_f32(static_cast<uint16_t>(v >> 16));
    }
#pragma unroll
    for (int i = 0; i < kConvStrip; ++i) {
        for (int k = 0; k < K - 1; ++k) {
            h0[k] = h0[k + 1];
            h1[k] = h1[k + 1];
        }
        h0[K - 1] = bf16_to_f32(static_cast<uint16_t>(xv[i] & 0xffff));
        h1[K - 1] = bf16_to_f32(static_cast<uint16_t>(xv[i] >> 16));
        float s0 = b0, s1 = b1;
        for (int k = 0; k < K; ++k) {
            s0 += h0[k] * w0[k];
            s1 += h1[k] * w1[k];
        }
        s0 = silu_fast(s0);
        s1 = silu_fast(s1);
        __builtin_amdgcn_raw_buffer_store_b32(f32x2_to_bf16x2(s0, s1), ru, lane_off + (t0 + i) * row, 0, 0);
    }
}

struct BlockLayout {
    size_t xi, z, u, xdbl, delta, y, bytes;
};

static BlockLayout block_layout(const KMMamba1Weights *w, long B, long L) {
    BlockLayout l{};
    const size_t T = static_cast<size_t>(B) * L;
    const size_t act = align_up(T * w->d_inner * 2, 256);
    size_t off = 0;
    l.xi = off; off += act;
    l.z = off; off += act;
    l.u = off; off += act;
    l.delta = off; off += act;
    l.y = off; off += act;
    l.xdbl = off; off += align_up(T * (w->dt_rank + 2 * w->d_state) * 2, 256);
    l.bytes = off;
    return l;
}

static bool block_ok(const KMMamba1Weights *w, const void *x, const void *out, long B, long L) {
    if (!w || !x || !out || !w->W_in || !w->conv_w || !w->W_x || !w->W_dt || !w->dt_bias ||
        !w->A || !w->W_out) {
        set_error("km_mamba1_block_fwd: NULL pointer");
        return false;
    }
    if (B <= 0 || L <= 0 || w->dim <= 0 || w->d_inner <= 0 || w->d_state <= 0 || w->d_state > 64 ||
        w->d_conv <= 0 || w->d_conv > 8 || w->dt_rank <= 0 || w->dim % 8 || w->d_inner % 8 ||
        w->dt_rank % 8 || (w->dt_rank + 2 * w->d_state) % 8) {
        set_error("km_mamba1_block_fwd: unsupported shape dim=%ld d_inner=%ld d_state=%ld "
                  "d_conv=%ld dt_rank=%ld (dim, d_inner, dt_rank, dt_rank+2*d_state multiples "
                  "of 8; d_state <= 64; d_conv <= 8)", w->dim, w->d_inner, w->d_state, w->d_conv,
                  w->dt_rank);
        return false;
    }
    return true;
}

size_t mamba1_workspace(const KMMamba1Weights *w, long B, long L) {
    if (!w || B <= 0 || L <= 0) return 0;
    return block_layout(w, B, L).bytes;
}

int mamba1_block_fwd(const KMMamba1Weights *w, const void *x, void *out, long B, long L,
                     void *workspace, size_t ws_bytes, hipStream_t s) {
    if (!block_ok(w, x, out, B, L)) return -1;
    if (!gpu_ready()) return -1;
    const BlockLayout lay = block_layout(w, B, L);
    char *ws = static_cast<char *>(workspace);
    if (ws) {
        if (ws_bytes < lay.bytes) {
            set_error("km_mamba1_block_fwd: workspace of %zu bytes, %zu needed", ws_bytes, lay.bytes);
            return -1;
        }
    } else {
        ws = static_cast<char *>(Workspace::reserve(lay.bytes, s, WsUse::Block));
        if (!ws) return -1;
    }
    const long T = B * L, di = w->d_inner, N = w->d_state, R = w->dt_rank, NX = R + 2 * N;
    auto *xi = ws + lay.xi, *z = ws + lay.z, *u = ws + lay.u, *xdbl = ws + lay.xdbl,
         *delta = ws + lay.delta, *y = ws + lay.y;
    const uint16_t *Win = static_cast<const uint16_t *>(w->W_in);

    // Every projection runs on the hand-written bf16 MFMA GEMM (km_gemm_bf16).
    auto plain = [&](const KMGemm &g) { return gemm_bf16_launch(&g, s); };
    KMGemm g{};
    g.c_dtype = KM_BF16;
    // in_proj: x and z halves of one product (columns [0, di) -> xi,
    // [di, 2 di) -> z), one launch
    g.A = x; g.B = Win; g.C = xi; g.M = T; g.N = 2 * di; g.K = w->dim;
    g.lda = w->dim; g.ldb = w->dim; g.ldc = di; g.epilogue = KM_EPI_NONE;
    if (gemm_bf16_launch_split(&g, z, di, s) != 0) return -1;
    g.N = di;
    // causal depthwise conv1d + SiLU
    {
        dim3 grid(static_cast<unsigned>((di / 2 + 255) / 256),
                  static_cast<unsigned>((L + kConvStrip - 1) / kConvStrip), static_cast<unsigned>(B));
        // The conv kernel addresses one sequence (plus a strip past its end)
        // with 32-bit byte offsets.
        if (grid.y > 65535 || grid.z > 65535 || (L + kConvStrip) * di * 2 > 0x7fffffffL) {
            set_error("km_mamba1_block_fwd: sequence or batch too large");
            return -1;
        }
        const auto *xin = reinterpret_cast<const uint32_t *>(xi);
        auto *uo = reinterpret_cast<uint32_t *>(u);
        switch (w->d_conv) {
        case 4: hipLaunchKernelGGL(conv1d_silu_bf16<4>, grid, dim3(256), 0, s, xin, w->conv_w, w->conv_b, uo, L, di, 4); break;
        case 3: hipLaunchKernelGGL(conv1d_silu_bf16<3>, grid, dim3(256), 0, s, xin, w->conv_w, w->conv_b, uo, L, di, 3); break;
        case 2: hipLaunchKernelGGL(conv1d_silu_bf16<2>, grid, dim3(256), 0, s, xin, w->conv_w, w->conv_b, uo, L, di, 2); break;
        default: hipLaunchKernelGGL(conv1d_silu_bf16<0>, grid, dim3(256), 0, s, xin, w->conv_w, w->conv_b, uo, L, di,
                                    static_cast<int>(w->d_conv)); break;
        }
        KM_HIP_TRY(hipGetLastError());
    }
    // x_proj -> [dt_low | B | C]
    g.A = u; g.B = w->W_x; g.C = xdbl; g.M = T; g.N = NX; g.K = di;
    g.lda = di; g.ldb = di; g.ldc = NX;
    if (plain(g) != 0) return -1;
    // dt_proj + bias + softplus
    g.A = xdbl; g.B = w->W_dt; g.C = delta; g.M = T; g.N = di; g.K = R;
    g.lda = NX; g.ldb = R; g.ldc = di; g.bias = w->dt_bias; g.epilogue = KM_EPI_SOFTPLUS;
    if (gemm_bf16_launch(&g, s) != 0) return -1;
    // selective scan with the skip and SiLU(z) gate fused into its store
    KMScan1DFwd k{};
    k.x = u; k.delta = delta; k.A = w->A;
    k.Bm = reinterpret_cast<uint16_t *>(xdbl) + R;
    k.Cm = reinterpret_cast<uint16_t *>(xdbl) + R + N;
    k.y = y; k.B = B; k.L = L; k.D = di; k.N = N;
    k.bc_sb = L * NX; k.bc_st = NX; k.bc_sd = 0;
    k.dtype = KM_BF16; k.clamp = w->clamp;
    k.z = z; k.Dskip = w->Dskip;
    if (scan1d_fwd_launch(&k, s, true) != 0) return -1;
    // out_proj
    KMGemm o{};
    o.A = y; o.B = w->W_out; o.C = out; o.M = T; o.N = w->dim; o.K = di;
    o.lda = di; o.ldb = di; o.ldc = w->dim; o.c_dtype = KM_BF16; o.epilogue = KM_EPI_NONE;
    return plain(o);
}

}  // namespace km

extern "C" {

size_t km_mamba1_block_workspace_bytes(const KMMamba1Weights *w, long B, long L) {
    km::clear_error();
    return km::mamba1_workspace(w, B, L);
}

int km_mamba1_block_fwd(const KMMamba1Weights *w, const void *x, void *out, long B, long L,
                        void *workspace, size_t workspace_bytes, void *stream) {
    km::clear_error();
    return km::mamba1_block_fwd(w, x, out, B, L, workspace, workspace_bytes,
                                static_cast<hipStream_t>(stream));
}

}  // extern "C"

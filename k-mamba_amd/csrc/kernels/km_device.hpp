// km_device.hpp - device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace km {

constexpr float kLog2e = 1.4426950408889634f;

// Steps between the forward-state checkpoints the Scan1D backward recomputes
// from (KM_SCAN1D_CKPT_STEPS of the public header).
constexpr int kCkptSteps = 32;

// Element type tags. Storage is fp32 or bfloat16; arithmetic is always fp32.
struct f32_t  { using storage = float; };
struct bf16_t { using storage = uint16_t; };

__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even fp32 -> bf16 on the gfx950 converter
// (v_cvt_pk_bf16_f32): the same bits as (u + 0x7fff + ((u >> 16) & 1)) >> 16
// for every non-NaN input, NaN kept NaN with its quiet bit set.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two values in one instruction: a in the low half, b in the high half.
typedef __bf16 km_bf16x2 __attribute__((ext_vector_type(2)));
typedef float km_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((km_f32x2{a, b}), km_bf16x2));
}

template <typename T> struct io;
template <> struct io<f32_t> {
    using S = float;
    static __device__ __forceinline__ float ld(const void *p, long i) {
        return static_cast<const float *>(p)[i];
    }
    static __device__ __forceinline__ void st(void *p, long i, float v) {
        static_cast<float *>(p)[i] = v;
    }
};
template <> struct io<bf16_t> {
    using S = uint16_t;
    static __device__ __forceinline__ float ld(const void *p, long i) {
        return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
    }
    static __device__ __forceinline__ void st(void *p, long i, float v) {
        static_cast<uint16_t *>(p)[i] = f32_to_bf16(v);
    }
};

// v(lane) + v(lane ^ 32) in every lane, on the VALU (gfx950
// v_permlane32_swap: the upper half of one copy trades places with the lower
// half of the other, so the two results hold each lane's value and its
// partner's). Same sum, bit for bit, as v + __shfl_xor(v, 32), without the
// LDS round trip of ds_bpermute.
__device__ __forceinline__ float sum_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// v(lane) + v(lane ^ 16) (v_permlane16_swap trades odd and even 16-lane rows).
__device__ __forceinline__ float sum_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// 2^x on the transcendental unit (v_exp_f32, ~1 ulp).
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// DPP lane move within rows of 16 lanes (ctrl: row_ror, mirrors, quad_perm).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                  0xf, 0xf, false));
}

// Reduce-scatter over the 16 lanes of each row, on DPP VALU operands only:
// lane l contributes yr[0..TW) and returns the row's total of value
// (l % 16) / (16 / TW). Each step keeps half of the remaining values and
// adds the partner's copy of that half; partners differ in one lane bit per
// step (xor 8 by row_ror:8, xor 7 by row_half_mirror, xor 2 and xor 1 by
// quad_perm), so the four steps cover all 16 lanes, as a butterfly does.
template <int CTRL, int BIT, int CNT, int TW>
__device__ __forceinline__ void readout_step(float (&cur)[TW], int l) {
    if constexpr (CNT > 1) {
        constexpr int H = CNT / 2;
        const bool hi = (l & BIT) != 0;
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const float keep = hi ? cur[H + i] : cur[i];
            const float send = hi ? cur[i] : cur[H + i];
            cur[i] = keep + dpp<CTRL>(send);
        }
    } else {
        cur[0] += dpp<CTRL>(cur[0]);
    }
}
template <int TW>
__device__ __forceinline__ float row_readout(const float (&yr)[TW]) {
    static_assert(TW == 4 || TW == 8 || TW == 16, "16 / TW lanes per column");
    const int l = threadIdx.x & 15;
    float cur[TW];
#pragma unroll
    for (int i = 0; i < TW; ++i) cur[i] = yr[i];
    readout_step<0x128, 8, TW>(cur, l);                         // row_ror:8 (l ^ 8)
    readout_step<0x141, 4, (TW > 2 ? TW / 2 : 1)>(cur, l);      // row_half_mirror (l ^ 7)
    readout_step<0x4E, 2, (TW > 4 ? TW / 4 : 1)>(cur, l);       // quad_perm [2,3,0,1] (l ^ 2)
    readout_step<0xB1, 1, (TW > 8 ? TW / 8 : 1)>(cur, l);       // quad_perm [1,0,3,2] (l ^ 1)
    return cur[0];
}

// Workgroup id in an order where consecutive ids share an XCD: the hardware
// deals workgroups to the 8 XCDs round-robin (XCD x runs ids x, x + 8, ...);
// this maps XCD x's ids to one contiguous range, so neighbouring tiles (which
// share operands) meet in one L2.
__device__ __forceinline__ long xcd_remap(long b, long nb) {
    const long q = nb / 8, r = nb % 8, x = b % 8;
    return x * q + (x < r ? x : r) + b / 8;
}

// (row block, column block) of a 2D grid of gx column blocks, numbered
// row-major in XCD order.
__device__ __forceinline__ void xcd_tile(long &mb, long &nb) {
    const long gx = gridDim.x, lin = static_cast<long>(blockIdx.y) * gx + blockIdx.x;
    const long t = xcd_remap(lin, gx * gridDim.y);
    mb = t / gx;
    nb = t % gx;
}

// SiLU v * sigmoid(v) = v / (1 + e^-v) on the hardware exp2 and reciprocal
// (about 1 ulp each) instead of the library exp and the IEEE division
// sequence; e^-v = inf gives rcp = 0, the limit.
__device__ __forceinline__ float silu_fast(float v) {
    return v * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-v * kLog2e));
}

// softplus log(1 + e^v) on the hardware exp2 / log2 (5 instructions instead
// of the library exp and log with their range reduction); v > 20 returns v,
// where log(1 + e^v) rounds to v in fp32 anyway.
constexpr float kLn2 = 0.6931471805599453f;
__device__ __forceinline__ float softplus_fast(float v) {
    return v > 20.f ? v : kLn2 * __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(v * kLog2e));
}

// Raw buffer resource over [base, base + bytes): loads past the end return 0
// and stores past the end are dropped by the hardware range check. Word 3 is
// the gfx9 raw-buffer format (no swizzle, 32-bit data).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, long bytes) {
    const int n = bytes > 0x7fffffffL ? 0x7fffffff : static_cast<int>(bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, n, 0x00020000);
}

// Element loads/stores through a buffer resource. voff: per-lane byte offset
// (range-checked); soff: wave-uniform SGPR byte offset, which the gfx9 raw
// buffer range check does NOT cover, so callers keep it 0 unless the access
// is known to be in bounds.
template <typename T> struct bio;
template <> struct bio<f32_t> {
    static constexpr int size = 4;
    static __device__ __forceinline__ float ld(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
    }
    static __device__ __forceinline__ void st(__amdgpu_buffer_rsrc_t r, int voff, int soff, float v) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, voff, soff, 0);
    }
    // Agent-coherent load (cache policy sc1): misses the CU's L1 and reads
    // the XCD's L2, so it sees stores another CU of the same XCD completed.
    static __device__ __forceinline__ float ld_agent(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 16));
    }
};
template <> struct bio<bf16_t> {
    static constexpr int size = 2;
    static __device__ __forceinline__ float ld(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
        return bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0));
    }
    static __device__ __forceinline__ void st(__amdgpu_buffer_rsrc_t r, int voff, int soff, float v) {
        __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(v), r, voff, soff, 0);
    }
};

}  // namespace km

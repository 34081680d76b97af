// mamba3_block.hip - the reference Mamba-3 block forward on gfx950.
//
// Reference: src/mamba_block.c:89-120 (controller projections), :413-466
// (scan), :471-501 (forward). Per batch element, with R = mimo rank:
//   u_t = SiLU(W_in x_t), dt_t = clamp(softplus(delta_proj . x_t)),
//   lambda_t = sigmoid(lambda_proj . x_t), B_t = W_B x_t + b_B, C_t = W_C x_t + b_C
//   h_t = alpha_t * R(theta) h_{t-1} + beta_t * Bu_{t-1} + gamma_t * Bu_t
//   y_t[r] = sum_n C_t[r, n] h_t[n],  out_t = x_t + W_out y_t
// with alpha = e^(dt a_n), beta = (1 - lambda) dt alpha, gamma = lambda dt.
//
// GPU schedule (five kernels, one pass each):
//   1. proj: P = X . Wcat^T, the R + 2 + 2NR controller rows of every token
//      at once (fp32 SGEMM, 64x64 register-blocked tiles through LDS).
//   2. prep: per (t, n) the step's decay a_t = alpha and its drive
//      c_t = beta Bu_{t-1} + gamma Bu_t, which do not depend on h.
//   3. scan: h_t = a_t * R(theta) h_{t-1} + c_t, one lane per state pair,
//      the only sequential part; operands prefetched a step ahead.
//   4. readout: Y[t, r] = sum_n C_t[r, n] h_t[n].
//   5. out: out = x + W_out Y.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "km_device.hpp"
#include "../km_runtime.hpp"
#include "kmamba.h"
#include "kmamba_km.h"
#include "km_topology.h"
#include "wavefront_plan.h"

namespace km {

struct M3Args {
    const float *x;       // [T, D]
    float *out;           // [T, D]
    const float *Wcat;    // [J, D]: W_in (R) | delta_proj (1) | lambda_proj (1) | W_B (NR) | W_C (NR)
    const float *W_out;   // [D, R]
    const float *A;       // [N]
    const float *bB, *bC; // [NR]
    const float *theta;   // [N/2]
    float *P;             // [T, J]
    float *a, *c;         // [T, N]
    float *H;             // [T, N]
    float *Y;             // [T, R]
    long T, L, D, N, R, J;
    int has_delta, has_lambda;
    float dt_scale, dt_min, dt_max;
};

// ---- 1. projections ------------------------------------------------------
constexpr int kPT = 64, kPJ = 64, kPK = 16;

__global__ void __launch_bounds__(256) m3_proj(M3Args p) {
    __shared__ float sx[kPK][kPT + 4];
    __shared__ float sw[kPK][kPJ + 4];
    const int tid = threadIdx.x;
    const int tr = tid / 16, tc = tid % 16;           // 16 x 16 threads, 4 x 4 outputs each
    const long t0 = static_cast<long>(blockIdx.x) * kPT;
    const long j0 = static_cast<long>(blockIdx.y) * kPJ;
    float acc[4][4] = {};
    for (long k0 = 0; k0 < p.D; k0 += kPK) {
        // 64 rows x 16 k of X and of Wcat: 1024 values each, 4 per thread.
        for (int i = tid; i < kPT * kPK; i += 256) {
            const int r = i / kPK, kk = i % kPK;
            const long t = t0 + r, k = k0 + kk;
            sx[kk][r] = (t < p.T && k < p.D) ? p.x[t * p.D + k] : 0.f;
            const long j = j0 + r;
            sw[kk][r] = (j < p.J && k < p.D) ? p.Wcat[j * p.D + k] : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kPK; ++kk) {
            float xv[4], wv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xv[i] = sx[kk][tr * 4 + i];
                wv[i] = sw[kk][tc * 4 + i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(xv[i], wv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const long t = t0 + tr * 4 + i;
        if (t >= p.T) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const long jj = j0 + tc * 4 + j;
            if (jj < p.J) p.P[t * p.J + jj] = acc[i][j];
        }
    }
}

// ---- 2. per-step decay and drive --------------------------------------------
__device__ __forceinline__ float silu_f(float v) { return v / (1.f + expf(-v)); }

__device__ __forceinline__ void m3_ctrl(const M3Args &p, long t, float &dt, float &lam) {
    const float *row = p.P + t * p.J;
    if (p.has_delta) {
        float v = logf(1.f + expf(row[p.R]));
        v = v < p.dt_min ? p.dt_min : v;
        dt = v > p.dt_max ? p.dt_max : v;
    } else {
        dt = p.dt_scale;
    }
    lam = p.has_lambda ? 1.f / (1.f + expf(-row[p.R + 1])) : 0.5f;
}

// Bu_t[n] = sum_r (W_B x_t + b_B)[r, n] * SiLU(W_in x_t)[r].
__device__ __forceinline__ float m3_bu(const M3Args &p, long t, long n) {
    const float *row = p.P + t * p.J;
    float s = 0.f;
    for (long r = 0; r < p.R; ++r)
        s += (row[p.R + 2 + r * p.N + n] + p.bB[r * p.N + n]) * silu_f(row[r]);
    return s;
}

__global__ void __launch_bounds__(256) m3_prep(M3Args p) {
    const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= p.T * p.N) return;
    const long t = i / p.N, n = i % p.N;
    const long l = t % p.L;                            // step within the sequence
    float dt, lam;
    m3_ctrl(p, t, dt, lam);
    const float alpha = expf(dt * p.A[n]);
    const float bu = m3_bu(p, t, n);
    const float pbu = (l > 0) ? m3_bu(p, t - 1, n) : 0.f;
    p.a[i] = alpha;
    p.c[i] = (1.f - lam) * dt * alpha * pbu + lam * dt * bu;
}

// ---- 3. the recurrence ------------------------------------------------------
// One lane per state pair (2i, 2i+1) of one batch element; an odd last state
// has no partner and no rotation. Waves hold 64 pairs of consecutive batch
// elements' flattened (b, pair) index.
__global__ void __launch_bounds__(64) m3_scan(M3Args p, long npairs) {
    const long gid = static_cast<long>(blockIdx.x) * 64 + threadIdx.x;
    const long nb = p.T / p.L;
    if (gid >= nb * npairs) return;
    const long b = gid / npairs, pi = gid % npairs;
    const long n0 = 2 * pi, n1 = n0 + 1;
    const bool pair = n1 < p.N;
    const float th = pair ? p.theta[pi] : 0.f;
    const float cv = pair ? cosf(th) : 1.f, sv = pair ? sinf(th) : 0.f;
    const long base = b * p.L * p.N;
    float h0 = 0.f, h1 = 0.f;
    float a0n = p.a[base + n0], c0n = p.c[base + n0];
    float a1n = pair ? p.a[base + n1] : 0.f, c1n = pair ? p.c[base + n1] : 0.f;
    for (long l = 0; l < p.L; ++l) {
        const float a0 = a0n, c0 = c0n, a1 = a1n, c1 = c1n;
        if (l + 1 < p.L) {                               // next step's operands
            const long o = base + (l + 1) * p.N;
            a0n = p.a[o + n0];
            c0n = p.c[o + n0];
            if (pair) {
                a1n = p.a[o + n1];
                c1n = p.c[o + n1];
            }
        }
        const long o = base + l * p.N;
        if (pair) {
            const float r0 = cv * h0 - sv * h1, r1 = sv * h0 + cv * h1;
            h0 = fmaf(a0, r0, c0);
            h1 = fmaf(a1, r1, c1);
            p.H[o + n0] = h0;
            p.H[o + n1] = h1;
        } else {
            h0 = fmaf(a0, h0, c0);
            p.H[o + n0] = h0;
        }
    }
}

// ---- 4. readout, 5. output ---------------------------------------------------
__global__ void __launch_bounds__(256) m3_readout(M3Args p) {
    const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= p.T * p.R) return;
    const long t = i / p.R, r = i % p.R;
    const float *row = p.P + t * p.J + p.R + 2 + p.N * p.R + r * p.N;
    const float *h = p.H + t * p.N;
    float s = 0.f;
    for (long n = 0; n < p.N; ++n) s = fmaf(row[n] + p.bC[r * p.N + n], h[n], s);
    p.Y[i] = s;
}

__global__ void __launch_bounds__(256) m3_out(M3Args p) {
    const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= p.T * p.D) return;
    const long t = i / p.D, d = i % p.D;
    float s = 0.f;
    for (long r = 0; r < p.R; ++r) s = fmaf(p.W_out[d * p.R + r], p.Y[t * p.R + r], s);
    p.out[i] = p.x[i] + s;
}

static long grid256(long n) { return (n + 255) / 256; }

int mamba3_launch(M3Args &a, hipStream_t s) {
    if (a.T <= 0) return 0;
    if (grid256(a.T * std::max(a.N, a.D)) > 0x7fffffffL) {
        set_error("mamba_block_forward: problem too large");
        return -1;
    }
    dim3 gp(static_cast<unsigned>((a.T + kPT - 1) / kPT), static_cast<unsigned>((a.J + kPJ - 1) / kPJ));
    if (gp.y > 65535) {
        set_error("mamba_block_forward: too many projection rows");
        return -1;
    }
    hipLaunchKernelGGL(m3_proj, gp, dim3(256), 0, s, a);
    hipLaunchKernelGGL(m3_prep, dim3(grid256(a.T * a.N)), dim3(256), 0, s, a);
    const long npairs = (a.N + 1) / 2;
    const long lanes = (a.T / a.L) * npairs;
    hipLaunchKernelGGL(m3_scan, dim3((lanes + 63) / 64), dim3(64), 0, s, a, npairs);
    hipLaunchKernelGGL(m3_readout, dim3(grid256(a.T * a.R)), dim3(256), 0, s, a);
    hipLaunchKernelGGL(m3_out, dim3(grid256(a.T * a.D)), dim3(256), 0, s, a);
    KM_HIP_TRY(hipGetLastError());
    return 0;
}

static size_t mimo_r(const MBConfig &c) { return c.mimo_rank > 1 ? c.mimo_rank : 1; }

static int alloc_matrix(MBMatrix *m, size_t rows, size_t cols) {
    m->rows = rows;
    m->cols = cols;
    m->data = static_cast<float *>(calloc(rows * cols ? rows * cols : 1, sizeof(float)));
    return m->data ? 0 : -1;
}

}  // namespace km

extern "C" {

MambaBlock *mamba_block_create(const MBConfig *config) {
    km::clear_error();
    if (!config) return nullptr;
    MambaBlock *b = static_cast<MambaBlock *>(calloc(1, sizeof(MambaBlock)));
    if (!b) return nullptr;
    b->config = *config;
    if (b->config.mimo_rank == 0) b->config.mimo_rank = 1;
    if (km_normalize_spatial_topology(&b->config.spatial_ndims, b->config.spatial_dims,
                                      b->config.seq_len, b->config.use_convnd,
                                      &b->config.convnd_ndims, b->config.convnd_K) != 0) {
        km::set_error("mamba_block_create: invalid spatial topology");
        mamba_block_free(b);
        return nullptr;
    }
    const size_t R = km::mimo_r(b->config), N = b->config.state_size, D = b->config.dim;
    const size_t L = b->config.seq_len;
    if (km::alloc_matrix(&b->W_in, R, D) || km::alloc_matrix(&b->W_out, D, R) ||
        km::alloc_matrix(&b->A_log, N, 1) || km::alloc_matrix(&b->W_B, N * R, D) ||
        km::alloc_matrix(&b->W_C, N * R, D) || km::alloc_matrix(&b->delta_proj, 1, D) ||
        km::alloc_matrix(&b->lambda_proj, 1, D)) {
        mamba_block_free(b);
        return nullptr;
    }
    const size_t TS = N / 2 > 0 ? N / 2 : 1;
    b->b_B = static_cast<float *>(calloc(N * R ? N * R : 1, sizeof(float)));
    b->b_C = static_cast<float *>(calloc(N * R ? N * R : 1, sizeof(float)));
    b->theta = static_cast<float *>(calloc(TS, sizeof(float)));
    b->hidden = static_cast<float *>(calloc(N ? N : 1, sizeof(float)));
    b->delta = static_cast<float *>(calloc(L ? L : 1, sizeof(float)));
    b->scan_B = static_cast<float *>(calloc(L * N * R ? L * N * R : 1, sizeof(float)));
    b->scan_C = static_cast<float *>(calloc(L * N * R ? L * N * R : 1, sizeof(float)));
    b->scan_delta = static_cast<float *>(calloc(L * N ? L * N : 1, sizeof(float)));
    b->scan_h = static_cast<float *>(calloc(N ? N : 1, sizeof(float)));
    b->wavefront_plan = km_wavefront_plan_create(b->config.spatial_dims, b->config.spatial_ndims);
    if (!b->b_B || !b->b_C || !b->theta || !b->hidden || !b->delta || !b->scan_B || !b->scan_C ||
        !b->scan_delta || !b->scan_h || !b->wavefront_plan) {
        mamba_block_free(b);
        return nullptr;
    }
    if (b->config.use_convnd && b->config.convnd_K > 0) {
        // The reference sizes these in bytes and clears them as floats
        // (src/mamba_block.c:223-233); here both are float counts.
        long n = b->config.convnd_ndims * b->config.convnd_K * static_cast<long>(D);
        if (n == 0 && b->config.spatial_ndims > 0)
            n = b->config.spatial_ndims * b->config.convnd_K * static_cast<long>(D);
        b->convnd_kernel = static_cast<float *>(calloc(n > 0 ? n : 1, sizeof(float)));
        b->convnd_bias = static_cast<float *>(calloc(D ? D : 1, sizeof(float)));
        if (!b->convnd_kernel || !b->convnd_bias) {
            mamba_block_free(b);
            return nullptr;
        }
    }
    return b;
}

void mamba_block_free(MambaBlock *b) {
    if (!b) return;
    free(b->W_in.data); free(b->W_out.data); free(b->A_log.data); free(b->W_B.data);
    free(b->W_C.data); free(b->delta_proj.data); free(b->lambda_proj.data);
    free(b->b_B); free(b->b_C); free(b->theta); free(b->hidden); free(b->delta);
    free(b->scan_B); free(b->scan_C); free(b->scan_delta); free(b->scan_h);
    if (b->wavefront_plan) km_wavefront_plan_free(b->wavefront_plan);
    free(b->convnd_kernel); free(b->convnd_bias);
    free(b);
}

void mamba_block_init(MambaBlock *b) {
    if (!b) return;
    // The reference divides by RAND_MAX converted to float, as here.
    const float kRandMax = static_cast<float>(RAND_MAX);
    for (size_t i = 0; i < b->config.state_size; i++) b->A_log.data[i] = -1.0f;
    MBMatrix *mats[] = {&b->W_in, &b->W_out, &b->W_B, &b->W_C};
    for (MBMatrix *M : mats) {
        const float scale = sqrtf(6.0f / static_cast<float>(M->rows + M->cols));
        for (size_t i = 0; i < M->rows * M->cols; i++)
            M->data[i] = (static_cast<float>(rand()) / kRandMax * 2.0f - 1.0f) * scale;
    }
    const size_t R = km::mimo_r(b->config), N = b->config.state_size;
    memset(b->b_B, 0, N * R * sizeof(float));
    memset(b->b_C, 0, N * R * sizeof(float));
    const float base = 2.0f * 3.14159f / static_cast<float>(N);
    for (size_t i = 0; i < (N / 2 > 0 ? N / 2 : 1); i++)
        b->theta[i] = (static_cast<float>(rand()) / kRandMax) * base;
    for (size_t i = 0; i < b->delta_proj.rows * b->delta_proj.cols; i++)
        b->delta_proj.data[i] = (static_cast<float>(rand()) / kRandMax - 0.5f) * 0.02f;
    for (size_t i = 0; i < b->lambda_proj.rows * b->lambda_proj.cols; i++)
        b->lambda_proj.data[i] = (static_cast<float>(rand()) / kRandMax - 0.5f) * 0.02f;
}

void mamba_block_forward(MambaBlock *b, float *output, const float *input, size_t batch_size) {
    km::clear_error();
    if (!b || !output || !input || batch_size == 0) {
        km::set_error("mamba_block_forward: invalid arguments");
        return;
    }
    const MBConfig &c = b->config;
    const long L = static_cast<long>(c.seq_len), D = static_cast<long>(c.dim);
    const long N = static_cast<long>(c.state_size), R = static_cast<long>(km::mimo_r(c));
    if (L <= 0 || D <= 0 || N <= 0 || !b->W_in.data || !b->W_out.data || !b->A_log.data ||
        !b->W_B.data || !b->W_C.data || !b->b_B || !b->b_C || !b->theta) {
        km::set_error("mamba_block_forward: incomplete block");
        return;
    }
    if (!km::gpu_ready()) return;
    const long T = static_cast<long>(batch_size) * L, NR = N * R;
    const bool has_delta = b->delta_proj.rows > 0 && b->delta_proj.data;
    const bool has_lambda = b->lambda_proj.rows > 0 && b->lambda_proj.data;
    const long J = R + 2 + 2 * NR;
    const long TS = N / 2 > 0 ? N / 2 : 1;
    const bool dev_io = km::is_device_ptr(input) && km::is_device_ptr(output);
    km::Staging::lock();
    do {
        const size_t io_bytes = dev_io ? 0 : 2 * km::align_up(sizeof(float) * T * D, 256);
        const size_t bytes = io_bytes + sizeof(float) * (J * D + D * R + N + 2 * NR + TS) + 8 * 256 +
                             sizeof(float) * (T * J + 3 * T * N + T * R) + 8 * 256;
        void *base = km::Staging::reserve(bytes);
        if (!base) break;
        km::Carver cv(base);
        float *x = dev_io ? const_cast<float *>(input) : cv.take<float>(T * D);
        float *o = dev_io ? output : cv.take<float>(T * D);
        float *Wcat = cv.take<float>(J * D);
        float *Wout = cv.take<float>(D * R);
        float *A = cv.take<float>(N);
        float *bB = cv.take<float>(NR), *bC = cv.take<float>(NR);
        float *th = cv.take<float>(TS);
        bool ok = true;
        auto h2d = [&](void *dst, const void *src, size_t n) {
            ok = ok && hipMemcpy(dst, src, n, hipMemcpyHostToDevice) == hipSuccess;
        };
        if (!dev_io) h2d(x, input, sizeof(float) * T * D);
        h2d(Wcat, b->W_in.data, sizeof(float) * R * D);
        if (has_delta) h2d(Wcat + R * D, b->delta_proj.data, sizeof(float) * D);
        if (has_lambda) h2d(Wcat + (R + 1) * D, b->lambda_proj.data, sizeof(float) * D);
        h2d(Wcat + (R + 2) * D, b->W_B.data, sizeof(float) * NR * D);
        h2d(Wcat + (R + 2 + NR) * D, b->W_C.data, sizeof(float) * NR * D);
        h2d(Wout, b->W_out.data, sizeof(float) * D * R);
        h2d(A, b->A_log.data, sizeof(float) * N);
        h2d(bB, b->b_B, sizeof(float) * NR);
        h2d(bC, b->b_C, sizeof(float) * NR);
        h2d(th, b->theta, sizeof(float) * TS);
        if (!ok) {
            km::set_error("mamba_block_forward: host-to-device copy failed");
            break;
        }
        km::M3Args a{};
        a.x = x; a.out = o; a.Wcat = Wcat; a.W_out = Wout; a.A = A; a.bB = bB; a.bC = bC;
        a.theta = th;
        a.P = cv.take<float>(T * J);
        a.a = cv.take<float>(T * N);
        a.c = cv.take<float>(T * N);
        a.H = cv.take<float>(T * N);
        a.Y = cv.take<float>(T * R);
        a.T = T; a.L = L; a.D = D; a.N = N; a.R = R; a.J = J;
        a.has_delta = has_delta; a.has_lambda = has_lambda;
        a.dt_scale = c.dt_scale; a.dt_min = c.dt_min; a.dt_max = c.dt_max;
        if (km::mamba3_launch(a, nullptr) != 0) break;
        if (hipStreamSynchronize(nullptr) != hipSuccess) {
            km::set_error("mamba_block_forward: %s", hipGetErrorString(hipGetLastError()));
            break;
        }
        if (!dev_io && hipMemcpy(output, o, sizeof(float) * T * D, hipMemcpyDeviceToHost) != hipSuccess)
            km::set_error("mamba_block_forward: device-to-host copy failed");
    } while (false);
    km::Staging::unlock();
}

}  // extern "C"

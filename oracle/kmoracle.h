/* kmoracle.h - CPU restatement of the reference k-mamba hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP
 * kernels of libkmamba: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it. The product never links it and
 * has no CPU fallback to it.
 *
 * Each function restates one reference function in the same arithmetic order
 * (fp32, no FMA contraction, glibc expf), citing the reference file:line it
 * follows. Struct layouts mirror the reference headers (8-byte pointers and
 * longs) so the same ctypes structures drive the oracle and the library.
 */
#ifndef KMORACLE_H
#define KMORACLE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    float *x, *A, *B, *C, *delta, *h, *y;
    long L, D, M;
} OrcScanParams;                         /* ref include/scan.h:45-56 */

typedef struct {
    float *x, *A, *B, *C, *delta, *h0, *h, *dy, *dx, *dA, *dB, *dC, *ddelta;
    long L, D, M;
} OrcScanBackwardParams;                 /* ref include/scan.h:61-78 */

typedef struct {
    float *x, *A, *A_diag, *B, *C, *delta, *h0, *h, *dy, *dx, *dA, *dB, *dC, *ddelta;
    long L, D;
} OrcScanBackwardSharedParams;           /* ref include/scan.h:83-100 */

typedef struct {
    float *x, *A1, *A2, *B, *C, *delta1, *delta2, *h, *y;
    long d1, d2, D, M;
} OrcScan2DParams;                       /* ref include/scan.h:117-131 */

typedef struct {
    const long *dims;
    long ndims, D, M;
    const float *x, *A, *B, *C, *delta;
    float *h, *y;
    const float *theta, *lambda;
} OrcScanNDParams;                       /* ref include/scan_nd.h:40-55 */

typedef struct {
    float *input;
    const float *kernel, *bias;
    float *output, *dy, *dinput, *dkernel, *dbias;
    const long *dims;
    long ndims, D, K;
} OrcConvNDParams;                       /* ref include/convnd.h:10-23 */

typedef struct {
    long *dims;
    long ndims, total_points, max_level, max_level_size;
    long *level_starts, *level_offsets;
} OrcPlan;                               /* ref include/wavefront_plan.h:27-35 */

/* ---- Scan1D ---------------------------------------------------------- */
void orc_scan1d(OrcScanParams *p);
void orc_scan1d_batched(const float *x, const float *delta, const float *A,
                        const float *Bm, const float *Cm, float *y,
                        float *h, float *h_hist,
                        long B, long L, long D, long N,
                        long bc_sb, long bc_st, long bc_sd,
                        int clamp, int nthreads);
void orc_scan1d_backward(OrcScanBackwardParams *p);
void orc_scan1d_backward_m1_shared_bc(OrcScanBackwardSharedParams *p);
float orc_m1_asm_taylor(float x, int simple);
void orc_scan1d_backward_m1_shared_bc_asm(OrcScanBackwardSharedParams *p, int simple);
void orc_scan1d_batched_backward(const float *x, const float *delta, const float *A,
                                 const float *Bm, const float *Cm, const float *dy,
                                 const float *h0, const float *h_hist,
                                 float *dx, float *ddelta, float *dA,
                                 float *dB, float *dC,
                                 long B, long L, long D, long N,
                                 long bc_sb, long bc_st, long bc_sd, int nthreads);

/* ---- Scan2D / ScanND -------------------------------------------------- */
void orc_scan2d(OrcScan2DParams *p);
int  orc_scannd_validate(const OrcScanNDParams *p);
int  orc_scannd_ref_with_plan(OrcScanNDParams *p, const OrcPlan *plan, int nthreads);
int  orc_scannd_ref(OrcScanNDParams *p, int nthreads);
int  orc_scannd(OrcScanNDParams *p, int nthreads);

/* Adjoint of scannd_ref (no counterpart in the reference, which has no
 * ScanND backward): for L = sum dy . y with h the forward's states (p->h),
 *   g[p]     = dy[p] C[p] + sum_a [i_a < dims_a - 1] exp(delta_a[p+s_a] A_a) g[p+s_a]
 *   dC[p]    = dy[p] h[p];  dB[p] = g[p] dtbar[p] x[p]
 *   dx[p]    = sum_m g dtbar B
 *   ddelta_a = sum_m g B x / ndims + [i_a > 0] sum_m g A_a e_a[p] h[p-s_a]
 *   dA_a     = sum_p [i_a > 0] g delta_a[p] e_a[p] h[p-s_a]
 * with e_a[p] = exp(delta_a[p] A_a) and dtbar = sum_a delta_a / ndims as the
 * forward forms them (src/scan_nd.c:105-108, :174-188). g runs in reverse
 * row-major order (every p + s_a precedes p); g is kept in dB's memory until
 * dB is formed. Sums over m and over p run in ascending order. */
int  orc_scannd_backward(const OrcScanNDParams *p, const float *dy, float *dx, float *ddelta,
                         float *dA, float *dB, float *dC);

/* ---- ConvND ----------------------------------------------------------- */
long orc_convnd_kernel_volume(long ndims, long K);
void orc_convnd_forward(OrcConvNDParams *p, int nthreads);
void orc_convnd_backward(OrcConvNDParams *p);

/* ---- Mamba-3 block forward -------------------------------------------- */
/* Parameters of one MambaBlock (ref include/kmamba.h:116-150) as plain
 * arrays: W_in [R, D], W_out [D, R], A_log [N], W_B / W_C [N*R, D],
 * delta_proj / lambda_proj [D] (NULL = absent), b_B / b_C [N*R],
 * theta [N/2]. */
typedef struct {
    const float *W_in, *W_out, *A_log, *W_B, *W_C, *delta_proj, *lambda_proj;
    const float *b_B, *b_C, *theta;
    long L, D, N, R;
    float dt_scale, dt_min, dt_max;
} OrcMamba3;

/* mamba_block_forward_ws (ref src/mamba_block.c:471-501) for input and
 * output [batch, L, D]. */
void orc_mamba3_forward(const OrcMamba3 *p, const float *input, float *output, long batch);

/* The reference's gemm_f32 (kernels/gemm_f32.c:13-31): C[M,N] = A[M,K] B[K,N]
 * row-major, C zeroed, then C[i,j] += A[i,k] * B[k,j] with k ascending per
 * element (two roundings per term, as the reference built without FMA
 * contraction). Rows run in parallel; each element's order is fixed. */
void orc_gemm_f32(const float *A, const float *B, float *C, long M, long K, long N);

/* The reference activations (include/kmamba_kernels.h:35-49 through
 * kernels/activations_f32.c:7-29): y[i] = x[i] / (1 + expf(-x[i])) and
 * y[i] = logf(1 + expf(x[i])), fp32. */
void orc_silu_f32(const float *x, float *y, long n);
void orc_softplus_f32(const float *x, float *y, long n);

/* ---- Wavefront / plan / topology -------------------------------------- */
int  orc_wavefront_validate_dims(const long *dims, long ndims);
long orc_wavefront_total_points(const long *dims, long ndims);
long orc_wavefront_max_level(const long *dims, long ndims);
long orc_wavefront_row_major_offset(const long *dims, const long *idx, long ndims);
long orc_wavefront_level_size(const long *dims, long ndims, long level);
OrcPlan *orc_plan_create(const long *dims, long ndims);
void orc_plan_free(OrcPlan *plan);
int  orc_make_row_major_strides(const long *dims, long ndims, long *strides);
void orc_unravel_index(long linear, const long *dims, const long *strides, long ndims, long *coords);
long orc_ravel_index(const long *coords, const long *dims, const long *strides, long ndims);
long orc_power_long(long base, long exp);

#ifdef __cplusplus
}
#endif

#endif

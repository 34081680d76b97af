/* scan.h - selective-scan entry points of libkmamba (MI355X build).
 *
 * Drop-in for the reference header include/scan.h. Struct layouts are
 * byte-identical to the reference (seven or more 8-byte pointers followed by
 * 8-byte longs) because existing callers and the reference's NASM offset
 * table (include/scan.inc:11-85) depend on them.
 *
 * Every function here runs on the GPU. The host-pointer functions
 * (scan1d, scan1d_backward, scan2d, ...) stage caller memory to the device,
 * run the HIP kernels and copy the results back; if the caller already passes
 * device (or managed) pointers no staging happens. There is no CPU compute
 * path in this library: when no GPU is usable the void functions leave their
 * outputs untouched and record an error readable with km_last_error()
 * (kmamba_km.h).
 */
#ifndef KMAMBA_SCAN_H
#define KMAMBA_SCAN_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Selective scan 1D, forward.
 *   x, delta, y : [L, D]
 *   A           : [D, M]
 *   B, C        : [L, D, M]
 *   h           : [D, M] running state, read as the initial state and
 *                 overwritten with the final state (reference asm semantics,
 *                 cpu/scan1d.asm:127-143)
 *   h_t = clamp(exp(delta_t*A) * h_{t-1} + (B_t*delta_t) * x_t, +-1000)
 *   y_t = sum_m C_t * h_t
 * Layout replaces include/scan.h:45-56 of the reference. */
typedef struct {
    float *x;
    float *A;
    float *B;
    float *C;
    float *delta;
    float *h;
    float *y;
    long   L;
    long   D;
    long   M;
} ScanParams;

/* Replaces scan1d (cpu/scan1d.asm:40-179, declared include/scan.h:58). */
void scan1d(ScanParams *p);

/* Selective scan 1D, backward, generic [L, D, M] layout.
 * h is the post-update state history [L, D, M]; h0 the optional initial
 * state [D, M]. All gradient outputs are overwritten (zeroed first).
 * Layout replaces include/scan.h:61-78 of the reference. */
typedef struct {
    float *x;
    float *A;
    float *B;
    float *C;
    float *delta;
    float *h0;
    float *h;
    float *dy;
    float *dx;
    float *dA;
    float *dB;
    float *dC;
    float *ddelta;
    long   L;
    long   D;
    long   M;
} ScanBackwardParams;

/* Replaces scan1d_backward (cpu/scan1d_backward.c:297-306, include/scan.h:80). */
void scan1d_backward(ScanBackwardParams *p);

/* Backward for M=1 with B, C shared over time ([D]) and delta shared over
 * channels ([L]). A_diag, when given, is exp(delta*A) precomputed [L, D].
 * Layout replaces include/scan.h:83-100 of the reference. */
typedef struct {
    float *x;
    float *A;
    float *A_diag;
    float *B;
    float *C;
    float *delta;
    float *h0;
    float *h;
    float *dy;
    float *dx;
    float *dA;
    float *dB;
    float *dC;
    float *ddelta;
    long   L;
    long   D;
} ScanBackwardSharedParams;

/* Replaces scan1d_backward_m1_shared_bc (cpu/scan1d_backward.c:182-191,
 * include/scan.h:102). */
void scan1d_backward_m1_shared_bc(ScanBackwardSharedParams *p);

/* Replace scan1d_backward_m1_shared_bc_asm and _simple_asm (include/scan.h:
 * 103-104; cpu/scan1d_backward_m1_shared_bc.asm and _simple.asm, which the
 * reference's build does not assemble). The same recurrence; without
 * A_diag the decay is those routines' Taylor polynomial
 * 1 + x + x^2/2 + x^3/6 of x = delta*A (not expf). L = 0 clears dA, dB, dC;
 * D = 0 clears ddelta. A missing buffer or a negative size sets
 * km_last_error() and writes nothing (the routines would fault). */
void scan1d_backward_m1_shared_bc_asm(ScanBackwardSharedParams *p);
void scan1d_backward_m1_shared_bc_simple_asm(ScanBackwardSharedParams *p);

/* Selective scan 2D over a d1 x d2 grid, anti-diagonal dependency order:
 *   h(i,j) = exp(dt1*A1) h(i-1,j) + exp(dt2*A2) h(i,j-1) + B*((dt1+dt2)/2)*x
 *   y(i,j) = sum_m C h(i,j)
 * x, delta1, delta2, y: [d1*d2, D]; A1, A2: [D, M]; B, C, h: [d1*d2, D, M]
 * (h receives the full state field). No clamp.
 * Layout replaces include/scan.h:117-131 of the reference. */
typedef struct {
    float *x;
    float *A1;
    float *A2;
    float *B;
    float *C;
    float *delta1;
    float *delta2;
    float *h;
    float *y;
    long   d1;
    long   d2;
    long   D;
    long   M;
} Scan2DParams;

/* Replaces scan2d (cpu/scan2d.asm:48-285, include/scan.h:133). */
void scan2d(Scan2DParams *p);

/* Device-pointer API (reference: include/scan.h:136-153, guarded there by
 * __CUDACC__; declared unconditionally here).
 *   om_scan1d_forward: B, C, h are [L, D, M]; h receives the full state
 *   history; the initial state is zero; the +-1000 clamp is applied per step
 *   as in the CPU path. Replaces cuda/scan1d.cu:258-310.
 *   om_scan1d_backward: h is the forward history [L, D, M]; zero initial
 *   state. Replaces cuda/scan1d_backward.cu:113-137.
 * Both are synchronous; on error they record it (km_last_error) and return
 * without exiting the process. */
void om_scan1d_forward(
    const float *d_x,  const float *d_A,
    const float *d_B,  const float *d_C,
    const float *d_dt,
    float *d_y, float *d_h,
    int L, int D, int M
);

void om_scan1d_backward(
    const float *d_dy,
    const float *d_x,  const float *d_A,
    const float *d_B,  const float *d_C,
    const float *d_dt, const float *d_h,
    float *d_dx, float *d_dA,
    float *d_dB, float *d_dC, float *d_ddt,
    int L, int D, int M
);

#ifdef __cplusplus
}
#endif

#endif /* KMAMBA_SCAN_H */

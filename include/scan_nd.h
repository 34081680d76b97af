/* scan_nd.h - ND selective scan over a causal grid (MI355X build).
 *
 *   x      : [P, D]            (P = prod(dims))
 *   A      : [ndims, D, M]
 *   B, C   : [P, D, M]
 *   delta  : [ndims, P, D]
 *   h      : [P, D, M]         (receives the full state field)
 *   y      : [P, D]
 *   dt_bar(p,d) = (sum_axis delta(axis,p,d)) / ndims
 *   h(p,d,m)    = dt_bar * (B*x) + sum_axis[idx>0] exp(delta(axis)*A(axis)) h(p - e_axis)
 *   y(p,d)      = sum_m C h
 * Dependencies follow the wavefront level sum(idx).
 *
 * Drop-in for the reference include/scan_nd.h:40-73. The struct layout is
 * unchanged. dims stays a host pointer for every entry point, including the
 * device-pointer one.
 */
#ifndef KMAMBA_SCAN_ND_H
#define KMAMBA_SCAN_ND_H

#include "wavefront_plan.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    const long  *dims;
    long         ndims;
    long         D;
    long         M;
    const float *x;
    const float *A;
    const float *B;
    const float *C;
    const float *delta;
    float       *h;
    float       *y;
    /* Mamba-3 extensions of the reference (rotation angles [D/2], per-point
     * lambda [P]), used by the lambda branch of scannd_ref
     * (src/scan_nd.c:59-210) when lambda is non-NULL:
     *   h = bpa*((1-lambda)*dt_bar*aavg) + bu*(lambda*dt_bar)
     *       + sum_a alpha_a * hrot[p - e_a]
     * with bu = B*x, alpha_a = exp(delta_a * min(A_a, -1e-5)), bpa and aavg
     * the averages over the predecessors of B[prev]*x[prev] and alpha_a, and
     * hrot a predecessor's states after the rotation of channel pairs
     * (2i, 2i+1) by theta[i] (the states themselves when theta is NULL).
     * The reference keeps hrot in a [D, M] buffer it indexes by point
     * (out of bounds); this library keeps the [P, D, M] field that indexing
     * implies. theta without lambda has no effect. scannd() applies the
     * branch for ndims >= 3 only, as the reference dispatcher does. */
    const float *theta;
    const float *lambda;
} ScanNDParams;

/* 1 when sizes and pointers are valid, else 0 (ref src/scan_nd.c:17-29). */
int scannd_validate(const ScanNDParams *p);

/* Generic ND scan, host pointers, wavefront semantics of
 * src/scan_nd.c:235-247 (no clamp; full h written). 0 ok, -1 error. */
int scannd_ref(ScanNDParams *p);

/* Same, with a caller-built plan that must match dims (ref :31-233). */
int scannd_ref_with_plan(ScanNDParams *p, const KMWavefrontPlan *plan);

/* Dispatching entry (ref :249-308): ndims == 1 follows scan1d semantics
 * (h is a running [D, M] state, +-1000 clamp), ndims == 2 follows scan2d,
 * ndims >= 3 follows scannd_ref. Host pointers. 0 ok, -1 error. */
int scannd(ScanNDParams *p);

/* Device-pointer ND scan with scannd_ref semantics for every ndims
 * (ref cuda/scan_nd.cu:337-400, declared include/scan_nd.h:72). Synchronous.
 * 0 ok, -1 error. */
int om_scannd_forward(ScanNDParams *p);

#ifdef __cplusplus
}
#endif

#endif /* KMAMBA_SCAN_ND_H */

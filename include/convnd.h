/* convnd.h - dense per-channel causal ND convolution (MI355X build).
 *
 *   out[n, d] = bias[d] + sum_{k in [0,K)^ndims} in[n - (K-1-k), d] * W[k, d]
 * Taps that fall below 0 on any axis are skipped (zero padding on the low
 * side only), stride 1. input/output/dy/dinput: [P, D]; kernel/dkernel:
 * [K^ndims, D] with the kernel index row-major over axes; bias/dbias: [D].
 *
 * Drop-in for the reference include/convnd.h:10-52; layout unchanged.
 */
#ifndef CONVND_H
#define CONVND_H

#include <stddef.h>
#include "wavefront_plan.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    float *input;           /* [prod(dims), D] */
    const float *kernel;    /* [K^ndims, D] */
    const float *bias;      /* [D] or NULL */
    float *output;          /* [prod(dims), D] */
    float *dy;              /* [prod(dims), D], backward only */
    float *dinput;          /* [prod(dims), D], backward only */
    float *dkernel;         /* [K^ndims, D], backward only */
    float *dbias;           /* [D] or NULL, backward only */
    const long *dims;       /* [ndims], host pointer */
    long ndims;
    long D;
    long K;
} ConvNDParams;

typedef enum {
    CONVND_FORWARD = 1,
    CONVND_BACKWARD = 2,
    CONVND_COMPLETE = 3
} ConvNDMode;

/* K^ndims, or 0 when ndims <= 0 or K <= 0 (ref src/convnd.c:58-61). */
long convnd_kernel_volume(long ndims, long K);

/* Forward with a caller plan matching dims; host pointers
 * (ref src/convnd.c:67-129). */
void convnd_forward_wavefront(ConvNDParams *p, const KMWavefrontPlan *plan);

/* Backward (dinput, dkernel, dbias overwritten) with a caller plan; host
 * pointers (ref src/convnd.c:135-202). */
void convnd_backward_wavefront(ConvNDParams *p, const KMWavefrontPlan *plan);

/* Unified entry, host pointers (ref src/convnd.c:208-244). */
void convnd(ConvNDParams *p, ConvNDMode mode);

/* Device-pointer forward / backward (ref cuda/convnd.cu:258-436, declared
 * include/convnd.h:48-51 under __CUDACC__). Synchronous. 0 ok, -1 error. */
int om_convnd_forward(ConvNDParams *p);
int om_convnd_backward(ConvNDParams *p);

#ifdef __cplusplus
}
#endif

#endif

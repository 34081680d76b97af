/* kmamba.h - Mamba-3 block API of libkmamba (MI355X build).
 *
 * Drop-in for the block part of the reference include/kmamba.h:17-150 and
 * :228-235: the same MBMatrix, MBConfig and MambaBlock layouts (8-byte
 * pointers, size_t and long) and the same create / free / init / forward
 * entry points. The forward runs on the GPU (mamba_block_forward takes host
 * or device pointers for input and output, as the reference's host call
 * does). The reference's optimizer and training entry points are not part
 * of this library: opt_state stays NULL in blocks it creates.
 */
#ifndef KMAMBA_H
#define KMAMBA_H

#include <stddef.h>
#include <stdint.h>

#include "km_topology.h"
#include "wavefront_plan.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    float *data;
    size_t rows;
    size_t cols;
} MBMatrix;                                   /* ref include/kmamba.h:17-24 */

typedef struct {
    size_t dim;
    size_t state_size;
    size_t seq_len;
    size_t mimo_rank;
    float dt_scale;
    float dt_min;
    float dt_max;
    int use_fp16;
    int use_bf16;
    float loss_scale;
    long spatial_ndims;
    long spatial_dims[KMAMBA_MAX_NDIMS];
    int use_convnd;
    long convnd_K;
    long convnd_ndims;
} MBConfig;                                   /* ref include/kmamba.h:27-54 */

/* Optimizer state of the reference's training API; opaque here. */
typedef struct km_mb_optim_state MBOptimState;

typedef struct {
    MBConfig config;
    MBMatrix W_in;          /* [R, dim] */
    MBMatrix W_out;         /* [dim, R] */
    MBMatrix A_log;         /* [state_size, 1]: the decay rate a (alpha = exp(dt * a)) */
    MBMatrix W_B;           /* [N*R, dim] */
    MBMatrix W_C;           /* [N*R, dim] */
    MBMatrix delta_proj;    /* [1, dim] */
    float *b_B;             /* [N*R] */
    float *b_C;             /* [N*R] */
    float *theta;           /* [max(N/2, 1)] rotation angles per state pair */
    MBMatrix lambda_proj;   /* [1, dim] */
    KMWavefrontPlan *wavefront_plan;
    float *convnd_kernel;
    float *convnd_bias;
    float *hidden;
    float *delta;
    float *scan_B;
    float *scan_C;
    float *scan_delta;
    float *scan_h;
    MBOptimState *opt_state;
} MambaBlock;                                 /* ref include/kmamba.h:116-150 */

/* Allocates a block for config (ref src/mamba_block.c:177-238); NULL on
 * invalid topology or allocation failure. Parameters start at zero. */
MambaBlock *mamba_block_create(const MBConfig *config);

/* Frees a block made by mamba_block_create (ref src/mamba_block.c:240-263). */
void mamba_block_free(MambaBlock *block);

/* Reference initialisation (ref src/mamba_block.c:269-289): A_log = -1,
 * W_in / W_out / W_B / W_C uniform in +-sqrt(6 / (rows + cols)) from rand(),
 * b_B = b_C = 0, theta uniform in [0, 2*pi/N), delta_proj and lambda_proj
 * uniform in +-0.01; the same rand() call order as the reference. */
void mamba_block_init(MambaBlock *block);

/* Mamba-3 forward (ref src/mamba_block.c:471-501, :814-831) on the GPU for
 * input and output [batch, seq_len, dim] fp32, host or device pointers:
 *   u_t = SiLU(W_in x_t); dt_t = clamp(softplus(delta_proj . x_t), dt_min, dt_max);
 *   lambda_t = sigmoid(lambda_proj . x_t); B_t = W_B x_t + b_B; C_t = W_C x_t + b_C
 *   h_t = e^(dt_t a) * R(theta) h_{t-1} + (1 - lambda_t) dt_t e^(dt_t a) Bu_{t-1}
 *         + lambda_t dt_t Bu_t,        Bu_t[n] = sum_r B_t[r, n] u_t[r]
 *   y_t[r] = sum_n C_t[r, n] h_t[n];   out_t = x_t + W_out y_t
 * Returns silently on invalid arguments, as the reference; the reason is in
 * km_last_error(). */
void mamba_block_forward(MambaBlock *block, float *output, const float *input, size_t batch_size);

#ifdef __cplusplus
}
#endif

#endif /* KMAMBA_H */

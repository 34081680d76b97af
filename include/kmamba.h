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

/* ------------------------------------------------------------------------
 * The stacked model (ref include/kmamba.h:159-223, src/kmamba.c): token
 * embedding, n_layers Mamba-3 blocks, output head. Layouts are those of the
 * reference's CPU build (no KMAMBA_BUILD_CUDA member). Parameters live in
 * host memory as in the reference; the forward runs on the GPU. Training
 * (kmamba_enable_training, kmamba_train_*) is not part of this library.
 * ---------------------------------------------------------------------- */

/* Optimizer settings (ref include/kmamba_kernels.h:78-85); kept for the
 * KMamba layout. */
typedef struct {
    float lr;
    float mu;
    float beta2;
    float eps;
    float clip_norm;
    float weight_decay;
} MBOptimConfig;

typedef struct {
    size_t vocab_size;
    size_t dim;
    size_t state_size;
    size_t seq_len;
    size_t n_layers;
    size_t mimo_rank;             /* 0 or 1: SISO */
    float dt_scale;
    float dt_min;
    float dt_max;
    long spatial_ndims;           /* 0: the implicit 1D shape [seq_len] */
    long spatial_dims[KMAMBA_MAX_NDIMS];
    int use_convnd;
    long convnd_K;
    long convnd_ndims;
    int weight_tying;             /* 1: head shares the embedding's memory */
} KMambaConfig;                               /* ref include/kmamba.h:159-183 */

typedef struct {
    KMambaConfig cfg;
    float *embedding;             /* [vocab_size, dim] row-major */
    float *head;                  /* [dim, vocab_size] row-major (the embedding when tied) */
    MambaBlock **layers;          /* [n_layers] */
    int for_training;
    MBOptimConfig opt_blocks;
    float lr_embed_head;
    float weight_decay;
    float *m_embedding;
    float *v_embedding;
    float *m_head;
    float *v_head;
    size_t step_embed_head;
    float last_grad_norm;
    float last_grad_over_clip;
    int last_grad_would_clip;
} KMamba;                                     /* ref include/kmamba.h:185-223 */

/* Allocates a model (ref src/kmamba.c:102-152): NULL when vocab_size, dim,
 * seq_len or n_layers is 0, the spatial topology is invalid, or memory
 * runs out. Parameters start at zero. */
KMamba *kmamba_create(const KMambaConfig *cfg);

/* Frees a model and its blocks (ref src/kmamba.c:154-175). */
void kmamba_free(KMamba *m);

/* srand(seed), then Xavier-uniform embedding and (untied) head and the
 * blocks' initialisation, in the reference's rand() order
 * (ref src/kmamba.c:177-188). Returns 0, or -1 for NULL. */
int kmamba_init(KMamba *m, uint32_t seed);

/* Checkpoint version 4 (ref src/kmamba.c:216-294): an 80-byte header
 * ("KMAMBA", version, sizes, dt range), the embedding, the head, then per
 * layer W_in, W_out, A_log, W_B, W_C, b_B, b_C, delta_proj, lambda_proj,
 * theta as raw fp32. Returns 0, or -1 (error in km_last_error()). */
int kmamba_save(const KMamba *m, const char *path);

/* Reads a checkpoint written by kmamba_save (versions <= 4; versions below
 * 4 load as mimo_rank 1) into a new untied model (ref src/kmamba.c:296-342).
 * for_training must be 0: training is not part of this library (NULL with
 * an error otherwise); opt_blocks, lr_embed_head and weight_decay are then
 * unused. NULL on a missing file, a bad header or a short read. */
KMamba *kmamba_load(const char *path, int for_training, const MBOptimConfig *opt_blocks,
                    float lr_embed_head, float weight_decay);

/* Inference on one sequence (ref src/kmamba.c:344-372): tokens [seq_len]
 * (ids >= vocab_size embed as zeros), logits_out [seq_len, vocab_size], both
 * host memory; logits = h . head with h the last block's output. Clears the
 * blocks' hidden and scan_h as the reference does. Runs on the GPU: the
 * head is uploaded on every call, as the parameters are host-owned. Calls
 * that overlap on one device race on the library's device workspace.
 * Returns 0, or -1 (error in km_last_error()). */
int kmamba_forward(KMamba *m, const uint32_t *tokens, float *logits_out);

#ifdef __cplusplus
}
#endif

#endif /* KMAMBA_H */

/* kmamba_km.h - libkmamba extensions with no single counterpart in the
 * reference API: batched and strided scan layouts, bf16 I/O, explicit HIP
 * streams and error reporting.
 *
 * All pointers are device pointers. Entry points are asynchronous on the
 * given stream (a hipStream_t passed as void*, NULL for the null stream) and
 * return 0 on success, -1 on invalid arguments or a launch failure; the
 * reason is available from km_last_error(). The only device allocation is
 * the library's per-device scratch, made on first use (and when a larger one
 * is needed) by entry points that need scratch and were given none.
 */
#ifndef KMAMBA_KM_H
#define KMAMBA_KM_H

#include <stddef.h>

#include "scan_nd.h"
#include "convnd.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Last error message of the calling thread ("" when none). */
const char *km_last_error(void);
void km_clear_error(void);

/* Library version string. */
const char *km_version(void);

/* Device memory the library holds in its caches (bytes, every device):
 * the host-pointer staging arenas and the per-(device, stream) scratch
 * blocks of entry points called without a workspace. */
size_t km_device_bytes_held(void);

/* Frees the library's scratch blocks tied to `stream` on the current device
 * (after waiting for the stream). Call it before destroying a stream that
 * library calls ran on, so its blocks do not stay allocated; the library
 * also frees the least recently used blocks of other streams by itself
 * when its table of 64 blocks is full. Returns the bytes freed. */
size_t km_release_stream(void *stream);

typedef enum {
    KM_F32 = 0,   /* IEEE fp32 */
    KM_BF16 = 1   /* bfloat16 storage, fp32 arithmetic, round-to-nearest-even on store */
} KMDtype;

/* Batched, strided Scan1D forward.
 *
 * Generalises the reference scan1d (cpu/scan1d.asm:40-179) to a batch and to
 * B/C operands shared over channels. For every b, d, n and t:
 *   e     = exp(delta[b,t,d] * A[d,n])
 *   h     = e * h + B(b,t,d,n) * (delta[b,t,d] * x[b,t,d])
 *   h     = clamp(h, -1000, 1000)            when clamp != 0
 *   y[b,t,d] = sum_n C(b,t,d,n) * h
 * x, delta, y : [B, L, D] contiguous, dtype
 * A           : [D, N] fp32
 * B(b,t,d,n)  : Bm[b*bc_sb + t*bc_st + d*bc_sd + n], dtype (same for Cm).
 *               Shared over channels: bc_sd = 0 (e.g. [B, L, N]).
 *               Reference API layout [L, D, N]: bc_sd = N, bc_st = D*N.
 * h0          : [B, D, N] fp32 initial state, NULL for zero
 * h_final     : [B, D, N] fp32 final state, may be NULL (may alias h0)
 * h_hist      : [B, L, D, N] fp32 state after every step, may be NULL
 * h_ckpt      : [B, ceil(L/32), D, N] fp32 state after every 32nd step (and
 *               after the last step), may be NULL: the checkpoints the
 *               backward recomputes states from
 * y may be NULL when only states are wanted.
 * z           : [B, L, D] dtype gate, may be NULL; Dskip: [D] fp32, may be
 *               NULL. When given, y = (sum_n C*h + Dskip*x) * SiLU(z) (the
 *               Mamba-1 output gating, fused into the store; km_scan1d_bwd
 *               does not differentiate it).
 * The +-1000 clamp is not associative; the kernel runs the unclamped
 * chunked scan and re-runs any (b, channel group) whose state left
 * [-1000, 1000] with the sequential clamped recurrence, so results follow the
 * per-step clamp exactly as the reference CPU path does. */
typedef struct {
    const void  *x;
    const void  *delta;
    const float *A;
    const void  *Bm;
    const void  *Cm;
    void        *y;
    const float *h0;
    float       *h_final;
    float       *h_hist;
    long B, L, D, N;
    long bc_sb, bc_st, bc_sd;
    int  dtype;
    int  clamp;
    float       *h_ckpt;
    const void  *z;
    const float *Dskip;
} KMScan1DFwd;

#define KM_SCAN1D_CKPT_STEPS 32

int km_scan1d_fwd(const KMScan1DFwd *a, void *stream);

/* Batched, strided Scan1D backward: the adjoint of km_scan1d_fwd, per batch
 * element the reference scan1d_backward (cpu/scan1d_backward.c:248-295):
 *   ah = adj + dy*C;  dC = dy*h_t;  dB = ah*delta*x;  dA += ah*delta*e*h_{t-1}
 *   dx = sum_n ah*delta*B;  ddelta = sum_n ah*(A*e*h_{t-1} + B*x);  adj = ah*e
 * The forward clamp is not differentiated (as in the reference).
 * Forward states come from h_hist when given, else from h_ckpt (written by
 * km_scan1d_fwd) when given, else the library first recomputes checkpoints
 * into the workspace. Inputs as in KMScan1DFwd, plus:
 *   dy          : [B, L, D] dtype
 *   dx, ddelta  : [B, L, D] dtype (written)
 *   dA          : [D, N] fp32, summed over batch and time (written)
 *   dB, dC      : dtype. Shared over channels (bc_sd == 0): the sum over
 *                 channels, written at b*bc_sb + t*bc_st + n. Otherwise per
 *                 channel at the B/C strides. Strides must not alias over
 *                 batch or time (bc_sb, bc_st > 0 when B, L > 1).
 *   clamp       : the forward's clamp flag (used when states are recomputed)
 *   workspace   : device scratch of km_scan1d_bwd_workspace_bytes() bytes, or
 *                 NULL for the library's scratch of this (device, stream).
 *                 It holds per-workgroup partial sums (dA and, with shared
 *                 B/C, dB/dC per channel group; the group width depends on
 *                 the kernel the shape runs on) and, when neither h_hist
 *                 nor h_ckpt is given, the recomputed checkpoints.
 * dA (summed over batch and time) and the shared dB/dC (summed over
 * channels) are formed from those partials in a fixed order, with no
 * atomics: every output is identical run to run. */
typedef struct {
    const void  *x;
    const void  *delta;
    const float *A;
    const void  *Bm;
    const void  *Cm;
    const void  *dy;
    const float *h0;
    const float *h_hist;
    const float *h_ckpt;
    void        *dx;
    void        *ddelta;
    float       *dA;
    void        *dB;
    void        *dC;
    long B, L, D, N;
    long bc_sb, bc_st, bc_sd;
    int  dtype;
    int  clamp;
    void        *workspace;
    size_t       workspace_bytes;
} KMScan1DBwd;

size_t km_scan1d_bwd_workspace_bytes(const KMScan1DBwd *a);
int km_scan1d_bwd(const KMScan1DBwd *a, void *stream);

/* ConvND forward / backward on device pointers over `batch` independent
 * grids, enqueued on `stream` without a host synchronisation. Same
 * ConvNDParams as om_convnd_forward / om_convnd_backward (ref
 * include/convnd.h:10-51, cuda/convnd.cu:258-436), with input, output, dy and
 * dinput holding [batch, prod(dims), D]; kernel and bias are shared by the
 * batch, and dkernel / dbias sum over it. Backward overwrites dinput,
 * dkernel and dbias (dbias may be NULL). For 2D (K <= 4) and 3D (K <= 3)
 * grids dkernel and dbias are summed in a fixed order through the library's
 * per-device workspace (identical run to run; backward calls that overlap
 * on one device then race); other shapes sum them with fp32 atomics, whose
 * last bits may vary between runs.
 * Returns 0, or -1 with km_last_error() set. */
int km_convnd_fwd(const ConvNDParams *p, long batch, void *stream);
int km_convnd_bwd(const ConvNDParams *p, long batch, void *stream);

/* bf16 GEMM on the matrix cores (no counterpart in the reference, whose
 * kernels/gemm_f32.c:13-31 is a scalar fp32 triple loop):
 *   C[M, N] = epilogue(A[M, K] . B[N, K]^T + bias[N])
 * A, B: bf16 row-major with leading dimensions lda, ldb (B as [out, in]
 * weights); C: c_dtype (KM_F32 or KM_BF16) with ldc; bias fp32 [N] or NULL.
 * Accumulation in fp32. K, lda and ldb must be multiples of 8. */
typedef enum {
    KM_EPI_NONE = 0,
    KM_EPI_SOFTPLUS = 1,   /* log(1 + e^v) (ref include/kmamba_kernels.h:47-49) */
    KM_EPI_SILU = 2        /* v / (1 + e^-v) (ref include/kmamba_kernels.h:35-37) */
} KMEpilogue;

typedef struct {
    const void  *A;
    const void  *B;
    void        *C;
    const float *bias;
    long M, N, K;
    long lda, ldb, ldc;
    int  c_dtype;
    int  epilogue;
} KMGemm;

int km_gemm_bf16(const KMGemm *g, void *stream);

/* Mamba-1 block forward (configs[4]; no single reference function, composed
 * of the reference pieces: kernels/gemm_f32.c projections, the causal convnd
 * in 1D, SiLU / softplus of include/kmamba_kernels.h:35-49 and the scan1d
 * recurrence). With di = d_inner, N = d_state, R = dt_rank:
 *   xi = x W_in[0:di]^T;  z = x W_in[di:2di]^T
 *   u  = SiLU(causal_conv1d(xi, conv_w) + conv_b)
 *   [dt_low | B | C] = u W_x^T
 *   delta = softplus(dt_low W_dt^T + dt_bias)
 *   y  = (scan(u, delta, A, B, C) + Dskip*u) * SiLU(z)
 *   out = y W_out^T
 * x, out: [B, L, dim] bf16. Weights: W_in [2*di, dim], W_x [R + 2N, di],
 * W_dt [di, R], W_out [dim, di] bf16; conv_w [d_conv, di], conv_b [di] (may
 * be NULL), dt_bias [di], A [di, N], Dskip [di] (may be NULL) fp32.
 * clamp: the +-1000 state clamp of the reference scan (1) or none (0).
 * workspace: km_mamba1_block_workspace_bytes() bytes of device memory, or
 * NULL for the library's scratch of this (device, stream). Every projection
 * runs on km_gemm_bf16's bf16 MFMA kernels. */
typedef struct {
    long dim, d_inner, d_state, d_conv, dt_rank;
    const void  *W_in;
    const float *conv_w;
    const float *conv_b;
    const void  *W_x;
    const void  *W_dt;
    const float *dt_bias;
    const float *A;
    const float *Dskip;
    const void  *W_out;
    int clamp;
} KMMamba1Weights;

size_t km_mamba1_block_workspace_bytes(const KMMamba1Weights *w, long B, long L);
int km_mamba1_block_fwd(const KMMamba1Weights *w, const void *x, void *out, long B, long L,
                        void *workspace, size_t workspace_bytes, void *stream);

/* ScanND forward on device pointers, enqueued on `stream` (NULL = default
 * stream) without a host synchronisation. Same parameters, layout and
 * semantics as om_scannd_forward (ref include/scan_nd.h:72), including the
 * Mamba-3 lambda branch (theta and lambda device memory). Returns 0, or -1
 * with km_last_error() set. */
int km_scannd_fwd(const ScanNDParams *p, void *stream);

/* Status of the latest km_scannd_fwd / km_scannd_fwd_noalloc /
 * km_scannd_bwd call enqueued on `stream` (current device). Waits for the
 * stream, then returns 0 when that call's outputs are exact, 1 when one of
 * its dataflow waits (grids of 2 to 4 dimensions on the tile kernels) ran
 * out of its polling budget (KM_SCANND_FLOW_SPIN): that call then wrote NaN
 * into the affected tiles' states and outputs (the backward: its
 * gradients) and should be run again (the synchronous om_scannd_forward /
 * scannd re-run it on the band schedule by themselves), or -1 on error. A
 * km_scannd_bwd given a workspace keeps its status word there: keep the
 * workspace alive until the status is read. */
int km_scannd_status(void *stream);

/* km_scannd_fwd without any allocation. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * parameters, semantics and results as km_scannd_fwd. The dataflow schedule
 * of 2- to 4-dimensional grids keeps its counters, epoch and completion
 * flags in a fixed 1 MiB array in each GPU's memory (held until the process
 * ends) instead of a per-stream allocation; the epoch is advanced on the
 * device by each call, so a call captured in a HIP graph may be replayed.
 * 1D grids run on the Scan1D kernels that use no workspace. Grids needing
 * more than 262,128 (tile, channel group) flags, shapes of 2 or more
 * dimensions outside the tile kernels (D*M not a multiple of 64, or M not
 * dividing 64), and the Mamba-3 lambda branch (whose rotated states need
 * workspace) are rejected with -1 and km_last_error(). Every call on one
 * GPU shares that array: calls that overlap on one GPU (other streams,
 * other threads) race. */
int km_scannd_fwd_noalloc(const ScanNDParams *p, void *stream);

/* ScanND backward (no counterpart in the reference, which has no ScanND
 * adjoint; the adjoint of scannd_ref, src/scan_nd.c:74-192, for the loss
 * L = sum dy . y). With e_a[p] = exp(delta_a[p] A_a), dtbar = sum_a
 * delta_a / ndims and h the forward's states:
 *   g[p]     = dy[p] C[p] + sum_a [i_a < dims_a - 1] e_a[p + s_a] g[p + s_a]
 *   dC = dy h;  dB = g dtbar x;  dx = sum_m g dtbar B
 *   ddelta_a = sum_m g B x / ndims + [i_a > 0] sum_m g A_a e_a h[p - s_a]
 *   dA_a     = sum_p [i_a > 0] g delta_a e_a h[p - s_a]
 * Layouts as ScanNDParams (dims a host pointer): x, dy, dx [P, D];
 * delta, ddelta [ndims, P, D]; A, dA [ndims, D, M]; B, C, h, dB, dC
 * [P, D, M] (h: the states km_scannd_fwd wrote). All outputs are
 * overwritten; dA is summed in a fixed order (identical run to run).
 * M a power of two <= 64, or ndims * M <= 64. workspace: km_scannd_bwd_workspace_bytes()
 * bytes of device memory, or NULL for the library's scratch of this
 * (device, stream). The adjoint state runs against the forward's wavefront:
 * on 2D and 3D grids with D*M a multiple of 64 as one dataflow launch over
 * tiles on a device with 8 XCDs (KM_SCANND_SCHED=band: one launch per tile
 * band), otherwise one launch per anti-diagonal level, last to first. With
 * D*M a multiple of 2048 and 4 <= M <= 32 (3D: 8 <= M <= 32) that launch
 * runs on pencils and also forms every gradient (the workspace then holds
 * the pencils' boundary states, 1/4 of a [P, D, M] tensor in 2D, 1/2 in
 * 3D; KM_SCANND_BWD_FUSED=0: the sweep, then a separate gradient pass). */
typedef struct {
    const long  *dims;
    long ndims, D, M;
    const float *x;
    const float *A;
    const float *B;
    const float *C;
    const float *delta;
    const float *h;
    const float *dy;
    float *dx;
    float *ddelta;
    float *dA;
    float *dB;
    float *dC;
    void  *workspace;
    size_t workspace_bytes;
} KMScanNDBwd;

size_t km_scannd_bwd_workspace_bytes(const KMScanNDBwd *a);
int km_scannd_bwd(const KMScanNDBwd *a, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* KMAMBA_KM_H */

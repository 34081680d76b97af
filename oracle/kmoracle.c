/* kmoracle.c - CPU restatement of the reference k-mamba hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see kmoracle.h). Compiled with -ffp-contract=off
 * so every product and sum below is one fp32 rounding in the order written,
 * matching the scalar SSE code of the reference. Reductions that the
 * reference never performs at batch scale (over the batch, or over channels
 * for shared B/C) accumulate in fp64 and are marked as such.
 */
#include "kmoracle.h"

#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* memset of n floats; n = 0 leaves p alone (it may be NULL then, which
 * memset itself does not allow). */
static void orc_zero(float *p, long n) {
    if (n > 0) memset(p, 0, (size_t)n * sizeof(float));
}

/* Reference +-1000 state clamp, cpu/scan1d.asm:136-140: minss then maxss.
 * minss returns its second operand when the comparison is false, so NaN
 * maps to +1000. */
static inline float clamp_state(float hn) {
    hn = (hn < 1000.0f) ? hn : 1000.0f;
    hn = (hn > -1000.0f) ? hn : -1000.0f;
    return hn;
}

/* ======================================================================
 * Scan1D forward: cpu/scan1d.asm:53-169 (loop t, d, m; running h[D,M]).
 * ====================================================================== */
void orc_scan1d(OrcScanParams *p) {
    for (long t = 0; t < p->L; t++) {
        for (long d = 0; d < p->D; d++) {
            long td = t * p->D + d;
            float y = 0.0f;
            for (long m = 0; m < p->M; m++) {
                long dm = d * p->M + m;
                float dA = expf(p->delta[td] * p->A[dm]);          /* :90-101 */
                float dB = p->B[td * p->M + m] * p->delta[td];     /* :114-121 */
                float hn = dA * p->h[dm] + dB * p->x[td];          /* :131-134 */
                hn = clamp_state(hn);                              /* :136-140 */
                p->h[dm] = hn;                                     /* :143 */
                y = y + p->C[td * p->M + m] * hn;                  /* :147-152 */
            }
            p->y[td] = y;                                          /* :157-162 */
        }
    }
}

/* Batched / strided form of the same recurrence: for each batch element b
 * the reference scan1d runs on x[b], delta[b] with B(b,t,d,n) read through
 * strides (bc_sd = 0 broadcasts a [B, L, N] operand over channels). Per
 * (b, d) the arithmetic is exactly orc_scan1d's, so splitting the work over
 * (b, d) between threads does not change any result bit.
 * h: [B, D, N] in/out running state (may be NULL: zero initial, not
 * written). h_hist: optional [B, L, D, N] post-update states. */
void orc_scan1d_batched(const float *x, const float *delta, const float *A,
                        const float *Bm, const float *Cm, float *y,
                        float *h, float *h_hist,
                        long B, long L, long D, long N,
                        long bc_sb, long bc_st, long bc_sd,
                        int clamp, int nthreads) {
    long work = B * D;
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
    #pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (long w = 0; w < work; w++) {
        long b = w / D, d = w % D;
        float state[64];
        float *st = state;
        float *heap = NULL;
        if (N > 64) { heap = (float *)malloc((size_t)N * sizeof(float)); st = heap; }
        for (long m = 0; m < N; m++) st[m] = h ? h[(b * D + d) * N + m] : 0.0f;
        for (long t = 0; t < L; t++) {
            long td = (b * L + t) * D + d;
            long bc = b * bc_sb + t * bc_st + d * bc_sd;
            float acc = 0.0f;
            for (long m = 0; m < N; m++) {
                float dA = expf(delta[td] * A[d * N + m]);
                float dB = Bm[bc + m] * delta[td];
                float hn = dA * st[m] + dB * x[td];
                if (clamp) hn = clamp_state(hn);
                st[m] = hn;
                if (h_hist) h_hist[td * N + m] = hn;
                acc = acc + Cm[bc + m] * hn;
            }
            y[td] = acc;
        }
        if (h) for (long m = 0; m < N; m++) h[(b * D + d) * N + m] = st[m];
        free(heap);
    }
}

/* ======================================================================
 * Scan1D backward: cpu/scan1d_backward.c:193-306.
 * ====================================================================== */
static void bwd_zero(OrcScanBackwardParams *p) {            /* :199-205 */
    orc_zero(p->dx, p->L * p->D);
    orc_zero(p->dA, p->D * p->M);
    orc_zero(p->dB, p->L * p->D * p->M);
    orc_zero(p->dC, p->L * p->D * p->M);
    orc_zero(p->ddelta, p->L * p->D);
}

static void bwd_m1(OrcScanBackwardParams *p) {              /* :207-246 */
    float *adj = (float *)calloc((size_t)p->D, sizeof(float));
    bwd_zero(p);
    if (!adj) return;
    for (long t = p->L - 1; t >= 0; t--) {
        for (long d = 0; d < p->D; d++) {
            long td = t * p->D + d;
            float dt = p->delta[td], xt = p->x[td], dy = p->dy[td];
            float a = p->A[d], b = p->B[td], c = p->C[td];
            float dA = expf(dt * a);
            float hp = 0.0f;
            if (t > 0) hp = p->h[(t - 1) * p->D + d];
            else if (p->h0) hp = p->h0[d];
            float ah = adj[d] + dy * c;
            p->dC[td] += dy * p->h[td];
            p->dB[td] += ah * dt * xt;
            p->dA[d] += ah * dt * dA * hp;
            p->dx[td] += ah * dt * b;
            p->ddelta[td] += ah * (a * dA * hp + b * xt);
            adj[d] = ah * dA;
        }
    }
    free(adj);
}

static void bwd_generic(OrcScanBackwardParams *p) {         /* :248-295 */
    long D = p->D, M = p->M;
    float *adj = (float *)calloc((size_t)(D * M), sizeof(float));
    bwd_zero(p);
    if (!adj) return;
    for (long t = p->L - 1; t >= 0; t--) {
        for (long d = 0; d < D; d++) {
            long td = t * D + d;
            float dt = p->delta[td], xt = p->x[td], dy = p->dy[td];
            float ddt = 0.0f;
            for (long m = 0; m < M; m++) {
                long dm = d * M + m, tdm = td * M + m;
                float a = p->A[dm], b = p->B[tdm], c = p->C[tdm];
                float dA = expf(dt * a);
                float hp = 0.0f;
                if (t > 0) hp = p->h[(t - 1) * D * M + dm];
                else if (p->h0) hp = p->h0[dm];
                float ah = adj[dm] + dy * c;
                p->dC[tdm] += dy * p->h[tdm];
                p->dB[tdm] += ah * dt * xt;
                p->dA[dm] += ah * dt * dA * hp;
                p->dx[td] += ah * dt * b;
                ddt += ah * (a * dA * hp + b * xt);
                adj[dm] = ah * dA;
            }
            p->ddelta[td] += ddt;
        }
    }
    free(adj);
}

void orc_scan1d_backward(OrcScanBackwardParams *p) {        /* :297-306 */
    if (!p || !p->x || !p->A || !p->B || !p->C || !p->delta || !p->h || !p->dy ||
        !p->dx || !p->dA || !p->dB || !p->dC || !p->ddelta ||
        p->L <= 0 || p->D <= 0 || p->M <= 0) return;
    if (p->M == 1) bwd_m1(p);
    else bwd_generic(p);
}

/* M=1 shared-B/C backward: scalar path cpu/scan1d_backward.c:23-70 and the
 * AVX2 path :72-180 (taken when A_diag != NULL && D >= 8). The AVX2 path
 * differs in arithmetic order only in ddt, which it accumulates in eight
 * lane partials over d in blocks of 8, reduces lanes 0..7 in order, then adds
 * the scalar tail; that order is restated here without intrinsics. */
void orc_scan1d_backward_m1_shared_bc(OrcScanBackwardSharedParams *p) {
    if (!p || !p->x || !p->A || !p->B || !p->C || !p->delta || !p->h || !p->dy ||
        !p->dx || !p->dA || !p->dB || !p->dC || !p->ddelta || p->L <= 0 || p->D <= 0)
        return;                                                     /* :17-21 */
    long L = p->L, D = p->D;
    int avx_order = (p->A_diag && D >= 8);                          /* :185 */
    orc_zero(p->dx, L * D);
    orc_zero(p->dA, D);
    orc_zero(p->dB, D);
    orc_zero(p->dC, D);
    orc_zero(p->ddelta, L);
    float *adj = (float *)calloc((size_t)D, sizeof(float));
    if (!adj) return;
    for (long t = L - 1; t >= 0; t--) {
        float dt = p->delta[t];
        float ddt = 0.0f;
        float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        long vec_end = avx_order ? (D / 8) * 8 : 0;
        const float *hprev_row = NULL;
        if (t > 0) hprev_row = p->h + (t - 1) * D;
        else if (p->h0) hprev_row = p->h0;
        for (long d = 0; d < D; d++) {
            long td = t * D + d;
            float xt = p->x[td], dy = p->dy[td];
            float a = p->A[d], b = p->B[d], c = p->C[d];
            float dA = p->A_diag ? p->A_diag[td] : expf(dt * a);
            float hp = hprev_row ? hprev_row[d] : 0.0f;
            float ah = adj[d] + dy * c;
            p->dC[d] += dy * p->h[td];
            p->dB[d] += ah * dt * xt;
            p->dA[d] += ah * dt * dA * hp;
            p->dx[td] += ah * dt * b;
            float term = ah * (a * dA * hp + b * xt);
            if (d < vec_end) lanes[d & 7] += term;                  /* :144-146 */
            else {
                if (d == vec_end && avx_order)
                    for (int l = 0; l < 8; l++) ddt += lanes[l];    /* :151-155 */
                ddt += term;
            }
            adj[d] = ah * dA;
        }
        if (avx_order && vec_end == D)
            for (int l = 0; l < 8; l++) ddt += lanes[l];
        p->ddelta[t] += ddt;
    }
    free(adj);
}

/* The decay of the M=1 assembly routines when A_diag is NULL: the
 * third-order Taylor polynomial 1 + x + x^2/2 + x^3/6 of exp(x), x =
 * delta*A, in their instruction order (cpu/scan1d_backward_m1_shared_bc.asm:
 * 220-231 with x^3/6 = (x^3 * 0.5) * 0.33333334; _simple.asm:212-225 with
 * x^3 * 0.16666667). It is not expf: at x = -1 it gives 1/3, not e^-1. */
float orc_m1_asm_taylor(float x, int simple) {
    float x2 = x * x;
    float acc = x + x2 * 0.5f;
    float x3 = x2 * x;
    x3 = simple ? x3 * 0.16666667f : (x3 * 0.5f) * 0.33333334f;
    acc = acc + x3;
    return acc + 1.0f;
}

/* Restatement of scan1d_backward_m1_shared_bc_asm
 * (cpu/scan1d_backward_m1_shared_bc.asm, simple = 0) and
 * scan1d_backward_m1_shared_bc_simple_asm (_simple.asm, simple = 1), which
 * the reference declares (include/scan.h:103-104) but its build never
 * assembles. Same recurrence as the C function, in the instructions' order:
 * vfmadd231 as fmaf, every other operation rounded on its own. The AVX2
 * routine walks channels eight at a time while d + 8 <= D (ddelta terms
 * accumulated by fma into the lane d mod 8, :178-277) and the rest one at a
 * time (mul then add into a scalar, :279-377); ddelta[t] is then
 * ((l0+l4) + (l1+l5)) + ((l2+l6) + (l3+l7)) + tail, added to the zeroed
 * ddelta[t] (:379-388). The scalar routine adds ah * inner in channel order.
 * Validation is the routine's own: only p is checked (:63-65, calloc of adj_h :70-76); L = 0 zeroes
 * dA, dB, dC, and D = 0 zeroes ddelta. */
void orc_scan1d_backward_m1_shared_bc_asm(OrcScanBackwardSharedParams *p, int simple) {
    if (!p) return;
    long L = p->L, D = p->D;
    float *adj = (float *)calloc((size_t)(D > 0 ? D : 1), sizeof(float));
    if (!adj) return;
    orc_zero(p->dx, L * D);              /* :78-113 */
    orc_zero(p->dA, D);
    orc_zero(p->dB, D);
    orc_zero(p->dC, D);
    orc_zero(p->ddelta, L);
    for (long t = L - 1; t >= 0; t--) {
        const float dt = p->delta[t];
        const float *hprev = t > 0 ? p->h + (t - 1) * D : p->h0;   /* NULL: zero state */
        float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float tail = 0.0f;
        long d = 0;
        for (int pass = 0; pass < 2; pass++) {
            long end = (pass == 0) ? (simple ? 0 : (D >= 8 ? D - D % 8 : 0)) : D;
            for (; d < end; d++) {
                long td = t * D + d;
                float xt = p->x[td], gy = p->dy[td];
                float a = p->A[d], b = p->B[d], c = p->C[d];
                float e = p->A_diag ? p->A_diag[td] : orc_m1_asm_taylor(dt * a, simple);
                float hp = hprev ? hprev[d] : 0.0f;
                float ah = gy * c + adj[d];
                p->dC[d] = fmaf(gy, p->h[td], p->dC[d]);
                float ahdt = ah * dt;
                p->dB[d] = fmaf(ahdt, xt, p->dB[d]);
                p->dA[d] = fmaf(ahdt * e, hp, p->dA[d]);
                p->dx[td] = ahdt * b;
                float inner = fmaf(b, xt, (a * e) * hp);
                if (pass == 0) lanes[d & 7] = fmaf(ah, inner, lanes[d & 7]);
                else tail = tail + ah * inner;
                adj[d] = ah * e;
            }
        }
        float s = simple ? tail
                         : ((lanes[0] + lanes[4]) + (lanes[1] + lanes[5])) +
                               ((lanes[2] + lanes[6]) + (lanes[3] + lanes[7])) + tail;
        p->ddelta[t] = s + p->ddelta[t];
    }
    free(adj);
}

/* Batched backward with strided B/C, the adjoint of orc_scan1d_batched
 * without clamp. Per batch element it is cpu/scan1d_backward.c:248-295 with
 * B, C read through strides and dy, x, delta, h of that element; dx and
 * ddelta keep the reference fp32 order. dA [D, N] sums over batch and time,
 * and, when bc_sd == 0 (B/C shared over channels), dB/dC [B, L, N] sum the
 * per-channel gradients over d; these three reductions accumulate in fp64.
 * When bc_sd != 0, dB/dC are written per channel at the strided positions.
 * h0: [B, D, N] or NULL; h_hist: [B, L, D, N] forward states. */
void orc_scan1d_batched_backward(const float *x, const float *delta, const float *A,
                                 const float *Bm, const float *Cm, const float *dy,
                                 const float *h0, const float *h_hist,
                                 float *dx, float *ddelta, float *dA,
                                 float *dB, float *dC,
                                 long B, long L, long D, long N,
                                 long bc_sb, long bc_st, long bc_sd, int nthreads) {
    int shared = (bc_sd == 0);
    if (N > 64) return;
    if (nthreads < 1) nthreads = 1;
    long bcsz = shared ? B * L * N : 0;
    double *dA64 = (double *)calloc((size_t)(D * N), sizeof(double));
    double *dB64 = shared ? (double *)calloc((size_t)nthreads * bcsz, sizeof(double)) : NULL;
    double *dC64 = shared ? (double *)calloc((size_t)nthreads * bcsz, sizeof(double)) : NULL;
    if (!dA64 || (shared && (!dB64 || !dC64))) { free(dA64); free(dB64); free(dC64); return; }

#ifdef _OPENMP
    #pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (long d = 0; d < D; d++) {
        int tid = 0;
#ifdef _OPENMP
        tid = omp_get_thread_num();
#endif
        float adj[64];
        for (long b = 0; b < B; b++) {
            for (long m = 0; m < N; m++) adj[m] = 0.0f;
            for (long t = L - 1; t >= 0; t--) {
                long td = (b * L + t) * D + d;
                long bc = b * bc_sb + t * bc_st + d * bc_sd;
                float dt = delta[td], xt = x[td], g = dy[td];
                float dxv = 0.0f, ddt = 0.0f;
                for (long m = 0; m < N; m++) {
                    float a = A[d * N + m], bb = Bm[bc + m], c = Cm[bc + m];
                    float e = expf(dt * a);
                    float hp = 0.0f;
                    if (t > 0) hp = h_hist[(td - D) * N + m];
                    else if (h0) hp = h0[(b * D + d) * N + m];
                    float ah = adj[m] + g * c;
                    float dCv = g * h_hist[td * N + m];
                    float dBv = ah * dt * xt;
                    dA64[d * N + m] += (double)(ah * dt * e * hp);
                    dxv += ah * dt * bb;
                    ddt += ah * (a * e * hp + bb * xt);
                    adj[m] = ah * e;
                    if (shared) {
                        long o = (b * L + t) * N + m;
                        dB64[tid * bcsz + o] += (double)dBv;
                        dC64[tid * bcsz + o] += (double)dCv;
                    } else {
                        dB[bc + m] = dBv;
                        dC[bc + m] = dCv;
                    }
                }
                dx[td] = dxv;
                ddelta[td] = ddt;
            }
        }
    }
    for (long i = 0; i < D * N; i++) dA[i] = (float)dA64[i];
    if (shared) {
        for (long o = 0; o < bcsz; o++) {
            double sb = 0.0, sc = 0.0;
            for (int t = 0; t < nthreads; t++) { sb += dB64[t * bcsz + o]; sc += dC64[t * bcsz + o]; }
            long b = o / (L * N), rem = o % (L * N), t = rem / N, m = rem % N;
            dB[b * bc_sb + t * bc_st + m] = (float)sb;
            dC[b * bc_sb + t * bc_st + m] = (float)sc;
        }
    }
    free(dA64); free(dB64); free(dC64);
}

/* ======================================================================
 * Scan2D: cpu/scan2d.asm:66-275 (anti-diagonal k = i + j, i ascending).
 * ====================================================================== */
void orc_scan2d(OrcScan2DParams *p) {
    long d1 = p->d1, d2 = p->d2, D = p->D, M = p->M, DM = D * M;
    for (long k = 0; k < d1 + d2 - 1; k++) {                        /* :66-72 */
        long imin = k - d2 + 1; if (imin < 0) imin = 0;              /* :74-82 */
        long imax = k; if (imax > d1 - 1) imax = d1 - 1;             /* :84-92 */
        for (long i = imin; i <= imax; i++) {
            long j = k - i, pos = i * d2 + j;
            for (long d = 0; d < D; d++) {
                long pd = pos * D + d;
                float y = 0.0f;
                for (long m = 0; m < M; m++) {
                    long dm = d * M + m, q = pos * DM + dm;
                    float h1 = (i > 0) ? p->h[(pos - d2) * DM + dm] : 0.0f;   /* :148-159 */
                    float h2 = (j > 0) ? p->h[(pos - 1) * DM + dm] : 0.0f;    /* :161-172 */
                    float a1 = expf(p->delta1[pd] * p->A1[dm]);               /* :179-185 */
                    float a2 = expf(p->delta2[pd] * p->A2[dm]);               /* :190-199 */
                    float dB = p->B[q] * ((p->delta1[pd] + p->delta2[pd]) * 0.5f); /* :204-224 */
                    float hn = ((a1 * h1) + (a2 * h2)) + (dB * p->x[pd]);     /* :232-239 */
                    p->h[q] = hn;                                             /* :241-243 */
                    y = y + p->C[q] * hn;                                     /* :245-251 */
                }
                p->y[pd] = y;
            }
        }
    }
}

/* ======================================================================
 * Wavefront enumeration and plan, restated by brute force so that it pins
 * the product's closed-form implementation independently.
 * src/wavefront_nd.c:134-279, src/wavefront_plan.c:35-132.
 * ====================================================================== */
int orc_wavefront_validate_dims(const long *dims, long ndims) {
    if (!dims || ndims <= 0) return 0;
    for (long i = 0; i < ndims; i++) if (dims[i] <= 0) return 0;
    return 1;
}

long orc_wavefront_total_points(const long *dims, long ndims) {
    if (!orc_wavefront_validate_dims(dims, ndims)) return -1;
    long total = 1;
    for (long i = 0; i < ndims; i++) {
        if (total > LONG_MAX / dims[i]) return -1;
        total *= dims[i];
    }
    return total;
}

long orc_wavefront_max_level(const long *dims, long ndims) {
    if (!orc_wavefront_validate_dims(dims, ndims)) return -1;
    long lvl = 0;
    for (long i = 0; i < ndims; i++) {
        if (lvl > LONG_MAX - (dims[i] - 1)) return -1;
        lvl += dims[i] - 1;
    }
    return lvl;
}

long orc_wavefront_row_major_offset(const long *dims, const long *idx, long ndims) {
    if (!orc_wavefront_validate_dims(dims, ndims) || !idx) return -1;
    long off = 0;
    for (long a = 0; a < ndims; a++) {
        if (idx[a] < 0 || idx[a] >= dims[a]) return -1;
        if (off > (LONG_MAX - idx[a]) / dims[a]) return -1;
        off = off * dims[a] + idx[a];
    }
    return off;
}

/* Counts points with coordinate sum == level by enumerating every point. */
long orc_wavefront_level_size(const long *dims, long ndims, long level) {
    long maxl = orc_wavefront_max_level(dims, ndims);
    long P = orc_wavefront_total_points(dims, ndims);
    if (maxl < 0 || P < 0 || level < 0 || level > maxl) return -1;
    long cnt = 0;
    for (long off = 0; off < P; off++) {
        long rem = off, s = 0;
        for (long a = ndims - 1; a >= 0; a--) { s += rem % dims[a]; rem /= dims[a]; }
        if (s == level) cnt++;
    }
    return cnt;
}

/* Plan by a stable counting sort of all row-major offsets by level: within a
 * level offsets come out ascending, which is the reference's lexicographic
 * emission order (src/wavefront_nd.c:84-109). */
OrcPlan *orc_plan_create(const long *dims, long ndims) {
    long P = orc_wavefront_total_points(dims, ndims);
    long maxl = orc_wavefront_max_level(dims, ndims);
    if (P <= 0 || maxl < 0) return NULL;
    OrcPlan *pl = (OrcPlan *)calloc(1, sizeof(*pl));
    long *lvl = (long *)malloc((size_t)P * sizeof(long));
    if (!pl || !lvl) { free(pl); free(lvl); return NULL; }
    pl->dims = (long *)malloc((size_t)ndims * sizeof(long));
    pl->level_starts = (long *)calloc((size_t)(maxl + 2), sizeof(long));
    pl->level_offsets = (long *)malloc((size_t)P * sizeof(long));
    if (!pl->dims || !pl->level_starts || !pl->level_offsets) {
        orc_plan_free(pl); free(lvl); return NULL;
    }
    memcpy(pl->dims, dims, (size_t)ndims * sizeof(long));
    pl->ndims = ndims; pl->total_points = P; pl->max_level = maxl;
    for (long off = 0; off < P; off++) {
        long rem = off, s = 0;
        for (long a = ndims - 1; a >= 0; a--) { s += rem % dims[a]; rem /= dims[a]; }
        lvl[off] = s;
        pl->level_starts[s + 1]++;
    }
    for (long l = 0; l <= maxl; l++) {
        long sz = pl->level_starts[l + 1];
        if (sz > pl->max_level_size) pl->max_level_size = sz;
        pl->level_starts[l + 1] = pl->level_starts[l] + sz;
    }
    long *cur = (long *)malloc((size_t)(maxl + 1) * sizeof(long));
    if (!cur) { orc_plan_free(pl); free(lvl); return NULL; }
    memcpy(cur, pl->level_starts, (size_t)(maxl + 1) * sizeof(long));
    for (long off = 0; off < P; off++) pl->level_offsets[cur[lvl[off]]++] = off;
    free(cur); free(lvl);
    return pl;
}

void orc_plan_free(OrcPlan *pl) {
    if (!pl) return;
    free(pl->dims); free(pl->level_starts); free(pl->level_offsets); free(pl);
}

/* src/km_topology.c:24-81 */
int orc_make_row_major_strides(const long *dims, long ndims, long *strides) {
    if (!dims || !strides || ndims <= 0 || ndims > 8) return 0;
    if (!orc_wavefront_validate_dims(dims, ndims)) return 0;
    long s = 1;
    for (long a = ndims - 1; a >= 0; a--) { strides[a] = s; s *= dims[a]; }
    return 1;
}

void orc_unravel_index(long linear, const long *dims, const long *strides, long ndims, long *coords) {
    if (!dims || !strides || !coords || ndims <= 0 || ndims > 8 || linear < 0) return;
    for (long a = 0; a < ndims; a++) coords[a] = (linear / strides[a]) % dims[a];
}

long orc_ravel_index(const long *coords, const long *dims, const long *strides, long ndims) {
    if (!coords || !dims || !strides || ndims <= 0 || ndims > 8) return -1;
    long off = 0;
    for (long a = 0; a < ndims; a++) {
        if (coords[a] < 0 || coords[a] >= dims[a]) return -1;
        off += coords[a] * strides[a];
    }
    return off;
}

long orc_power_long(long base, long exp) {
    if (exp < 0) return 0;
    if (base == 0 && exp == 0) return 0;
    long r = 1;
    for (long i = 0; i < exp; i++) r *= base;
    return r;
}

/* ======================================================================
 * ScanND reference: src/scan_nd.c:17-308, lambda == NULL branch
 * (Appendix order :95-192). The idx scratch is private per point, which
 * removes the reference's shared-idx race (src/scan_nd.c:34, :86-95).
 * ====================================================================== */
int orc_scannd_validate(const OrcScanNDParams *p) {          /* :17-29 */
    if (!p || !p->dims) return 0;
    if (p->ndims <= 0 || p->D <= 0 || p->M <= 0) return 0;
    if (!p->x || !p->A || !p->B || !p->C || !p->delta || !p->h || !p->y) return 0;
    if (!orc_wavefront_validate_dims(p->dims, p->ndims)) return 0;
    if (orc_wavefront_total_points(p->dims, p->ndims) <= 0) return 0;
    return 1;
}

static void scannd_point(OrcScanNDParams *p, long P, const long *strides, long offset) {
    long idx[8];
    long D = p->D, M = p->M, nd = p->ndims;
    orc_unravel_index(offset, p->dims, strides, nd, idx);
    for (long d = 0; d < D; d++) {
        float x_val = p->x[offset * D + d];
        float dt_bar = 0.0f, y_acc = 0.0f;
        for (long a = 0; a < nd; a++) dt_bar += p->delta[(a * P + offset) * D + d];  /* :105-107 */
        dt_bar /= (float)nd;                                                           /* :108 */
        for (long m = 0; m < M; m++) {
            long dm = d * M + m, pdm = offset * D * M + dm;
            float bu = p->B[pdm] * x_val;                                              /* :115 */
            float hn = dt_bar * bu;                                                    /* :174 */
            for (long a = 0; a < nd; a++) {                                            /* :175-184 */
                if (idx[a] > 0) {
                    long prev = offset - strides[a];
                    float dt_a = p->delta[(a * P + offset) * D + d];
                    float av = p->A[(a * D + d) * M + m];
                    float decay = expf(dt_a * av);
                    hn += decay * p->h[prev * D * M + dm];
                }
            }
            p->h[pdm] = hn;                                                            /* :187 */
            y_acc += p->C[pdm] * hn;                                                   /* :188 */
        }
        p->y[offset * D + d] = y_acc;                                                  /* :191 */
    }
}

/* Mamba-3 branch (lambda != NULL), src/scan_nd.c:59-72 and :95-210. The
 * reference sizes its rotated-state buffer h_rot [D, M] but indexes it with
 * point offsets (prev * D * M + dm, :166, :200-205), and reads it whether
 * or not theta rotated anything: out-of-bounds and uninitialised reads, so
 * its output is undefined. This restatement follows the evident intent:
 * hrot [P, D, M] holds each point's state after the pair rotation R(theta)
 * (channels 2i, 2i+1 by theta[i]; an odd last channel unrotated), or the
 * state itself when theta is NULL, and predecessors are read from it. The
 * predecessor "Bu_prev" (:121-127, :164) is B[prev] * x[prev], which the
 * reference stores per point (:169). Arithmetic order as written at
 * :104-191: bu, then per axis the predecessor sums, then the averages,
 * beta = (1 - lambda) * dt_bar * alpha_avg, gamma = lambda * dt_bar,
 * h = bu_prev_avg * beta + bu * gamma, then alpha_a * hrot[prev_a] per axis,
 * with A clamped to at most -1e-5 in this branch (:129, :157). */
static void scannd_point_m3(OrcScanNDParams *p, long P, const long *strides, long offset,
                            float *hrot) {
    long idx[8];
    long D = p->D, M = p->M, nd = p->ndims;
    orc_unravel_index(offset, p->dims, strides, nd, idx);
    float lam = p->lambda[offset];                                                     /* :99 */
    for (long d = 0; d < D; d++) {
        float x_val = p->x[offset * D + d];
        float dt_bar = 0.0f, y_acc = 0.0f;
        for (long a = 0; a < nd; a++) dt_bar += p->delta[(a * P + offset) * D + d];
        dt_bar /= (float)nd;
        for (long m = 0; m < M; m++) {
            long dm = d * M + m, pdm = offset * D * M + dm;
            float bu = p->B[pdm] * x_val;                                              /* :115 */
            float bu_prev_acc = 0.0f, decay_acc = 0.0f;
            int n_pred = 0;
            for (long a = 0; a < nd; a++) {                                            /* :123-142 */
                if (idx[a] > 0) {
                    long prev = offset - strides[a];
                    float dt_a = p->delta[(a * P + offset) * D + d];
                    float av = p->A[(a * D + d) * M + m];
                    if (av > -1e-5f) av = -1e-5f;
                    float alpha = expf(dt_a * av);
                    bu_prev_acc += p->B[prev * D * M + dm] * p->x[prev * D + d];
                    decay_acc += alpha;
                    n_pred++;
                }
            }
            float bu_prev_avg = (n_pred > 0) ? (bu_prev_acc / (float)n_pred) : 0.0f;   /* :148 */
            float alpha_avg = (n_pred > 0) ? (decay_acc / (float)n_pred) : 0.0f;
            float beta = (1.0f - lam) * dt_bar * alpha_avg;
            float gamma = lam * dt_bar;
            float hn = bu_prev_avg * beta + bu * gamma;                                /* :155 */
            if (n_pred > 0) {
                for (long a = 0; a < nd; a++) {                                        /* :156-167 */
                    if (idx[a] > 0) {
                        long prev = offset - strides[a];
                        float dt_a = p->delta[(a * P + offset) * D + d];
                        float av = p->A[(a * D + d) * M + m];
                        if (av > -1e-5f) av = -1e-5f;
                        float alpha = expf(dt_a * av);
                        hn += alpha * hrot[prev * D * M + dm];
                    }
                }
            }
            p->h[pdm] = hn;
            y_acc += p->C[pdm] * hn;
        }
        p->y[offset * D + d] = y_acc;
    }
    /* The point's states as its successors read them (:194-209). */
    float *hr = hrot + offset * D * M;
    const float *hs = p->h + offset * D * M;
    if (!p->theta) {
        for (long i = 0; i < D * M; i++) hr[i] = hs[i];
        return;
    }
    for (long d = 0; d + 1 < D; d += 2) {
        float th = p->theta[d >> 1];
        float cv = cosf(th), sv = sinf(th);
        for (long m = 0; m < M; m++) {
            float h0 = hs[d * M + m], h1 = hs[(d + 1) * M + m];
            hr[d * M + m] = cv * h0 - sv * h1;
            hr[(d + 1) * M + m] = sv * h0 + cv * h1;
        }
    }
    if (D & 1)
        for (long m = 0; m < M; m++) hr[(D - 1) * M + m] = hs[(D - 1) * M + m];
}

int orc_scannd_ref_with_plan(OrcScanNDParams *p, const OrcPlan *plan, int nthreads) {
    if (!orc_scannd_validate(p)) return -1;
    if (!plan || plan->ndims != p->ndims) return -1;
    for (long a = 0; a < p->ndims; a++) if (plan->dims[a] != p->dims[a]) return -1;
    long strides[8];
    if (!orc_make_row_major_strides(p->dims, p->ndims, strides)) return -1;
    long P = plan->total_points;
    if (nthreads < 1) nthreads = 1;
    /* theta without lambda has no effect (the rotation lives in the lambda
     * branch, :59-72). */
    float *hrot = NULL;
    if (p->lambda) {
        hrot = (float *)malloc(sizeof(float) * (size_t)P * (size_t)p->D * (size_t)p->M);
        if (!hrot) return -1;
    }
    for (long level = 0; level <= plan->max_level; level++) {
        long s0 = plan->level_starts[level], s1 = plan->level_starts[level + 1];
#ifdef _OPENMP
        #pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
        for (long i = s0; i < s1; i++) {
            if (hrot) scannd_point_m3(p, P, strides, plan->level_offsets[i], hrot);
            else scannd_point(p, P, strides, plan->level_offsets[i]);
        }
    }
    free(hrot);
    return 0;
}

int orc_scannd_ref(OrcScanNDParams *p, int nthreads) {        /* :235-247 */
    if (!orc_scannd_validate(p)) return -1;
    OrcPlan *pl = orc_plan_create(p->dims, p->ndims);
    if (!pl) return -1;
    int rc = orc_scannd_ref_with_plan(p, pl, nthreads);
    orc_plan_free(pl);
    return rc;
}

/* Adjoint of scannd_ref; see kmoracle.h. */
int orc_scannd_backward(const OrcScanNDParams *p, const float *dy, float *dx, float *ddelta,
                        float *dA, float *dB, float *dC) {
    if (!p || !p->dims || p->ndims <= 0 || p->ndims > 8 || p->D <= 0 || p->M <= 0) return -1;
    if (!p->x || !p->A || !p->B || !p->C || !p->delta || !p->h || !dy) return -1;
    if (!dx || !ddelta || !dA || !dB || !dC) return -1;
    if (p->lambda) return -1;   /* no adjoint of the Mamba-3 branch */
    if (!orc_wavefront_validate_dims(p->dims, p->ndims)) return -1;
    long strides[8], idx[8];
    if (!orc_make_row_major_strides(p->dims, p->ndims, strides)) return -1;
    const long nd = p->ndims, D = p->D, M = p->M;
    const long P = orc_wavefront_total_points(p->dims, nd);
    float *g = dB;
    for (long q = P - 1; q >= 0; q--) {
        orc_unravel_index(q, p->dims, strides, nd, idx);
        for (long d = 0; d < D; d++) {
            const float dyv = dy[q * D + d];
            for (long m = 0; m < M; m++) {
                const long dm = d * M + m;
                float gv = dyv * p->C[q * D * M + dm];
                for (long a = 0; a < nd; a++) {
                    if (idx[a] + 1 < p->dims[a]) {
                        const long nx = q + strides[a];
                        const float e = expf(p->delta[(a * P + nx) * D + d] * p->A[(a * D + d) * M + m]);
                        gv += e * g[nx * D * M + dm];
                    }
                }
                g[q * D * M + dm] = gv;
            }
        }
    }
    for (long i = 0; i < nd * D * M; i++) dA[i] = 0.0f;
    for (long q = 0; q < P; q++) {
        orc_unravel_index(q, p->dims, strides, nd, idx);
        for (long d = 0; d < D; d++) {
            const float xv = p->x[q * D + d], dyv = dy[q * D + d];
            float dtb = 0.0f;
            for (long a = 0; a < nd; a++) dtb += p->delta[(a * P + q) * D + d];
            dtb /= (float)nd;
            float sx = 0.0f, sbx = 0.0f, sdel[8];
            for (long a = 0; a < nd; a++) sdel[a] = 0.0f;
            for (long m = 0; m < M; m++) {
                const long dm = d * M + m, pdm = q * D * M + dm;
                const float gv = g[pdm], bv = p->B[pdm];
                dC[pdm] = dyv * p->h[pdm];
                sx += gv * dtb * bv;
                sbx += gv * bv * xv;
                for (long a = 0; a < nd; a++) {
                    if (idx[a] > 0) {
                        const float dta = p->delta[(a * P + q) * D + d];
                        const float av = p->A[(a * D + d) * M + m];
                        const float e = expf(dta * av);
                        const float gh = gv * e * p->h[(q - strides[a]) * D * M + dm];
                        sdel[a] += gh * av;
                        dA[(a * D + d) * M + m] += gh * dta;
                    }
                }
                dB[pdm] = gv * dtb * xv;
            }
            dx[q * D + d] = sx;
            for (long a = 0; a < nd; a++) ddelta[(a * P + q) * D + d] = sbx / (float)nd + sdel[a];
        }
    }
    return 0;
}

/* CPU dispatch of scannd (src/scan_nd.c:265-307): 1D -> scan1d with h as a
 * running [D, M] state, 2D -> scan2d, otherwise scannd_ref. */
int orc_scannd(OrcScanNDParams *p, int nthreads) {
    if (!orc_scannd_validate(p)) return -1;
    if (p->ndims == 1) {
        OrcScanParams s = { (float *)p->x, (float *)p->A, (float *)p->B, (float *)p->C,
                            (float *)p->delta, p->h, p->y, p->dims[0], p->D, p->M };
        orc_scan1d(&s);
        return 0;
    }
    if (p->ndims == 2) {
        long P = orc_wavefront_total_points(p->dims, 2);
        OrcScan2DParams s;
        s.x = (float *)p->x; s.A1 = (float *)p->A; s.A2 = (float *)(p->A + p->D * p->M);
        s.B = (float *)p->B; s.C = (float *)p->C;
        s.delta1 = (float *)p->delta; s.delta2 = (float *)(p->delta + P * p->D);
        s.h = p->h; s.y = p->y; s.d1 = p->dims[0]; s.d2 = p->dims[1]; s.D = p->D; s.M = p->M;
        orc_scan2d(&s);
        return 0;
    }
    return orc_scannd_ref(p, nthreads);
}

/* ======================================================================
 * ConvND: src/convnd.c:58-244.
 * ====================================================================== */
long orc_convnd_kernel_volume(long ndims, long K) {          /* :58-61 */
    if (ndims <= 0 || K <= 0) return 0;
    long v = 1;
    for (long i = 0; i < ndims; i++) v *= K;
    return v;
}

static void conv_strides(const long *dims, long nd, long *st) {  /* :50-56 */
    long s = 1;
    for (long a = nd; a-- > 0;) { st[a] = s; s *= dims[a]; }
}

/* Forward (:67-129). Point order does not affect results; taps run
 * kl = 0..K^N-1 with the last axis fastest, skipping out-of-range taps. */
void orc_convnd_forward(OrcConvNDParams *p, int nthreads) {
    if (!p || !p->input || !p->kernel || !p->output || !p->dims ||
        p->ndims <= 0 || p->D <= 0 || p->K <= 0) return;
    long nd = p->ndims, D = p->D, K = p->K, st[8];
    long P = orc_wavefront_total_points(p->dims, nd);
    long KV = orc_convnd_kernel_volume(nd, K);
    if (P <= 0 || nd > 8) return;
    conv_strides(p->dims, nd, st);
    if (nthreads < 1) nthreads = 1;
#ifdef _OPENMP
    #pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (long out = 0; out < P; out++) {
        long oc[8], rem = out;
        for (long a = nd; a-- > 0;) { oc[a] = rem % p->dims[a]; rem /= p->dims[a]; }  /* :43-48 */
        for (long d = 0; d < D; d++) {
            float sum = p->bias ? p->bias[d] : 0.0f;                           /* :96 */
            for (long kl = 0; kl < KV; kl++) {
                long tmp = kl, src = 0; int valid = 1;
                for (long a = nd; a-- > 0;) {                                   /* :103-114 */
                    long ka = tmp % K; tmp /= K;
                    long sc = oc[a] - (K - 1 - ka);
                    if (sc < 0 || sc >= p->dims[a]) { valid = 0; break; }
                    src += sc * st[a];
                }
                if (!valid) continue;
                sum += p->input[src * D + d] * p->kernel[kl * D + d];           /* :117-118 */
            }
            p->output[out * D + d] = sum;                                       /* :121 */
        }
    }
}

/* Backward (:135-202): zero the gradients, then levels from max_level down
 * to 0 and points of a level in plan order, serially. */
void orc_convnd_backward(OrcConvNDParams *p) {
    if (!p || !p->input || !p->kernel || !p->dy || !p->dinput || !p->dkernel ||
        !p->dims || p->ndims <= 0 || p->D <= 0 || p->K <= 0) return;
    long nd = p->ndims, D = p->D, K = p->K, st[8];
    long P = orc_wavefront_total_points(p->dims, nd);
    long KV = orc_convnd_kernel_volume(nd, K);
    if (P <= 0 || nd > 8) return;
    OrcPlan *pl = orc_plan_create(p->dims, nd);
    if (!pl) return;
    conv_strides(p->dims, nd, st);
    orc_zero(p->dinput, P * D);
    orc_zero(p->dkernel, KV * D);
    if (p->dbias) orc_zero(p->dbias, D);
    for (long level = pl->max_level; level >= 0; level--) {
        for (long i = pl->level_starts[level]; i < pl->level_starts[level + 1]; i++) {
            long out = pl->level_offsets[i], oc[8], rem = out;
            for (long a = nd; a-- > 0;) { oc[a] = rem % p->dims[a]; rem /= p->dims[a]; }
            for (long d = 0; d < D; d++) {
                float g = p->dy[out * D + d];
                if (p->dbias) p->dbias[d] += g;
                for (long kl = 0; kl < KV; kl++) {
                    long tmp = kl, src = 0; int valid = 1;
                    for (long a = nd; a-- > 0;) {
                        long ka = tmp % K; tmp /= K;
                        long sc = oc[a] - (K - 1 - ka);
                        if (sc < 0 || sc >= p->dims[a]) { valid = 0; break; }
                        src += sc * st[a];
                    }
                    if (!valid) continue;
                    p->dkernel[kl * D + d] += g * p->input[src * D + d];
                    p->dinput[src * D + d] += g * p->kernel[kl * D + d];
                }
            }
        }
    }
    orc_plan_free(pl);
}


/* ======================================================================
 * Mamba-3 block forward: src/mamba_block.c:89-120 (controller), :413-466
 * (scan), :471-501 (forward). gemv rows sum j = 0..D-1 in order
 * (kernels/gemm_f32.c:48-58); SiLU, softplus, sigmoid as
 * include/kmamba_kernels.h:35-49.
 * ====================================================================== */
static void m3_gemv(const float *A, const float *x, float *y, long M, long N) {
    for (long i = 0; i < M; i++) {                      /* gemm_f32.c:51-57 */
        float sum = 0.0f;
        for (long j = 0; j < N; j++) sum += A[i * N + j] * x[j];
        y[i] = sum;
    }
}

void orc_mamba3_forward(const OrcMamba3 *p, const float *input, float *output, long batch) {
    if (!p || !input || !output) return;
    long L = p->L, D = p->D, N = p->N, R = p->R > 1 ? p->R : 1, NR = N * R;
    float *z = malloc((size_t)R * sizeof(float));
    float *u = malloc((size_t)(L * R) * sizeof(float));
    float *dl = malloc((size_t)L * sizeof(float));
    float *lam = malloc((size_t)L * sizeof(float));
    float *Bs = malloc((size_t)(L * NR) * sizeof(float));
    float *Cs = malloc((size_t)(L * NR) * sizeof(float));
    float *y = malloc((size_t)(L * R) * sizeof(float));
    float *yp = malloc((size_t)D * sizeof(float));
    float *h = malloc((size_t)N * sizeof(float));
    float *hr = malloc((size_t)N * sizeof(float));
    float *bu = malloc((size_t)N * sizeof(float));
    float *pbu = malloc((size_t)N * sizeof(float));
    if (!z || !u || !dl || !lam || !Bs || !Cs || !y || !yp || !h || !hr || !bu || !pbu) goto out;
    for (long b = 0; b < batch; b++) {
        const float *in = input + b * L * D;
        float *o = output + b * L * D;
        for (long t = 0; t < L; t++) {
            const float *xt = in + t * D;
            m3_gemv(p->W_in, xt, z, R, D);                               /* :98-99 */
            for (long r = 0; r < R; r++) u[t * R + r] = z[r] / (1.0f + expf(-z[r]));
            if (p->delta_proj) {                                         /* :102-108 */
                float dv;
                m3_gemv(p->delta_proj, xt, &dv, 1, D);
                dv = logf(1.0f + expf(dv));
                if (dv < p->dt_min) dv = p->dt_min;
                if (dv > p->dt_max) dv = p->dt_max;
                dl[t] = dv;
            } else {
                dl[t] = p->dt_scale;
            }
            if (p->lambda_proj) {                                        /* :112-118 */
                float lr;
                m3_gemv(p->lambda_proj, xt, &lr, 1, D);
                lam[t] = 1.0f / (1.0f + expf(-lr));
            } else {
                lam[t] = 0.5f;
            }
            m3_gemv(p->W_B, xt, Bs + t * NR, NR, D);                     /* :488-493 */
            m3_gemv(p->W_C, xt, Cs + t * NR, NR, D);
            for (long i = 0; i < NR; i++) {
                Bs[t * NR + i] += p->b_B[i];
                Cs[t * NR + i] += p->b_C[i];
            }
        }
        orc_zero(h, N);                        /* :422 */
        orc_zero(pbu, N);
        for (long t = 0; t < L; t++) {
            float dt = dl[t], lt = lam[t];
            const float *bt = Bs + t * NR, *ct = Cs + t * NR, *ut = u + t * R;
            for (long i = 0; i + 1 < N; i += 2) {                        /* :431-437 */
                float th = p->theta[i >> 1], cv = cosf(th), sv = sinf(th);
                float h0 = h[i], h1 = h[i + 1];
                hr[i] = cv * h0 - sv * h1;
                hr[i + 1] = sv * h0 + cv * h1;
            }
            if (N & 1) hr[N - 1] = h[N - 1];
            orc_zero(bu, N);                   /* :440-443 */
            for (long r = 0; r < R; r++)
                for (long n = 0; n < N; n++) bu[n] += bt[r * N + n] * ut[r];
            for (long n = 0; n < N; n++) {                               /* :446-452 */
                float a = p->A_log[n];
                float alpha = expf(dt * a);
                float beta = (1.0f - lt) * dt * alpha;
                float gamma = lt * dt;
                h[n] = alpha * hr[n] + beta * pbu[n] + gamma * bu[n];
            }
            for (long r = 0; r < R; r++) {                               /* :455-459 */
                float yr = 0.0f;
                for (long n = 0; n < N; n++) yr += ct[r * N + n] * h[n];
                y[t * R + r] = yr;
            }
            memcpy(pbu, bu, (size_t)N * sizeof(float));                 /* :462 */
        }
        for (long t = 0; t < L; t++) {                                   /* :496-499 */
            m3_gemv(p->W_out, y + t * R, yp, D, R);
            for (long d = 0; d < D; d++) o[t * D + d] = in[t * D + d] + yp[d];
        }
    }
out:
    free(z); free(u); free(dl); free(lam); free(Bs); free(Cs); free(y); free(yp);
    free(h); free(hr); free(bu); free(pbu);
}

/* ref kernels/gemm_f32.c:13-31; see kmoracle.h. */
void orc_gemm_f32(const float *A, const float *B, float *C, long M, long K, long N) {
    if (!A || !B || !C || M <= 0 || N <= 0) return;
    #pragma omp parallel for schedule(static)
    for (long i = 0; i < M; i++) {
        float *c = C + i * N;
        for (long j = 0; j < N; j++) c[j] = 0.0f;
        for (long k = 0; k < K; k++) {
            const float a = A[i * K + k];
            const float *b = B + k * N;
            for (long j = 0; j < N; j++) c[j] = c[j] + a * b[j];
        }
    }
}

/* SiLU and softplus of the reference (include/kmamba_kernels.h:35-37 and
 * :47-49, applied elementwise by kernels/activations_f32.c:7-29):
 * x / (1 + expf(-x)) and logf(1 + expf(x)), fp32, glibc expf/logf, no
 * overflow guard (softplus of x > ~88.7 is +inf, SiLU of x < ~-88.7 is -0). */
void orc_silu_f32(const float *x, float *y, long n) {
    for (long i = 0; i < n; i++) {
        const float den = 1.0f + expf(-x[i]);
        y[i] = x[i] / den;
    }
}

void orc_softplus_f32(const float *x, float *y, long n) {
    for (long i = 0; i < n; i++) {
        const float arg = 1.0f + expf(x[i]);
        y[i] = logf(arg);
    }
}

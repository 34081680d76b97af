/* A plain C caller of libkmamba, built with gcc against include/ and
 * lib/libkmamba.so only (no torch, no Python): the way existing k-mamba C
 * code uses the drop-in. It runs the reference host-pointer API scan1d on a
 * small problem and prints y, the final state and the library's error
 * string, for tests/test_c_caller.py to compare with the oracle. Then the
 * model API: kmamba_create / init / forward on a small model, kmamba_save,
 * kmamba_load and a second forward, which must give identical logits; the
 * tokens and logits go to KM_C_CALLER_MODEL, the checkpoint to
 * KM_C_CALLER_CKPT. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kmamba.h"

#include "kmamba_cuda_utils.h"
#include "kmamba_km.h"
#include "mamba_scan.h"
#include "wavefront_plan.h"

int main(void) {
    const long L = 33, D = 40, M = 16;
    float *x = malloc(sizeof(float) * L * D), *dt = malloc(sizeof(float) * L * D);
    float *y = calloc(L * D, sizeof(float)), *A = malloc(sizeof(float) * D * M);
    float *B = malloc(sizeof(float) * L * D * M), *C = malloc(sizeof(float) * L * D * M);
    float *h = calloc(D * M, sizeof(float));
    unsigned s = 12345u;
#define RND() ((s = s * 1664525u + 1013904223u), (float)((s >> 8) & 0xffff) / 65536.0f)
    for (long i = 0; i < L * D; i++) { x[i] = 2.0f * RND() - 1.0f; dt[i] = 0.01f + 0.49f * RND(); }
    for (long i = 0; i < D * M; i++) { A[i] = -0.01f - 0.99f * RND(); h[i] = RND() - 0.5f; }
    for (long i = 0; i < L * D * M; i++) { B[i] = RND() - 0.5f; C[i] = RND() - 0.5f; }
    long dims[2] = {16, 16};
    KMWavefrontPlan *plan = km_wavefront_plan_create(dims, 2);
    printf("plan max_level %ld max_level_size %ld\n", plan->max_level, plan->max_level_size);
    km_wavefront_plan_free(plan);
    printf("available %d devices %d backend %d\n", kmamba_cuda_available(), kmamba_cuda_device_count(),
           (int)kmamba_backend_select());
    FILE *f = fopen(getenv("KM_C_CALLER_IN") ? getenv("KM_C_CALLER_IN") : "/dev/null", "wb");
    if (f) {
        fwrite(x, 4, L * D, f); fwrite(dt, 4, L * D, f); fwrite(A, 4, D * M, f);
        fwrite(B, 4, L * D * M, f); fwrite(C, 4, L * D * M, f); fwrite(h, 4, D * M, f);
        fclose(f);
    }
    MambaScan1DParams p = {x, A, B, C, dt, h, y, L, D, M};
    mamba_scan1d_forward(&p);
    printf("error '%s'\n", km_last_error());
    f = fopen(getenv("KM_C_CALLER_OUT") ? getenv("KM_C_CALLER_OUT") : "/dev/null", "wb");
    if (f) { fwrite(y, 4, L * D, f); fwrite(h, 4, D * M, f); fclose(f); }
    if (km_last_error()[0]) return 1;

    const char *ckpt = getenv("KM_C_CALLER_CKPT");
    if (!ckpt) return 0;
    KMambaConfig cfg;
    memset(&cfg, 0, sizeof(cfg));
    cfg.vocab_size = 50; cfg.dim = 16; cfg.state_size = 8; cfg.seq_len = 12; cfg.n_layers = 2;
    cfg.mimo_rank = 1; cfg.dt_scale = 0.1f; cfg.dt_min = 1e-3f; cfg.dt_max = 0.1f;
    KMamba *m = kmamba_create(&cfg);
    if (!m || kmamba_init(m, 2024) != 0) { printf("model create failed: %s\n", km_last_error()); return 2; }
    uint32_t tok[12];
    for (int t = 0; t < 12; t++) tok[t] = (uint32_t)((t * 7 + 3) % 53);   /* 50..52 are past the vocabulary */
    float *lg1 = malloc(sizeof(float) * 12 * 50), *lg2 = malloc(sizeof(float) * 12 * 50);
    if (kmamba_forward(m, tok, lg1) != 0 || kmamba_save(m, ckpt) != 0) {
        printf("model forward/save failed: %s\n", km_last_error());
        return 3;
    }
    KMamba *m2 = kmamba_load(ckpt, 0, NULL, 0.0f, 0.0f);
    if (!m2 || kmamba_forward(m2, tok, lg2) != 0) { printf("model load failed: %s\n", km_last_error()); return 4; }
    const int same = memcmp(lg1, lg2, sizeof(float) * 12 * 50) == 0;
    printf("model logits identical after reload: %d\n", same);
    f = fopen(getenv("KM_C_CALLER_MODEL") ? getenv("KM_C_CALLER_MODEL") : "/dev/null", "wb");
    if (f) { fwrite(tok, 4, 12, f); fwrite(lg1, 4, 12 * 50, f); fclose(f); }
    kmamba_free(m);
    kmamba_free(m2);
    free(lg1);
    free(lg2);
    return same ? 0 : 5;
}

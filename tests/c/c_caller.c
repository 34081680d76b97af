/* A plain C caller of libkmamba, built with gcc against include/ and
 * lib/libkmamba.so only (no torch, no Python): the way existing k-mamba C
 * code uses the drop-in. It runs the reference host-pointer API scan1d on a
 * small problem and prints y, the final state and the library's error
 * string, for tests/test_c_caller.py to compare with the oracle. */
#include <stdio.h>
#include <stdlib.h>

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
    return km_last_error()[0] ? 1 : 0;
}

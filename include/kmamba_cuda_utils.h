/* kmamba_cuda_utils.h - GPU detection and backend selection.
 *
 * Drop-in for the reference include/kmamba_cuda_utils.h:16-63. The names
 * keep the reference's "cuda" spelling because callers link against them;
 * in this library they query HIP devices.
 *
 * KMAMBA_BACKEND=auto|gpu|cuda selects the GPU. KMAMBA_BACKEND=cpu is
 * accepted for compatibility, but this library has no CPU compute path:
 * compute entry points then fail with -1 (or record an error for void
 * functions) instead of silently computing something else.
 */
#ifndef KMAMBA_CUDA_UTILS_H
#define KMAMBA_CUDA_UTILS_H

#ifdef __cplusplus
extern "C" {
#endif

/* 1 when a HIP device is present and usable (ref cuda/kmamba_cuda_utils.cu:14-45). */
int kmamba_cuda_available(void);
/* Number of HIP devices, 0 when none (ref :47-53). */
int kmamba_cuda_device_count(void);
/* Current HIP device, -1 when none (ref :55-61). */
int kmamba_cuda_current_device(void);

typedef enum {
    KMAMBA_BACKEND_AUTO = 0,
    KMAMBA_BACKEND_CPU = 1,
    KMAMBA_BACKEND_GPU = 2
} KMambaBackend;

/* Global preference, set from KMAMBA_BACKEND by kmamba_backend_init. */
extern KMambaBackend kmamba_backend_preference;

/* Parses KMAMBA_BACKEND (case-insensitive) into the preference
 * (ref src/kmamba_cuda_utils.c:37-57). Thread-safe. */
void kmamba_backend_init(void);

/* Effective backend: GPU when preferred/auto and a device is usable, else CPU
 * (ref :60-81). Device detection is cached after the first call. */
KMambaBackend kmamba_backend_select(void);

#define KMAMBA_IF_CUDA(expr) expr

/* Reference convenience macro (include/kmamba_cuda_utils.h:57-63).
 * kmamba_backend_init is idempotent here, so the once-flag is only an
 * optimisation. */
#define KMAMBA_AUTO_BACKEND() \
    static int _kmamba_backend_init_done = 0; \
    if (!_kmamba_backend_init_done) { \
        kmamba_backend_init(); \
        _kmamba_backend_init_done = 1; \
    } \
    KMambaBackend backend = kmamba_backend_select()

#ifdef __cplusplus
}
#endif

#endif /* KMAMBA_CUDA_UTILS_H */

/* km_shape.h - overflow-checked shape arithmetic shared by the host helpers
 * (wavefront enumeration, plans, topology). Internal header: nothing here is
 * part of the C ABI.
 *
 * Every predicate returns 1 when the operation is defined and representable
 * and 0 otherwise; results go through an out-pointer that is written only on
 * success. */
#ifndef KM_SHAPE_H
#define KM_SHAPE_H

#include <stddef.h>

/* A grid shape: 1 <= rank <= max_rank (no limit when max_rank <= 0) and
 * every extent >= 1. */
static inline int km_shape_valid(const long *dims, long rank, long max_rank) {
    if (!dims || rank <= 0 || (max_rank > 0 && rank > max_rank)) return 0;
    for (const long *d = dims; d != dims + rank; ++d)
        if (*d <= 0) return 0;
    return 1;
}

static inline int km_add_ok(long a, long b, long *out) {
    long r;
    if (__builtin_add_overflow(a, b, &r)) return 0;
    *out = r;
    return 1;
}

/* Products of non-negative extents only. */
static inline int km_mul_ok(long a, long b, long *out) {
    long r;
    if (a < 0 || b < 0 || __builtin_mul_overflow(a, b, &r)) return 0;
    *out = r;
    return 1;
}

static inline int km_umul_ok(size_t a, size_t b, size_t *out) {
    size_t r;
    if (__builtin_mul_overflow(a, b, &r)) return 0;
    *out = r;
    return 1;
}

#endif /* KM_SHAPE_H */

/* wavefront_nd.h - bounded, causal ND wavefront enumeration (host code).
 *
 * level(idx) = idx[0] + ... + idx[ndims-1]. Points of one level are
 * independent for any operator whose dependencies point to lower levels.
 * Within a level, points are visited in lexicographic index order, which is
 * ascending row-major offset order.
 *
 * Drop-in for the reference header include/wavefront_nd.h:21-60; results are
 * bit-identical to src/wavefront_nd.c.
 */
#ifndef KMAMBA_WAVEFRONT_ND_H
#define KMAMBA_WAVEFRONT_ND_H

#ifdef __cplusplus
extern "C" {
#endif

typedef int (*WavefrontNDVisitFn)(
    const long *idx,
    long ndims,
    long level,
    long ordinal_in_level,
    void *user
);

/* 1 when ndims > 0 and every dims[axis] > 0 (ref src/wavefront_nd.c:134-140). */
int wavefront_nd_validate_dims(const long *dims, long ndims);

/* Product of dims, or -1 on invalid input / overflow (ref :142-151). */
long wavefront_nd_total_points(const long *dims, long ndims);

/* Sum of (dims[axis]-1), or -1 on invalid input / overflow (ref :153-162). */
long wavefront_nd_max_level(const long *dims, long ndims);

/* Row-major offset of idx, or -1 when out of range / overflow (ref :164-176). */
long wavefront_nd_row_major_offset(const long *dims, const long *idx, long ndims);

/* Number of points on a level, or -1 when invalid (ref :178-198). */
long wavefront_nd_level_size(const long *dims, long ndims, long level);

/* Visits one level in lexicographic order. idx_scratch may be NULL,
 * otherwise it must hold ndims longs. Returns 0 when the level was fully
 * visited, the callback's nonzero code on early stop, -1 on invalid input
 * (ref :200-237). */
int wavefront_nd_for_level(const long *dims, long ndims, long level,
                           long *idx_scratch,
                           WavefrontNDVisitFn visit,
                           void *user);

/* Visits levels 0..max_level, same return convention (ref :239-279). */
int wavefront_nd_for_each_level(const long *dims, long ndims,
                                long *idx_scratch,
                                WavefrontNDVisitFn visit,
                                void *user);

#ifdef __cplusplus
}
#endif

#endif /* KMAMBA_WAVEFRONT_ND_H */

/* wavefront_nd.c - ND wavefront enumeration (host).
 *
 * Same results as the reference src/wavefront_nd.c:134-279, computed without
 * recursion or per-call heap allocation:
 *   - level sizes come from a bounded-composition count (dynamic programming
 *     over axes, O(ndims * level * max_dim));
 *   - a level is enumerated with an odometer over axes 0..ndims-2 whose
 *     per-axis range is clipped by the remaining level and the capacity of
 *     the trailing axes, so the visit order is lexicographic exactly like the
 *     reference's recursive emitter (:84-109).
 */
#include "wavefront_nd.h"

#include <limits.h>
#include <stdlib.h>

#include "km_shape.h"


int wavefront_nd_validate_dims(const long *dims, long ndims) {
    return km_shape_valid(dims, ndims, 0);
}

long wavefront_nd_total_points(const long *dims, long ndims) {
    long total = 1;
    if (!wavefront_nd_validate_dims(dims, ndims)) return -1;
    for (long a = 0; a < ndims; a++)
        if (!km_mul_ok(total, dims[a], &total)) return -1;
    return total;
}

long wavefront_nd_max_level(const long *dims, long ndims) {
    long lvl = 0;
    if (!wavefront_nd_validate_dims(dims, ndims)) return -1;
    for (long a = 0; a < ndims; a++)
        if (!km_add_ok(lvl, dims[a] - 1, &lvl)) return -1;
    return lvl;
}

long wavefront_nd_row_major_offset(const long *dims, const long *idx, long ndims) {
    long off = 0;
    if (!wavefront_nd_validate_dims(dims, ndims) || !idx) return -1;
    for (long a = 0; a < ndims; a++) {
        if (idx[a] < 0 || idx[a] >= dims[a]) return -1;
        if (!km_mul_ok(off, dims[a], &off)) return -1;
        if (!km_add_ok(off, idx[a], &off)) return -1;
    }
    return off;
}

/* Number of idx with 0 <= idx[a] < dims[a] and sum(idx) == level.
 * cnt[s] holds the count for the axes folded so far; each new axis is a
 * sliding-window sum of width dims[a]. */
long wavefront_nd_level_size(const long *dims, long ndims, long level) {
    long maxl = wavefront_nd_max_level(dims, ndims);
    if (maxl < 0 || level < 0 || level > maxl) return -1;
    long *cnt = (long *)calloc((size_t)(level + 1), sizeof(long));
    long *nxt = (long *)calloc((size_t)(level + 1), sizeof(long));
    if (!cnt || !nxt) { free(cnt); free(nxt); return -1; }
    cnt[0] = 1;
    long reach = 0;   /* largest reachable sum so far, capped at level */
    for (long a = 0; a < ndims; a++) {
        long nreach = reach + dims[a] - 1;
        if (nreach > level) nreach = level;
        long window = 0;
        for (long s = 0; s <= nreach; s++) {
            if (s <= reach && !km_add_ok(window, cnt[s], &window)) { free(cnt); free(nxt); return -1; }
            long drop = s - dims[a];
            if (drop >= 0 && drop <= reach) window -= cnt[drop];
            nxt[s] = window;
        }
        for (long s = 0; s <= nreach; s++) cnt[s] = nxt[s];
        reach = nreach;
    }
    long r = (level <= reach) ? cnt[level] : 0;
    free(cnt); free(nxt);
    return r;
}

/* Visits one level. cap[a] = sum_{b > a} (dims[b]-1) bounds what the axes
 * after a can absorb, so axis a ranges over
 * [max(0, rem - cap[a]), min(dims[a]-1, rem)] (same clipping as the
 * reference's emitter) and the last axis takes the remainder. */
static int visit_level(const long *dims, long ndims, long level, long *idx,
                       const long *cap, WavefrontNDVisitFn visit, void *user) {
    long rem[ndims + 1];
    long hi[ndims];
    long ordinal = 0;
    long last = ndims - 1;

    if (ndims == 1) {
        if (level >= dims[0]) return 0;
        idx[0] = level;
        return visit(idx, ndims, level, 0, user);
    }
    /* Start every axis at its lowest admissible value. */
    rem[0] = level;
    for (long a = 0; a < last; a++) {
        long lo = rem[a] - cap[a];
        if (lo < 0) lo = 0;
        hi[a] = (dims[a] - 1 < rem[a]) ? dims[a] - 1 : rem[a];
        if (lo > hi[a]) return 0;   /* level empty (cannot happen for valid levels) */
        idx[a] = lo;
        rem[a + 1] = rem[a] - lo;
    }
    for (;;) {
        idx[last] = rem[last];
        int rc = visit(idx, ndims, level, ordinal++, user);
        if (rc != 0) return rc;
        /* Advance the odometer: bump the deepest axis that still has room. */
        long a = last - 1;
        while (a >= 0 && idx[a] >= hi[a]) a--;
        if (a < 0) return 0;
        idx[a]++;
        rem[a + 1] = rem[a] - idx[a];
        for (long b = a + 1; b < last; b++) {
            long lo = rem[b] - cap[b];
            if (lo < 0) lo = 0;
            hi[b] = (dims[b] - 1 < rem[b]) ? dims[b] - 1 : rem[b];
            idx[b] = lo;
            rem[b + 1] = rem[b] - lo;
        }
    }
}

static int build_caps(const long *dims, long ndims, long *cap) {
    long s = 0;
    for (long a = ndims - 1; a >= 0; a--) {
        cap[a] = s;
        if (!km_add_ok(s, dims[a] - 1, &s)) return 0;
    }
    return 1;
}

int wavefront_nd_for_level(const long *dims, long ndims, long level,
                           long *idx_scratch, WavefrontNDVisitFn visit, void *user) {
    if (!wavefront_nd_validate_dims(dims, ndims) || !visit) return -1;
    long local_idx[ndims];
    long cap[ndims];
    long maxl = wavefront_nd_max_level(dims, ndims);
    if (maxl < 0 || level < 0 || level > maxl) return -1;
    if (!build_caps(dims, ndims, cap)) return -1;
    return visit_level(dims, ndims, level, idx_scratch ? idx_scratch : local_idx, cap, visit, user);
}

int wavefront_nd_for_each_level(const long *dims, long ndims,
                                long *idx_scratch, WavefrontNDVisitFn visit, void *user) {
    if (!wavefront_nd_validate_dims(dims, ndims) || !visit) return -1;
    long local_idx[ndims];
    long cap[ndims];
    long maxl = wavefront_nd_max_level(dims, ndims);
    if (maxl < 0) return -1;
    if (!build_caps(dims, ndims, cap)) return -1;
    long *idx = idx_scratch ? idx_scratch : local_idx;
    for (long level = 0; level <= maxl; level++) {
        int rc = visit_level(dims, ndims, level, idx, cap, visit, user);
        if (rc != 0) return rc;
    }
    return 0;
}

/* wavefront_plan.c - reusable wavefront plan (host).
 *
 * Produces the same tables as the reference km_wavefront_plan_create
 * (src/wavefront_plan.c:35-101) in O(P + ndims * max_level):
 *   1. the level-size distribution of the whole grid comes from one
 *      bounded-composition count (sliding window over each axis);
 *   2. level_starts is its exclusive prefix sum, with
 *      level_starts[max_level + 1] = P;
 *   3. one odometer pass over the grid in row-major order appends every
 *      offset to its level's bucket, so offsets inside a level are ascending,
 *      which is the reference's lexicographic emission order.
 */
#include "wavefront_plan.h"

#include <stdlib.h>
#include <string.h>

KMWavefrontPlan *km_wavefront_plan_create(const long *dims, long ndims) {
    long P = wavefront_nd_total_points(dims, ndims);
    long maxl = wavefront_nd_max_level(dims, ndims);
    if (P <= 0 || maxl < 0) return NULL;

    KMWavefrontPlan *plan = (KMWavefrontPlan *)calloc(1, sizeof(*plan));
    if (!plan) return NULL;
    plan->dims = (long *)malloc((size_t)ndims * sizeof(long));
    plan->level_starts = (long *)calloc((size_t)(maxl + 2), sizeof(long));
    plan->level_offsets = (long *)malloc((size_t)P * sizeof(long));
    long *cnt = (long *)calloc((size_t)(maxl + 1), sizeof(long));
    long *nxt = (long *)calloc((size_t)(maxl + 1), sizeof(long));
    long *idx = (long *)calloc((size_t)ndims, sizeof(long));
    if (!plan->dims || !plan->level_starts || !plan->level_offsets || !cnt || !nxt || !idx) {
        free(cnt); free(nxt); free(idx);
        km_wavefront_plan_free(plan);
        return NULL;
    }
    memcpy(plan->dims, dims, (size_t)ndims * sizeof(long));
    plan->ndims = ndims;
    plan->total_points = P;
    plan->max_level = maxl;

    /* 1. level sizes: fold axes into the distribution of coordinate sums. */
    cnt[0] = 1;
    long reach = 0;
    for (long a = 0; a < ndims; a++) {
        long nreach = reach + dims[a] - 1;
        long window = 0;
        for (long s = 0; s <= nreach; s++) {
            if (s <= reach) window += cnt[s];
            long drop = s - dims[a];
            if (drop >= 0 && drop <= reach) window -= cnt[drop];
            nxt[s] = window;
        }
        memcpy(cnt, nxt, (size_t)(nreach + 1) * sizeof(long));
        reach = nreach;
    }

    /* 2. level starts. */
    long cursor = 0;
    for (long l = 0; l <= maxl; l++) {
        plan->level_starts[l] = cursor;
        if (cnt[l] > plan->max_level_size) plan->max_level_size = cnt[l];
        cursor += cnt[l];
    }
    plan->level_starts[maxl + 1] = cursor;
    if (cursor != P) {
        free(cnt); free(nxt); free(idx);
        km_wavefront_plan_free(plan);
        return NULL;
    }

    /* 3. bucket fill in row-major order (cnt reused as per-level cursor). */
    memcpy(cnt, plan->level_starts, (size_t)(maxl + 1) * sizeof(long));
    long level = 0;
    for (long off = 0; off < P; off++) {
        plan->level_offsets[cnt[level]++] = off;
        for (long a = ndims - 1; a >= 0; a--) {
            if (++idx[a] < dims[a]) { level++; break; }
            level -= dims[a] - 1;
            idx[a] = 0;
        }
    }
    free(cnt); free(nxt); free(idx);
    return plan;
}

void km_wavefront_plan_free(KMWavefrontPlan *plan) {
    if (!plan) return;
    free(plan->dims);
    free(plan->level_starts);
    free(plan->level_offsets);
    free(plan);
}

int km_wavefront_plan_matches_dims(const KMWavefrontPlan *plan, const long *dims, long ndims) {
    if (!plan || !dims || ndims <= 0) return 0;
    if (plan->ndims != ndims) return 0;
    for (long a = 0; a < ndims; a++)
        if (plan->dims[a] != dims[a]) return 0;
    return 1;
}

long km_wavefront_plan_level_size(const KMWavefrontPlan *plan, long level) {
    if (!plan || level < 0 || level > plan->max_level) return -1;
    return plan->level_starts[level + 1] - plan->level_starts[level];
}

const long *km_wavefront_plan_level_offsets(const KMWavefrontPlan *plan, long level) {
    if (!plan || level < 0 || level > plan->max_level) return NULL;
    return plan->level_offsets + plan->level_starts[level];
}

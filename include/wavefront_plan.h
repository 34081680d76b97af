/* wavefront_plan.h - reusable wavefront plan for ND operators (host code).
 *
 * A plan holds only grid topology: dims, the level boundaries and the
 * row-major offsets grouped by level (ascending within a level). It is shared
 * by scanND and convND. Drop-in for the reference header
 * include/wavefront_plan.h:27-52; the tables are bit-identical to
 * km_wavefront_plan_create in src/wavefront_plan.c:35-101.
 */
#ifndef KMAMBA_WAVEFRONT_PLAN_H
#define KMAMBA_WAVEFRONT_PLAN_H

#include "wavefront_nd.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    long *dims;           /* [ndims] */
    long ndims;
    long total_points;
    long max_level;
    long max_level_size;
    long *level_starts;   /* [max_level + 2]; level_starts[max_level+1] = total_points */
    long *level_offsets;  /* [total_points] row-major offsets grouped by level */
} KMWavefrontPlan;

/* Builds a plan, or NULL on invalid dims / allocation failure.
 * The caller owns the plan and frees it with km_wavefront_plan_free.
 * Replaces src/wavefront_plan.c:35-101. */
KMWavefrontPlan *km_wavefront_plan_create(const long *dims, long ndims);

/* Frees a plan and its tables; NULL is accepted (ref :103-109). */
void km_wavefront_plan_free(KMWavefrontPlan *plan);

/* 1 when the plan was built for exactly dims/ndims (ref :111-122). */
int km_wavefront_plan_matches_dims(const KMWavefrontPlan *plan,
                                   const long *dims,
                                   long ndims);

/* Size of a level, or -1 when invalid (ref :124-127). */
long km_wavefront_plan_level_size(const KMWavefrontPlan *plan, long level);

/* Offsets of a level, or NULL when invalid (ref :129-132). */
const long *km_wavefront_plan_level_offsets(const KMWavefrontPlan *plan, long level);

#ifdef __cplusplus
}
#endif

#endif /* KMAMBA_WAVEFRONT_PLAN_H */

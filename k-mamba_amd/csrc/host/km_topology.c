/* km_topology.c - ND shape helpers of the block topology (host code).
 *
 * Observable behaviour follows the reference src/km_topology.c:8-110, edge
 * cases included: ranks are limited to KMAMBA_MAX_NDIMS, km_power_long(0, 0)
 * is 0, unravel leaves its output untouched on invalid input, and a rank <= 0
 * topology is the implicit 1D shape [seq_len].
 *
 * Design: every shape query goes through one descriptor, built in a single
 * pass from the last axis to the first (validity, checked point count and
 * row-major strides together), on the overflow-checked arithmetic of
 * km_shape.h that the wavefront enumeration and the plans also use. Strides,
 * like the reference's products in `long`, wrap modulo 2^64; they are formed
 * unsigned here, so without undefined behaviour. */
#include "km_topology.h"

#include <limits.h>

#include "km_shape.h"

typedef struct {
    int valid;              /* rank in [1, KMAMBA_MAX_NDIMS], every extent >= 1 */
    int count_fits;         /* the point count fits in size_t */
    size_t count;           /* number of points when count_fits */
    unsigned long stride[KMAMBA_MAX_NDIMS];   /* row-major, wrapping */
} topo_desc;

static topo_desc topo_describe(const long *dims, long ndims) {
    topo_desc t = {0};
    if (!km_shape_valid(dims, ndims, KMAMBA_MAX_NDIMS)) return t;
    t.valid = 1;
    t.count_fits = 1;
    t.count = 1;
    unsigned long wrap = 1;
    for (long a = ndims - 1; a >= 0; --a) {
        t.stride[a] = wrap;
        wrap *= (unsigned long)dims[a];
        if (t.count_fits && !km_umul_ok(t.count, (size_t)dims[a], &t.count)) t.count_fits = 0;
    }
    return t;
}

int km_spatial_dims_product(const long *dims, long ndims, size_t *product_out) {
    const topo_desc t = topo_describe(dims, ndims);
    if (!product_out || !t.valid || !t.count_fits) return 0;
    *product_out = t.count;
    return 1;
}

int km_make_row_major_strides(const long *dims, long ndims, long *strides_out) {
    const topo_desc t = topo_describe(dims, ndims);
    if (!strides_out || !t.valid) return 0;
    for (long a = 0; a < ndims; ++a) strides_out[a] = (long)t.stride[a];
    return 1;
}

/* Rank check shared by the index conversions, which take caller strides. */
static int rank_ok(long ndims) { return ndims > 0 && ndims <= KMAMBA_MAX_NDIMS; }

void km_unravel_index(long linear, const long *dims, const long *strides, long ndims,
                      long *coords_out) {
    if (linear < 0 || !dims || !strides || !coords_out || !rank_ok(ndims)) return;
    /* Any stride set is accepted, as in the reference; a zero stride or
     * extent (a division by zero there) is rejected here before anything is
     * written. */
    long c[KMAMBA_MAX_NDIMS];
    for (long a = 0; a < ndims; ++a) {
        if (strides[a] == 0 || dims[a] == 0) return;
        c[a] = (linear / strides[a]) % dims[a];
    }
    for (long a = 0; a < ndims; ++a) coords_out[a] = c[a];
}

long km_ravel_index(const long *coords, const long *dims, const long *strides, long ndims) {
    if (!coords || !dims || !strides || !rank_ok(ndims)) return -1;
    unsigned long off = 0;   /* wraps like the reference's long sum */
    for (long a = 0; a < ndims; ++a) {
        if (coords[a] < 0 || coords[a] >= dims[a]) return -1;
        off += (unsigned long)coords[a] * (unsigned long)strides[a];
    }
    return (long)off;
}

long km_power_long(long base, long exp) {
    if (exp < 0 || (exp == 0 && base == 0)) return 0;
    /* Square-and-multiply modulo 2^64: the same bits as repeated
     * multiplication, in O(log exp) steps. */
    unsigned long acc = 1, sq = (unsigned long)base;
    for (unsigned long e = (unsigned long)exp; e; e >>= 1) {
        if (e & 1) acc *= sq;
        sq *= sq;
    }
    return (long)acc;
}

int km_normalize_spatial_topology(long *spatial_ndims, long *spatial_dims, size_t seq_len,
                                  int use_convnd, long *convnd_ndims, long convnd_K) {
    if (!spatial_ndims || !spatial_dims || seq_len > (size_t)LONG_MAX) return -1;
    const int implicit = *spatial_ndims <= 0;
    if (implicit) {
        /* The implicit 1D topology [seq_len], with the unused axes cleared. */
        spatial_dims[0] = (long)seq_len;
        for (long a = 1; a < KMAMBA_MAX_NDIMS; ++a) spatial_dims[a] = 0;
        *spatial_ndims = 1;
    }
    const topo_desc t = topo_describe(spatial_dims, *spatial_ndims);
    if (!t.valid || !t.count_fits || t.count != seq_len) return -1;
    if (!use_convnd) return 0;
    /* The ConvND rank defaults to, and must equal, the spatial rank. */
    if (!convnd_ndims || convnd_K <= 0) return -1;
    if (*convnd_ndims <= 0) *convnd_ndims = *spatial_ndims;
    return *convnd_ndims == *spatial_ndims ? 0 : -1;
}

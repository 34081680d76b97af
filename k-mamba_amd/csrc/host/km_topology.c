/* km_topology.c - ND shape helpers of the block topology (host code).
 *
 * Behaviour of the reference src/km_topology.c:8-110, edge cases included:
 * ranks are limited to KMAMBA_MAX_NDIMS, km_power_long(0, 0) is 0, unravel
 * leaves its output untouched on invalid input, and a rank <= 0 topology is
 * the implicit 1D shape [seq_len]. The arithmetic is the overflow-checked
 * shape arithmetic of km_shape.h; strides, like the reference's products in
 * `long`, wrap modulo 2^64 (computed unsigned here, so without undefined
 * behaviour). */
#include "km_topology.h"

#include <limits.h>

#include "km_shape.h"

/* The rank and extents every helper below accepts. */
static int topo_shape_ok(const long *dims, long ndims) {
    return km_shape_valid(dims, ndims, KMAMBA_MAX_NDIMS);
}

int km_spatial_dims_product(const long *dims, long ndims, size_t *product_out) {
    if (!product_out || !topo_shape_ok(dims, ndims)) return 0;
    size_t total = 1;
    for (long a = 0; a < ndims; ++a)
        if (!km_umul_ok(total, (size_t)dims[a], &total)) return 0;
    *product_out = total;
    return 1;
}

int km_make_row_major_strides(const long *dims, long ndims, long *strides_out) {
    if (!strides_out || !topo_shape_ok(dims, ndims)) return 0;
    /* Suffix products: the last axis is contiguous. */
    unsigned long run = 1;
    for (long a = ndims; a-- > 0;) {
        strides_out[a] = (long)run;
        run *= (unsigned long)dims[a];
    }
    return 1;
}

void km_unravel_index(long linear, const long *dims, const long *strides, long ndims,
                      long *coords_out) {
    if (linear < 0 || !dims || !strides || !coords_out || ndims <= 0 || ndims > KMAMBA_MAX_NDIMS)
        return;
    /* Any stride set is accepted, as in the reference; a zero stride or
     * extent (a division by zero there) is invalid input here. */
    for (long a = 0; a < ndims; ++a)
        if (strides[a] == 0 || dims[a] == 0) return;
    for (long a = 0; a < ndims; ++a) {
        const long along = linear / strides[a];
        coords_out[a] = along % dims[a];
    }
}

long km_ravel_index(const long *coords, const long *dims, const long *strides, long ndims) {
    if (!coords || !dims || !strides || ndims <= 0 || ndims > KMAMBA_MAX_NDIMS) return -1;
    unsigned long off = 0;   /* wraps like the reference's long sum */
    for (long a = 0; a < ndims; ++a) {
        const long c = coords[a];
        if (c < 0 || c >= dims[a]) return -1;
        off += (unsigned long)c * (unsigned long)strides[a];
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
    if (*spatial_ndims <= 0) {
        /* Implicit 1D topology [seq_len]; unused axes cleared. */
        for (long a = 0; a < KMAMBA_MAX_NDIMS; ++a) spatial_dims[a] = a ? 0 : (long)seq_len;
        *spatial_ndims = 1;
    }
    size_t points = 0;
    if (!km_spatial_dims_product(spatial_dims, *spatial_ndims, &points) || points != seq_len)
        return -1;
    if (!use_convnd) return 0;
    /* The ConvND rank defaults to, and must equal, the spatial rank. */
    if (!convnd_ndims || convnd_K <= 0) return -1;
    if (*convnd_ndims <= 0) *convnd_ndims = *spatial_ndims;
    return (*convnd_ndims == *spatial_ndims) ? 0 : -1;
}

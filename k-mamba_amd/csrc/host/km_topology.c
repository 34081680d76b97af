/* km_topology.c - ND shape helpers (host). Semantics of the reference
 * src/km_topology.c:8-110, including its edge cases (km_power_long(0, 0) is
 * 0, unravel is a no-op on invalid input). */
#include "km_topology.h"

#include <limits.h>
#include <string.h>

#include "wavefront_nd.h"

int km_spatial_dims_product(const long *dims, long ndims, size_t *product_out) {
    if (!dims || !product_out || ndims <= 0 || ndims > KMAMBA_MAX_NDIMS) return 0;
    if (!wavefront_nd_validate_dims(dims, ndims)) return 0;
    size_t prod = 1;
    for (long a = 0; a < ndims; a++) {
        size_t e = (size_t)dims[a];
        if (prod > ((size_t)-1) / e) return 0;
        prod *= e;
    }
    *product_out = prod;
    return 1;
}

int km_make_row_major_strides(const long *dims, long ndims, long *strides_out) {
    if (!dims || !strides_out || ndims <= 0 || ndims > KMAMBA_MAX_NDIMS) return 0;
    if (!wavefront_nd_validate_dims(dims, ndims)) return 0;
    long s = 1;
    for (long a = ndims - 1; a >= 0; a--) {
        strides_out[a] = s;
        s *= dims[a];
    }
    return 1;
}

void km_unravel_index(long linear, const long *dims, const long *strides,
                      long ndims, long *coords_out) {
    if (!dims || !strides || !coords_out || ndims <= 0 || ndims > KMAMBA_MAX_NDIMS) return;
    if (linear < 0) return;
    for (long a = 0; a < ndims; a++)
        coords_out[a] = (linear / strides[a]) % dims[a];
}

long km_ravel_index(const long *coords, const long *dims, const long *strides, long ndims) {
    if (!coords || !dims || !strides || ndims <= 0 || ndims > KMAMBA_MAX_NDIMS) return -1;
    long off = 0;
    for (long a = 0; a < ndims; a++) {
        if (coords[a] < 0 || coords[a] >= dims[a]) return -1;
        off += coords[a] * strides[a];
    }
    return off;
}

long km_power_long(long base, long exp) {
    if (exp < 0) return 0;
    if (base == 0 && exp == 0) return 0;
    /* Integer power by squaring in unsigned arithmetic: identical to the
     * reference's repeated multiplication modulo 2^64, without signed
     * overflow. */
    unsigned long r = 1, b = (unsigned long)base;
    while (exp > 0) {
        if (exp & 1) r *= b;
        exp >>= 1;
        if (exp) b *= b;
    }
    return (long)r;
}

int km_normalize_spatial_topology(long *spatial_ndims, long *spatial_dims, size_t seq_len,
                                  int use_convnd, long *convnd_ndims, long convnd_K) {
    size_t total;
    if (!spatial_ndims || !spatial_dims) return -1;
    if (seq_len > (size_t)LONG_MAX) return -1;
    if (*spatial_ndims <= 0) {
        memset(spatial_dims, 0, (size_t)KMAMBA_MAX_NDIMS * sizeof(long));
        *spatial_ndims = 1;
        spatial_dims[0] = (long)seq_len;
    }
    if (!km_spatial_dims_product(spatial_dims, *spatial_ndims, &total)) return -1;
    if (total != seq_len) return -1;
    if (use_convnd) {
        if (!convnd_ndims || convnd_K <= 0) return -1;
        if (*convnd_ndims <= 0) *convnd_ndims = *spatial_ndims;
        if (*convnd_ndims != *spatial_ndims) return -1;
    }
    return 0;
}

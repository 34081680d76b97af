/* km_topology.h - ND shape helpers (host code).
 * Drop-in for the reference header include/km_topology.h:10-46, same
 * semantics as src/km_topology.c:8-110. */
#ifndef KMAMBA_TOPOLOGY_H
#define KMAMBA_TOPOLOGY_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KMAMBA_MAX_NDIMS 8

/* Product of dims into *product_out; 0 on invalid input or size_t overflow,
 * 1 on success (ref src/km_topology.c:8-22). */
int km_spatial_dims_product(const long *dims, long ndims, size_t *product_out);

/* strides[axis] = prod(dims[axis+1..]); 1 on success, 0 on invalid input
 * (ref :24-37). */
int km_make_row_major_strides(const long *dims, long ndims, long *strides_out);

/* coords[axis] = (linear / strides[axis]) % dims[axis]; no-op on invalid
 * input or negative linear (ref :39-50). */
void km_unravel_index(long linear,
                      const long *dims,
                      const long *strides,
                      long ndims,
                      long *coords_out);

/* sum coords[axis]*strides[axis], or -1 when a coordinate is out of range
 * (ref :52-67). */
long km_ravel_index(const long *coords,
                    const long *dims,
                    const long *strides,
                    long ndims);

/* base^exp for exp >= 0; 0 when exp < 0 or when base == 0 && exp == 0
 * (ref :69-81). */
long km_power_long(long base, long exp);

/* Normalises a block's spatial topology: ndims <= 0 means the implicit 1D
 * shape [seq_len]; the product must equal seq_len; with use_convnd the conv
 * rank defaults to, and must equal, the spatial rank. 0 on success, -1 on
 * error (ref :83-110). */
int km_normalize_spatial_topology(long *spatial_ndims,
                                  long *spatial_dims,
                                  size_t seq_len,
                                  int use_convnd,
                                  long *convnd_ndims,
                                  long convnd_K);

#ifdef __cplusplus
}
#endif

#endif /* KMAMBA_TOPOLOGY_H */

/* mamba_scan_2d.h - public k-mamba alias of the 2D scan.
 * Drop-in for the reference include/mamba_scan_2d.h:8-10. */
#ifndef MAMBA_SCAN_2D_H
#define MAMBA_SCAN_2D_H

#include "scan.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef Scan2DParams MambaScan2DParams;

void mamba_scan2d_forward(MambaScan2DParams *p);

#ifdef __cplusplus
}
#endif

#endif

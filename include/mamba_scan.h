/* mamba_scan.h - public k-mamba aliases of the 1D scan API.
 * Drop-in for the reference include/mamba_scan.h:9-16 (aliases defined in
 * cpu/mamba_scan.c:8-22). */
#ifndef MAMBA_SCAN_H
#define MAMBA_SCAN_H

#include "scan.h"
#include "mamba_scan_2d.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef ScanParams               MambaScan1DParams;
typedef ScanBackwardParams       MambaScan1DBackwardParams;
typedef ScanBackwardSharedParams MambaScan1DBackwardM1Params;

void mamba_scan1d_forward(MambaScan1DParams *p);
void mamba_scan1d_backward(MambaScan1DBackwardParams *p);
void mamba_scan1d_backward_m1_shared_bc(MambaScan1DBackwardM1Params *p);

#ifdef __cplusplus
}
#endif

#endif

/*
 * mdnav_calib.h — measurement helper exported by libmdnav.so.  No counterpart
 * in the reference: a plain device-to-device copy kernel of known size whose
 * FETCH_SIZE / WRITE_SIZE counter readings calibrate the HBM-traffic figures
 * reported for the hot-path kernels.
 */
#ifndef MDNAV_CALIB_H
#define MDNAV_CALIB_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Copies `bytes` (multiple of 16) between two fresh device buffers `repeats`
 * times with a streaming kernel; returns the mean kernel time in *ms. */
int mdn_calib_copy(uint64_t bytes, uint32_t repeats, double* ms);

#ifdef __cplusplus
}
#endif

#endif /* MDNAV_CALIB_H */

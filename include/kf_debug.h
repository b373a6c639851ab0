/*
 * kf_debug.h — entry points of the instrumented build libkfhip_timeline.so
 * (kernelforge.jl_amd/build.py compiles the scan and reduction sources with
 * -DKF_TIMELINE into it). None of them is exported by the production
 * libkfhip.so. They exist for tests and profiling only; none has a
 * counterpart in the reference.
 */
#ifndef KF_DEBUG_H
#define KF_DEBUG_H

#include "kf.h"

#ifdef __cplusplus
extern "C" {
#endif

/* On the calling host thread, later kf_scan calls leave tile `tile`
 * unpublished and give up after `spin_limit` lookback polls, so that the
 * give-up path runs with every kernel exiting normally; tile < 0 restores
 * normal operation. */
int kf_debug_scan_giveup(int64_t tile, uint32_t spin_limit);

/* The same for the reduction fold: workgroup `workgroup` of a folding
 * launch does not publish its partial and the waiting workgroup gives up
 * after `spin_limit` polls; workgroup < 0 restores normal operation. */
int kf_debug_reduce_giveup(int workgroup, uint32_t spin_limit);

/* Per-tile records of the scan into `buf`, 6 64-bit words per tile: four
 * 100 MHz realtime stamps (start, tile scanned, prefix known, stores
 * issued), the XCD id and the HW_ID word; null stops recording. */
int kf_debug_scan_timeline(void* buf);

/* Per-workgroup records of the folding one-launch reductions into `buf`,
 * 6 64-bit words per workgroup: three 100 MHz realtime stamps (start,
 * loads folded into the partial, slot published or fold done), the XCD id,
 * the HW_ID word and the grid size; null stops recording. */
int kf_debug_reduce_timeline(void* buf);

#ifdef __cplusplus
}
#endif
#endif

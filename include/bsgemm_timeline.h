/*
 * bsgemm_timeline.h — profiling hook of the phase-timeline build of libbsgemm
 * (libbsgemm_timeline.so, compiled from the same sources with -DBSG_TIMELINE).  No counterpart in
 * the reference and not part of the shipped library: it exists to measure where a GEMM launch
 * spends its time.
 *
 * After bsg_timeline_attach(buf, slots, slot_groups), GEMM launches enqueued by this process write,
 * per work-group g, 8 uint64 at buf[(launch % slots) * slot_groups * 8 + g * 8 + i]:
 *   i = 0 entry, 1 block list staged, 2 first block's weights consumed, 3 main loop done,
 *       4 outputs or partials issued, 5 end (own stores acknowledged)   -- 100 MHz wall clock
 *   i = 6 bit 0: 1 when the work-group stored Y (under split-K: the last arriver of its tile);
 *         bits 1..63: the latest main-loop end (same clock) over the work-group's waves
 *   i = 7 (XCC id << 32) | HW_ID register
 * Launches with more than slot_groups work-groups record nothing.  buf = NULL detaches.
 * The shipped libbsgemm.so exports the same symbol and returns BSG_ERR_UNSUPPORTED for any
 * non-NULL buf (its kernels carry no stamps).
 */
#ifndef BSGEMM_TIMELINE_H
#define BSGEMM_TIMELINE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int bsg_timeline_attach(void* buf, int64_t slots, int64_t slot_groups);

/* Frequency of the stamps' wall clock on the current device, in kHz (-1 on a HIP error).  Both
 * builds implement it. */
int64_t bsg_timeline_clock_khz(void);

#ifdef __cplusplus
}
#endif

#endif /* BSGEMM_TIMELINE_H */

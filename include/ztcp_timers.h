/*
 * ztcp_timers.h -- phase timers of the fused kernels (diagnostic build only).
 *
 * No counterpart in the reference.  Declared by libztcp_hip_timers.so, the
 * build of the same sources with -DZTCP_PHASE_TIMERS; the product library
 * libztcp_hip.so does not export it.  In that build every fused egress and
 * ingress launch (up to ZTCP_TIMER_MAX_WORKGROUPS workgroups) writes one
 * record of ZTCP_TIMER_SLOTS 64-bit words per workgroup: shader-clock counts
 * (s_memtime) of the phases of the workgroup's wave roles, relative to the
 * clock at which they left the workgroup's first barrier, and the absolute
 * shader and 100 MHz reference clocks at its first and last barrier.  The
 * slot meanings are the TimerSlot enumerators of
 * vlx-tee_amd/csrc/ztcp_rows.h.
 */
#ifndef ZTCP_TIMERS_H
#define ZTCP_TIMERS_H

#include <stdint.h>

/* Every entry point is exported from the library, which is built with hidden
 * default visibility: the library exports exactly what its headers declare. */
#ifndef ZTCP_API
#if defined(__GNUC__) || defined(__clang__)
#define ZTCP_API __attribute__((visibility("default")))
#else
#define ZTCP_API
#endif
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define ZTCP_TIMER_SLOTS 48
#define ZTCP_TIMER_MAX_WORKGROUPS 4096
#define ZTCP_TRACE_ROWS 1024

/* Copies the records of the last fused launch of `direction` (0 = egress,
 * 1 = ingress) on the current device into `out` (HOST, max_words words),
 * after synchronizing the device.  Returns the number of words written
 * (workgroups * ZTCP_TIMER_SLOTS), 0 when no fused launch was recorded, or a
 * negative ZTCP_E* code. */
ZTCP_API int64_t ztcp_phase_timers_read(int32_t direction, uint64_t* out, int64_t max_words);

/* Workgroup 0's row trace of the same launch: 4 * ZTCP_TRACE_ROWS 32-bit
 * words.  Clocks since its first barrier: out[r] when payload row r reached
 * the ring, out[ZTCP_TRACE_ROWS + r] when the MAC / verify wave absorbed it;
 * for a group of four rows starting at r whose ready flags that wave found
 * incomplete, the clocks it then waited for the group's rows
 * (out[2 * ZTCP_TRACE_ROWS + r], zero for every other row);
 * out[3 * ZTCP_TRACE_ROWS + r] is zero.  Rows past the payload keep whatever
 * an earlier launch left in the first two words.  Returns 4 * ZTCP_TRACE_ROWS,
 * 0 when no fused launch was recorded, or a negative ZTCP_E* code. */
ZTCP_API int64_t ztcp_phase_trace_read(int32_t direction, uint32_t* out, int64_t max_words);

#ifdef __cplusplus
}
#endif
#endif /* ZTCP_TIMERS_H */

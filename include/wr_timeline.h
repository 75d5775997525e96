/*
 * wr_timeline.h -- measurement hook of libwarp_route_hip.so: per-workgroup
 * timestamps of the single-token fused kernel (k_fused_ffn), from which
 * bench.py --timeline builds the phase timelines it reports.  Not part of the
 * drop-in boundary (include/warp_route.h) and without counterpart in the
 * reference.  The kernel records them only in a library built with
 * WR_HIPCC_FLAGS=-DWR_TIMELINE=1 (warp-route_amd/build.py); a default build
 * exports the function, records nothing and returns -1 from it.
 */
#ifndef WR_TIMELINE_H
#define WR_TIMELINE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define WR_TL_API __attribute__((visibility("default")))
#else
#define WR_TL_API
#endif

/* Records per workgroup and the largest grid recorded (larger grids record
 * their first WR_TIMELINE_MAX_BLOCKS workgroups). */
#define WR_TIMELINE_EVENTS 8
#define WR_TIMELINE_MAX_BLOCKS 16384

/* Record i of workgroup b is rec[b * WR_TIMELINE_EVENTS + i].  Times are the
 * GPU's constant-rate wall clock (hipDeviceAttributeWallClockRate, kHz):
 *   0  workgroup start
 *   1  expert selection done
 *   2  down: first weight tile's loads issued; gate/up with x staged in LDS:
 *      the x copy and the first round of weight loads landed (else 0)
 *   3  gate/up: last arrival counted, the workgroup's end; down: hand-off
 *      release seen by the workgroup
 *   4  down: workgroup end (gate/up: 0)
 * and
 *   5  hardware ids: XCD id in bits 0-3, the HW_ID register in bits 32-63
 *   6  role: 0 gate/up, 1 down
 *   7  gate/up: the last chunk's rows computed, before their stores (down: 0)
 */

/* Copies the records of the last k_fused_ffn launch on the current device
 * into host memory (rec, room for max_blocks workgroups), after
 * synchronising `stream` (a hipStream_t as void*).  Returns the number of
 * workgroups copied, -1 if the library was built without WR_TIMELINE, or -2
 * on a HIP error. */
WR_TL_API int64_t wr_timeline_read(uint64_t *rec, int64_t max_blocks, void *stream);

/* Rate of the timestamps' clock on the current device in kHz, or -2 on a
 * HIP error (in any build). */
WR_TL_API int64_t wr_timeline_clock_khz(void);

#ifdef __cplusplus
}
#endif

#endif /* WR_TIMELINE_H */

/*
 * wr_probe.h -- C-ABI of libwr_probe.so, a measurement utility beside the
 * MoE library: a read-only HBM streaming kernel that gives the achievable
 * read bandwidth of MI355X for the same bytes a MoE layer reads.  It is not
 * part of the drop-in boundary (include/warp_route.h) and has no counterpart
 * in the reference; bench.py uses it for the ceiling it reports beside the
 * layer's roofline fraction.
 */
#ifndef WR_PROBE_H
#define WR_PROBE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define WR_PROBE_API __attribute__((visibility("default")))
#else
#define WR_PROBE_API
#endif

#define WR_PROBE_MAX_RANGES 8

/* Reads every byte of n_ranges device ranges (ptrs[i], bytes[i]; each
 * pointer 16-byte aligned and each size a multiple of 16) once, with 16-byte
 * non-temporal loads, in one launch of blocks_per_cu * CUs workgroups of 256
 * threads that stride over the ranges, `unroll` (1, 2, 4 or 8) loads in
 * flight per lane.  The loaded data is folded into a value that is written
 * to *sink only if it equals a constant no real data produces, so the loads
 * cannot be elided and nothing is normally written.  Returns 0, or -1 for
 * invalid arguments (checked before any HIP call), or -2 if the launch
 * failed. */
WR_PROBE_API int wr_probe_read(const void *const *ptrs, const int64_t *bytes, int n_ranges,
                               int blocks_per_cu, int unroll, uint32_t *sink, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* WR_PROBE_H */

/*
 * wr_probe.h -- C-ABI of libwr_probe.so, a measurement utility beside the
 * MoE library: a read-only HBM streaming kernel that gives the achievable
 * read bandwidth of MI355X for the same bytes a MoE layer reads, and the rate
 * of the gate/up phase's own read order over them.  It is not
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
#define WR_PROBE_MAX_EXPERTS 8

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

/* Reads the gate and up matrices of n_experts packed experts (experts[i]:
 * the gate matrix, I rows of row_bytes; the up matrix right after it) in
 * the order a gate/up work pattern reads them, with the same loads as
 * wr_probe_read, in one launch of `blocks` workgroups of 256 threads that
 * loop over their share of the work:
 *   pattern 0: the single-token kernel's gate/up slots -- slot v covers rows
 *              8 (v mod I/8) .. + 8 of expert v / (I/8), wave w rows 2w and
 *              2w + 1 of the slot in both matrices, 4 KB of each row per
 *              round (four 1 KB loads per lane), rounds one after another;
 *   pattern 1: workgroup-level grid stride over groups of 4 rows of both
 *              matrices, wave w the w-th quarter of each row (row_bytes / 4096
 *              1 KB loads per lane per row), all 4 rows in one round.
 * row_bytes must be 4096 or 8192 and I a multiple of 8.  Returns 0, -1 for
 * invalid arguments (checked before any HIP call) or -2 if the launch
 * failed.  Like wr_probe_read, it writes *sink only in a case no real data
 * produces. */
WR_PROBE_API int wr_probe_gateup(const void *const *experts, int n_experts, int64_t row_bytes,
                                 int I, int pattern, int blocks, uint32_t *sink, void *stream);

/* Reads the down matrices of n_experts experts (down[i]: h rows of row_bytes,
 * the intermediate dimension of 16-bit weights) in groups of 4 rows, workgroup
 * b taking groups b, b + blocks, ...:
 *   pattern 0: the single-token kernel's down order -- the group's 1 KB column
 *              chunks of all experts (the last of a row partial),
 *              wave w taking q = w, w + 4, ..., four chunks of all 4 rows per
 *              round (16 loads per lane), rounds one after another;
 *   pattern 1: row-contiguous -- wave w reads row w of the group, expert after
 *              expert, 16 consecutive 1 KB loads per round.
 * row_bytes must be a multiple of 16 and at most 65536, h a positive
 * multiple of 4; rows must start 16-byte aligned.  Returns 0, -1 for invalid arguments (checked before any HIP
 * call) or -2 if the launch failed; *sink as for wr_probe_read. */
WR_PROBE_API int wr_probe_down(const void *const *down, int n_experts, int64_t row_bytes, int h,
                               int pattern, int blocks, uint32_t *sink, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* WR_PROBE_H */

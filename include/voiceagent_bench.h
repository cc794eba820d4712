/*
 * voiceagent_bench.h — bench-only diagnostics (libvoiceagent_bench.so).
 *
 * Not part of the drop-in ABI (include/voiceagent_attn.h) and with no
 * counterpart in the reference: bench.py uses it to measure the HBM read
 * floor that the decode kernel's bandwidth is read against, the mixed
 * read/write floor of the varlen launches, and one CU's read rate against
 * the bytes it keeps in flight.
 */
#ifndef VOICEAGENT_BENCH_H
#define VOICEAGENT_BENCH_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* load paths of va_bench_hbm_read */
#define VA_PROBE_PLAIN 0    /* plain 16-byte loads, 4 in flight per lane          */
#define VA_PROBE_NT 1       /* non-temporal 16-byte loads, 8 in flight per lane   */
#define VA_PROBE_LDS_DMA 2  /* non-temporal global_load_lds_dwordx4, 16 KiB in    */
                            /* flight per wave (the decode kernel's load path)    */

/* Streaming read of `bytes` contiguous bytes at `src` (16-byte aligned) in one
 * launch of `workgroups` 512-lane workgroups, each reading one contiguous
 * slice through load path `mode`.  `sink` needs `workgroups` 32-bit words and
 * is, in practice, never written.  Returns 0, or -1 on a bad argument (the
 * message is in va_bench_last_error()). */
int va_bench_hbm_read(const void* src, size_t bytes, int workgroups, int mode, void* sink,
                      void* stream);

/* Mixed stream in one launch of `workgroups` 512-lane workgroups: reads
 * `read_bytes` at `src` and writes `write_bytes` at `dst` (16-byte aligned,
 * non-overlapping), both contiguous, with non-temporal loads and stores; each
 * workgroup takes one contiguous slice of max(read_bytes, write_bytes).  The
 * floor that a launch reading and writing those byte counts is read against.
 * Returns 0, or -1 on a bad argument (va_bench_last_error()). */
int va_bench_hbm_copy(const void* src, size_t read_bytes, void* dst, size_t write_bytes,
                      int workgroups, void* stream);

/* One launch of `workgroups` 512-lane workgroups whose kernel does nothing:
 * the fixed cost of a launch of that grid (dispatch, completion and the
 * caches' hand-over to the next kernel), which every attention launch pays
 * before it moves a byte.  Returns 0, or -1 on a bad argument
 * (va_bench_last_error()). */
int va_bench_empty(int workgroups, void* stream);

/* Per-CU read rate against the bytes in flight: one launch of `workgroups`
 * 512-lane workgroups, each holding a 128 KiB LDS ring (so one per CU and
 * no two on one CU), workgroup w reading the `bytes_per_wg` bytes at
 * src + w bytes_per_wg (1 KiB aligned, inside `src_bytes`) in 1 KiB units
 * per wave: `dma_kib_per_wave` (0, 4, 8 or 16) through non-temporal LDS DMA
 * and `vgpr_kib_per_wave` (0, 4 or 8) through non-temporal register loads,
 * that many in flight per wave at every request.  `times` (device) receives
 * two 64-bit s_memrealtime stamps (100 MHz) per workgroup, start and end;
 * `sink` needs one 32-bit word per workgroup and is, in practice, never
 * written.  Returns 0, or -1 on a bad argument (va_bench_last_error()). */
int va_bench_hbm_depth(const void* src, size_t src_bytes, size_t bytes_per_wg, int workgroups,
                       int dma_kib_per_wave, int vgpr_kib_per_wave, void* times, void* sink,
                       void* stream);

const char* va_bench_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* VOICEAGENT_BENCH_H */

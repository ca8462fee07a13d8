/*
 * pa_probe.h -- streaming-rate probes of libpa_bench_probe.so.
 *
 * Measurement helpers for the benchmark (no reference counterpart, and not
 * part of the decode path's C ABI): the practical HBM rates that bound the
 * decode and write kernels.  Status codes are pa_mi355x.h's.
 */
#ifndef PA_PROBE_H
#define PA_PROBE_H

#include <stddef.h>
#include <stdint.h>

#include "pa_mi355x.h"

#ifdef __cplusplus
extern "C" {
#endif

/* pa_probe_read_contiguous sweeps `bytes` from `src` with 16-byte loads;
 * pa_probe_read_chunks reads `num_chunks` chunks of `chunk_bytes` (1024,
 * 2048 or a multiple of 4096) at src + order[i] * chunk_bytes, skipping order
 * values past `bytes`.  Both keep a checksum that is written to `sink` only on
 * a practically impossible value, so the loads cannot be optimised away. */
pa_status_t pa_probe_read_contiguous(const void* src, size_t bytes, uint32_t* sink, int32_t grid,
                                     pa_stream_t stream);
pa_status_t pa_probe_read_chunks(const void* src, size_t bytes, const int32_t* order,
                                 int32_t num_chunks, int32_t chunk_bytes, uint32_t* sink,
                                 int32_t grid, pa_stream_t stream);
/* pa_probe_read_write reads `read_bytes` (a multiple of 16) from `src` and
 * writes read_bytes / 2 to `dst` (below 4 GiB), both contiguous: the
 * practical rate of a stream with the INT8 write kernel's read : write ratio. */
pa_status_t pa_probe_read_write(const void* src, size_t read_bytes, void* dst, int32_t grid,
                                pa_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PA_PROBE_H */

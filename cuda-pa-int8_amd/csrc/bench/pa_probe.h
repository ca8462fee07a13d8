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

/* pa_probe_decode_stream issues exactly the loads of one grid decode launch
 * (the single-launch kinds, head_dim 128, at most 16 query heads per kv head)
 * and folds the loaded words into a checksum instead of computing attention:
 * its time is the memory system's for the decode's address stream.  The
 * arguments are those of the decode call, plus the plan it runs under
 * (pa_decode_plan_detail of pa_mi355x_tuning.h): partition_tokens, waves (4
 * or 8) and load_flags (bit 0: non-temporal V rows, bit 1: non-temporal K
 * rows, FP16 only).  int8_kv selects the INT8 layout (k_scales / v_scales
 * required). */
pa_status_t pa_probe_decode_stream(int32_t int8_kv, const void* q, const void* k_cache,
                                   const void* v_cache, const float* k_scales,
                                   const float* v_scales, const int32_t* block_table,
                                   const int32_t* context_lens, int32_t num_seqs,
                                   int32_t num_heads, int32_t num_kv_heads, int32_t block_size,
                                   int32_t num_blocks, int32_t max_blocks_per_seq,
                                   int32_t max_context_len, int32_t partition_tokens,
                                   int32_t waves, int32_t load_flags, uint32_t* sink,
                                   pa_stream_t stream);

/* pa_probe_quant_write runs the INT8 write kernel's launch (fp16 key / value,
 * per-token scales, head_dim 128) with the same loads and stores but no
 * quantization: each element's high byte is stored, and a scale of 1.  Its
 * time is the memory system's for the write kernel's address stream.  The
 * arguments are those of pa_reshape_and_cache_int8 (x = 8); the caches are
 * overwritten. */
pa_status_t pa_probe_quant_write(const void* key, const void* value, int64_t key_token_stride,
                                 int64_t key_head_stride, int64_t value_token_stride,
                                 int64_t value_head_stride, const int64_t* slot_mapping,
                                 int32_t num_tokens, int32_t num_kv_heads, void* k_cache,
                                 void* v_cache, float* k_scales, float* v_scales,
                                 int32_t num_blocks, int32_t block_size, pa_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PA_PROBE_H */

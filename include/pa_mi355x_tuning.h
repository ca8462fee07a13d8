/*
 * pa_mi355x_tuning.h -- test and tuning hooks of libpa_mi355x.so.
 *
 * No reference counterpart, and not part of the serving interface: these
 * force choices the planner otherwise makes itself, for parity tests that
 * must cover every code path and for partition / occupancy sweeps.  Each
 * setting belongs to the calling thread (thread-local) and affects that
 * thread's later planning, workspace-size queries and launches alike, so set
 * it before sizing a workspace; other threads keep the automatic choices.
 * Results never depend on them beyond the decode tolerance.
 */
#ifndef PA_MI355X_TUNING_H
#define PA_MI355X_TUNING_H

#include <stdint.h>

#include "pa_mi355x.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Waves per decode work-group: 4 or 8; 0 restores the automatic choice (8
 * for head_dim <= 128, else 4, and 4 for the split-K kinds with INT8 KV or
 * several query-head chunks per kv head). */
pa_status_t pa_decode_set_waves_per_group(int32_t waves);

/* Work distribution.  0 = automatic: the in-kernel schedule for the split-K
 * kinds with up to 1024 sequences, the grid otherwise; 1 = grid: one
 * work-group per (unit, split) slot of the host plan; 2 = in-kernel schedule:
 * persistent work-groups, one per resident slot, claim (split, kv head, head
 * chunk) items of a compact work list that every work-group derives from
 * context_lens; 3 = stream partition (split-K kinds, up to 1024 sequences):
 * the chunks of all (sequence, kv head) streams form one list, and every
 * resident work-group takes an equal contiguous range of it. */
pa_status_t pa_decode_set_schedule(int32_t mode);

/* The most query heads one work-group serves: 16 or 32 (two MFMA column
 * tiles, head_dim <= 128 only); 0 restores the automatic choice. */
pa_status_t pa_decode_set_max_head_tile(int32_t heads);

/* Cache hint of the V-row loads (K rows load plain, except in FP16 grid
 * launches whose splits hold at least 1024 tokens, which follow V).
 * 0 = automatic: non-temporal when each kv head's tiles are read by one
 * work-group and the call reads more than 32 MB of K/V, plain otherwise;
 * 1 = plain; 2 = non-temporal. */
pa_status_t pa_decode_set_load_policy(int32_t mode);

/* The plan this thread's calls would run under for these arguments (the
 * settings above included).  info receives up to n (<= 7) entries: [0] tokens
 * per split, [1] splits, [2] waves per work-group, [3] query heads per
 * work-group, [4] work distribution (1 grid, 2 in-kernel schedule, 3 stream
 * partition), [5] load hints (bit 0: non-temporal V rows, bit 1: non-temporal
 * K rows), [6] 1 when the splits are merged in the decode launch. */
pa_status_t pa_decode_plan_detail(pa_decode_kind_t kind, int32_t num_seqs, int32_t num_heads,
                                  int32_t head_dim, int32_t num_kv_heads, int32_t block_size,
                                  int32_t max_blocks_per_seq, int32_t max_context_len,
                                  int32_t partition_tokens, int32_t* info, int32_t n);

#ifdef __cplusplus
}
#endif

#endif /* PA_MI355X_TUNING_H */

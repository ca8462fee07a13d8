// Launch-level interface between the C ABI (pa_capi.cpp) and the kernel
// translation units (pa_decode_*.hip, pa_quant.hip).  Host-only types.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "pa_mi355x.h"

namespace pa {

constexpr int kIterTokens = 64;      // partition granularity (one wave iteration for head_dim <= 128)
constexpr int kMaxGroupTile = 16;    // query heads of one MFMA column tile
// Query heads one work-group serves for head_dim <= 128: two column tiles,
// so that each K/V load feeds up to 32 heads (MQA 32/1 in one work-group).
constexpr int kMaxHeadTile = 32;
// Largest split, per 4 waves of a work-group.  The planner never exceeds it
// (forced partitions included), so the block ids of one split fit in LDS.
// 8192 rather than 4096 for head_dim <= 128: uniform long contexts get half
// as many items per work-group, each paying its start once (MI355X, bench
// config 4 INT8 64k / 128k: 189.9 -> 185.9 us / 369.6 -> 362.8 us).  With
// head_dim 256 the larger block list would not fit two 4-wave groups per CU.
constexpr int max_partition_per_4_waves(int head_dim) { return head_dim > 128 ? 4096 : 8192; }
constexpr int kMinBlockSize = 8;
// In-kernel scheduling (persistent work-groups over a compact work list):
// the lengths of up to kSchedMaxSeqs sequences are staged in LDS; a ragged
// batch is cut into about kSchedItemsPerGroup items per resident work-group.
constexpr int kSchedMaxSeqs = 1024;
constexpr int kSchedItemsPerGroup = 4;
constexpr int kSchedQueueStride = 32;   // words between the 8 claim counters (128 B)
// Arrival counters: one per unit, then, for units of many splits (merged in
// two levels by the single launches), kMergeGroups per unit for the groups
// of splits.
constexpr int kMergeGroups = 4;

// Shape of one decode launch, shared by every decode kernel.
// The decode kernels take (block_table, context_lens, DecodeShape, ...) as
// their first arguments and the library is built to preload the first 14
// argument dwords into SGPRs: the two pointers and the first ten fields
// below, which is all a work-group needs to find its work item and issue its
// block-id and context-length loads without first fetching its arguments.
struct DecodeShape {
  int nchunk;       // group / head_tile
  int num_items;    // num_seqs * nsplit: (sequence, split) items of the grid form
  int nsplit;       // splits present in the grid
  int num_kv_heads;
  int partition;    // tokens per split, multiple of kIterTokens
  int max_blocks;   // block_table row stride
  int bs_log2;
  int block_size;
  int num_seqs;
  int num_blocks;
  int num_heads;
  int group;        // num_heads / num_kv_heads
  int head_tile;    // query heads per work-group (<= kMaxGroupTile)
  float scale_log2; // softmax scale * log2(e)
};

struct DecodeLaunch {
  void* out;
  const void* q;
  const void* k_cache;
  const void* v_cache;
  const float* k_scales;
  const float* v_scales;
  const int32_t* block_table;
  const int32_t* context_lens;
  float* part_acc;     // [units, nsplit, head_tile, head_dim]
  float* part_ml;      // [units, nsplit, head_tile, 2]
  uint32_t* counters;  // [units]
  int head_dim;
  int waves;           // waves per decode work-group: 4 or 8 (head_dim <= 128)
  bool int8_kv;
  bool fused;          // true: single launch with last-arriver merge; false: partition + reduce
                       // (the in-kernel schedule is always fused)
  bool nt_loads;       // non-temporal V-row loads (one head chunk per kv head)
  bool k_nt;           // non-temporal K-row loads too (FP16 grid launches, long splits)
  DecodeShape shape;
  // In-kernel schedule (sched = true): `groups` resident work-groups claim
  // (row, kv head) items; the partials hold `rows_max` slot rows.  Stream
  // partition (stream_part = true): `groups` work-groups take equal
  // contiguous ranges of the chunk list; the partials hold 2 * groups slots
  // and sched_info receives the chunk prefix.
  bool sched;
  bool stream_part;
  int groups;
  int rows_max;
  int pmin, pmax;      // partition bounds, multiples of 64 (equal when forced)
  int pmin_uniform;    // lower bound for equal lengths (<= pmin)
  int* sched_info;     // stream partition: [2 + num_seqs] chunk total, then prefix
  uint32_t* queue;     // 8 claim counters, zero between launches
  hipStream_t stream;
};

// One decode call's arguments as the C ABI passes them (pa_mi355x.h), minus
// the device memory and the stream.
struct DecodeCall {
  pa_decode_kind_t kind;
  void* out;
  const void* q;
  const void* k_cache;
  const void* v_cache;
  const float* k_scales;
  const float* v_scales;
  const int32_t* block_table;
  const int32_t* context_lens;
  float scale;
  int32_t block_size;
  int32_t num_seqs;
  int32_t num_heads;
  int32_t head_dim;
  int32_t num_kv_heads;
  int32_t num_blocks;
  int32_t x;
  int32_t max_blocks;
  int32_t max_context_len;
  int32_t partition_tokens;
};

// Defined in pa_capi.cpp, for the no-alloc entry point (pa_noalloc.hip).
// decode_sizes_capped validates and plans `c` with at most `ws_cap` bytes of
// workspace (the in-kernel schedule's row capacity is lowered to fit) and
// returns the counter and workspace bytes the call then uses, or
// PA_ERR_SCRATCH_LIMIT; no device access.  decode_launch_capped does the
// same and launches.
pa_status_t decode_sizes_capped(const DecodeCall& c, size_t ws_cap, size_t* counter_bytes,
                                size_t* workspace_bytes);
pa_status_t decode_launch_capped(const DecodeCall& c, void* counters, size_t counter_bytes,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream);

// Head dims the library is built for: every multiple of 8 in [8, 256].  The
// decode kernels are instantiated once per head_dim from pa_decode_inst.hip
// (compiled with -DPA_HEAD_DIM=D); the write kernels take the same set.
#define PA_FOR_EACH_HEAD_DIM(X)                                                          \
  X(8) X(16) X(24) X(32) X(40) X(48) X(56) X(64) X(72) X(80) X(88) X(96) X(104) X(112)  \
  X(120) X(128) X(136) X(144) X(152) X(160) X(168) X(176) X(184) X(192) X(200) X(208)   \
  X(216) X(224) X(232) X(240) X(248) X(256)

// Per head_dim D: the launcher of every decode kind, and the resident
// work-groups of a persistent decode kernel (the in-kernel schedule, or the
// stream partition) for a wave count and 1 or 2 column tiles (0 if it
// cannot run).
#define PA_DECLARE_DECODE_D(D)                                                          \
  hipError_t launch_decode_d##D(const DecodeLaunch& l);                                 \
  int resident_groups_d##D(bool stream_part, int waves, bool int8_kv, int column_tiles);
PA_FOR_EACH_HEAD_DIM(PA_DECLARE_DECODE_D)
#undef PA_DECLARE_DECODE_D

// Zeroes `bytes` (a multiple of 4) at `p` with a fill kernel on `stream`
// (pa_fill.hip).  A HIP graph may capture it: no memset node is recorded.
hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream);

struct QuantLaunch {
  const void* key;
  const void* value;
  int64_t key_token_stride;
  int64_t key_head_stride;
  int64_t value_token_stride;
  int64_t value_head_stride;
  const int64_t* slot_mapping;
  int num_tokens;
  int num_kv_heads;
  int head_dim;
  void* k_cache;
  void* v_cache;
  float* k_scales;
  float* v_scales;
  // Per-tensor mode: one given fp32 scale for every K (V) element, read on
  // the device; both NULL for the per-token mode.
  const float* k_scale_in;
  const float* v_scale_in;
  int num_blocks;
  int block_size;
  bool bf16_input;   // key / value are bf16 (else fp16)
  hipStream_t stream;
};

// Defined in pa_quant.hip.
hipError_t launch_quant_write_i8(const QuantLaunch& l);

struct CacheWriteLaunch {
  const void* key;
  const void* value;
  int64_t key_token_stride;
  int64_t key_head_stride;
  int64_t value_token_stride;
  int64_t value_head_stride;
  const int64_t* slot_mapping;
  int num_tokens;
  int num_kv_heads;
  int head_dim;
  void* k_cache;
  void* v_cache;
  int num_blocks;
  int block_size;
  hipStream_t stream;
};

// Defined in pa_cache_write.hip.
hipError_t launch_cache_write_f16(const CacheWriteLaunch& l);

}  // namespace pa

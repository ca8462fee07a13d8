// extern "C" entry points of libpa_mi355x.so (declared in include/pa_mi355x.h).
//
// Host side only: argument validation (the reference's TORCH_CHECKs made
// device-free), split planning, workspace carving and kernel dispatch.
#include "pa_mi355x.h"
#include "pa_mi355x_tuning.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "pa_internal.hpp"

namespace pa {
namespace {

// Dispatch on head_dim to the per-head_dim instantiations.
hipError_t launch_decode(const DecodeLaunch& l) {
  switch (l.head_dim) {
#define PA_CASE(D) \
  case D: return launch_decode_d##D(l);
    PA_FOR_EACH_HEAD_DIM(PA_CASE)
#undef PA_CASE
    default: return hipErrorInvalidValue;
  }
}

int resident_groups(int head_dim, bool stream_part, int waves, bool int8_kv, int column_tiles) {
  switch (head_dim) {
#define PA_CASE(D) \
  case D: return resident_groups_d##D(stream_part, waves, int8_kv, column_tiles);
    PA_FOR_EACH_HEAD_DIM(PA_CASE)
#undef PA_CASE
    default: return 0;
  }
}

}  // namespace
}  // namespace pa

namespace {

constexpr int kRefTile = 128;        // reference TILE (paged_attention_v3_warp.cu:20)
// Split planning, from partition-size sweeps on MI355X (bench configs 2-4):
// about 2048 resident waves (2 per SIMD with the pipelined loop) in as few
// splits as possible gave the best times; smaller partitions pay more merge
// round trips, larger ones leave CUs idle.
constexpr int kTargetWaves = 2048;   // waves one decode launch aims for (256 CUs x 8)
constexpr int kMinPartition = 256;   // per 4 waves: one 64-token iteration each
// Shortest item of the in-kernel schedule on ragged lengths, in tokens at
// head_dim <= 128 (half that above, where a token holds twice the bytes),
// whatever the group size; FP16 in 8-wave groups (one per CU) goes down to
// kSchedMinItemTokensF16.
constexpr int kSchedMinItemTokens = 2048;
constexpr int kSchedMinItemTokensF16 = 1536;
// Test and tuning overrides (pa_mi355x_tuning.h), per calling thread.
thread_local int g_waves_override = 0;
thread_local int g_schedule_mode = 0;   // 0 auto, 1 grid, 2 in-kernel schedule
thread_local int g_load_mode = 0;       // 0 auto, 1 plain, 2 non-temporal cache-tile loads
thread_local int g_head_tile_cap = 0;   // 0 auto, else the most query heads per work-group
constexpr long long kNtMinBytes = 32ll << 20;   // non-temporal loads above this much K/V
constexpr int kKntMinPartition = 1024;          // non-temporal K rows from this split size
// Split-K launches that read at most this much K/V (bound: every sequence at
// the checked maximum or the block-table capacity) take the single-launch plan.
constexpr long long kSplitKGridMaxBytes = 64ll << 20;
// Upper bound on resident decode work-groups used to size the partial
// buffers of the in-kernel schedule (256 CUs x 2 groups on MI355X).
constexpr int kSchedGroupsBound = 1024;
constexpr size_t kAlign = 256;

bool is_f16(pa_decode_kind_t k) { return k == PA_DECODE_WARP_F16 || k == PA_DECODE_SPLITK_F16; }
bool is_fused(pa_decode_kind_t k) { return k == PA_DECODE_WARP_F16 || k == PA_DECODE_WARP_I8; }
bool supported_head_dim(int d) {
  switch (d) {
#define PA_CASE(D) case D:
    PA_FOR_EACH_HEAD_DIM(PA_CASE)
#undef PA_CASE
    return true;
    default: return false;
  }
}
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
int ilog2(int v) {
  int r = 0;
  while ((1 << r) < v) ++r;
  return r;
}

// Largest divisor of the GQA group size that fits one work-group's head tile
// of at most `cap` query heads.
int head_tile_for(int group, int cap) {
  for (int t = std::min(group, cap); t >= 1; --t)
    if (group % t == 0) return t;
  return 1;
}

struct Plan {
  int head_tile = 1;
  int nchunk = 1;
  int units = 0;
  int waves = 4;
  int partition = 0;
  int nsplit = 1;
  // In-kernel schedule: partials hold rows_max slot rows of units_per_row
  // units; the kernel picks the partition in [pmin, pmax].
  bool sched = false;
  // Stream partition: equal contiguous chunk ranges per work-group; the
  // partials hold 2 slots per work-group.
  bool stream = false;
  int rows_max = 0;
  int rows_min = 0;       // rows at the upper partition bound: the least the partials may hold
  int pmin = 0, pmax = 0;
  int pmin_uniform = 0;   // lower bound the kernel uses when all lengths are equal
  bool nt_loads = false;  // non-temporal V-row loads
  bool k_nt = false;      // non-temporal K-row loads too
  bool fused = false;     // splits merged in the same launch (last-arriving work-group)
};

Plan make_plan(pa_decode_kind_t kind, int num_seqs, int num_heads, int num_kv_heads,
               int head_dim, int block_size, int max_blocks, int max_context_len,
               int partition_tokens) {
  Plan p;
  const int group = num_heads / num_kv_heads;
  // Work distribution.  The split-K kinds (long and ragged contexts) use the
  // in-kernel schedule: no empty work-groups and largest-first items (config
  // 5 of the bench: 10-37% faster than the grid).  The single-launch kinds
  // keep the grid, which saves the schedule's start-up for equal lengths.
  const int mode = g_schedule_mode;
  const long long cap = (long long)max_blocks * block_size;
  long long ctx = max_context_len > 0 ? std::min<long long>(max_context_len, cap) : cap;
  if (ctx < 1) ctx = 1;
  // K/V bytes of the launch if every sequence held `ctx` tokens.
  const long long kv_bytes = (long long)num_seqs * num_kv_heads * ctx * head_dim * 2 *
                             (is_f16(kind) ? 2 : 1);
  // Split-K kinds on small launches take the single-launch plan: the host
  // grid, splits merged in the launch, no schedule to build first.  There the
  // schedule's start-up (context lengths, then the schedule, then the block
  // ids) and its item floor (1536-2048 tokens per work-group) cost more than the
  // grid's empty work-groups: every ragged launch of a few dozen MB took 18.5-20 us
  // under the schedule.  Same box, alternating, schedule -> grid: one sequence,
  // 12/2, 1k / 16k tokens 9.43 -> 7.48 / 12.56 -> 11.07 us (INT8 16k 14.78 ->
  // 10.84); the reference's b1 x 4096 8/8 10.57 -> 9.04 and b8 x 4096 8/1 11.11 ->
  // 9.80; ragged 24 x median 1024 (bound 57 MB) 19.26 -> 10.97, 4 ragged up to
  // 9000 (37 MB) 19.18 -> 12.16; a 16k-capacity table holding 1k tokens 9.20 ->
  // 8.12.  Past 64 MB ragged batches turn (against the schedule with its
  // load-aware floor): 16 x median 2048 (164 MB) 17.0 -> 21.8, MQA 16 x median
  // 2048 (100 MB INT8) 17.5 -> 28.9, config 5 2-4x.
  if (mode == 0 && !is_fused(kind) && kv_bytes <= kSplitKGridMaxBytes)
    kind = is_f16(kind) ? PA_DECODE_WARP_F16 : PA_DECODE_WARP_I8;
  p.sched = mode == 2 || (mode == 0 && !is_fused(kind));
  // The stream partition serves the split-K kinds (its merge is the reduce
  // launch); its chunk list must count in 32 bits: at most S * ceil(cap / 32)
  // chunks per kv head.
  p.stream = mode == 3 && !is_fused(kind) &&
             (long long)num_seqs * ((cap + 31) / 32) * num_heads < (1ll << 31);
  if (num_seqs > pa::kSchedMaxSeqs) p.sched = p.stream = false;
  if (p.stream) p.sched = false;
  // Split merge: the single-launch kinds merge in the launch by definition;
  // under the in-kernel schedule the split-K kinds do too (the last
  // work-group of a unit merges its splits while the other work-groups still
  // stream) instead of a separate reduce launch.  Same-box A/B on MI355X,
  // split-K + reduce -> merged: MQA 32/1 of bench config 5 FP16 68.2 -> 60.5 us,
  // INT8 49.5 -> 44.5 us; config 4 32k INT8 95.6 -> 90.6 us; config 2 29.7 ->
  // 28.2 us; config 5 32/8 INT8 174.4 -> 169.4 us (FP16 279 -> 284 us, the one
  // loss).  The grid and stream forms of split-K keep their reduce launch.
  p.fused = is_fused(kind) || p.sched;
  // Head tile: up to 32 query heads (two MFMA column tiles) for head_dim <=
  // 128.  Under the in-kernel schedule only for FP16: there the K/V rows of a
  // kv head are read by one work-group instead of meeting in L2 from two
  // (MQA 32/1 on 8 x 32k, same box: 45.0 -> 42.9 us; config 5's ragged MQA
  // about even); INT8 keeps 16, whose single-tile form has the 16-byte W8
  // loads (8 x 32k INT8: 35.3 us with 16-head tiles, 40.6 with 32).
  int tile_cap = (head_dim <= 128 && (!p.sched || is_f16(kind))) ? pa::kMaxHeadTile
                                                                 : pa::kMaxGroupTile;
  // The hook sets the cap outright (two column tiles need head_dim <= 128).
  if (g_head_tile_cap > 0)
    tile_cap = std::min(g_head_tile_cap, head_dim <= 128 ? pa::kMaxHeadTile : pa::kMaxGroupTile);
  p.head_tile = head_tile_for(group, tile_cap);
  p.nchunk = group / p.head_tile;
  p.units = num_seqs * num_kv_heads * p.nchunk;
  const int ov = g_waves_override;
  p.waves = (ov == 4 || ov == 8) ? ov : 8;
  // Split-K kinds with INT8 KV or with several head chunks per kv head: two
  // 4-wave work-groups per CU, so that one group's item start (block ids, then
  // the first K/V round trip) overlaps the other's streaming.  Same-process
  // A/B on MI355X (bench config 5, 256 ragged sequences): INT8 188 -> 181 us,
  // MQA 32/1 INT8 57.0 -> 48.7 us, MQA FP16 72.4 -> 67.1 us; uniform config 4
  // INT8 +0.5-1.3%; FP16 with one chunk gains nothing (ragged +1.4%).
  if (ov == 0 && !is_fused(kind) && (!is_f16(kind) || p.nchunk > 1)) p.waves = 4;
  if (ov == 0 && p.stream) p.waves = 4;
  // Single-launch kinds with one 16-head column tile that read enough to be
  // bandwidth-bound: one 4-wave work-group per CU, with the partition an
  // 8-wave plan would take (up to the 4-wave cap of 8192 tokens, which keeps
  // a split's block ids in LDS), so each SIMD serves one wave's chunk math.  Same
  // box, alternating processes: INT8 config 3 48.2 -> 47.6 us, config 2 16.9
  // -> 16.6, config 4 32k 91.6 -> 90.3 (64k +0.6%); FP16 config 3 85.8 ->
  // 83.9, config 2 25.6 -> 25.3, the reference's GQA shapes 0.8-1.4%.  The
  // 32-head form (8-byte INT8 loads, 32 tokens per iteration) keeps 8 waves
  // (INT8 MQA 32/1 on 8 x 32k 33.0 -> 40.6 us with 4), and so do launches
  // below kNtMinBytes, which are latency-bound (config 1 4.8 -> 5.7 us with 4).
  const bool quad = ov == 0 && is_fused(kind) && head_dim <= 128 && p.head_tile <= 16 &&
                    kv_bytes > kNtMinBytes;
  if (quad) p.waves = 4;
  if (head_dim > 128) p.waves = 4;     // LDS of the 8-wave merge exceeds 64 KB
  long long part;
  // Caps the serial work of a work-group and keeps a split's block ids in LDS.
  const long long hi = (long long)pa::max_partition_per_4_waves(head_dim) * p.waves / 4;
  if (partition_tokens > 0) {
    part = std::min<long long>(partition_tokens, hi);
  } else {
    const long long units = std::max(1, p.units);
    const int plan_waves = quad ? 8 : p.waves;   // the group size the split count assumes
    const long long groups = kTargetWaves / plan_waves;
    const long long lo = (long long)kMinPartition * plan_waves / 4;
    part = (ctx * units + groups - 1) / groups;
    part = (part + kMinPartition - 1) / kMinPartition * kMinPartition;
    part = std::min(std::max(part, lo), hi);
  }
  part = (part + pa::kIterTokens - 1) / pa::kIterTokens * pa::kIterTokens;
  part = std::min<long long>(part, (ctx + pa::kIterTokens - 1) / pa::kIterTokens * pa::kIterTokens);
  p.partition = (int)part;
  p.nsplit = (int)((ctx + part - 1) / part);

  // V-row loads: non-temporal when every K/V byte is read by exactly one
  // work-group (one head chunk per kv head); MI355X streams them faster (plain
  // V: config 3 FP16 +10%, INT8 +6%; K rows follow their own rule, see
  // load_tile and k_nt below).  With several head chunks per kv head the
  // chunks find the tiles in the L2 only with plain loads (MQA 32/1 of
  // config 5: 71 us plain, 95 us non-temporal).
  // A launch that reads little (bound: every sequence at `ctx` tokens) is
  // latency-bound and its tiles may still sit in the 256 MB Infinity Cache
  // from an earlier call, which plain loads can hit (config 1: 4.6 us plain,
  // 6.0 us non-temporal); non-temporal loads start at 32 MB.
  const int lm = g_load_mode;
  p.nt_loads = lm == 2 || (lm == 0 && p.nchunk == 1 && kv_bytes > kNtMinBytes);

  // K rows non-temporal as well: FP16 grid launches whose splits hold at least
  // kKntMinPartition tokens (same box, caches rotated over 4x the Infinity
  // Cache: config 3 FP16 89.6 -> 86.4 us; with one 4-wave group per CU,
  // config 2's 1024-token splits 25.38 -> 25.22 us and the reference's GQA
  // shapes 0.4-1.4%; INT8 measured faster with plain K).
  p.k_nt = p.nt_loads && is_f16(kind) && !p.sched && !p.stream &&
           p.partition >= kKntMinPartition;
  if (p.sched) {
    if (partition_tokens > 0) {
      p.pmin = p.pmax = p.pmin_uniform = p.partition;
    } else {
      // Shorter items pay their fixed start-up and merge costs too often
      // (forced-partition sweeps of bench config 5 on MI355X, same box: 2048
      // against 1024 tokens, INT8 in 4-wave groups, 32/8 161.9 -> 156.2 us,
      // MQA 32/1 41.2 -> 39.7 us).  FP16 in 8-wave groups, one per CU, has
      // half the work-groups and gains from 1536 where the floor binds (MQA
      // 32/1, same box: config 5 56.2 -> 54.2 us; lognormal mixes of 512 x
      // median 512 60.1 -> 56.1 and 64 x median 2048 36.2 -> 33.0; 128 x
      // median 4096 108.9 -> 111.1); with 8 kv heads the floor does not bind.
      const int floor_tokens =
          (is_f16(kind) && p.waves == 8) ? kSchedMinItemTokensF16 : kSchedMinItemTokens;
      p.pmin = head_dim <= 128 ? floor_tokens : floor_tokens / 2;
      // Equal lengths: one item per resident work-group, down to the grid
      // plan's bound (config 2 would otherwise run on half the work-groups).
      p.pmin_uniform = kMinPartition * p.waves / 4;
      p.pmax = (int)hi;
    }
    // rows <= S + ceil(T / P), and the kernel keeps T / P <= max(groups * K / Hkv,
    // S * cap / pmax) (see build_schedule).
    const long long by_items =
        ((long long)kSchedGroupsBound * pa::kSchedItemsPerGroup + num_kv_heads - 1) / num_kv_heads;
    const long long by_cap = ((long long)num_seqs * cap + p.pmax - 1) / p.pmax;
    p.rows_max = (int)std::min<long long>(1 << 30, num_seqs + std::max(by_items, by_cap) + 1);
    p.rows_min = (int)std::min<long long>(1 << 30, num_seqs + by_cap + 1);
  }
  return p;
}

// Counters (zero between calls): the 8 claim counters of the in-kernel
// schedule at a fixed offset, then one arrival counter per unit, then
// kMergeGroups per unit for the two-level merge of long units.  Workspace
// (scratch): the stream partition's chunk record (stream partition only),
// then the split partials.
constexpr size_t kQueueBytes = 8 * pa::kSchedQueueStride * sizeof(uint32_t);
size_t counter_region(int units) {
  return align_up(kQueueBytes) + align_up((size_t)units * (1 + pa::kMergeGroups) * sizeof(uint32_t));
}

struct WsLayout {
  size_t info = 0, ml = 0, acc = 0, total = 0;
};

size_t slot_count(const Plan& p, int num_seqs) {
  if (p.stream) return 2 * (size_t)kSchedGroupsBound;
  return p.sched ? (size_t)p.rows_max * p.units / std::max(1, num_seqs)
                 : (size_t)p.units * p.nsplit;
}

WsLayout ws_layout(const Plan& p, int head_dim, int num_seqs) {
  WsLayout w;
  const size_t slots = slot_count(p, num_seqs);
  w.info = p.stream ? align_up((size_t)(2 + num_seqs) * sizeof(int)) : 0;
  w.ml = align_up(slots * p.head_tile * 2 * sizeof(float));
  w.acc = align_up(slots * p.head_tile * head_dim * sizeof(float));
  w.total = w.info + w.ml + w.acc;
  return w;
}

// Validates a call and plans it.  `ws_fit` > 0 caps the workspace: the
// in-kernel schedule's row capacity is lowered until its partials fit (the
// kernel then doubles its partition when the rows would exceed them), down to
// the rows it needs at the longest partition; a call that still does not fit
// gets PA_ERR_SCRATCH_LIMIT.  No device access.
pa_status_t decode_plan_call(const pa::DecodeCall& c, size_t ws_fit, Plan* plan, WsLayout* layout) {
  const pa_status_t st = pa_validate_decode(c.kind, c.num_seqs, c.num_heads, c.head_dim,
                                            c.num_kv_heads, c.num_blocks, c.block_size, c.x,
                                            c.max_blocks);
  if (st != PA_OK || c.num_seqs == 0) return st;
  if (!c.out || !c.q || !c.k_cache || !c.v_cache || !c.block_table || !c.context_lens)
    return PA_ERR_NULL_POINTER;
  if (!is_f16(c.kind) && (!c.k_scales || !c.v_scales)) return PA_ERR_NULL_POINTER;

  Plan p = make_plan(c.kind, c.num_seqs, c.num_heads, c.num_kv_heads, c.head_dim, c.block_size,
                     c.max_blocks, c.max_context_len, c.partition_tokens);
  if (!p.sched) {
    // The grid form launches (sequence, split) items rounded up to groups of 8,
    // times the kv heads and head chunks; a dispatch counts work-items in 32 bits.
    const long long items = (long long)c.num_seqs * p.nsplit;
    const long long groups = (items + 7) / 8 * 8 * c.num_kv_heads * p.nchunk;
    if (groups * p.waves * 64 > 0xFFFFFFFFll) return PA_ERR_BAD_SHAPE;
  }
  WsLayout wl = ws_layout(p, c.head_dim, c.num_seqs);
  if (ws_fit > 0 && wl.total > ws_fit && p.stream) {
    // the stream partition's partials do not fit: the in-kernel schedule,
    // whose row capacity can shrink, serves the call
    const int saved = g_schedule_mode;
    g_schedule_mode = 2;
    p = make_plan(c.kind, c.num_seqs, c.num_heads, c.num_kv_heads, c.head_dim, c.block_size,
                  c.max_blocks, c.max_context_len, c.partition_tokens);
    g_schedule_mode = saved;
    wl = ws_layout(p, c.head_dim, c.num_seqs);
  }
  if (ws_fit > 0 && wl.total > ws_fit) {
    if (!p.sched) return PA_ERR_SCRATCH_LIMIT;
    Plan lo = p;
    lo.rows_max = p.rows_min;
    if (ws_layout(lo, c.head_dim, c.num_seqs).total > ws_fit) return PA_ERR_SCRATCH_LIMIT;
    int a = p.rows_min, b = p.rows_max;   // largest row capacity that fits, in [a, b)
    while (b - a > 1) {
      lo.rows_max = a + (b - a) / 2;
      if (ws_layout(lo, c.head_dim, c.num_seqs).total <= ws_fit) a = lo.rows_max;
      else b = lo.rows_max;
    }
    p.rows_max = a;
    wl = ws_layout(p, c.head_dim, c.num_seqs);
  }
  *plan = p;
  *layout = wl;
  return PA_OK;
}

pa_status_t decode_common(const pa::DecodeCall& c, void* counters, size_t counter_bytes,
                          void* workspace, size_t workspace_bytes, pa_stream_t stream,
                          size_t ws_fit) {
  Plan p;
  WsLayout wl;
  const pa_status_t st = decode_plan_call(c, ws_fit, &p, &wl);
  if (st != PA_OK || c.num_seqs == 0) return st;
  if (!counters || counter_bytes < counter_region(p.units)) return PA_ERR_WORKSPACE;
  if (!workspace || workspace_bytes < wl.total) return PA_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(workspace) % kAlign != 0 ||
      reinterpret_cast<uintptr_t>(counters) % kAlign != 0)
    return PA_ERR_WORKSPACE;
  const pa_decode_kind_t kind = c.kind;
  void* out = c.out;
  const int num_seqs = c.num_seqs, num_heads = c.num_heads, head_dim = c.head_dim;
  const int num_kv_heads = c.num_kv_heads, block_size = c.block_size;

  pa::DecodeLaunch l{};
  l.out = out;
  l.q = c.q;
  l.k_cache = c.k_cache;
  l.v_cache = c.v_cache;
  l.k_scales = c.k_scales;
  l.v_scales = c.v_scales;
  l.block_table = c.block_table;
  l.context_lens = c.context_lens;
  char* cn = static_cast<char*>(counters);
  l.queue = reinterpret_cast<uint32_t*>(cn);
  l.counters = reinterpret_cast<uint32_t*>(cn + align_up(kQueueBytes));
  char* ws = static_cast<char*>(workspace);
  l.sched_info = reinterpret_cast<int*>(ws);
  l.part_ml = reinterpret_cast<float*>(ws + wl.info);
  l.part_acc = reinterpret_cast<float*>(ws + wl.info + wl.ml);
  l.sched = p.sched;
  l.stream_part = p.stream;
  l.rows_max = p.rows_max;
  l.pmin = p.pmin;
  l.pmin_uniform = p.pmin_uniform;
  l.pmax = p.pmax;
  if (p.sched || p.stream) {
    const bool i8 = !is_f16(kind);
    l.groups = pa::resident_groups(head_dim, p.stream, p.waves, i8,
                                   p.head_tile > pa::kMaxGroupTile ? 2 : 1);
    if (l.groups <= 0) return PA_ERR_LAUNCH;
    l.groups = std::min(l.groups, kSchedGroupsBound);
  }
  l.head_dim = head_dim;
  l.waves = p.waves;
  l.int8_kv = !is_f16(kind);
  l.fused = p.fused;
  l.nt_loads = p.nt_loads;
  l.k_nt = p.k_nt;
  l.stream = reinterpret_cast<hipStream_t>(stream);
  pa::DecodeShape& sh = l.shape;
  sh.num_seqs = num_seqs;
  sh.num_heads = num_heads;
  sh.num_kv_heads = num_kv_heads;
  sh.group = num_heads / num_kv_heads;
  sh.head_tile = p.head_tile;
  sh.nchunk = p.nchunk;
  sh.block_size = block_size;
  sh.bs_log2 = ilog2(block_size);
  sh.num_blocks = c.num_blocks;
  sh.max_blocks = c.max_blocks;
  sh.partition = p.partition;
  sh.nsplit = p.nsplit;
  sh.num_items = num_seqs * p.nsplit;
  sh.scale_log2 = c.scale * 1.4426950408889634f;

  return pa::launch_decode(l) == hipSuccess ? PA_OK : PA_ERR_LAUNCH;
}

}  // namespace

namespace pa {

pa_status_t decode_sizes_capped(const DecodeCall& c, size_t ws_cap, size_t* counter_bytes,
                                size_t* workspace_bytes) {
  Plan p;
  WsLayout wl;
  const pa_status_t st = decode_plan_call(c, ws_cap, &p, &wl);
  if (st != PA_OK) return st;
  *counter_bytes = c.num_seqs == 0 ? 0 : counter_region(p.units);
  *workspace_bytes = c.num_seqs == 0 ? 0 : wl.total;
  return PA_OK;
}

pa_status_t decode_launch_capped(const DecodeCall& c, void* counters, size_t counter_bytes,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return decode_common(c, counters, counter_bytes, workspace, workspace_bytes,
                       reinterpret_cast<pa_stream_t>(stream), workspace_bytes);
}

}  // namespace pa

extern "C" {

const char* pa_status_string(pa_status_t s) {
  switch (s) {
    case PA_OK: return "ok";
    case PA_ERR_NULL_POINTER: return "a required pointer is NULL";
    case PA_ERR_BAD_SHAPE: return "tensor sizes are inconsistent or out of range";
    case PA_ERR_BAD_BLOCK_SIZE: return "block_size must divide TILE and be a multiple of 8 (16 for int8)";
    case PA_ERR_UNSUPPORTED: return "head_dim must be a multiple of 8 in [8, 256] and x must be 8";
    case PA_ERR_WORKSPACE: return "counters or workspace NULL, misaligned or smaller than required";
    case PA_ERR_LAUNCH: return "the HIP runtime rejected the kernel launch";
    case PA_ERR_EMPTY_CONTEXT: return "context_lens must be >= 1 (empty sequences unsupported)";
    case PA_ERR_SCRATCH_LIMIT:
      return "the call needs more device scratch than the no-alloc entry point's static array";
  }
  return "unknown status";
}

const char* pa_version(void) { return "pa_mi355x 0.2 (gfx950)"; }

pa_status_t pa_validate_decode(pa_decode_kind_t kind, int32_t num_seqs, int32_t num_heads,
                               int32_t head_dim, int32_t num_kv_heads, int32_t num_blocks,
                               int32_t block_size, int32_t x, int32_t max_blocks_per_seq) {
  if (kind < PA_DECODE_WARP_F16 || kind > PA_DECODE_SPLITK_I8) return PA_ERR_BAD_SHAPE;
  // block_size rule of the reference launchers (v3:149-150, v5:167-168).
  const int mult = is_f16(kind) ? 8 : 16;
  if (block_size <= 0 || block_size % mult != 0 || kRefTile % block_size != 0)
    return PA_ERR_BAD_BLOCK_SIZE;
  if (x != 8) return PA_ERR_UNSUPPORTED;   // int8 rule of v5:176; the fp16 K loads assume it too
  if (!supported_head_dim(head_dim)) return PA_ERR_UNSUPPORTED;
  if (num_seqs < 0 || num_heads < 1 || num_kv_heads < 1 || num_heads % num_kv_heads != 0)
    return PA_ERR_BAD_SHAPE;
  if (num_seqs > 0 && (num_blocks < 1 || max_blocks_per_seq < 1)) return PA_ERR_BAD_SHAPE;
  if ((long long)max_blocks_per_seq * block_size > (1LL << 30)) return PA_ERR_BAD_SHAPE;
  return PA_OK;
}

pa_status_t pa_check_context_lens(const int32_t* host_context_lens, int32_t num_seqs,
                                  int32_t* max_len) {
  if (num_seqs > 0 && !host_context_lens) return PA_ERR_NULL_POINTER;
  int32_t mx = 0;
  for (int32_t i = 0; i < num_seqs; ++i) {
    if (host_context_lens[i] < 1) return PA_ERR_EMPTY_CONTEXT;
    mx = std::max(mx, host_context_lens[i]);
  }
  if (max_len) *max_len = mx;
  return PA_OK;
}

pa_status_t pa_decode_plan(pa_decode_kind_t kind, int32_t num_seqs, int32_t num_heads,
                           int32_t head_dim, int32_t num_kv_heads, int32_t block_size,
                           int32_t max_blocks_per_seq, int32_t max_context_len,
                           int32_t partition_tokens, int32_t* out_partition_tokens,
                           int32_t* out_num_splits) {
  pa_status_t st = pa_validate_decode(kind, num_seqs, num_heads, head_dim, num_kv_heads, 1,
                                      block_size, 8, std::max(1, max_blocks_per_seq));
  if (st != PA_OK) return st;
  const Plan p = make_plan(kind, num_seqs, num_heads, num_kv_heads, head_dim, block_size,
                           std::max(1, max_blocks_per_seq), max_context_len, partition_tokens);
  if (out_partition_tokens) *out_partition_tokens = p.partition;
  if (out_num_splits) *out_num_splits = p.nsplit;
  return PA_OK;
}

pa_status_t pa_decode_plan_detail(pa_decode_kind_t kind, int32_t num_seqs, int32_t num_heads,
                                  int32_t head_dim, int32_t num_kv_heads, int32_t block_size,
                                  int32_t max_blocks_per_seq, int32_t max_context_len,
                                  int32_t partition_tokens, int32_t* info, int32_t n) {
  if (!info && n > 0) return PA_ERR_NULL_POINTER;
  pa_status_t st = pa_validate_decode(kind, num_seqs, num_heads, head_dim, num_kv_heads, 1,
                                      block_size, 8, std::max(1, max_blocks_per_seq));
  if (st != PA_OK) return st;
  const Plan p = make_plan(kind, num_seqs, num_heads, num_kv_heads, head_dim, block_size,
                           std::max(1, max_blocks_per_seq), max_context_len, partition_tokens);
  const int32_t v[7] = {p.partition, p.nsplit, p.waves, p.head_tile,
                        p.stream ? 3 : (p.sched ? 2 : 1),
                        (p.nt_loads ? 1 : 0) | (p.k_nt ? 2 : 0), p.fused ? 1 : 0};
  for (int i = 0; i < n && i < 7; ++i) info[i] = v[i];
  return PA_OK;
}

size_t pa_decode_workspace_bytes(pa_decode_kind_t kind, int32_t num_seqs, int32_t num_heads,
                                 int32_t head_dim, int32_t num_kv_heads, int32_t block_size,
                                 int32_t max_blocks_per_seq, int32_t max_context_len,
                                 int32_t partition_tokens) {
  if (num_heads < 1 || num_kv_heads < 1 || num_heads % num_kv_heads != 0 || block_size < 1)
    return 0;
  const Plan p = make_plan(kind, std::max(0, num_seqs), num_heads, num_kv_heads, head_dim,
                           block_size, std::max(1, max_blocks_per_seq), max_context_len,
                           partition_tokens);
  return ws_layout(p, head_dim, std::max(0, num_seqs)).total;
}

pa_status_t pa_decode_set_waves_per_group(int32_t waves) {
  if (waves != 0 && waves != 4 && waves != 8) return PA_ERR_BAD_SHAPE;
  g_waves_override = waves;
  return PA_OK;
}

size_t pa_decode_counter_bytes(int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads) {
  if (num_heads < 1 || num_kv_heads < 1 || num_heads % num_kv_heads != 0) return 0;
  const int group = num_heads / num_kv_heads;
  // Head tiles of at most 16 query heads (the head_dim-256 rule): the most
  // units any head_dim gives, so the bound holds without knowing it.
  const int units =
      std::max(0, num_seqs) * num_kv_heads * (group / head_tile_for(group, pa::kMaxGroupTile));
  return counter_region(units);
}

pa_status_t pa_decode_set_schedule(int32_t mode) {
  if (mode < 0 || mode > 3) return PA_ERR_BAD_SHAPE;
  g_schedule_mode = mode;
  return PA_OK;
}

pa_status_t pa_decode_set_max_head_tile(int32_t heads) {
  if (heads != 0 && heads != 16 && heads != 32) return PA_ERR_BAD_SHAPE;
  g_head_tile_cap = heads;
  return PA_OK;
}

pa_status_t pa_decode_set_load_policy(int32_t mode) {
  if (mode < 0 || mode > 2) return PA_ERR_BAD_SHAPE;
  g_load_mode = mode;
  return PA_OK;
}

pa_status_t pa_decode_counters_reset(void* counters, size_t bytes, pa_stream_t stream) {
  if (bytes == 0) return PA_OK;
  if (!counters) return PA_ERR_NULL_POINTER;
  if (bytes % 4 != 0 || reinterpret_cast<uintptr_t>(counters) % 4 != 0) return PA_ERR_BAD_SHAPE;
  return pa::launch_fill_zero(counters, bytes, reinterpret_cast<hipStream_t>(stream)) == hipSuccess
             ? PA_OK
             : PA_ERR_LAUNCH;
}

// The four decode entry points differ only in the kind they pass on.
#define PA_DECODE_ENTRY_F16(NAME, KIND)                                                          \
  pa_status_t NAME(void* out, const void* q, const void* k_cache, const void* v_cache,          \
                   const int32_t* block_table, const int32_t* context_lens, float scale,        \
                   int32_t block_size, int32_t num_seqs, int32_t num_heads, int32_t head_dim,   \
                   int32_t num_kv_heads, int32_t num_blocks, int32_t x,                         \
                   int32_t max_blocks_per_seq, int32_t max_context_len,                         \
                   int32_t partition_tokens, void* counters, size_t counter_bytes,              \
                   void* workspace, size_t workspace_bytes, pa_stream_t stream) {               \
    const pa::DecodeCall c{KIND,         out,          q,         k_cache,                      \
                           v_cache,      nullptr,      nullptr,   block_table,                  \
                           context_lens, scale,        block_size, num_seqs,                    \
                           num_heads,    head_dim,     num_kv_heads, num_blocks,                \
                           x,            max_blocks_per_seq, max_context_len, partition_tokens}; \
    return decode_common(c, counters, counter_bytes, workspace, workspace_bytes, stream, 0);   \
  }
#define PA_DECODE_ENTRY_I8(NAME, KIND)                                                           \
  pa_status_t NAME(void* out, const void* q, const void* k_cache, const void* v_cache,          \
                   const float* k_scales, const float* v_scales, const int32_t* block_table,    \
                   const int32_t* context_lens, float scale, int32_t block_size,                \
                   int32_t num_seqs, int32_t num_heads, int32_t head_dim,                       \
                   int32_t num_kv_heads, int32_t num_blocks, int32_t x,                         \
                   int32_t max_blocks_per_seq, int32_t max_context_len,                         \
                   int32_t partition_tokens, void* counters, size_t counter_bytes,              \
                   void* workspace, size_t workspace_bytes, pa_stream_t stream) {               \
    const pa::DecodeCall c{KIND,         out,          q,         k_cache,                      \
                           v_cache,      k_scales,     v_scales,  block_table,                  \
                           context_lens, scale,        block_size, num_seqs,                    \
                           num_heads,    head_dim,     num_kv_heads, num_blocks,                \
                           x,            max_blocks_per_seq, max_context_len, partition_tokens}; \
    return decode_common(c, counters, counter_bytes, workspace, workspace_bytes, stream, 0);   \
  }

PA_DECODE_ENTRY_F16(pa_paged_decode_attn_warp, PA_DECODE_WARP_F16)
PA_DECODE_ENTRY_F16(pa_paged_decode_attn_splitk, PA_DECODE_SPLITK_F16)
PA_DECODE_ENTRY_I8(pa_paged_decode_attn_warp_int8, PA_DECODE_WARP_I8)
PA_DECODE_ENTRY_I8(pa_paged_decode_attn_splitk_int8, PA_DECODE_SPLITK_I8)

}  // extern "C"

namespace {

// Checks shared by the cache-write entry points: 16-byte row loads and row
// stores need 16-byte aligned rows and bases.
pa_status_t check_write_args(const void* key, const void* value, int64_t kts, int64_t khs,
                             int64_t vts, int64_t vhs, const int64_t* slot_mapping,
                             int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                             const void* k_cache, const void* v_cache, int32_t num_blocks,
                             int32_t block_size, int32_t x, int32_t block_mult) {
  if (block_size <= 0 || block_size % block_mult != 0 || kRefTile % block_size != 0)
    return PA_ERR_BAD_BLOCK_SIZE;
  if (x != 8 || !supported_head_dim(head_dim)) return PA_ERR_UNSUPPORTED;
  if (num_tokens < 0 || num_kv_heads < 1 || num_blocks < 1) return PA_ERR_BAD_SHAPE;
  if (num_tokens == 0) return PA_OK;
  if (!key || !value || !slot_mapping || !k_cache || !v_cache) return PA_ERR_NULL_POINTER;
  const int64_t strides[4] = {kts, khs, vts, vhs};
  for (int64_t s : strides)
    if (s < 0 || s % 8 != 0) return PA_ERR_BAD_SHAPE;
  const void* ptrs[4] = {key, value, k_cache, v_cache};
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return PA_ERR_BAD_SHAPE;
  return PA_OK;
}

pa_status_t quant_write(const void* key, const void* value, int64_t key_token_stride,
                        int64_t key_head_stride, int64_t value_token_stride,
                        int64_t value_head_stride, const int64_t* slot_mapping,
                        int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                        void* k_cache, void* v_cache, float* k_scales, float* v_scales,
                        const float* k_scale_in, const float* v_scale_in, int32_t num_blocks,
                        int32_t block_size, int32_t x, pa_stream_t stream, bool bf16_input) {
  const pa_status_t st = check_write_args(
      key, value, key_token_stride, key_head_stride, value_token_stride, value_head_stride,
      slot_mapping, num_tokens, num_kv_heads, head_dim, k_cache, v_cache, num_blocks, block_size,
      x, 16);
  if (st != PA_OK || num_tokens == 0) return st;
  if (!k_scales || !v_scales) return PA_ERR_NULL_POINTER;
  pa::QuantLaunch l{};
  l.key = key;
  l.value = value;
  l.key_token_stride = key_token_stride;
  l.key_head_stride = key_head_stride;
  l.value_token_stride = value_token_stride;
  l.value_head_stride = value_head_stride;
  l.slot_mapping = slot_mapping;
  l.num_tokens = num_tokens;
  l.num_kv_heads = num_kv_heads;
  l.head_dim = head_dim;
  l.k_cache = k_cache;
  l.v_cache = v_cache;
  l.k_scales = k_scales;
  l.v_scales = v_scales;
  l.k_scale_in = k_scale_in;
  l.v_scale_in = v_scale_in;
  l.num_blocks = num_blocks;
  l.block_size = block_size;
  l.bf16_input = bf16_input;
  l.stream = reinterpret_cast<hipStream_t>(stream);
  return pa::launch_quant_write_i8(l) == hipSuccess ? PA_OK : PA_ERR_LAUNCH;
}

}  // namespace

extern "C" {

pa_status_t pa_reshape_and_cache_int8(const void* key, const void* value,
                                      int64_t key_token_stride, int64_t key_head_stride,
                                      int64_t value_token_stride, int64_t value_head_stride,
                                      const int64_t* slot_mapping, int32_t num_tokens,
                                      int32_t num_kv_heads, int32_t head_dim, void* k_cache,
                                      void* v_cache, float* k_scales, float* v_scales,
                                      int32_t num_blocks, int32_t block_size, int32_t x,
                                      pa_stream_t stream) {
  return quant_write(key, value, key_token_stride, key_head_stride, value_token_stride,
                     value_head_stride, slot_mapping, num_tokens, num_kv_heads, head_dim, k_cache,
                     v_cache, k_scales, v_scales, nullptr, nullptr, num_blocks, block_size, x,
                     stream, false);
}

pa_status_t pa_reshape_and_cache_int8_bf16(const void* key, const void* value,
                                           int64_t key_token_stride, int64_t key_head_stride,
                                           int64_t value_token_stride, int64_t value_head_stride,
                                           const int64_t* slot_mapping, int32_t num_tokens,
                                           int32_t num_kv_heads, int32_t head_dim, void* k_cache,
                                           void* v_cache, float* k_scales, float* v_scales,
                                           int32_t num_blocks, int32_t block_size, int32_t x,
                                           pa_stream_t stream) {
  return quant_write(key, value, key_token_stride, key_head_stride, value_token_stride,
                     value_head_stride, slot_mapping, num_tokens, num_kv_heads, head_dim, k_cache,
                     v_cache, k_scales, v_scales, nullptr, nullptr, num_blocks, block_size, x,
                     stream, true);
}

pa_status_t pa_reshape_and_cache_int8_static(
    const void* key, const void* value, int64_t key_token_stride, int64_t key_head_stride,
    int64_t value_token_stride, int64_t value_head_stride, const int64_t* slot_mapping,
    int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim, void* k_cache, void* v_cache,
    float* k_scales, float* v_scales, const float* k_scale, const float* v_scale,
    int32_t num_blocks, int32_t block_size, int32_t x, pa_stream_t stream) {
  if (num_tokens > 0 && (!k_scale || !v_scale)) return PA_ERR_NULL_POINTER;
  return quant_write(key, value, key_token_stride, key_head_stride, value_token_stride,
                     value_head_stride, slot_mapping, num_tokens, num_kv_heads, head_dim, k_cache,
                     v_cache, k_scales, v_scales, k_scale, v_scale, num_blocks, block_size, x,
                     stream, false);
}

pa_status_t pa_reshape_and_cache_int8_static_bf16(
    const void* key, const void* value, int64_t key_token_stride, int64_t key_head_stride,
    int64_t value_token_stride, int64_t value_head_stride, const int64_t* slot_mapping,
    int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim, void* k_cache, void* v_cache,
    float* k_scales, float* v_scales, const float* k_scale, const float* v_scale,
    int32_t num_blocks, int32_t block_size, int32_t x, pa_stream_t stream) {
  if (num_tokens > 0 && (!k_scale || !v_scale)) return PA_ERR_NULL_POINTER;
  return quant_write(key, value, key_token_stride, key_head_stride, value_token_stride,
                     value_head_stride, slot_mapping, num_tokens, num_kv_heads, head_dim, k_cache,
                     v_cache, k_scales, v_scales, k_scale, v_scale, num_blocks, block_size, x,
                     stream, true);
}

pa_status_t pa_reshape_and_cache_f16(const void* key, const void* value,
                                     int64_t key_token_stride, int64_t key_head_stride,
                                     int64_t value_token_stride, int64_t value_head_stride,
                                     const int64_t* slot_mapping, int32_t num_tokens,
                                     int32_t num_kv_heads, int32_t head_dim, void* k_cache,
                                     void* v_cache, int32_t num_blocks, int32_t block_size,
                                     int32_t x, pa_stream_t stream) {
  const pa_status_t st = check_write_args(
      key, value, key_token_stride, key_head_stride, value_token_stride, value_head_stride,
      slot_mapping, num_tokens, num_kv_heads, head_dim, k_cache, v_cache, num_blocks, block_size,
      x, 8);
  if (st != PA_OK || num_tokens == 0) return st;
  pa::CacheWriteLaunch l{};
  l.key = key;
  l.value = value;
  l.key_token_stride = key_token_stride;
  l.key_head_stride = key_head_stride;
  l.value_token_stride = value_token_stride;
  l.value_head_stride = value_head_stride;
  l.slot_mapping = slot_mapping;
  l.num_tokens = num_tokens;
  l.num_kv_heads = num_kv_heads;
  l.head_dim = head_dim;
  l.k_cache = k_cache;
  l.v_cache = v_cache;
  l.num_blocks = num_blocks;
  l.block_size = block_size;
  l.stream = reinterpret_cast<hipStream_t>(stream);
  return pa::launch_cache_write_f16(l) == hipSuccess ? PA_OK : PA_ERR_LAUNCH;
}

}  // extern "C"

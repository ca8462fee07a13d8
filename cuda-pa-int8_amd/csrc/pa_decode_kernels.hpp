// Paged-attention decode kernels for gfx950 (FP16 and INT8 KV), MFMA form.
//
// Work decomposition
//   A work item is (sequence, kv_head, split).  A work-group of 4 or 8 waves serves
//   one work item for the whole group of query heads that share the kv head
//   (up to 16 per MFMA column tile, two tiles at head_dim <= 128; larger
//   groups in several head chunks), so every K/V byte fetched from HBM feeds
//   all of them (the reference launches one block per query head and re-reads
//   KV G times, kernels/paged_attention_v3_warp.cu:159).  The split's tokens are cut into
//   wave iterations (64 tokens for head_dim <= 128, else 32) dealt
//   round-robin to the waves (a fixed assignment, so results are bitwise
//   reproducible); each wave keeps its own online-softmax state and the waves
//   merge through LDS at the end.
//
// Both products are 16-wide MFMAs (v_mfma_f32_16x16x32_f16):
//   QK:  S^T[16 token rows][16 heads] += K[rows][32 dims] x Q^T[32 dims][heads]
//   PV:  O^T[16 dims][16 heads]       += V^T[dims][32 tokens] x P^T[tokens][heads]
//   Lane l = (r = l & 15, g = l >> 4).  The B operands hold one query head per
//   lane column, so after QK lane (r, g) owns head r and the scores of the 8
//   consecutive tokens tok0 + 32p + 8g .. +7 (p = pair of 16-token slabs);
//   those are exactly the P^T values the same lane feeds to the PV MFMA, and
//   the PV result O^T lands in the same lane (head r, dims 16t + 4g + e).
//   Softmax rescaling is therefore lane-local; only the per-head max and sum
//   are combined over the 4 lanes of a head (permlane swaps).  K rows are
//   assigned to MFMA rows so that row 4g + e of the first QK MFMA of a pair is
//   token tok0 + 32p + 8g + e and of the second one token + 4.
//   The softmax scale is folded into exp2 via scale*log2(e); the running
//   (max, sum) update is the reference's (paged_attention_v3_warp.cu:84-122).
//
// INT8 (paged_attention_v5_warp_int8.cu:80-108 semantics): int8 K and V are
//   converted to fp16 holding 1152 + value (exact, 3 ops per 4 values); the K
//   bias is removed from the scores with 1152*sum(q) per head.  V enters the
//   PV products biased: each chunk's weight sums sum(w) per head come from
//   one more MFMA against a ones operand, and 1152*sum(w) is subtracted from
//   the fp32 accumulator after the chunk's products, so no bias carries from
//   one chunk to the next.  That subtraction cancels in fp32: the chunk's
//   biased sums are at most 1279*sum(w), so its error stays within a few
//   roundings of 2^-24 * 1279 * sum(w), below 2.3e-4 times the weight-averaged
//   s_v in the output (about 2e-6 of a token's largest |v| = 127 s_v).  s_k
//   multiplies each score; s_v is folded into the fp16 softmax weight, scaled
//   by 2^e with e chosen per iteration from the largest s_v so the weights
//   stay normal and below fp16's range; the running sum l accumulates the
//   unscaled weight.
//
// Splits: FUSED (the single-launch grid kernel, and the scheduled split-K
//   kernel) writes per-split partials with device-coherent (write-through)
//   stores, waits for them, counts arrivals with a device-scope atomic, and
//   the last work-group of a unit merges with device-coherent loads in the
//   same launch (units with many splits in two levels).  The grid and stream
//   forms of split-K merge in a separate reduce kernel
//   (paged_attention_v4_splitk.cu:156-187).
#pragma once

#include <math.h>

#include <type_traits>

#include "pa_device.hpp"
#include "pa_internal.hpp"

namespace pa {

constexpr int kThreads = 4 * kWave;   // split-K reduce work-group
// s_waitcnt immediate (gfx9 encoding) that waits for LDS/scalar memory only:
// vmcnt and expcnt at their maxima, lgkmcnt = 0.
constexpr int kWaitLgkm0 = 0xC07F;
constexpr float kNegInf = -INFINITY;

// Work-group barrier for LDS traffic only: this thread's LDS accesses are
// complete (lgkmcnt 0) before it, and, unlike __syncthreads, it waits for no
// vector-memory operation, so K/V loads already issued stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef float f2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f4_t mfma16(h8_t a, h8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Max / sum over the four lanes l, l^16, l^32, l^48 (the lanes of head r).
__device__ __forceinline__ float head_max(float v) {
  v = cross_row16(v, OpMax());
  return cross_half32(v, OpMax());
}
__device__ __forceinline__ float head_sum(float v) {
  v = cross_row16(v, OpSum());
  return cross_half32(v, OpSum());
}

// Loads of cache tiles.  NTL: non-temporal, for tiles that no other
// work-group of the launch reads (one head chunk per kv head); otherwise plain,
// so the head chunks that share a kv head find its tiles in the L2.  V rows
// take the non-temporal form under NTL: a V load instruction covers whole
// 128-B lines.  Each K line is read half by one instruction and half by the
// next (the two token halves of a row group), and non-temporal K lines can
// leave the L2 in between (INT8 config 3 fetched 7% more), so K rows load
// plain except under KNT, which the planner sets for FP16 grid launches with
// splits of >= 1024 tokens, where non-temporal K measured faster (config 3
// FP16 3.6%, config 2 0.6%; plain K stays ahead for INT8, ragged batches and
// shorter splits).
template <typename T, bool NTL>
__device__ __forceinline__ T load_tile(const void* p) {
  if constexpr (NTL) return load_stream<T>(p);
  else return *reinterpret_cast<const T*>(p);
}

// Value of quad position b (lane 4k + b) in every lane of quad k.  b must
// fold to a constant (unrolled loops).
__device__ __forceinline__ float quad_bcast(float v, int b) {
  switch (b) {
    case 0: return dpp_mov<0x00>(v);
    case 1: return dpp_mov<0x55>(v);
    case 2: return dpp_mov<0xAA>(v);
    default: return dpp_mov<0xFF>(v);
  }
}

// 8 int8 values -> 8 fp16 values holding 1152 + value.
__device__ __forceinline__ h8_t i8x8_biased(uint2 w) {
  uint32_t d[4];
  i8x4_to_biased_h2(w.x, d[0], d[1]);
  i8x4_to_biased_h2(w.y, d[2], d[3]);
  return __builtin_bit_cast(h8_t, d);
}
// Zero the fp16 elements e >= n of an 8-element row (tokens past the end may
// hold NaN bits, and 0 * NaN would poison the PV product).
__device__ __forceinline__ uint4 keep_first(uint4 v, int n) {
  uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t m = (2 * k + 1 < n) ? 0xFFFFFFFFu : ((2 * k < n) ? 0x0000FFFFu : 0u);
    d[k] &= m;
  }
  return make_uint4(d[0], d[1], d[2], d[3]);
}

// Buffer resource over [base, base + bytes).  The base must be uniform over
// the wave (it lives in scalar registers); offsets past `bytes` read zeros and
// drop writes.
constexpr int kBufWord3 = 0x00020000;   // 32-bit data format, raw (untyped) access
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kBufWord3);
}
// Cache policy of buffer accesses: device-coherent (sc1) stores write
// through to memory, device-coherent loads do not hit in a stale L2 line; the
// same bits the compiler uses for agent-scope atomic loads and stores.
constexpr int kPolicyDevice = 16;

// Folds the partials of splits [0, ns) of one unit, in split order, into the
// running (max, sum, accumulators) (M, L, A) of NI consecutive items of one
// head: (head h, dims 4(c0 + i) .. 4(c0 + i) + 3), i < NI; M = -inf: nothing
// folded yet.  The partial of split sp sits in slot slot_of(sp): acc[gt][D]
// (relative to its max) and (m, l) per head.  SB splits go out as one batch of
// loads (NI accumulator chunks and one (m, l) pair each), so a unit of ns
// splits costs ceil(ns / SB) round trips per thread.
// COHERENT: device-coherent loads (partials written in this launch).
template <int D, bool COHERENT, int NI, int SB, typename SlotOf>
__device__ __forceinline__ void fold_splits(const float* __restrict__ pacc,
                                            const float* __restrict__ pml, SlotOf slot_of, int gt,
                                            int h, int c0, int ns, float& M, float& L,
                                            f4_t (&A)[NI]) {
  constexpr int POL = COHERENT ? kPolicyDevice : 0;
  const uint32_t acc_bytes = (uint32_t)(gt * D * 4), ml_bytes = (uint32_t)(gt * 8);
  for (int s0 = 0; s0 < ns; s0 += SB) {
    f4_t v[SB][NI];
    f2_t ml[SB];
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      // Past the last split the last one is re-read (and weighted 0), so
      // every load of the batch is unconditional.
      const size_t slot = slot_of(min(s0 + u, ns - 1));
      const auto ra = buf_rsrc(pacc + slot * gt * D, acc_bytes);
      const auto rm = buf_rsrc(pml + slot * gt * 2, ml_bytes);
#pragma unroll
      for (int i = 0; i < NI; ++i)
        v[u][i] = __builtin_bit_cast(
            f4_t, __builtin_amdgcn_raw_buffer_load_b128(ra, (h * D + 4 * (c0 + i)) * 4, 0, POL));
      ml[u] = __builtin_bit_cast(f2_t, __builtin_amdgcn_raw_buffer_load_b64(rm, h * 8, 0, POL));
    }
    float mb = M;
#pragma unroll
    for (int u = 0; u < SB; ++u)
      if (s0 + u < ns) mb = fmaxf(mb, ml[u].x);
    const float fo = M == kNegInf ? 0.f : exp2f_fast(M - mb);
#pragma unroll
    for (int i = 0; i < NI; ++i) A[i] *= fo;
    L *= fo;
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const float f = (s0 + u < ns && ml[u].x != kNegInf) ? exp2f_fast(ml[u].x - mb) : 0.f;
#pragma unroll
      for (int i = 0; i < NI; ++i) A[i] += v[u][i] * f;
      L += ml[u].y * f;
    }
    M = mb;
  }
}

// The normalised fp16 output of item (head h, dims 4c .. 4c + 3).
template <int D>
__device__ __forceinline__ void write_out_item(half_t* __restrict__ out, size_t out_base, int h,
                                               int c, float L, f4_t A) {
  const float inv = L > 0.f ? 1.f / L : 0.f;
  const uint2 pk = make_uint2(pack_h2(A[0] * inv, A[1] * inv), pack_h2(A[2] * inv, A[3] * inv));
  *reinterpret_cast<uint2*>(out + out_base + (size_t)h * D + 4 * c) = pk;
}

// Where a merge puts its items: the normalised fp16 output rows of the unit.
template <int D>
struct OutSink {
  half_t* out;
  size_t base;
  __device__ __forceinline__ void operator()(int h, int c, float, float L, f4_t A) const {
    write_out_item<D>(out, base, h, c, L, A);
  }
};

// ... or one partial (the fold of a group of splits, relative to its max) in
// the slot behind `racc`.  The (max, sum) pairs wait in LDS (`ml_lds`, two
// floats per head) until every thread has read the group's own pairs, since
// the destination slot is one of the group's: the caller stores them after a
// barrier.  Each accumulator item is read and rewritten by one thread only.
template <int D>
struct SlotSink {
  __amdgpu_buffer_rsrc_t racc;
  float* ml_lds;
  __device__ __forceinline__ void operator()(int h, int c, float M, float L, f4_t A) const {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4_t, A), racc, (h * D + 4 * c) * 4,
                                           0, kPolicyDevice);
    if (c == 0) {
      ml_lds[2 * h] = M;
      ml_lds[2 * h + 1] = L;
    }
  }
};

// Items (head, 4-dim chunk) tid * NI .. + NI - 1, + THREADS * NI, ... of a unit:
// NI consecutive chunks of one head per thread (D / 4 is a multiple of NI).
template <int D, int THREADS, bool COHERENT, int NI, int SB, typename SlotOf, typename Sink>
__device__ __forceinline__ void merge_splits_by(const float* __restrict__ pacc,
                                                const float* __restrict__ pml, SlotOf slot_of,
                                                int gt, int ns, int tid, const Sink& sink) {
  constexpr int CH = D / 4;
  static_assert(CH % NI == 0, "a thread's chunks lie in one head");
  const int nitems = gt * CH;
  for (int base = tid * NI; base < nitems; base += THREADS * NI) {
    const int h = base / CH, c0 = base - h * CH;
    float M = kNegInf, L = 0.f;
    f4_t A[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) A[i] = (f4_t){0.f, 0.f, 0.f, 0.f};
    fold_splits<D, COHERENT, NI, SB>(pacc, pml, slot_of, gt, h, c0, ns, M, L, A);
#pragma unroll
    for (int i = 0; i < NI; ++i) sink(h, c0 + i, M, L, A[i]);
  }
}

// Merge the `ns` partials of one unit (gt heads) into `sink`, without LDS or
// barriers.  With more items than threads each thread takes 2 or 4
// consecutive chunks of one head: they share the (m, l) loads, and all of a
// batch's loads are in flight together (up to about 24 per thread), so the
// round trips a thread waits for are ceil(ns / SB) rather than one per 8
// splits and chunk.  The batch follows ns: the re-read padding of a short last
// batch costs load slots (config 2, 4 splits: 16-split batches measured 3-4%
// slower than 4-split ones).  Same box, against one chunk per thread in
// batches of 8: bench config 3 warp_int8 50.4 -> 48.6 us, MQA 32/1 INT8 of
// config 5 44.8 -> 42.6 us.
template <int D, int THREADS, bool COHERENT, typename SlotOf, typename Sink>
__device__ __forceinline__ void merge_splits_into(const float* __restrict__ pacc,
                                                  const float* __restrict__ pml, SlotOf slot_of,
                                                  int gt, int ns, const Sink& sink) {
  constexpr int CH = D / 4;
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));   // nothing lane-dependent is hoisted out of a caller's loop
  const int nitems = gt * CH;
#define PA_MERGE_BY(NI, SB) \
  merge_splits_by<D, THREADS, COHERENT, NI, SB>(pacc, pml, slot_of, gt, ns, tid, sink)
  if constexpr (CH % 4 == 0) {
    if (nitems > 2 * THREADS) {
      if (ns <= 4) PA_MERGE_BY(4, 4);
      else PA_MERGE_BY(4, 6);
      return;
    }
  }
  if constexpr (CH % 2 == 0) {
    if (nitems > THREADS) {
      if (ns <= 4) PA_MERGE_BY(2, 4);
      else if (ns <= 8 || (ns > 10 && ns <= 16)) PA_MERGE_BY(2, 8);
      else PA_MERGE_BY(2, 10);
      return;
    }
  }
  if (ns <= 4) PA_MERGE_BY(1, 4);
  else if (ns <= 8) PA_MERGE_BY(1, 8);
  else PA_MERGE_BY(1, 16);
#undef PA_MERGE_BY
}

// Merge the `ns` partials of one unit and write its fp16 output rows.
template <int D, int THREADS, bool COHERENT, typename SlotOf>
__device__ __forceinline__ void merge_splits(const float* __restrict__ pacc,
                                             const float* __restrict__ pml,
                                             half_t* __restrict__ out, SlotOf slot_of, int gt,
                                             size_t out_base, int ns) {
  merge_splits_into<D, THREADS, COHERENT>(pacc, pml, slot_of, gt, ns, OutSink<D>{out, out_base});
}

// Block ids of one split: at most max_partition_per_4_waves(D) * NW / 4 tokens,
// starting anywhere inside a block of >= kMinBlockSize tokens.
template <int D, int NW>
constexpr int split_blocks_max() {
  return max_partition_per_4_waves(D) * NW / 4 / kMinBlockSize + 1;
}

// Row padding of the wave-merge slots: lane (r, g) touches row r, so rows
// D floats apart would put the 16 lanes of one g on the same LDS banks.
constexpr int kMergeRowPad = 4;
// Occupancy the decode kernels are built for: 2 waves per SIMD, so 8 waves
// (one 8-wave or two 4-wave work-groups) share a CU's 160 KB of LDS.
constexpr int kWavesPerCU = 8;
constexpr size_t kLdsPerCU = 160 * 1024 - 4096;   // (margin for allocation granularity)

template <int D, int NW>
struct alignas(16) DecodeSmem {   // (one column tile at a time)
  float a[NW][16][D + kMergeRowPad];   // each wave's accumulator: per head, per dim (+ pad)
  float m[NW][16];
  float l[NW][16];
  int blk[split_blocks_max<D, NW>()];     // the split's block ids
  int last;
};

// One split of one unit, processed by a whole work-group.
struct SplitWork {
  int seq, kvh, chunk, split;
  int ctx;         // context length (clamped)
  int partition;   // tokens per split
  int ns;          // splits of this unit
  size_t slot0;    // partial slot of split 0 of this unit
  int stride;      // partial slots between consecutive splits
};

// Where one decode call's caches live (the same for every wave).
struct CacheView {
  const uint8_t* kc;
  const uint8_t* vc;
  const float* ksc;   // INT8 only
  const float* vsc;
  int hkv;            // kv heads
  int bs;             // block size (a power of two)
  int num_blocks;     // valid block ids are [0, num_blocks)
};

// The work of one wave on one 32- or 64-token chunk of one (sequence, kv
// head) stream at a time: its K/V/scale loads, the QK product, the online
// softmax and the PV product, and the running state of its query heads.  CT:
// 16-head MFMA column tiles (1, or 2 for head tiles of 17..32 query heads:
// each K/V register load then feeds both tiles).  The decode kernels drive it
// with block ids from wherever they keep them (LDS for a split, registers
// for a stream); all positions are tokens of the stream.
//
// Token layout of a chunk starting at tok0, for lane (r = lane & 15, g = lane >> 4);
// the pair mapping:
//   K rows: token tok0 + 32p + 8(r>>2) + (r&3) feeds MFMA row r of pair p's first QK
//           MFMA, + 4 its second (W8: tokens tok0 + 16(r>>2) + 8p + 2(r&3) and + 1);
//   scores / V: the lane's 8 score tokens are tok0 + 32p + 8g .. +7 (W8: tok0 + 16g +
//           8p .. +7), exactly its P^T operand of PV, and its V rows are dims 16t + r;
// the group mapping (GM, below):
//   K rows: token tok0 + 16m + r feeds MFMA row r of group m's QK MFMA (m = 2p, 2p + 1:
//           pair p's first and second);
//   scores / V: the lane's 8 score tokens are tok0 + 32p + 4g .. +3 and tok0 + 32p +
//           16 + 4g .. +3.
// A token at or past t_end is read at token `fb` instead (a valid token of the
// same stream: its block id is looked up the same way) and masked.
template <int D, int CT, bool I8, bool GM = false>
struct DecodeWave {
  static_assert(D % 8 == 0 && D >= 8 && D <= 256, "head_dim: a multiple of 8 in [8, 256]");
  static_assert(CT == 1 || (CT == 2 && D <= 128), "two column tiles only for head_dim <= 128");
  static constexpr int KC = (D + 31) / 32;   // 32-dim k-chunks of one QK product
  static constexpr int NT = (D + 15) / 16;   // 16-dim output tiles of PV
  static constexpr int DG = D / 8;           // 8-dim groups of a K row
  // With head_dim % 32 != 0 the last k-chunk holds 8, 16 or 24 dims: its dim
  // groups 4(KC-1) + g with 4(KC-1) + g >= DG lie past the row.  Those lanes
  // load the row's last group instead (in bounds) and feed zeros to the MFMA;
  // their query operand is zero as well.
  static constexpr bool KPAD = (D % 32) != 0;
  // With head_dim % 16 == 8 the last output tile holds 8 dims: its V rows r
  // >= 8 lie past the row.  Those lanes load row r - 8 instead (in bounds);
  // the products land in accumulator rows 8..15 of the tile (lanes g >= 2),
  // which are never stored.
  static constexpr bool VPAD = (D % 16) != 0;
  // 32-token pairs per chunk: two, except with head_dim 256 (whose
  // accumulators are twice as large) and with two column tiles (whose query
  // operands, scores and accumulators are twice as many); either way the
  // registers of one wave stay within the 256 of two waves per SIMD.
  static constexpr int PAIRS = (D <= 128 && CT == 1) ? 2 : 1;
  static constexpr int IT = 32 * PAIRS;      // tokens per chunk
  static constexpr int ESZ = I8 ? 1 : 2;     // bytes per cache element
  using LVec = typename std::conditional<I8, uint2, uint4>::type;   // 8 elements
  // INT8 with head_dim <= 128 and one column tile uses 16-byte loads
  // throughout (W8): a K load holds one dim group of two adjacent tokens (t,
  // t + 1), which feed the same row of the two QK MFMAs of a pair, and a V
  // load holds 16 tokens of one dim, which feed both pairs.  Each lane loads
  // the scales of 4 tokens and the others reach the lanes that need them by
  // quad DPP broadcasts.
  static constexpr bool W8 = I8 && D <= 128 && CT == 1;
  // FP16 with head_dim > 128: the query operand is read from LDS at each QK
  // (its KC * 4 registers would not fit beside the accumulators and the K/V
  // rows in flight within 256 VGPRs; they spilled).  The work-group stages
  // the tile once (stage_query), rows of QROW halves.
  static constexpr bool QLDS = !I8 && D > 128;
  // GM, the group mapping (FP16, the grid kernels): MFMA row tile m of a
  // chunk is the 16-token group tok0 + 16m .. + 15, so lane (r, g) loads K
  // row r of its group (8 dims, 16 B) and eight lanes read one whole 128-B
  // line of a dim group, where the mapping above reads half lines (four
  // lanes).  After QK lane (r, g) holds tokens 4g .. 4g + 3 of each group,
  // so its V operand of pair p is tokens 4g .. 4g + 3 of groups 2p and 2p + 1
  // (two 8-byte loads, 512 contiguous bytes per instruction).  Every load of
  // a group half comes from one wave-uniform block.  On MI355X the read
  // stream of config 2 ran 2.6% faster this way (a third fewer L2 requests,
  // all of whole lines; one work-group pulled 24-29% more bandwidth), and
  // the decode 1.3% (config 2) and 1.2% (config 3 FP16) faster.  The grid
  // kernels use it for FP16 launches with non-temporal loads
  // (decode_kernel); the scheduled split-K kernels measured slower with it
  // (ragged 32/8 +0.9%) and keep the pair mapping of the token layout above,
  // as do the stream partition, INT8 and small launches.
  static_assert(!(GM && I8), "the group mapping is FP16 only");
  static constexpr int NG = 2 * PAIRS;   // 16-token groups per chunk
  static constexpr int QROW = D + 8;   // (row stride 16 B off a bank multiple)

  // Block ids of a lane's K rows and V rows (W8: one 16-token group each).
  struct Blocks {
    int kb[PAIRS];
    int vb[PAIRS];
    // GM: blocks of tokens 16m and 16m + 8 of each group m (wave-uniform;
    // equal unless block_size is 8)
    int gb[2 * NG];
  };
  // W8: the scales of the 4 tokens tok0 + 16g + 4(r & 3) + i and the valid
  // tokens among the lane's 8 of each pair.  They are loaded one chunk
  // ahead, with the K rows, so the softmax does not wait for the V rows (the
  // memory counter completes in order): `wa` holds the next chunk's, and
  // each chunk copies them out before loading the following ones.
  struct W8Buf {
    float4 ks4, vs4;
    int nvalid[PAIRS];
  };

  int r, g;
  // Running (max, sum) of query head r + 16 ct, its accumulator (dims 16t +
  // 4g + e), and the exponent the INT8 weights are scaled by (FP16: 14).
  float m_run[CT], l_part[CT];
  f4_t acc[CT][NT];
  int e_cur;
  // Query operand: lane (r, g) holds q[head r + 16 ct][32kk + 8g .. +7]
  // (QLDS: read from qs instead); INT8: the K bias 1152 * sum(q) per head.
  h8_t qreg[CT][KC];
  const half_t* qs;
  float qbias[CT];
  // Loads of the chunk in flight.
  LVec kx[PAIRS][KC], ky[PAIRS][KC], vr[PAIRS][NT];
  float ksv[PAIRS][8], vsv[PAIRS][8];   // INT8 scales of this lane's 8 tokens
  int nvalid[PAIRS];                    // valid tokens among this lane's 8
  int nv2[PAIRS][2];                    // GM: valid tokens among its 4 of group 2p + h
  uint4 kw[PAIRS][KC];                  // W8: K rows of tokens (t, t + 1)
  uint4 vw[NT];                         // W8: V rows of 16 tokens
  W8Buf wa;

  __device__ __forceinline__ void init(int lane) {
    r = lane & 15;
    g = lane >> 4;
    reset();
  }

  // Empty state: no token seen yet.
  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      m_run[ct] = kNegInf;
      l_part[ct] = 0.f;
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[ct][t] = (f4_t){0.f, 0.f, 0.f, 0.f};
    }
    e_cur = I8 ? 0 : 14;
  }

  // The query operand of the gt heads starting at q row `row0` (sequence *
  // num_heads + first head).
  __device__ __forceinline__ void load_q(const half_t* __restrict__ q, size_t row0, int gt) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const bool hv = r + 16 * ct < gt;
      const half_t* qrow = q + (row0 + (hv ? r + 16 * ct : 0)) * D + 8 * g;
#pragma unroll
      for (int kk = 0; kk < KC; ++kk) {
        const bool dv = !KPAD || kk < KC - 1 || 4 * kk + g < DG;
        const uint4 v = (hv && dv) ? *reinterpret_cast<const uint4*>(qrow + 32 * kk)
                                   : make_uint4(0, 0, 0, 0);
        qreg[ct][kk] = __builtin_bit_cast(h8_t, v);
      }
    }
  }

  // QLDS: the query operand of k-chunk kk from the staged tile.  The padding
  // lanes of a short last chunk would read past the row's D halves (the row's
  // unwritten pad, or the next row); they take zeros, since whatever bits lie
  // there could be an fp16 NaN or infinity, and 0 * NaN poisons the MFMA sum.
  __device__ __forceinline__ h8_t q_operand(int ct, int kk) const {
    if constexpr (QLDS) {
      if (KPAD && kk == KC - 1 && 4 * kk + g >= DG) return (h8_t){};
      return *reinterpret_cast<const h8_t*>(qs + r * QROW + 32 * kk + 8 * g);
    } else {
      return qreg[ct][kk];
    }
  }

  // V row of output tile t that lane (r, g) loads, relative to dim r: 16t,
  // or for the padding rows of a half last tile 16t - 8 (see VPAD).
  __device__ __forceinline__ int vdim(int t) const {
    return (VPAD && t == NT - 1 && r >= 8) ? 16 * t - 8 : 16 * t;
  }

  // INT8: the K bias of each head, once the query operand has arrived.
  __device__ __forceinline__ void compute_qbias() {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      qbias[ct] = 0.f;
      if constexpr (I8) {
        float s = 0.f;
#pragma unroll
        for (int kk = 0; kk < KC; ++kk) {
          const uint4 v = __builtin_bit_cast(uint4, qreg[ct][kk]);
          s = dot2(v.x, 0x3C003C00u, s);
          s = dot2(v.y, 0x3C003C00u, s);
          s = dot2(v.z, 0x3C003C00u, s);
          s = dot2(v.w, 0x3C003C00u, s);
        }
        qbias[ct] = 1152.f * head_sum(s);
      }
    }
  }

  // The tokens whose block ids this lane's loads of the chunk at tok0 need
  // (out-of-range tokens replaced by fb): kt for the K rows, vt for the V rows.
  __device__ __forceinline__ void block_tokens(int tok0, int t_end, int fb, int (&kt)[PAIRS],
                                               int (&vt)[PAIRS]) const {
    if constexpr (W8) {
      // K rows of lane (r, g) lie in the 16-token group tok0 + 16(r >> 2), its V
      // rows and scales in tok0 + 16g; a group never straddles a block
      // (block_size is a multiple of 16).
      const int kg = tok0 + 16 * (r >> 2);
      const int tg = tok0 + 16 * g;
      kt[0] = kg < t_end ? kg : fb;
      vt[0] = tg < t_end ? tg : fb;
      return;
    }
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
      const int kg = tok0 + 32 * p + 8 * (r >> 2);
      const int tg = tok0 + 32 * p + 8 * g;
      kt[p] = kg < t_end ? kg : fb;
      vt[p] = tg < t_end ? tg : fb;
    }
  }

  // Dim-group offset (relative to the lane's group g) of k-chunk kk's K row
  // load: 4 kk, or for the padding lanes of a 16-dim last chunk the row's
  // last group.
  __device__ __forceinline__ int kgroup(int kk) const {
    return (!KPAD || 4 * kk + g < DG) ? 4 * kk : DG - 1 - g;
  }

  // K rows of kv head kvh.
  template <bool KNT>
  __device__ __forceinline__ void issue_k(const CacheView& cv, int kvh, int tok0, int t_end, int fb,
                                          const Blocks& b) {
    if constexpr (W8) {
      // Row r of pair p: tokens tok0 + 16(r >> 2) + 8p + 2(r & 3) and + 1.
      const int kg = tok0 + 16 * (r >> 2);
      const int kgc = kg < t_end ? kg : fb;
      const int kb = (unsigned)b.kb[0] < (unsigned)cv.num_blocks ? b.kb[0] : 0;
      const uint8_t* kp = cv.kc + ((((size_t)kb * cv.hkv + kvh) * (D / 8) + g) * cv.bs +
                                   (kgc & (cv.bs - 1)) + 2 * (r & 3)) * 8;
#pragma unroll
      for (int p = 0; p < PAIRS; ++p)
#pragma unroll
        for (int kk = 0; kk < KC; ++kk)
          kw[p][kk] = load_tile<uint4, KNT>(kp + (size_t)kgroup(kk) * cv.bs * 8 + 64 * p);
      return;
    }
    if constexpr (GM) {
      // Row r of group m: token 16m + r (a group past the end reads the
      // first group of the split instead, masked).
#pragma unroll
      for (int m = 0; m < NG; ++m) {
        const int g0 = tok0 + 16 * m;
        const int gs = g0 < t_end ? g0 : fb;
        const int bk = r < 8 ? b.gb[2 * m] : b.gb[2 * m + 1];
        const int kb = (unsigned)bk < (unsigned)cv.num_blocks ? bk : 0;
        const uint8_t* kp = cv.kc + ((((size_t)kb * cv.hkv + kvh) * (D / 8) + g) * cv.bs +
                                     ((gs + r) & (cv.bs - 1))) * 16;
#pragma unroll
        for (int kk = 0; kk < KC; ++kk) {
          const LVec x = load_tile<LVec, KNT>(kp + (size_t)kgroup(kk) * cv.bs * 16);
          if (m & 1) ky[m >> 1][kk] = x;
          else kx[m >> 1][kk] = x;
        }
      }
      return;
    }
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
      const int kg = tok0 + 32 * p + 8 * (r >> 2);
      const int kgc = kg < t_end ? kg : fb;
      const int kb = (unsigned)b.kb[p] < (unsigned)cv.num_blocks ? b.kb[p] : 0;
      const int koff = (kgc & (cv.bs - 1)) + (r & 3);
      const uint8_t* kp =
          cv.kc + ((((size_t)kb * cv.hkv + kvh) * (D / 8) + g) * cv.bs + koff) * 8 * ESZ;
#pragma unroll
      for (int kk = 0; kk < KC; ++kk) {
        const uint8_t* p0 = kp + (size_t)kgroup(kk) * cv.bs * 8 * ESZ;
        kx[p][kk] = load_tile<LVec, KNT>(p0);
        ky[p][kk] = load_tile<LVec, KNT>(p0 + 4 * 8 * ESZ);
      }
    }
  }

  // W8: the scales and valid counts of a chunk (see W8Buf).
  __device__ __forceinline__ void issue_scales(const CacheView& cv, int kvh, int tok0, int t_end,
                                               int fb, const Blocks& b, W8Buf& B) const {
    const int tg = tok0 + 16 * g;
    const int tgc = tg < t_end ? tg : fb;
    const bool vok = (unsigned)b.vb[0] < (unsigned)cv.num_blocks;
    const int vb = vok ? b.vb[0] : 0;
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
      const int t0 = tg + 8 * p;
      B.nvalid[p] = (vok && t0 < t_end) ? min(8, t_end - t0) : 0;
    }
    const size_t slot = ((size_t)vb * cv.hkv + kvh) * cv.bs + (tgc & (cv.bs - 1)) + 4 * (r & 3);
    // (plain loads: a scale line holds several kv heads' scales)
    B.ks4 = *reinterpret_cast<const float4*>(cv.ksc + slot);
    B.vs4 = *reinterpret_cast<const float4*>(cv.vsc + slot);
  }

  // Where a chunk's V rows (and INT8 scales) are, once its block ids are
  // known: lets a caller reuse the block-id registers before issuing them.
  struct VPlan {
    const uint8_t* vp[PAIRS];   // the lane's first V row of each pair
    size_t slot[PAIRS];         // its tokens' first scale (INT8, not W8)
    int nvalid[PAIRS];          // valid tokens among its 8 of each pair (not W8)
    const uint8_t* vp2[PAIRS][2];   // GM: its first V row in groups 2p and 2p + 1
    int nv2[PAIRS][2];              // GM: valid tokens among its 4 of each
  };

  __device__ __forceinline__ VPlan plan_v(const CacheView& cv, int kvh, int tok0, int t_end,
                                          int fb, const Blocks& b) const {
    VPlan v;
    if constexpr (W8) {
      // V rows: dim 16t + r, tokens tok0 + 16g .. + 15 (pair p uses 8p .. 8p + 7).
      const int tg = tok0 + 16 * g;
      const int tgc = tg < t_end ? tg : fb;
      const int vb = (unsigned)b.vb[0] < (unsigned)cv.num_blocks ? b.vb[0] : 0;
      v.vp[0] = cv.vc + (((size_t)vb * cv.hkv + kvh) * D + r) * cv.bs + (tgc & (cv.bs - 1));
      return v;
    }
    if constexpr (GM) {
      // V rows: dim 16t + r, tokens 16m + 4g .. + 3 of groups m = 2p, 2p + 1.
#pragma unroll
      for (int p = 0; p < PAIRS; ++p)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int m = 2 * p + h;
          const int g0 = tok0 + 16 * m;
          const bool gin = g0 < t_end;
          const int gs = gin ? g0 : fb;
          const int bk = g < 2 ? b.gb[2 * m] : b.gb[2 * m + 1];
          const bool vok = (unsigned)bk < (unsigned)cv.num_blocks;
          const int vb = vok ? bk : 0;
          const int nv = t_end - (g0 + 4 * g);
          v.nv2[p][h] = (gin && vok) ? (nv < 0 ? 0 : (nv > 4 ? 4 : nv)) : 0;
          v.vp2[p][h] = cv.vc + ((((size_t)vb * cv.hkv + kvh) * D + r) * cv.bs +
                                 ((gs + 4 * g) & (cv.bs - 1))) * 2;
        }
      return v;
    }
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
      const int tg = tok0 + 32 * p + 8 * g;
      const bool tin = tg < t_end;
      const int tgc = tin ? tg : fb;
      const bool vok = (unsigned)b.vb[p] < (unsigned)cv.num_blocks;
      const int vb = vok ? b.vb[p] : 0;
      const int voff = tgc & (cv.bs - 1);
      v.nvalid[p] = (tin && vok) ? min(8, t_end - tg) : 0;
      v.slot[p] = ((size_t)vb * cv.hkv + kvh) * cv.bs + voff;
      v.vp[p] = cv.vc + ((((size_t)vb * cv.hkv + kvh) * D + r) * cv.bs + voff) * ESZ;
    }
    return v;
  }

  // V rows (dims 16t + r) and the lane's score tokens tok0 + 32p + 8g .. +7,
  // with their INT8 scales (not W8, which loads them with the K rows).
  template <bool NTL>
  __device__ __forceinline__ void issue_v(const CacheView& cv, const VPlan& v) {
    if constexpr (W8) {
#pragma unroll
      for (int t = 0; t < NT; ++t) vw[t] = load_tile<uint4, NTL>(v.vp[0] + (size_t)vdim(t) * cv.bs);
      return;
    }
    if constexpr (GM) {
#pragma unroll
      for (int p = 0; p < PAIRS; ++p) {
        nv2[p][0] = v.nv2[p][0];
        nv2[p][1] = v.nv2[p][1];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const uint2 lo = load_tile<uint2, NTL>(v.vp2[p][0] + (size_t)vdim(t) * cv.bs * 2);
          const uint2 hi = load_tile<uint2, NTL>(v.vp2[p][1] + (size_t)vdim(t) * cv.bs * 2);
          vr[p][t] = make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
      }
      return;
    }
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
      nvalid[p] = v.nvalid[p];
#pragma unroll
      for (int t = 0; t < NT; ++t)
        vr[p][t] = load_tile<LVec, NTL>(v.vp[p] + (size_t)vdim(t) * cv.bs * ESZ);
      if constexpr (I8) {
        const float4 a0 = *reinterpret_cast<const float4*>(cv.ksc + v.slot[p]);
        const float4 a1 = *reinterpret_cast<const float4*>(cv.ksc + v.slot[p] + 4);
        const float4 b0 = *reinterpret_cast<const float4*>(cv.vsc + v.slot[p]);
        const float4 b1 = *reinterpret_cast<const float4*>(cv.vsc + v.slot[p] + 4);
        ksv[p][0] = a0.x; ksv[p][1] = a0.y; ksv[p][2] = a0.z; ksv[p][3] = a0.w;
        ksv[p][4] = a1.x; ksv[p][5] = a1.y; ksv[p][6] = a1.z; ksv[p][7] = a1.w;
        vsv[p][0] = b0.x; vsv[p][1] = b0.y; vsv[p][2] = b0.z; vsv[p][3] = b0.w;
        vsv[p][4] = b1.x; vsv[p][5] = b1.y; vsv[p][6] = b1.z; vsv[p][7] = b1.w;
      }
    }
  }

  template <bool NTL>
  __device__ __forceinline__ void issue_v(const CacheView& cv, int kvh, int tok0, int t_end,
                                          int fb, const Blocks& b) {
    issue_v<NTL>(cv, plan_v(cv, kvh, tok0, t_end, fb, b));
  }

  // Tokens past the end or in invalid blocks exist only in the last chunk of
  // a stream or split (or with a corrupt block table).
  __device__ __forceinline__ bool mask_needed(const W8Buf& B) const {
    bool short_lane = false;
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
      if constexpr (W8) short_lane = short_lane || B.nvalid[p] < 8;
      else if constexpr (GM) short_lane = short_lane || nv2[p][0] < 4 || nv2[p][1] < 4;
      else short_lane = short_lane || nvalid[p] < 8;
    }
    return __builtin_amdgcn_ballot_w64(short_lane) != 0;
  }

  // ---- QK: scores of tokens tok0 + 32p + 8g + j for head r + 16 ct
  // (W8: tok0 + 16g + 8p + j); each converted K operand feeds every tile.
  __device__ __forceinline__ void qk(float (&s)[CT][PAIRS][8]) const {
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
      f4_t sx[CT], sy[CT];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        sx[ct] = (f4_t){0.f, 0.f, 0.f, 0.f};
        sy[ct] = (f4_t){0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int kk = 0; kk < KC; ++kk) {
        h8_t ax, ay;
        if constexpr (W8) {
          ax = i8x8_biased(make_uint2(kw[p][kk].x, kw[p][kk].y));   // token T
          ay = i8x8_biased(make_uint2(kw[p][kk].z, kw[p][kk].w));   // token T + 1
        } else if constexpr (I8) {
          ax = i8x8_biased(kx[p][kk]);
          ay = i8x8_biased(ky[p][kk]);
        } else {
          ax = __builtin_bit_cast(h8_t, kx[p][kk]);
          ay = __builtin_bit_cast(h8_t, ky[p][kk]);
        }
        if (KPAD && kk == KC - 1 && 4 * kk + g >= DG) {
          ax = (h8_t){};   // padding lanes of the last k-chunk (their q is zero too)
          ay = (h8_t){};
        }
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const h8_t qo = q_operand(ct, kk);
          sx[ct] = mfma16(ax, qo, sx[ct]);
          sy[ct] = mfma16(ay, qo, sy[ct]);
        }
      }
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (W8) {
            // rows 4g + e: tokens tok0 + 16g + 8p + 2e (sx) and + 1 (sy)
            s[ct][p][2 * e] = sx[ct][e];
            s[ct][p][2 * e + 1] = sy[ct][e];
          } else {
            s[ct][p][e] = sx[ct][e];
            s[ct][p][4 + e] = sy[ct][e];
          }
        }
    }
  }

  // ---- online softmax (lane-local except the per-head max) and PV.  c:
  // the softmax scale times log2(e); B: the chunk's W8 scales.
  __device__ __forceinline__ void softmax_pv(float (&s)[CT][PAIRS][8], bool need_mask, W8Buf& B,
                                             float c) {
    // W8: this lane's 4 scales; token 16g + 8p + j of the lane's row is held
    // by quad position 2p + (j >> 2), element j & 3.  The K scales carry the
    // softmax scale c before they are broadcast (the same products, 4 instead
    // of 16 multiplies).
    float ksa[4] = {B.ks4.x * c, B.ks4.y * c, B.ks4.z * c, B.ks4.w * c};
    float vsa[4] = {B.vs4.x, B.vs4.y, B.vs4.z, B.vs4.w};
    auto nval = [&](int p) {
      if constexpr (W8) return B.nvalid[p];
      else return nvalid[p];
    };
    if constexpr (W8) {
      if (need_mask) {
        // the row's valid tokens are its first nvalid[0] + nvalid[1]
        const int n16 = B.nvalid[0] + B.nvalid[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) vsa[i] = 4 * (r & 3) + i < n16 ? vsa[i] : 0.f;
      }
#pragma unroll
      for (int p = 0; p < PAIRS; ++p)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float ksj = quad_bcast(ksa[j & 3], 2 * p + (j >> 2));
          s[0][p][j] = (s[0][p][j] - qbias[0]) * ksj;
        }
    } else {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int p = 0; p < PAIRS; ++p)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            float v;
            if constexpr (I8) v = (s[ct][p][j] - qbias[ct]) * (ksv[p][j] * c);
            else v = s[ct][p][j] * c;
            s[ct][p][j] = v;
          }
    }
    if (need_mask) {
#pragma unroll
      for (int p = 0; p < PAIRS; ++p)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) {
            bool ok;
            if constexpr (GM) ok = (j & 3) < nv2[p][j >> 2];   // group 2p + (j >> 2)
            else ok = j < nval(p);
            s[ct][p][j] = ok ? s[ct][p][j] : kNegInf;
          }
          if constexpr (I8 && !W8) vsv[p][j] = j < nval(p) ? vsv[p][j] : 0.f;
        }
    }
    float m_use[CT], alpha_m[CT], alpha_acc[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      float mloc = kNegInf;
#pragma unroll
      for (int p = 0; p < PAIRS; ++p)
#pragma unroll
        for (int j = 0; j < 8; ++j) mloc = fmaxf(mloc, s[ct][p][j]);
      const float m_new = fmaxf(m_run[ct], head_max(mloc));
      m_use[ct] = m_new == kNegInf ? 0.f : m_new;
      alpha_m[ct] = exp2f_fast(m_run[ct] - m_use[ct]);   // rescales l
      alpha_acc[ct] = alpha_m[ct];                       // rescales acc (incl. weight exponent)
      m_run[ct] = m_new;
    }
    float wsc;
    if constexpr (I8) {
      float msv = 0.f;
      if constexpr (W8) {
        // The 64 tokens' scales are spread over the quads of a row and the 4 rows.
        msv = fmaxf(fmaxf(vsa[0], vsa[1]), fmaxf(vsa[2], vsa[3]));
        msv = fmaxf(msv, dpp_mov<kQuadXor1>(msv));
        msv = fmaxf(msv, dpp_mov<kQuadXor2>(msv));
      } else {
#pragma unroll
        for (int p = 0; p < PAIRS; ++p)
#pragma unroll
          for (int j = 0; j < 8; ++j) msv = fmaxf(msv, vsv[p][j]);
      }
      // Every head's lanes see the same tokens, so this max is wave-uniform.
      msv = bitsf(__builtin_amdgcn_readfirstlane(fbits(head_max(msv))));
      // Keep the weight exponent while the largest weight stays in [2^12, 2^15);
      // it is shared by every head (the scales belong to the tokens).
      const float top = __builtin_amdgcn_ldexpf(msv, e_cur);
      if (msv > 0.f && (top >= 32768.f || top < 4096.f)) {
        int e_new = 15 - __builtin_amdgcn_frexp_expf(msv);
        e_new = e_new < 0 ? 0 : (e_new > 30 ? 30 : e_new);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
          alpha_acc[ct] = __builtin_amdgcn_ldexpf(alpha_m[ct], e_new - e_cur);
        e_cur = e_new;
      }
      wsc = __builtin_amdgcn_ldexpf(1.f, e_cur);
    } else {
      wsc = 16384.f;
    }
    // W8: the V scales carry the weight scale 2^e before they are broadcast
    // (exact: a power of two; weights too small for the product to stay
    // normal round to an fp16 zero either way).
    if constexpr (W8) {
#pragma unroll
      for (int i = 0; i < 4; ++i) vsa[i] *= wsc;
    }
    h8_t pb[CT][PAIRS];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      float lsum = 0.f;
#pragma unroll
      for (int p = 0; p < PAIRS; ++p) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float pj = exp2f_fast(s[ct][p][j] - m_use[ct]);
          lsum += pj;
          float wj;
          if constexpr (W8) wj = pj * quad_bcast(vsa[j & 3], 2 * p + (j >> 2));
          else if constexpr (I8) wj = pj * vsv[p][j] * wsc;
          else wj = pj * wsc;
          pb[ct][p][j] = (half_t)wj;
        }
      }
      l_part[ct] = l_part[ct] * alpha_m[ct] + lsum;
      if (__builtin_amdgcn_ballot_w64(alpha_acc[ct] != 1.f) != 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[ct][t] *= alpha_acc[ct];
      }
    }

    // ---- PV: each converted V operand feeds every column tile.  INT8: V
    // enters as 1152 + v (its conversion without an unbias step per
    // element); ws sums each head's weights of this chunk (an MFMA with a ones
    // operand: every element of lane (r, g) holds head r's sum), and the
    // chunk's 1152 * sum(w) comes off after its products, so the accumulator
    // carries no bias from one chunk to the next.
    [[maybe_unused]] f4_t ws[CT];
    if constexpr (I8) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) ws[ct] = (f4_t){0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
      if constexpr (I8) {
        const h8_t ones = {1.f16, 1.f16, 1.f16, 1.f16, 1.f16, 1.f16, 1.f16, 1.f16};
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) ws[ct] = mfma16(ones, pb[ct][p], ws[ct]);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        h8_t av;
        if constexpr (W8) {
          av = i8x8_biased(p == 0 ? make_uint2(vw[t].x, vw[t].y) : make_uint2(vw[t].z, vw[t].w));
        } else if constexpr (I8) {
          av = i8x8_biased(vr[p][t]);
        } else {
          uint4 v = vr[p][t];
          if constexpr (GM) {
            if (need_mask) {   // each half of the row keeps its group's valid tokens
              const uint4 lo = keep_first(make_uint4(v.x, v.y, 0, 0), nv2[p][0]);
              const uint4 hi = keep_first(make_uint4(v.z, v.w, 0, 0), nv2[p][1]);
              v = make_uint4(lo.x, lo.y, hi.x, hi.y);
            }
          } else if (need_mask) {
            v = keep_first(v, nval(p));
          }
          av = __builtin_bit_cast(h8_t, v);
        }
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[ct][t] = mfma16(av, pb[ct][p], acc[ct][t]);
      }
    }
    if constexpr (I8) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const float b = 1152.f * ws[ct][0];
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[ct][t] -= b;
      }
    }
  }

  // The wave's state of column tile ct into the merge slots of LDS: (max,
  // sum) and the accumulator of head r (the tile's heads below nh).
  template <typename Smem>
  __device__ __forceinline__ void store_state(Smem& sm, int w, int ct, int nh) const {
    if (r >= nh) return;
    const float l_run = head_sum(l_part[ct]);
    const float unscale = __builtin_amdgcn_ldexpf(1.f, -e_cur);
    if (g == 0) {
      sm.m[w][r] = m_run[ct];
      sm.l[w][r] = l_run;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (VPAD && t == NT - 1 && g >= 2) continue;   // dims past the row (see VPAD)
      *reinterpret_cast<f4_t*>(&sm.a[w][r][16 * t + 4 * g]) = acc[ct][t] * unscale;
    }
  }
};

// The query tile of one head chunk (q rows row0 .. row0 + gt - 1, zeros for
// the tile's other rows) for waves that read their query operand from LDS
// (DecodeWave::QLDS): every thread of the work-group loads 16-byte pieces
// (load, issued before the context length is known) and stores them into
// rows of D + 8 halves (store) over the wave-merge slots, which hold nothing
// between a work item's start and its first wave-state store.
template <int D, int NW>
struct QueryStage {
  static constexpr int QROW = D + 8;
  static constexpr int PIECES = 16 * D / 8;
  static constexpr int N = (PIECES + NW * kWave - 1) / (NW * kWave);   // pieces per thread
  uint4 v[N];

  __device__ __forceinline__ void load(const half_t* __restrict__ q, size_t row0, int gt, int tid) {
#pragma unroll
    for (int k = 0; k < N; ++k) {
      const int i = tid + k * NW * kWave;
      const int row = i / (D / 8), cg = i % (D / 8);
      v[k] = (i < PIECES && row < gt)
                 ? *reinterpret_cast<const uint4*>(q + (row0 + row) * D + 8 * cg)
                 : make_uint4(0, 0, 0, 0);
    }
  }

  __device__ __forceinline__ void store(half_t* qs, int tid) const {
#pragma unroll
    for (int k = 0; k < N; ++k) {
      const int i = tid + k * NW * kWave;
      if (i < PIECES) *reinterpret_cast<uint4*>(qs + (i / (D / 8)) * QROW + 8 * (i % (D / 8))) = v[k];
    }
  }
};

// Where QLDS waves find the staged query tile: the start of the wave-merge slots.
template <typename Smem>
__device__ __forceinline__ half_t* query_stage_lds(Smem& sm) {
  static_assert(16 * (sizeof(sm.a[0][0]) / sizeof(float) + 8) * sizeof(half_t) <= sizeof(sm.a),
                "the query tile fits in the wave-merge slots");
  return reinterpret_cast<half_t*>(&sm.a[0][0][0]);
}

// The NW wave states of item (head hh of a column tile, dims 4c .. 4c + 3) in
// LDS, merged: accumulator relative to the max, the max and the sum.
template <int D, int NW, typename Smem>
__device__ __forceinline__ void wave_state_item(const Smem& sm, int hh, int c, f4_t& A, float& M,
                                                float& L) {
  float mw[NW];
  M = kNegInf;
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    mw[v] = sm.m[v][hh];
    M = fmaxf(M, mw[v]);
  }
  A = (f4_t){0.f, 0.f, 0.f, 0.f};
  L = 0.f;
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    const float f = mw[v] == kNegInf ? 0.f : exp2f_fast(mw[v] - M);
    L += sm.l[v][hh] * f;
    A += *reinterpret_cast<const f4_t*>(&sm.a[v][hh][4 * c]) * f;
  }
}

// One item's partial (acc, then (max, sum) per head) through the buffer
// resources racc / rml (device-coherent, write-through stores when COHERENT).
template <int D, bool COHERENT>
__device__ __forceinline__ void store_partial_item(__amdgpu_buffer_rsrc_t racc,
                                                   __amdgpu_buffer_rsrc_t rml, int h, int c,
                                                   f4_t A, float M, float L) {
  constexpr int POL = COHERENT ? kPolicyDevice : 0;
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4_t, A), racc, (h * D + 4 * c) * 4, 0,
                                         POL);
  if (c == 0) {
    const f2_t ml = {M, L};
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2_t, ml), rml, h * 8, 0, POL);
  }
}

// The NW wave states of column tile ct in LDS, merged per (head, 4-dim
// chunk) item by the work-group's threads: the normalised fp16 output when
// `final_out`, else a partial.
template <int D, int NW, bool COHERENT, typename Smem>
__device__ __forceinline__ void merge_wave_states(const Smem& sm, int ct, int nh,
                                                  int tid, bool final_out,
                                                  half_t* __restrict__ out, size_t out_base,
                                                  __amdgpu_buffer_rsrc_t racc,
                                                  __amdgpu_buffer_rsrc_t rml) {
  constexpr int CH = D / 4;
  for (int i = tid; i < nh * CH; i += NW * kWave) {
    const int hh = i / CH, c = i - hh * CH;
    const int h = 16 * ct + hh;             // head within the unit's tile
    f4_t A;
    float M, L;
    wave_state_item<D, NW>(sm, hh, c, A, M, L);
    if (final_out) write_out_item<D>(out, out_base, h, c, L, A);
    else store_partial_item<D, COHERENT>(racc, rml, h, c, A, M, L);
  }
}

// Two-level split merge of the single launches (see decode_split): units of
// at least kMerge2MinSplits splits whose partials hold at least
// kMerge2MinFloats accumulator values (256 KB) fold in kMergeGroups groups
// first.  Smaller merges are faster in one level: the second level adds an
// acknowledged store and an arrival to the end of the launch (8 sequences of
// 4096 tokens at 8/1 heads, 32 splits of 8 heads: 12.2 -> 12.5 us in two).
constexpr int kMerge2MinSplits = 12;
constexpr int kMerge2MinFloats = 64 * 1024;
static_assert(kMerge2MinSplits >= 2 * kMergeGroups, "every group holds two splits or more");
// First split of merge group gi of a unit of ns splits (gi = kMergeGroups: ns);
// split sp belongs to group sp * kMergeGroups / ns.
__device__ __forceinline__ int merge_group_first(int gi, int ns) {
  return (gi * ns + kMergeGroups - 1) / kMergeGroups;
}

// Waits until this thread's stores are acknowledged, then counts the
// work-group's arrival at *c (thread 0).  True, in every thread, for the
// work-group that arrives last of n.
template <typename Smem>
__device__ __forceinline__ bool arrive_last(Smem& sm, uint32_t* c, int n) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sm.last = prev == (uint32_t)(n - 1);
  }
  __syncthreads();
  return sm.last;
}

// The decode of one split of one unit by a whole work-group.  FUSED:
// a unit with one split writes its output here; partials are written
// device-coherent and the last work-group of the unit merges them (single
// launch).  Otherwise every split writes a partial for the split-K reduce.
// `after_issue` runs in every wave once the wave's first K/V loads are issued
// (the scheduled kernel claims its next item there, so that no wait for this
// split's data also waits for the claim).
// `resolve(ctx, ns)` supplies the context length and split count once the
// split's block-id loads are in flight (the grid kernel reads them from
// memory then) and returns false when the split holds no tokens.
template <int D, int NW, int CT, bool I8, bool FUSED, bool NTL, bool KNT, bool GM,
          typename Resolve, typename AfterIssue>
__device__ __forceinline__ void decode_split(
    const half_t* __restrict__ q, const uint8_t* __restrict__ kc, const uint8_t* __restrict__ vc,
    const float* __restrict__ ksc, const float* __restrict__ vsc, const int* __restrict__ bt,
    half_t* __restrict__ out, float* __restrict__ pacc, float* __restrict__ pml,
    uint32_t* __restrict__ cnt, const DecodeShape& sh, SplitWork wk,
    DecodeSmem<D, NW>& sm, Resolve&& resolve, AfterIssue&& after_issue) {
  using Wave = DecodeWave<D, CT, I8, GM>;
  using Blocks = typename Wave::Blocks;
  using W8Buf = typename Wave::W8Buf;
  constexpr int PAIRS = Wave::PAIRS;
  constexpr int IT = Wave::IT;
  constexpr bool W8 = Wave::W8;

  const int seq = wk.seq, kvh = wk.kvh, chunk = wk.chunk, split = wk.split;
  const int gt = sh.head_tile;
  const int t_begin = split * wk.partition;

  // The thread index is made opaque here so that no lane-dependent address
  // math is hoisted out of a caller's loop over splits (it would stay live,
  // in registers, across the whole split).
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int head0 = kvh * sh.group + chunk * gt;
  const int unit = (seq * sh.num_kv_heads + kvh) * sh.nchunk + chunk;
  const int* btrow = bt + (size_t)seq * sh.max_blocks;
  const int bsl = sh.bs_log2;
  const CacheView cv{kc, vc, ksc, vsc, sh.num_kv_heads, sh.block_size, sh.num_blocks};
  const float c = sh.scale_log2;

  Wave dw;
  dw.init(lane);

  // ---- the split's block ids, staged once in LDS.  Their loads cover every
  // block the split can touch and are issued before the context length is
  // known, so the two memory round trips overlap.
  const int b_first = t_begin >> bsl;
  constexpr int kStageRegs = (split_blocks_max<D, NW>() + NW * kWave - 1) / (NW * kWave);
  int nstage = min(((t_begin + wk.partition - 1) >> bsl) - b_first + 1, sh.max_blocks - b_first);
  nstage = nstage < 0 ? 0 : min(nstage, split_blocks_max<D, NW>());
  int staged[kStageRegs];
#pragma unroll
  for (int k = 0; k < kStageRegs; ++k) {
    const int i = tid + k * NW * kWave;
    staged[k] = i < nstage ? btrow[b_first + i] : 0;
  }
  [[maybe_unused]] QueryStage<D, NW> qst;
  if constexpr (Wave::QLDS) {
    qst.load(q, (size_t)seq * sh.num_heads + head0, gt, tid);
    dw.qs = query_stage_lds(sm);
  } else {
    dw.load_q(q, (size_t)seq * sh.num_heads + head0, gt);
  }
  dw.compute_qbias();

  if (!resolve(wk.ctx, wk.ns)) return;   // work-group uniform, before any barrier
  const int ns_eff = wk.ns;
  const int t_end = min(wk.ctx, t_begin + wk.partition);
  const int n_it = t_end > t_begin ? (t_end - t_begin + IT - 1) / IT : 0;
  const int nblk = t_end > t_begin ? min(((t_end - 1) >> bsl) - b_first + 1, nstage) : 0;
  if constexpr (Wave::QLDS) {
    lds_barrier();   // a previous work item's wave merge has read the slots
    qst.store(query_stage_lds(sm), tid);
  }
#pragma unroll
  for (int k = 0; k < kStageRegs; ++k) {
    const int i = tid + k * NW * kWave;
    if (i < nstage) sm.blk[i] = staged[k];
  }
  lds_barrier();   // the block ids above are visible; no wait for the query loads

  // ---- software-pipelined token loop: wave w takes chunks w, w + NW, ... of
  // the split.  Once the K rows of its current chunk have fed the QK MFMAs it
  // issues the K rows of its next chunk; the V rows (plus INT8 scales) follow
  // once the PV MFMAs have consumed the V registers.  HBM traffic of the next
  // chunk overlaps this chunk's math.
  auto load_blocks = [&](int it_, Blocks& b) {
    if constexpr (GM) {
      // the blocks of tokens 16m and 16m + 8 of each group (a group past the
      // end: of the split's first group)
      const int tok0 = t_begin + it_ * IT;
#pragma unroll
      for (int m = 0; m < Wave::NG; ++m) {
        const int g0 = tok0 + 16 * m;
        const int gs = g0 < t_end ? g0 : t_begin;
        const int lo = (gs >> bsl) - b_first, hi = ((gs + 8) >> bsl) - b_first;
        b.gb[2 * m] = __builtin_amdgcn_readfirstlane(sm.blk[lo < nblk ? lo : 0]);
        b.gb[2 * m + 1] = __builtin_amdgcn_readfirstlane(sm.blk[hi < nblk ? hi : 0]);
      }
      return;
    }
    int kt[PAIRS], vt[PAIRS];
    dw.block_tokens(t_begin + it_ * IT, t_end, t_begin, kt, vt);
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
      const int ki = (kt[p] >> bsl) - b_first;
      const int vi = (vt[p] >> bsl) - b_first;
      b.kb[p] = sm.blk[ki < nblk ? ki : 0];
      b.vb[p] = sm.blk[vi < nblk ? vi : 0];
    }
  };

  // The loop is rotated so that every load inside it is unconditional: the
  // body issues the next K, finishes the current chunk (softmax, PV), issues
  // the next V, then runs QK of the next chunk.  The wait for K inside the
  // body therefore never covers the V rows issued after it; the last chunk's
  // softmax and PV run after the loop.
  if (w < n_it) {
    {
      Blocks b0;
      load_blocks(w, b0);
      const int tok0 = t_begin + w * IT;
      if constexpr (W8) dw.issue_scales(cv, kvh, tok0, t_end, t_begin, b0, dw.wa);
      dw.template issue_k<KNT>(cv, kvh, tok0, t_end, t_begin, b0);
      __builtin_amdgcn_sched_barrier(0);
      dw.template issue_v<NTL>(cv, kvh, tok0, t_end, t_begin, b0);
      __builtin_amdgcn_sched_barrier(0);
    }
    after_issue();
    float s[CT][PAIRS][8];
    dw.qk(s);
    __builtin_amdgcn_sched_barrier(0);
    int nxt = w + NW;
    // One iteration: the next chunk's K rows (and, W8, its scales) go out,
    // this chunk's softmax and PV run, then the next V rows go out and the
    // next QK runs.
    while (nxt < n_it) {
      W8Buf cur = dw.wa;   // W8: this chunk's scales, loaded one chunk ago
      Blocks bn;
      load_blocks(nxt, bn);
      const int tok0 = t_begin + nxt * IT;
      if constexpr (W8) dw.issue_scales(cv, kvh, tok0, t_end, t_begin, bn, dw.wa);
      dw.template issue_k<KNT>(cv, kvh, tok0, t_end, t_begin, bn);
      __builtin_amdgcn_sched_barrier(0);
      dw.softmax_pv(s, dw.mask_needed(cur), cur, c);
      __builtin_amdgcn_sched_barrier(0);
      dw.template issue_v<NTL>(cv, kvh, tok0, t_end, t_begin, bn);
      __builtin_amdgcn_sched_barrier(0);
      dw.qk(s);
      __builtin_amdgcn_sched_barrier(0);
      nxt += NW;
    }
    dw.softmax_pv(s, dw.mask_needed(dw.wa), dw.wa, c);
  } else {
    after_issue();
  }

  // ---- per-wave results, column tile by column tile: every wave's state
  // goes to LDS; then the work-group's threads merge them and write the
  // output when the unit has one split, else this split's partial.
  const size_t out_base = ((size_t)seq * sh.num_heads + head0) * D;
  const size_t slot = wk.slot0 + (size_t)split * wk.stride;
  const auto racc = buf_rsrc(pacc + slot * gt * D, (uint32_t)(gt * D * 4));
  const auto rml = buf_rsrc(pml + slot * gt * 2, (uint32_t)(gt * 8));
  const bool final_here = FUSED && ns_eff == 1;
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int nh = min(16, gt - 16 * ct);   // query heads of this tile
    if (ct > 0) __syncthreads();            // the previous tile's merge has read its slots
    else if constexpr (Wave::QLDS) lds_barrier();   // every wave's last QK has read the query tile
    dw.store_state(sm, w, ct, nh);
    __syncthreads();
    merge_wave_states<D, NW, FUSED>(sm, ct, nh, tid, final_here, out, out_base, racc, rml);
  }
  if constexpr (FUSED) {
    if (ns_eff > 1) {
      // Each thread's partial stores are acknowledged before the arrival is
      // counted; the last work-group to arrive merges.  (An arrival counted
      // before the stores, so that the last work-group could keep its own
      // partial in registers, measured slower: the last one then waits for
      // the others' stores, by device-scope polling.)  A unit of few splits
      // or small partials has one counter and its last work-group merges
      // every split.  Larger merges take two levels, so that no
      // single work-group reads all the partials (one CU's bandwidth bound
      // that fold: 8 x 32k tokens at 32/1 heads spent 12 of 42 us in it):
      // the splits form kMergeGroups groups of consecutive splits, each
      // with its own counter; the last arrival of a group folds the group's
      // partials into the group's first slot, then counts one arrival at the
      // unit's counter, whose last arrival folds the groups' slots into the
      // output.  Every counter is back at zero when the unit is done.
      const size_t slot0 = wk.slot0, stride = wk.stride;
      auto slot_of = [=](int sp) { return slot0 + (size_t)sp * stride; };
      const bool two =
          ns_eff >= kMerge2MinSplits && (int64_t)ns_eff * gt * D >= kMerge2MinFloats;
      uint32_t* const cu = cnt + unit;
      uint32_t* cg = cu;
      int lo = 0, hi = ns_eff;
      if (two) {   // (the divisions stay off the one-level path: it ends every launch)
        const int grp = split * kMergeGroups / ns_eff;
        lo = merge_group_first(grp, ns_eff);
        hi = merge_group_first(grp + 1, ns_eff);
        const size_t n_units = (size_t)sh.num_seqs * sh.num_kv_heads * sh.nchunk;
        cg = cnt + n_units + (size_t)unit * kMergeGroups + grp;
      }
      if (arrive_last(sm, cg, hi - lo)) {
        if (!two) {
          merge_splits<D, NW * kWave, true>(pacc, pml, out, slot_of, gt, out_base, ns_eff);
        } else {
          static_assert(NW * 16 >= 2 * 16 * CT, "(max, sum) of every head of the tile fit sm.m");
          const size_t dst = slot_of(lo);
          float* const ml_lds = &sm.m[0][0];
          // (one batch shape for both levels: the code of the whole merge
          // stays small, and it runs cold at the end of the launch)
          merge_splits_by<D, NW * kWave, true, 2, 8>(
              pacc, pml, [=](int i) { return slot_of(lo + i); }, gt, hi - lo, tid,
              SlotSink<D>{buf_rsrc(pacc + dst * gt * D, (uint32_t)(gt * D * 4)), ml_lds});
          __syncthreads();   // every thread has read the group's (max, sum) pairs
          if (tid < gt) {
            const f2_t ml = {ml_lds[2 * tid], ml_lds[2 * tid + 1]};
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2_t, ml),
                                                  buf_rsrc(pml + dst * gt * 2, (uint32_t)(gt * 8)),
                                                  tid * 8, 0, kPolicyDevice);
          }
          if (tid == 0) __hip_atomic_store(cg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (arrive_last(sm, cu, kMergeGroups))
            merge_splits_by<D, NW * kWave, true, 2, kMergeGroups>(
                pacc, pml, [=](int gi) { return slot_of(merge_group_first(gi, ns_eff)); }, gt,
                kMergeGroups, tid, OutSink<D>{out, out_base});
          else
            return;
        }
        if (tid == 0) __hip_atomic_store(cu, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// The first ten DecodeShape fields as plain int kernel arguments (after the
// block-table and context-length pointers): aggregates are not preloaded into
// SGPRs, scalars are.  The kernels rebuild the shape from them.
#define PA_SHAPE_HEAD_PARAMS                                                              \
  int sh_nchunk, int sh_num_items, int sh_nsplit, int sh_num_kv_heads, int sh_partition, \
      int sh_max_blocks, int sh_bs_log2, int sh_block_size, int sh_num_seqs, int sh_num_blocks
#define PA_SHAPE_HEAD_ARGS(s)                                                             \
  (s).nchunk, (s).num_items, (s).nsplit, (s).num_kv_heads, (s).partition, (s).max_blocks, \
      (s).bs_log2, (s).block_size, (s).num_seqs, (s).num_blocks
#define PA_SHAPE_REBUILD(sh, tail)                                                        \
  DecodeShape sh = tail;                                                                  \
  sh.nchunk = sh_nchunk;                                                                  \
  sh.num_items = sh_num_items;                                                            \
  sh.nsplit = sh_nsplit;                                                                  \
  sh.num_kv_heads = sh_num_kv_heads;                                                      \
  sh.partition = sh_partition;                                                            \
  sh.max_blocks = sh_max_blocks;                                                          \
  sh.bs_log2 = sh_bs_log2;                                                                \
  sh.block_size = sh_block_size;                                                          \
  sh.num_seqs = sh_num_seqs;                                                              \
  sh.num_blocks = sh_num_blocks

// Work item of work-group wg in the grid form (XCD-aware); false past the
// plan's items.  With at least 8 (sequence, split) items, an item's kv heads
// and head chunks get work-group indices 8 apart, so they share blockIdx % 8
// (their XCD under round-robin dispatch), run at about the same time and meet
// in that XCD's L2: they read the same block-table lines, the head chunks of
// a kv head the same K/V tiles, and with INT8 all kv heads of a block the same
// scale lines (the block's scales are adjacent).  With fewer items that would
// leave XCDs idle, so the kv heads are spread over the XCDs and only the head
// chunks are grouped.
struct GridItem {
  int seq, kvh, chunk, split;
};

__device__ __forceinline__ bool grid_item(const DecodeShape& sh, int wg, GridItem& it) {
  const bool by_item = sh.num_items >= 8;
  const int per = by_item ? sh.num_kv_heads * sh.nchunk : sh.nchunk;
  const int grp = wg / (8 * per);
  const int rem = wg - grp * 8 * per;
  const int sub = rem >> 3;
  const int idx = grp * 8 + (rem & 7);
  if (by_item) {
    if (idx >= sh.num_items) return false;
    it.split = idx % sh.nsplit;
    it.seq = idx / sh.nsplit;
    it.kvh = sub / sh.nchunk;
    it.chunk = sub - it.kvh * sh.nchunk;
  } else {
    if (idx >= sh.num_items * sh.num_kv_heads) return false;
    it.split = idx % sh.nsplit;
    const int sk = idx / sh.nsplit;
    it.kvh = sk % sh.num_kv_heads;
    it.seq = sk / sh.num_kv_heads;
    it.chunk = sub;
  }
  return true;
}

// A context length clamped to what the block table holds and to what the
// grid's splits cover (no work-group reads past the table or the partials).
__device__ __forceinline__ int grid_ctx(const DecodeShape& sh, int ctx_raw) {
  const int cap = min(sh.max_blocks * sh.block_size, sh.nsplit * sh.partition);
  return ctx_raw < 0 ? 0 : (ctx_raw > cap ? cap : ctx_raw);
}

// Grid form: one work-group per (unit, split) slot of the host's plan.
template <int D, int NW, int CT, bool I8, bool FUSED, bool NTL, bool KNT>
__global__ void __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(2)))
decode_kernel(const int* __restrict__ bt, const int* __restrict__ ctxl, PA_SHAPE_HEAD_PARAMS,
              DecodeShape sh_tail, const half_t* __restrict__ q, const uint8_t* __restrict__ kc,
              const uint8_t* __restrict__ vc, const float* __restrict__ ksc,
              const float* __restrict__ vsc, half_t* __restrict__ out, float* __restrict__ pacc,
              float* __restrict__ pml, uint32_t* __restrict__ cnt) {
  PA_SHAPE_REBUILD(sh, sh_tail);
  static_assert(sizeof(DecodeSmem<D, NW>) * (kWavesPerCU / NW) <= kLdsPerCU, "LDS budget");
  __shared__ DecodeSmem<D, NW> sm;

  GridItem it;
  if (!grid_item(sh, blockIdx.x, it)) return;
  const int seq = it.seq, kvh = it.kvh, chunk = it.chunk, split = it.split;

  // The context length is used only after the split's block-id loads are
  // issued.  It is read with a vector load at the top: a scalar load would be
  // scheduled next to its first use, after the argument fetches of the query
  // pointer.
  int zero = 0;
  asm volatile("" : "+v"(zero));
  const int ctx_lane = ctxl[seq + zero];
  const int unit = (seq * sh.num_kv_heads + kvh) * sh.nchunk + chunk;
  const SplitWork wk{seq, kvh, chunk, split, 0, sh.partition, 0, (size_t)unit * sh.nsplit, 1};
  auto resolve = [&](int& ctx, int& ns) {
    ctx = grid_ctx(sh, __builtin_amdgcn_readfirstlane(ctx_lane));
    ns = ctx > 0 ? (ctx + sh.partition - 1) / sh.partition : 1;
    return split < ns;
  };
  // FP16 launches that read non-temporally (over 32 MB of K/V, one head
  // chunk per kv head) take the group mapping; small latency-bound ones keep
  // the pair mapping (config 1: 4.8 us against 5.4 us with groups).
  decode_split<D, NW, CT, I8, FUSED, NTL, KNT, !I8 && NTL>(q, kc, vc, ksc, vsc, bt, out, pacc, pml,
                                                         cnt, sh, wk, sm, resolve, [] {});
}

// ---------------------------------------------------------------------------
// In-kernel schedule: persistent work-groups over a compact work list.
//
// Every work-group reads the (clamped) context lengths and derives the same
// schedule in LDS.  The partition P is chosen from the total token count:
// about one item per resident work-group when all lengths are equal (the
// grid plan's shape), about kSchedItemsPerGroup items per work-group
// otherwise.  A row is one split of one sequence; rows that hold a full
// partition come first, the shorter last rows of the sequences after them,
// longest first (in kShortBuckets bands of P / kShortBuckets tokens), so that
// the items claimed last are the shortest and the launch does not wait on a
// long one started late.  An item is (row, kv head, head chunk).  Items are
// dealt to 8 claim classes by row, row % 8, with the kv heads and chunks of a
// row next to each other; work-group b serves class b % 8 (its XCD under the
// usual round-robin dispatch), starts with item b / 8 of its class
// and claims the next one from the class counter once the current item's
// first loads are issued.  Exactly as many claims as the class has items are
// made per launch, so the claim that returns the last index is the last one
// and resets the counter for the next launch; a class with no more items than
// work-groups makes none.  No work-group is launched for
// a split that a sequence does not have, whatever the block-table capacity or
// the spread of the lengths.
struct SchedArgs {
  uint32_t* queue;    // 8 claim counters, kSchedQueueStride words apart
  int rows_max;       // slot rows the partial buffers hold
  int pmin, pmax;     // partition bounds (multiples of kIterTokens)
  int pmin_uniform;   // lower bound when all lengths are equal (one item per work-group)
  float fill_scale;   // 1024 * kv heads * head chunks / CUs (see the ragged floor below)
};

constexpr int kShortBuckets = 4;   // (their counts pack into one 64-bit word)

struct SchedSmem {
  int full_pre[kSchedMaxSeqs + 1];        // exclusive prefix of full rows per sequence
  uint16_t part_pre[kSchedMaxSeqs + 1];   // exclusive prefix of short last rows (<= S)
  uint16_t rem[kSchedMaxSeqs];            // context length % P (P <= 16384)
  uint16_t short_seq[kSchedMaxSeqs];      // sequence of short row j (longest first)
  uint64_t band_scan[16];                 // per-wave totals of the band counts
  uint32_t red[3][16];               // per-wave sum (in 1024-token units), min, max
  int scan_f[16], scan_p[16];
  int next_item;
};

// Unsigned wave reductions (DPP inside rows, permlane swaps across them);
// every lane receives the result.
template <class Op>
__device__ __forceinline__ uint32_t wave_reduce_u(uint32_t v, Op op) {
  v = op(v, dpp_mov_u<kQuadXor1>(v));
  v = op(v, dpp_mov_u<kQuadXor2>(v));
  v = op(v, dpp_mov_u<kRowHalfMirror>(v));
  v = op(v, dpp_mov_u<kRowMirror>(v));
  auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = op(r[0], r[1]);
  auto t = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return op(t[0], t[1]);
}
struct OpAddU { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a + b; } };
struct OpMinU { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a < b ? a : b; } };
struct OpMaxU { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; } };

// Inclusive prefix sum over the wave of 64-bit values.
__device__ __forceinline__ uint64_t wave_scan_u64(uint64_t v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint64_t u = __shfl_up(v, o, kWave);
    if (lane >= o) v += u;
  }
  return v;
}

// Inclusive prefix sum over the wave.
__device__ __forceinline__ int wave_scan_i(int v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int u = __shfl_up(v, o, kWave);
    if (lane >= o) v += u;
  }
  return v;
}

// Largest s in [0, n) with pre[s] <= x (pre is non-decreasing, pre[0] = 0 <= x).
__device__ __forceinline__ int prefix_search(const int* pre, int n, int x) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (pre[mid] <= x) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

struct Schedule {
  int partition, n_full, n_rows;
  bool uniform;
};

// Unsigned division by a divisor fixed for many dividends (Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994,
// fig. 4.1): with l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1,
// n / d = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0), t = mulhi(m, n),
// exact for every 32-bit n and 1 <= d < 2^31.  The setup runs once per
// divisor (uniform, on the scalar unit); each quotient costs a multiply-high,
// a subtraction, an add and two shifts instead of a division sequence.
struct DivU32 {
  uint32_t m;
  int s1, s2;
  uint32_t d;
};
__device__ __forceinline__ DivU32 div_setup(uint32_t d) {
  const int l = d > 1 ? 32 - __builtin_clz(d - 1) : 0;   // ceil(log2 d)
  DivU32 v;
  v.m = (uint32_t)((((1ull << l) - d) << 32) / d + 1);
  v.s1 = l < 1 ? l : 1;
  v.s2 = l - 1 > 0 ? l - 1 : 0;
  v.d = d;
  return v;
}
__device__ __forceinline__ uint32_t div_q(const DivU32& v, uint32_t n) {
  const uint32_t t = __umulhi(v.m, n);
  return (t + ((n - t) >> v.s1)) >> v.s2;
}

// Inclusive prefix sum over the wave: Hillis-Steele steps inside each
// 16-lane row by DPP row shifts (a lane shifted in from outside its row reads
// 0), then the totals of the rows below it, read from lanes 15, 31 and 47.
// Every lane must be active.
__device__ __forceinline__ uint32_t wave_scan_dpp(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, true);   // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, true);   // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, true);   // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, true);   // row_shr:8
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 15);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 31);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 47);
  const int row = (threadIdx.x & (kWave - 1)) >> 4;
  return v + (row > 0 ? r0 : 0u) + (row > 1 ? r1 : 0u) + (row > 2 ? r2 : 0u);
}

// The schedule of at most 64 sequences, one per lane: every wave derives it
// on its own with wave-wide reductions and DPP scans, wave 0 writes the
// tables, and one barrier publishes them; the same schedule, table for table,
// as build_schedule, whose cross-wave reductions and scans (LDS round trips
// and barriers) it skips.  Measured on MI355X against build_schedule at the
// bench's shapes (same box, alternating): config 2 split-K 28.73 -> 27.55 us,
// config 4 32k INT8 90.43 -> 89.15 (FP16 166.61 -> 165.45), 8 x 32k MQA 35.08
// -> 34.05 (INT8 28.49 -> 27.15); 128k even.
template <int NTH>
__device__ __forceinline__ Schedule build_schedule_small(const int* __restrict__ ctxl,
                                                         const DecodeShape& sh,
                                                         const SchedArgs& sa, SchedSmem& ss) {
  constexpr int NWV = NTH / kWave;
  const int S = sh.num_seqs;
  const int lane = threadIdx.x & (kWave - 1);
  const bool writer = threadIdx.x < kWave;
  const bool in = lane < S;
  const int cap = sh.max_blocks * sh.block_size;
  int c = in ? ctxl[lane] : 0;
  c = c < 0 ? 0 : (c > cap ? cap : c);
  // Wave-uniform, read into scalar registers: otherwise the compiler takes
  // every value derived from them (the partition, the claim classes, the
  // item fields) as divergent, and the whole item loop grows (214 instead of
  // 191 VGPRs for the INT8 kernel, 8% slower at config 5's MQA).
  const uint32_t t = __builtin_amdgcn_readfirstlane(wave_reduce_u(in ? (uint32_t)c >> 10 : 0u, OpAddU()));
  const uint32_t a = __builtin_amdgcn_readfirstlane(wave_reduce_u(in ? (uint32_t)c : 0xFFFFFFFFu, OpMinU()));
  const uint32_t b = __builtin_amdgcn_readfirstlane(wave_reduce_u(in ? (uint32_t)c : 0u, OpMaxU()));
  Schedule sc;
  sc.uniform = a == b;
  {
    constexpr uint64_t kGroupsPerCU = kWavesPerCU / NWV;
    const uint64_t groups = sc.uniform ? (gridDim.x + kGroupsPerCU - 1) / kGroupsPerCU : gridDim.x;
    const uint64_t k = sc.uniform ? 1 : kSchedItemsPerGroup;
    const float want = __builtin_ceilf((float)t * (1024.f * (float)sh.num_kv_heads) /
                                       (float)(groups * k));
    uint64_t part = (uint64_t)fminf(want, (float)sa.pmax);
    part = (part + kIterTokens - 1) / kIterTokens * kIterTokens;
    // (the same bounds as build_schedule's)
    uint64_t f = (uint64_t)fminf(__builtin_ceilf((float)(t + (uint32_t)S) * sa.fill_scale),
                                 (float)sa.pmin);
    f = (f + kIterTokens - 1) / kIterTokens * kIterTokens;
    const uint64_t lo = (sc.uniform || f < (uint64_t)sa.pmin_uniform) ? (uint64_t)sa.pmin_uniform : f;
    part = part < lo ? lo : (part > (uint64_t)sa.pmax ? (uint64_t)sa.pmax : part);
    const uint64_t top = ((uint64_t)(b > 0 ? b : 1) + kIterTokens - 1) / kIterTokens * kIterTokens;
    sc.partition = (int)(part < top ? part : top);
  }
  while (true) {
    const int P = sc.partition;
    const int qv = (int)((uint32_t)c / (uint32_t)P);
    const int rv = c - qv * P;
    const bool shortrow = in && (rv != 0 || c == 0);
    const uint32_t fs = in ? (uint32_t)qv : 0u, ps = shortrow ? 1u : 0u;
    const uint32_t fi = wave_scan_dpp(fs), pi = wave_scan_dpp(ps);
    const int tf = __builtin_amdgcn_readlane((int)fi, kWave - 1);
    const int tp = __builtin_amdgcn_readlane((int)pi, kWave - 1);
    if (tf + tp > sa.rows_max && P < sa.pmax) {
      sc.partition = P * 2 < sa.pmax ? P * 2 : sa.pmax;
      continue;
    }
    int bb = -1;
    if (shortrow) {
      bb = kShortBuckets - 1;
#pragma unroll
      for (int k = 1; k < kShortBuckets; ++k) bb -= (rv * kShortBuckets >= k * P) ? 1 : 0;
    }
    // a band's earlier members (in sequence order) and the bands' sizes, two
    // bands per 32-bit scan (16 bits each)
    const uint32_t c01 = bb == 0 ? 1u : (bb == 1 ? 0x10000u : 0u);
    const uint32_t c23 = bb == 2 ? 1u : (bb == 3 ? 0x10000u : 0u);
    const uint32_t s01 = wave_scan_dpp(c01), s23 = wave_scan_dpp(c23);
    const uint32_t t01 = (uint32_t)__builtin_amdgcn_readlane((int)s01, kWave - 1);
    const uint32_t t23 = (uint32_t)__builtin_amdgcn_readlane((int)s23, kWave - 1);
    if (writer && in) {
      ss.full_pre[lane] = (int)(fi - fs);
      ss.part_pre[lane] = (uint16_t)(pi - ps);
      ss.rem[lane] = (uint16_t)rv;
      if (bb >= 0) {
        const int n0 = (int)(t01 & 0xFFFFu), n1 = (int)(t01 >> 16), n2 = (int)(t23 & 0xFFFFu);
        const uint32_t e01 = s01 - c01, e23 = s23 - c23;   // exclusive
        int pos;
        if (bb == 0) pos = (int)(e01 & 0xFFFFu);
        else if (bb == 1) pos = n0 + (int)(e01 >> 16);
        else if (bb == 2) pos = n0 + n1 + (int)(e23 & 0xFFFFu);
        else pos = n0 + n1 + n2 + (int)(e23 >> 16);
        ss.short_seq[pos] = (uint16_t)lane;
      }
    }
    if (writer && lane == 0) {
      ss.full_pre[S] = tf;
      ss.part_pre[S] = (uint16_t)tp;
    }
    sc.n_full = tf;
    sc.n_rows = tf + tp;
    break;
  }
  __syncthreads();
  return sc;
}

// Builds the schedule in LDS; every thread of the work-group takes part and
// returns the same values.  Thread t owns sequences [t*E, t*E + E).
template <int NTH>
__device__ Schedule build_schedule(const int* __restrict__ ctxl, const DecodeShape& sh,
                                   const SchedArgs& sa, SchedSmem& ss) {
  constexpr int E = (kSchedMaxSeqs + NTH - 1) / NTH;
  constexpr int NWV = NTH / kWave;
  const int S = sh.num_seqs;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & (kWave - 1);
  const int cap = sh.max_blocks * sh.block_size;
  int c[E];
  uint32_t tk = 0, mn = 0xFFFFFFFFu, mx = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = tid * E + e;
    int v = i < S ? ctxl[i] : 0;
    v = v < 0 ? 0 : (v > cap ? cap : v);
    c[e] = v;
    if (i < S) {
      tk += (uint32_t)v >> 10;   // the total only steers the partition choice
      mn = mn < (uint32_t)v ? mn : (uint32_t)v;
      mx = mx > (uint32_t)v ? mx : (uint32_t)v;
    }
  }
  tk = wave_reduce_u(tk, OpAddU());
  mn = wave_reduce_u(mn, OpMinU());
  mx = wave_reduce_u(mx, OpMaxU());
  if (lane == 0) {
    ss.red[0][w] = tk;
    ss.red[1][w] = mn;
    ss.red[2][w] = mx;
  }
  __syncthreads();
  uint64_t t = 0;
  uint32_t a = 0xFFFFFFFFu, b = 0;
#pragma unroll
  for (int i = 0; i < NWV; ++i) {
    t += ss.red[0][i];
    a = a < ss.red[1][i] ? a : ss.red[1][i];
    b = b > ss.red[2][i] ? b : ss.red[2][i];
  }
  Schedule sc;
  sc.uniform = a == b;
  {
    // P: about one item per CU for equal lengths (per resident work-group
    // with 8-wave groups; with two 4-wave groups per CU, fewer and longer
    // items measured faster: config 4 32k INT8 93.6 -> 91.8 us, and every
    // extra split is merged at the end), about kSchedItemsPerGroup per
    // work-group otherwise; within [pmin, pmax] and no longer than the
    // longest sequence.
    constexpr uint64_t kGroupsPerCU = kWavesPerCU / NWV;
    const uint64_t groups = sc.uniform ? (gridDim.x + kGroupsPerCU - 1) / kGroupsPerCU : gridDim.x;
    const uint64_t k = sc.uniform ? 1 : kSchedItemsPerGroup;
    // (in float: a 64-bit integer division is a long scalar sequence, and
    // every work-group evaluates the same operations on the same values)
    const float want = __builtin_ceilf((float)t * (1024.f * (float)sh.num_kv_heads) /
                                       (float)(groups * k));
    uint64_t part = (uint64_t)fminf(want, (float)sa.pmax);
    part = (part + kIterTokens - 1) / kIterTokens * kIterTokens;
    // The ragged lower bound keeps items of a few hundred tokens from paying
    // their fixed costs too often; with equal lengths every resident
    // work-group gets one item, so the smaller grid bound applies.  A ragged
    // launch with less work than one pmin item per CU lowers the bound to about
    // one item per CU (its token total is below (t + S) * 1024), down to the
    // equal-length bound: same box, alternating, 16 ragged sequences of median
    // 2048 at 12/2 20.48 -> 17.00 us (INT8 19.53 -> 14.53), 48 of median 512
    // 19.52 -> 12.87, MQA 32/1 16 x median 2048 INT8 22.08 -> 17.54.  Config 5
    // keeps its partitions and its times (within 0.5%).
    // (branch-free: both bounds are cheap scalar values; a branch here cost the
    // scheduled launches 0.2-1.1% through code layout alone)
    uint64_t f = (uint64_t)fminf(__builtin_ceilf((float)(t + (uint32_t)S) * sa.fill_scale),
                                 (float)sa.pmin);
    f = (f + kIterTokens - 1) / kIterTokens * kIterTokens;
    const uint64_t lo = (sc.uniform || f < (uint64_t)sa.pmin_uniform) ? (uint64_t)sa.pmin_uniform : f;
    part = part < lo ? lo : (part > (uint64_t)sa.pmax ? (uint64_t)sa.pmax : part);
    const uint64_t top = ((uint64_t)(b > 0 ? b : 1) + kIterTokens - 1) / kIterTokens * kIterTokens;
    sc.partition = (int)(part < top ? part : top);
  }
  // Exclusive scans of full rows (ctx / P) and short last rows (0 or 1); the
  // partition doubles (rarely) until the rows fit the partial buffers, which
  // hold them at the upper partition bound.
  while (true) {
    const int P = sc.partition;
    const DivU32 dv = div_setup((uint32_t)P);
    int fq[E], fr[E];   // c / P and c % P
    int fs = 0, ps = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = tid * E + e;
      fq[e] = (int)div_q(dv, (uint32_t)c[e]);
      fr[e] = c[e] - fq[e] * P;
      fs += i < S ? fq[e] : 0;
      ps += i < S ? ((fr[e] != 0 || c[e] == 0) ? 1 : 0) : 0;
    }
    const int fi = wave_scan_i(fs), pi = wave_scan_i(ps);
    if (lane == kWave - 1) {
      ss.scan_f[w] = fi;
      ss.scan_p[w] = pi;
    }
    __syncthreads();
    int fo = fi - fs, po = pi - ps, tf = 0, tp = 0;
#pragma unroll
    for (int i = 0; i < NWV; ++i) {
      const int f = ss.scan_f[i], q = ss.scan_p[i];
      if (i < w) {
        fo += f;
        po += q;
      }
      tf += f;
      tp += q;
    }
    if (tf + tp > sa.rows_max && P < sa.pmax) {
      __syncthreads();   // scan_f/scan_p are rewritten by the next pass
      sc.partition = P * 2 < sa.pmax ? P * 2 : sa.pmax;
      continue;
    }
    // Short rows in bands of P / kShortBuckets tokens, longest band first, in
    // sequence order inside a band.  Every work-group must derive the same
    // order (the items are claimed from shared counters), so a row's place in
    // its band is the number of earlier sequences in that band: one scan of
    // the band counts, packed 16 bits per band (S <= 1024) into one word.
    int band[E];
    uint64_t cnt = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = tid * E + e;
      const int r = fr[e];
      band[e] = -1;
      if (i < S) {
        ss.full_pre[i] = fo;
        ss.part_pre[i] = (uint16_t)po;
        ss.rem[i] = (uint16_t)r;
        fo += fq[e];
        if (r != 0 || c[e] == 0) {
          po += 1;
          // floor(r * kShortBuckets / P) by comparisons (r < P <= 8192)
          int b = kShortBuckets - 1;
#pragma unroll
          for (int k = 1; k < kShortBuckets; ++k) b -= (r * kShortBuckets >= k * P) ? 1 : 0;
          band[e] = b;
          cnt += 1ull << (16 * band[e]);
        }
      }
    }
    if (tid == 0) {
      ss.full_pre[S] = tf;
      ss.part_pre[S] = (uint16_t)tp;
    }
    const uint64_t incl = wave_scan_u64(cnt);
    if (lane == kWave - 1) ss.band_scan[w] = incl;
    __syncthreads();
    uint64_t before = 0, total = 0;
#pragma unroll
    for (int v = 0; v < NWV; ++v) {
      const uint64_t t = ss.band_scan[v];
      if (v < w) before += t;
      total += t;
    }
    // the bands' bases (exclusive prefix of their totals)
    int bbase[kShortBuckets];
    int acc_b = 0;
#pragma unroll
    for (int b = 0; b < kShortBuckets; ++b) {
      bbase[b] = acc_b;
      acc_b += (int)((total >> (16 * b)) & 0xFFFFu);
    }
    // this thread's first place in each band
    uint64_t at = before + incl - cnt;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = tid * E + e;
#pragma unroll
      for (int b = 0; b < kShortBuckets; ++b) {
        if (band[e] == b) {
          ss.short_seq[bbase[b] + (int)((at >> (16 * b)) & 0xFFFFu)] = (uint16_t)i;
          at += 1ull << (16 * b);
        }
      }
    }
    sc.n_full = tf;
    sc.n_rows = tf + tp;
    break;
  }
  __syncthreads();
  return sc;
}

template <int D, int NW, int CT, bool I8, bool NTL>
__global__ void __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(2)))
decode_sched_kernel(const int* __restrict__ bt, const int* __restrict__ ctxl,
                    PA_SHAPE_HEAD_PARAMS, DecodeShape sh_tail, const half_t* __restrict__ q,
                    const uint8_t* __restrict__ kc, const uint8_t* __restrict__ vc,
                    const float* __restrict__ ksc, const float* __restrict__ vsc,
                    half_t* __restrict__ out, float* __restrict__ pacc, float* __restrict__ pml,
                    uint32_t* __restrict__ cnt, SchedArgs sa) {
  PA_SHAPE_REBUILD(sh, sh_tail);
  static_assert((sizeof(DecodeSmem<D, NW>) + sizeof(SchedSmem)) * (kWavesPerCU / NW) <= kLdsPerCU,
                "LDS budget");
  __shared__ DecodeSmem<D, NW> sm;
  __shared__ SchedSmem ss;
  // (the hint keeps the larger batches' path laid out as the hot one: without
  // it config 5's INT8 MQA ran 2.5-3.7% slower, with the same registers)
  Schedule sc;
  if (__builtin_expect(sh.num_seqs > kWave, 1)) sc = build_schedule<NW * kWave>(ctxl, sh, sa, ss);
  else sc = build_schedule_small<NW * kWave>(ctxl, sh, sa, ss);

  const int S = sh.num_seqs, hkv = sh.num_kv_heads, nchunk = sh.nchunk;
  const int P = __builtin_amdgcn_readfirstlane(sc.partition);
  const int n_full = __builtin_amdgcn_readfirstlane(sc.n_full);
  // Claim classes.  Eight, one per XCD under the usual round-robin dispatch:
  // rows r with r % 8 == cls, each followed by its kv heads and head chunks,
  // so the chunks of one (row, kv head) run at about the same time on one XCD
  // and share its L2.  Ragged lengths with one chunk per kv head (no two
  // items read the same K/V rows) use one class over all work-groups, so
  // the XCDs that start first take work from the ones that start late (same
  // box: bench config 5 32/8 FP16 278.9 -> 274.2 us, INT8 163.7 -> 162.3;
  // equal lengths measured 0.3-2.6% slower with one class and keep eight).
  const int n_rows = __builtin_amdgcn_readfirstlane(sc.n_rows);
  const int per_row = hkv * nchunk;
  const int lg = (nchunk > 1 || sc.uniform) ? 3 : 0;   // log2 of the class count
  const int ncls = 1 << lg;
  const int cls = blockIdx.x & (ncls - 1);
  const int groups_c = ((int)gridDim.x - cls + ncls - 1) >> lg;
  const int items_c = (n_rows > cls ? (n_rows - cls + ncls - 1) >> lg : 0) * per_row;
  uint32_t* queue = sa.queue + cls * kSchedQueueStride;
  // Item indices are compared unsigned: whatever a claim counter holds, no
  // work-group leaves its class's item list.
  int idx = blockIdx.x >> lg;   // index within the class: static first item
  // With no more items than work-groups in the class (equal lengths give one
  // item per work-group) the static first items cover the class: no claims,
  // and the counter stays at zero.
  const bool claims = items_c > groups_c;
  while ((uint32_t)idx < (uint32_t)items_c) {
    // The next item is claimed once this item's first loads are out.
    uint32_t old = 0;
    auto claim = [&] {
      if (claims && threadIdx.x == 0) {
        // The address is kept from looking uniform: the compiler's
        // wave-aggregated form of a uniform-address atomic reads the answer
        // at once, and that wait (the memory counter completes in order)
        // would also wait for this item's first K/V rows.
        int z = 0;
        asm volatile("" : "+v"(z));
        old = __hip_atomic_fetch_add(queue + z, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    };
    const int row = cls + ncls * (idx / per_row);
    const int sub = idx - (idx / per_row) * per_row;
    const int kvh = sub / nchunk, chunk = sub - (sub / nchunk) * nchunk;
    // Item fields are work-group uniform: keep them in scalar registers.
    int seq, split;
    if (row < n_full) {
      seq = prefix_search(ss.full_pre, S, row);
      split = row - ss.full_pre[seq];
    } else {
      seq = ss.short_seq[row - n_full];
      split = ss.full_pre[seq + 1] - ss.full_pre[seq];
    }
    seq = __builtin_amdgcn_readfirstlane(seq);
    split = __builtin_amdgcn_readfirstlane(split);
    const int ns = __builtin_amdgcn_readfirstlane(
        (ss.full_pre[seq + 1] - ss.full_pre[seq]) + (ss.part_pre[seq + 1] - ss.part_pre[seq]));
    const int rowbase = __builtin_amdgcn_readfirstlane(ss.full_pre[seq] + ss.part_pre[seq]);
    // A full row ends at its partition boundary, a short last row at the
    // sequence's length.
    const int ctx = row < n_full ? (split + 1) * P
                                 : split * P + __builtin_amdgcn_readfirstlane((int)ss.rem[seq]);
    const SplitWork wk{seq, kvh, chunk, split, ctx, P, ns,
                       ((size_t)rowbase * hkv + kvh) * nchunk + chunk, hkv * nchunk};
    decode_split<D, NW, CT, I8, true, NTL, false, false>(q, kc, vc, ksc, vsc, bt, out, pacc, pml, cnt, sh,
                                              wk, sm, [](int&, int&) { return true; }, claim);
    // Every processed item of the class made one claim (the first item of
    // each work-group is static), so the claim that returns items_c - 1 is
    // the last one and resets the counter for the next launch.
    if (!claims) break;
    if (threadIdx.x == 0) {
      if (old == (uint32_t)(items_c - 1))
        __hip_atomic_store(queue, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ss.next_item = (int)((uint32_t)groups_c + old);
    }
    __syncthreads();
    idx = __builtin_amdgcn_readfirstlane(ss.next_item);
  }
}

// ---------------------------------------------------------------------------
// Stream partition (split-K kinds): every (sequence, kv head, head chunk)
// is a stream of IT-token chunks.  The streams of all sequences, in
// sequence order, form one list of N chunks, and work-group b of the G
// launched takes the contiguous range [b N / G, (b + 1) N / G): every
// work-group gets the same number of chunks, whatever the spread of the
// lengths, and no chunk is tied to a split boundary.  The waves of a
// work-group deal the range's chunks round-robin and stream through them with
// one software pipeline that does not stop at stream boundaries: the block
// ids of a wave's chunk after next are loaded while it works on the current
// one, and the K/V rows of its next chunk are in flight whatever stream that
// chunk belongs to.  Where the range's part of a stream ends, the waves merge
// their states through LDS: a stream that lies wholly inside the range gets
// its output written there; otherwise the part becomes one of the range's
// two partials (slot 2b for the part that starts the range, 2b + 1 for the
// one that ends it), which stream_reduce_kernel merges.

struct StreamSmemTail {
  int pre[kSchedMaxSeqs + 1];   // chunks of all streams of the sequences before s
  int ctx[kSchedMaxSeqs];       // context length of s (clamped)
  int scan[16];                 // per-wave totals of the prefix scan
};

template <int D, int NW>
struct alignas(16) StreamSmem {
  float a[NW][16][D + kMergeRowPad];   // each wave's accumulator: per head, per dim (+ pad)
  float m[NW][16];
  float l[NW][16];
  StreamSmemTail t;
};

// Position of global chunk x: sequence s, stream u of s (kv head u / nchunk,
// head chunk u % nchunk), chunk c of the stream; the stream holds nch chunks
// and ends before global chunk `end`.  Work-group uniform.
struct ChunkPos {
  int x, s, u, c, nch, end, ctx;
};

__device__ __forceinline__ ChunkPos locate_chunk(const StreamSmemTail& t, int S, int U, int x) {
  ChunkPos z;
  z.x = x;
  z.s = __builtin_amdgcn_readfirstlane(prefix_search(t.pre, S, x));
  const int p0 = __builtin_amdgcn_readfirstlane(t.pre[z.s]);
  z.nch = __builtin_amdgcn_readfirstlane((t.pre[z.s + 1] - p0) / U);
  const int off = x - p0;
  z.u = off / z.nch;
  z.c = off - z.u * z.nch;
  z.end = p0 + (z.u + 1) * z.nch;
  z.ctx = __builtin_amdgcn_readfirstlane(t.ctx[z.s]);
  return z;
}

// The chunk `by` places further on (x + by < N).
__device__ __forceinline__ ChunkPos advance_chunk(const StreamSmemTail& t, int S, int U,
                                                  const ChunkPos& z, int by) {
  if (z.x + by < z.end) {
    ChunkPos n = z;
    n.x += by;
    n.c += by;
    return n;
  }
  return locate_chunk(t, S, U, z.x + by);
}

// Per-sequence chunk counts (ceil(ctx / IT) for each of the U streams) and
// their exclusive prefix over the sequences; returns N, the total.
template <int NTH, int IT>
__device__ int stream_prefix(const int* __restrict__ ctxl, int S, int U, int cap,
                             StreamSmemTail& t) {
  constexpr int E = (kSchedMaxSeqs + NTH - 1) / NTH;
  constexpr int NWV = NTH / kWave;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & (kWave - 1);
  int c[E], n[E], sum = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = tid * E + e;
    int v = i < S ? ctxl[i] : 0;
    v = v < 0 ? 0 : (v > cap ? cap : v);
    c[e] = v;
    n[e] = (v + IT - 1) / IT * U;
    sum += n[e];
  }
  const int incl = wave_scan_i(sum);
  if (lane == kWave - 1) t.scan[w] = incl;
  __syncthreads();
  int off = incl - sum, total = 0;
#pragma unroll
  for (int i = 0; i < NWV; ++i) {
    const int v = t.scan[i];
    if (i < w) off += v;
    total += v;
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = tid * E + e;
    if (i < S) {
      t.pre[i] = off;
      t.ctx[i] = c[e];
      off += n[e];
    }
  }
  if (tid == 0) t.pre[S] = total;
  __syncthreads();
  return total;
}

template <int D, int NW, int CT, bool I8, bool NTL>
__global__ void __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(2)))
decode_stream_kernel(const int* __restrict__ bt, const int* __restrict__ ctxl,
                     PA_SHAPE_HEAD_PARAMS, DecodeShape sh_tail, const half_t* __restrict__ q,
                     const uint8_t* __restrict__ kc, const uint8_t* __restrict__ vc,
                     const float* __restrict__ ksc, const float* __restrict__ vsc,
                     half_t* __restrict__ out, float* __restrict__ pacc, float* __restrict__ pml,
                     int* __restrict__ info) {
  PA_SHAPE_REBUILD(sh, sh_tail);
  using Wave = DecodeWave<D, CT, I8>;
  using Blocks = typename Wave::Blocks;
  using W8Buf = typename Wave::W8Buf;
  constexpr int PAIRS = Wave::PAIRS;
  constexpr int IT = Wave::IT;
  constexpr bool W8 = Wave::W8;
  static_assert(sizeof(StreamSmem<D, NW>) * (kWavesPerCU / NW) <= kLdsPerCU, "LDS budget");
  __shared__ StreamSmem<D, NW> sm;

  const int S = sh.num_seqs, U = sh.num_kv_heads * sh.nchunk, gt = sh.head_tile;
  const int N = stream_prefix<NW * kWave, IT>(ctxl, S, U, sh.max_blocks * sh.block_size, sm.t);
  // The reduce reads N and the prefix.
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i <= S; i += NW * kWave) info[1 + i] = sm.t.pre[i];
    if (threadIdx.x == 0) info[0] = N;
  }
  // With fewer chunks than work-groups, the first N take one each.
  const int G = min((int)gridDim.x, N);
  if ((int)blockIdx.x >= G) return;
  const int A = (int)((long long)blockIdx.x * N / G);
  const int B = (int)((long long)(blockIdx.x + 1) * N / G);

  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int bsl = sh.bs_log2;
  const CacheView cv{kc, vc, ksc, vsc, sh.num_kv_heads, sh.block_size, sh.num_blocks};
  const float c = sh.scale_log2;
  Wave dw;
  dw.init(lane);

  // Block ids of chunk z for this lane's loads, from the block table.
  auto chunk_blocks = [&](const ChunkPos& z, Blocks& b) {
    int kt[PAIRS], vt[PAIRS];
    const int tok0 = z.c * IT;
    dw.block_tokens(tok0, z.ctx, tok0, kt, vt);
    const int* row = bt + (size_t)z.s * sh.max_blocks;
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
      b.kb[p] = row[kt[p] >> bsl];
      b.vb[p] = row[vt[p] >> bsl];
    }
  };
  auto kv_head = [&](const ChunkPos& z) { return z.u / sh.nchunk; };

  // Wave w's chunks are A + w, A + w + NW, ... below B.  A wave without a next
  // chunk keeps loading its last one (every load of the loop is
  // unconditional, so the waits inside it never cover a later load).
  const bool have = w < B - A;
  ChunkPos cur = locate_chunk(sm.t, S, U, have ? A + w : A);
  ChunkPos nxt = (cur.x + NW < B) ? advance_chunk(sm.t, S, U, cur, NW) : cur;
  // The loads go out in the loop's order: K rows, then the next block ids,
  // then V rows.
  Blocks bn;
  {
    Blocks b0;
    chunk_blocks(cur, b0);
    const int tok0 = cur.c * IT;
    if constexpr (W8) dw.issue_scales(cv, kv_head(cur), tok0, cur.ctx, tok0, b0, dw.wa);
    dw.template issue_k<false>(cv, kv_head(cur), tok0, cur.ctx, tok0, b0);
    const typename Wave::VPlan vplan = dw.plan_v(cv, kv_head(cur), tok0, cur.ctx, tok0, b0);
    chunk_blocks(nxt, bn);
    __builtin_amdgcn_sched_barrier(0);
    dw.template issue_v<NTL>(cv, vplan);
    __builtin_amdgcn_sched_barrier(0);
  }

  for (int seg_lo = A; seg_lo < B;) {
    // The range's part of one stream: [seg_lo, seg_hi).
    const ChunkPos sg = locate_chunk(sm.t, S, U, seg_lo);
    const int seg_hi = min(B, sg.end);
    const bool whole = seg_lo == sg.end - sg.nch && seg_hi == sg.end;
    const int kvh = kv_head(sg), chunk = sg.u - kvh * sh.nchunk;
    const int head0 = kvh * sh.group + chunk * gt;
    if constexpr (Wave::QLDS) {
      QueryStage<D, NW> qst;
      qst.load(q, (size_t)sg.s * sh.num_heads + head0, gt, tid);
      lds_barrier();   // the previous part's wave merge has read the slots
      qst.store(query_stage_lds(sm), tid);
      lds_barrier();
      dw.qs = query_stage_lds(sm);
    } else {
      dw.load_q(q, (size_t)sg.s * sh.num_heads + head0, gt);
    }
    dw.compute_qbias();
    dw.reset();
    while (have && cur.x < seg_hi) {
      float s[CT][PAIRS][8];
      dw.qk(s);
      __builtin_amdgcn_sched_barrier(0);
      // The next chunk's K rows (and, W8, its scales) go out; then the block
      // ids of the one after it, into the registers those rows came from.
      W8Buf curw = dw.wa;   // W8: this chunk's scales, loaded one chunk ago
      const int ntok0 = nxt.c * IT, nkvh = kv_head(nxt);
      if constexpr (W8) dw.issue_scales(cv, nkvh, ntok0, nxt.ctx, ntok0, bn, dw.wa);
      dw.template issue_k<false>(cv, nkvh, ntok0, nxt.ctx, ntok0, bn);
      const typename Wave::VPlan vplan = dw.plan_v(cv, nkvh, ntok0, nxt.ctx, ntok0, bn);
      const ChunkPos after = (nxt.x + NW < B) ? advance_chunk(sm.t, S, U, nxt, NW) : nxt;
      chunk_blocks(after, bn);
      __builtin_amdgcn_sched_barrier(0);
      dw.softmax_pv(s, dw.mask_needed(curw), curw, c);
      __builtin_amdgcn_sched_barrier(0);
      dw.template issue_v<NTL>(cv, vplan);
      __builtin_amdgcn_sched_barrier(0);
      // past the wave's last chunk the position stays beyond the range
      cur = (nxt.x != cur.x) ? nxt : ChunkPos{B, 0, 0, 0, 1, B + 1, 0};
      nxt = after;
    }
    // ---- the part's end: every wave's state (empty for a wave without a
    // chunk in it) merges through LDS, column tile by column tile.  The next
    // chunk's K/V rows are in flight: the barriers order LDS only.
    const size_t out_base = ((size_t)sg.s * sh.num_heads + head0) * D;
    const size_t slot = 2 * (size_t)blockIdx.x + (seg_lo == A ? 0 : 1);
    const auto racc = buf_rsrc(pacc + slot * gt * D, (uint32_t)(gt * D * 4));
    const auto rml = buf_rsrc(pml + slot * gt * 2, (uint32_t)(gt * 8));
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int nh = min(16, gt - 16 * ct);
      lds_barrier();   // the previous merge has read the slots
      dw.store_state(sm, w, ct, nh);
      lds_barrier();
      merge_wave_states<D, NW, false>(sm, ct, nh, tid, whole, out, out_base, racc, rml);
    }
    seg_lo = seg_hi;
  }
}

// Merge of the streams the stream partition split between work-groups: one
// work-group per (sequence, stream); a stream inside one work-group's range
// was written by it, a sequence without tokens gets zeros.
template <int D>
__global__ void __launch_bounds__(kThreads)
stream_reduce_kernel(const float* __restrict__ pacc, const float* __restrict__ pml,
                     const int* __restrict__ info, half_t* __restrict__ out, DecodeShape sh,
                     int groups) {
  const int U = sh.num_kv_heads * sh.nchunk;
  const int s = blockIdx.x / U, u = blockIdx.x - s * U;
  const int kvh = u / sh.nchunk, chunk = u - kvh * sh.nchunk;
  const int gt = sh.head_tile;
  const size_t out_base = ((size_t)s * sh.num_heads + kvh * sh.group + chunk * gt) * D;
  const int N = info[0], p0 = info[1 + s], p1 = info[2 + s];
  const int nch = (p1 - p0) / U;
  if (nch <= 0) {
    for (int i = threadIdx.x; i < gt * D / 4; i += kThreads)
      *reinterpret_cast<uint2*>(out + out_base + 4 * (size_t)i) = make_uint2(0, 0);
    return;
  }
  const long long G = min(groups, N);
  const long long x0 = p0 + (long long)u * nch, x1 = x0 + nch;
  // work-group of chunk x: the last one whose range starts at or before x
  auto group_of = [&](long long x) { return (int)(((x + 1) * G - 1) / N); };
  const int g0 = group_of(x0), g1 = group_of(x1 - 1);
  if (g0 == g1) return;
  const size_t first = 2 * (size_t)g0 + ((long long)g0 * N / G == x0 ? 0 : 1);
  merge_splits<D, kThreads, false>(
      pacc, pml, out, [=](int k) { return k == 0 ? first : 2 * (size_t)(g0 + k); }, gt, out_base,
      g1 - g0 + 1);
}

// Split-K reduce: one work-group per (seq, kv_head, head chunk).
template <int D>
__global__ void __launch_bounds__(kThreads)
splitk_reduce_kernel(const float* __restrict__ pacc, const float* __restrict__ pml,
                     const int* __restrict__ ctxl, half_t* __restrict__ out, DecodeShape sh) {
  const int unit = blockIdx.x;
  const int chunk = unit % sh.nchunk;
  const int sk = unit / sh.nchunk;
  const int kvh = sk % sh.num_kv_heads;
  const int seq = sk / sh.num_kv_heads;
  const int cap = min(sh.max_blocks * sh.block_size, sh.nsplit * sh.partition);
  int ctx = ctxl[seq];
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int ns_eff = ctx > 0 ? (ctx + sh.partition - 1) / sh.partition : 1;
  const int head0 = kvh * sh.group + chunk * sh.head_tile;
  const size_t slot0 = (size_t)unit * sh.nsplit;
  merge_splits<D, kThreads, false>(
      pacc, pml, out, [=](int sp) { return slot0 + (size_t)sp; }, sh.head_tile,
      ((size_t)seq * sh.num_heads + head0) * D, ns_eff);
}

template <int D, int NW, int CT, bool I8, bool NTL, bool KNT>
hipError_t launch_decode_grid(const DecodeLaunch& l, int grid) {
  const DecodeShape& sh = l.shape;
  const auto* q = static_cast<const half_t*>(l.q);
  const auto* kc = static_cast<const uint8_t*>(l.k_cache);
  const auto* vc = static_cast<const uint8_t*>(l.v_cache);
  auto* out = static_cast<half_t*>(l.out);
  if (l.fused) {
    decode_kernel<D, NW, CT, I8, true, NTL, KNT><<<grid, NW * kWave, 0, l.stream>>>(
        l.block_table, l.context_lens, PA_SHAPE_HEAD_ARGS(sh), sh, q, kc, vc, l.k_scales, l.v_scales, out, l.part_acc,
        l.part_ml, l.counters);
    return hipGetLastError();
  }
  decode_kernel<D, NW, CT, I8, false, NTL, KNT><<<grid, NW * kWave, 0, l.stream>>>(
      l.block_table, l.context_lens, PA_SHAPE_HEAD_ARGS(sh), sh, q, kc, vc, l.k_scales, l.v_scales, out, l.part_acc,
      l.part_ml, l.counters);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int units = sh.num_seqs * sh.num_kv_heads * sh.nchunk;
  splitk_reduce_kernel<D><<<units, kThreads, 0, l.stream>>>(l.part_acc, l.part_ml, l.context_lens,
                                                            out, sh);
  return hipGetLastError();
}

template <int D, int NW, int CT, bool I8, bool NTL>
hipError_t launch_decode_tiles(const DecodeLaunch& l) {
  const DecodeShape& sh = l.shape;
  if (l.stream_part) {
    const auto* q = static_cast<const half_t*>(l.q);
    const auto* kc = static_cast<const uint8_t*>(l.k_cache);
    const auto* vc = static_cast<const uint8_t*>(l.v_cache);
    auto* out = static_cast<half_t*>(l.out);
    decode_stream_kernel<D, NW, CT, I8, NTL><<<l.groups, NW * kWave, 0, l.stream>>>(
        l.block_table, l.context_lens, PA_SHAPE_HEAD_ARGS(sh), sh, q, kc, vc, l.k_scales,
        l.v_scales, out, l.part_acc, l.part_ml, l.sched_info);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int streams = sh.num_seqs * sh.num_kv_heads * sh.nchunk;
    stream_reduce_kernel<D><<<streams, kThreads, 0, l.stream>>>(l.part_acc, l.part_ml,
                                                                  l.sched_info, out, sh, l.groups);
    return hipGetLastError();
  }
  if (l.sched) {
    constexpr int kGroupsPerCU = kWavesPerCU / NW;
    const int cus = (l.groups + kGroupsPerCU - 1) / kGroupsPerCU;
    const SchedArgs sa{l.queue, l.rows_max, l.pmin, l.pmax, l.pmin_uniform,
                       1024.f * (float)(l.shape.num_kv_heads * l.shape.nchunk) /
                           (float)(cus > 0 ? cus : 1)};
    const auto* q = static_cast<const half_t*>(l.q);
    const auto* kc = static_cast<const uint8_t*>(l.k_cache);
    const auto* vc = static_cast<const uint8_t*>(l.v_cache);
    auto* out = static_cast<half_t*>(l.out);
    // The last work-group of each unit merges its splits in this launch.
    decode_sched_kernel<D, NW, CT, I8, NTL><<<l.groups, NW * kWave, 0, l.stream>>>(
        l.block_table, l.context_lens, PA_SHAPE_HEAD_ARGS(sh), sh, q, kc, vc, l.k_scales,
        l.v_scales, out, l.part_acc, l.part_ml, l.counters, sa);
    return hipGetLastError();
  }
  // Groups of 8 items with their kv heads and head chunks, or, below 8 items,
  // of 8 (item, kv head) pairs with their head chunks (see decode_kernel).
  const int grid = sh.num_items >= 8
                       ? (sh.num_items + 7) / 8 * 8 * sh.num_kv_heads * sh.nchunk
                       : (sh.num_items * sh.num_kv_heads + 7) / 8 * 8 * sh.nchunk;
  if constexpr (!I8 && NTL && CT == 1) {
    if (l.k_nt) return launch_decode_grid<D, NW, CT, I8, NTL, true>(l, grid);
  }
  return launch_decode_grid<D, NW, CT, I8, NTL, false>(l, grid);
}

// Two MFMA column tiles when a work-group serves more than 16 query heads
// (head_dim <= 128; the planner keeps head tiles of head_dim 256 at 16).
template <int D, int NW, bool I8, bool NTL>
hipError_t launch_decode_waves(const DecodeLaunch& l) {
  if constexpr (D <= 128) {
    if (l.shape.head_tile > kMaxGroupTile) return launch_decode_tiles<D, NW, 2, I8, NTL>(l);
  }
  return launch_decode_tiles<D, NW, 1, I8, NTL>(l);
}

template <int D, bool I8, bool NTL>
hipError_t launch_decode_loads(const DecodeLaunch& l) {
  if constexpr (D <= 128) {
    if (l.waves == 8) return launch_decode_waves<D, 8, I8, NTL>(l);
  }
  return launch_decode_waves<D, 4, I8, NTL>(l);
}

template <int D, bool I8>
hipError_t launch_decode_dtype(const DecodeLaunch& l) {
  return l.nt_loads ? launch_decode_loads<D, I8, true>(l) : launch_decode_loads<D, I8, false>(l);
}

template <int D>
hipError_t launch_decode_d(const DecodeLaunch& l) {
  return l.int8_kv ? launch_decode_dtype<D, true>(l) : launch_decode_dtype<D, false>(l);
}

// Resident work-groups of the persistent decode kernels for one head_dim
// (cached per device and variant): the in-kernel schedule (stream_part =
// false) or the stream partition.
template <int D, int NW, int CT>
int resident_query(bool int8_kv, bool stream_part, int* per_cu) {
  hipError_t e;
  if (stream_part)
    e = int8_kv ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
                      per_cu, decode_stream_kernel<D, NW, CT, true, true>, NW * kWave, 0)
                : hipOccupancyMaxActiveBlocksPerMultiprocessor(
                      per_cu, decode_stream_kernel<D, NW, CT, false, true>, NW * kWave, 0);
  else
    e = int8_kv ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
                      per_cu, decode_sched_kernel<D, NW, CT, true, true>, NW * kWave, 0)
                : hipOccupancyMaxActiveBlocksPerMultiprocessor(
                      per_cu, decode_sched_kernel<D, NW, CT, false, true>, NW * kWave, 0);
  return e == hipSuccess ? 0 : -1;
}

template <int D>
int resident_groups_d(bool stream_part, int waves, bool int8_kv, int column_tiles) {
  static int cache[64][16] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  const int nw = (D <= 128 && waves == 8) ? 8 : 4;
  const int ct = (D <= 128 && column_tiles == 2) ? 2 : 1;
  const int slot = (stream_part ? 8 : 0) + (ct == 2 ? 4 : 0) + (nw == 8 ? 2 : 0) + (int8_kv ? 1 : 0);
  if (cache[dev][slot] == 0) {
    int cus = 0, per_cu = 0, e = -1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    if constexpr (D <= 128) {
      if (nw == 8) e = ct == 2 ? resident_query<D, 8, 2>(int8_kv, stream_part, &per_cu)
                               : resident_query<D, 8, 1>(int8_kv, stream_part, &per_cu);
      else e = ct == 2 ? resident_query<D, 4, 2>(int8_kv, stream_part, &per_cu)
                       : resident_query<D, 4, 1>(int8_kv, stream_part, &per_cu);
    } else {
      e = resident_query<D, 4, 1>(int8_kv, stream_part, &per_cu);
    }
    if (e != 0 || per_cu <= 0 || cus <= 0) return 0;
    cache[dev][slot] = cus * per_cu;
  }
  return cache[dev][slot];
}

}  // namespace pa

// Paged-attention decode kernels for gfx950 (FP16 and INT8 KV), MFMA form.
//
// Work decomposition
//   A work item is (sequence, kv_head, split).  A work-group of 4 or 8 waves serves
//   one work item for the whole group of query heads that share the kv head
//   (up to 16), so every K/V byte fetched from HBM feeds all of them (the
//   reference launches one block per query head and re-reads KV G times,
//   kernels/paged_attention_v3_warp.cu:159).  The split's tokens are cut into
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
//   bias is removed from the scores with 1152*sum(q) per head and the V bias
//   with a packed fp16 subtraction.  s_k multiplies each score; s_v is folded
//   into the fp16 softmax weight, scaled by 2^e with e chosen per iteration
//   from the largest s_v so the weights stay normal and below fp16's range;
//   the running sum l accumulates the unscaled weight.
//
// Splits: FUSED (the single-launch warp variant) writes per-split partials
//   with device-coherent (write-through) stores, waits for them, counts
//   arrivals with a device-scope atomic, and the last work-group of a unit
//   merges with device-coherent loads in the same launch.  Otherwise
//   (split-K) a separate reduce kernel merges the partials
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
// long splits (>= 4096 tokens), where non-temporal K measured faster
// (config 3 FP16 3.6%; plain K stays ahead for INT8, ragged batches and
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
// 8 int8 values -> the same values in fp16 (exact).
__device__ __forceinline__ h8_t i8x8_exact(uint2 w) {
  uint32_t d[4];
  i8x4_to_biased_h2(w.x, d[0], d[1]);
  i8x4_to_biased_h2(w.y, d[2], d[3]);
#pragma unroll
  for (int k = 0; k < 4; ++k) d[k] = unbias_h2(d[k]);
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

// Merge the `ns` partials of one unit (gt heads) and write its fp16 output
// rows.  The partial of split sp sits in slot slot0 + sp * stride: acc[gt][D]
// (relative to its max) and (m, l) per head.  Thread i owns (head, 4-dim
// chunk) items i, i + THREADS, ... and merges them without LDS or barriers:
// the (m, l) pairs and accumulators of 8 splits at a time are loaded in one
// batch and folded into a running (max, sum, acc).
// COHERENT: device-coherent loads (partials written in this launch).
template <int D, int THREADS, bool COHERENT>
__device__ __forceinline__ void merge_splits(const float* __restrict__ pacc,
                                             const float* __restrict__ pml,
                                             half_t* __restrict__ out, size_t slot0, int stride,
                                             int gt, size_t out_base, int ns) {
  constexpr int CH = D / 4;
  constexpr int SB = 8;
  constexpr int POL = COHERENT ? kPolicyDevice : 0;
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));   // nothing lane-dependent is hoisted out of a caller's loop
  const int nitems = gt * CH;
  const uint32_t acc_bytes = (uint32_t)(gt * D * 4), ml_bytes = (uint32_t)(gt * 8);
  for (int i = tid; i < nitems; i += THREADS) {
    const int h = i / CH, c = i - h * CH;
    float M = kNegInf, L = 0.f;
    f4_t A = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < ns; s0 += SB) {
      f4_t v[SB];
      f2_t ml[SB];
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        // Past the last split the last one is re-read (and weighted 0), so
        // every load of the batch is unconditional.
        const size_t slot = slot0 + (size_t)min(s0 + u, ns - 1) * stride;
        const auto ra = buf_rsrc(pacc + slot * gt * D, acc_bytes);
        const auto rm = buf_rsrc(pml + slot * gt * 2, ml_bytes);
        v[u] = __builtin_bit_cast(f4_t, __builtin_amdgcn_raw_buffer_load_b128(ra, (h * D + 4 * c) * 4, 0, POL));
        ml[u] = __builtin_bit_cast(f2_t, __builtin_amdgcn_raw_buffer_load_b64(rm, h * 8, 0, POL));
      }
      float mb = M;
#pragma unroll
      for (int u = 0; u < SB; ++u)
        if (s0 + u < ns) mb = fmaxf(mb, ml[u].x);
      const float fo = M == kNegInf ? 0.f : exp2f_fast(M - mb);
      A *= fo;
      L *= fo;
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const float f = (s0 + u < ns && ml[u].x != kNegInf) ? exp2f_fast(ml[u].x - mb) : 0.f;
        A += v[u] * f;
        L += ml[u].y * f;
      }
      M = mb;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const uint2 pk = make_uint2(pack_h2(A[0] * inv, A[1] * inv), pack_h2(A[2] * inv, A[3] * inv));
    *reinterpret_cast<uint2*>(out + out_base + (size_t)h * D + 4 * c) = pk;
  }
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
struct alignas(16) DecodeSmem {
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

// The decode of one split.  FUSED: partials are written device-coherent and
// the last work-group of the unit merges them (single launch).  DIRECT1: a
// unit with one split writes its output here (else the split-K reduce does).
// `after_issue` runs in every wave once the wave's first K/V loads are issued
// (the scheduled kernel claims its next item there, so that no wait for this
// split's data also waits for the claim).
// `resolve(ctx, ns)` supplies the context length and split count once the
// split's block-id loads are in flight (the grid kernel reads them from
// memory then) and returns false when the split holds no tokens.
template <int D, int NW, bool I8, bool FUSED, bool DIRECT1, bool NTL, bool KNT,
          typename Resolve, typename AfterIssue>
__device__ __forceinline__ void decode_split(
    const half_t* __restrict__ q, const uint8_t* __restrict__ kc, const uint8_t* __restrict__ vc,
    const float* __restrict__ ksc, const float* __restrict__ vsc, const int* __restrict__ bt,
    half_t* __restrict__ out, float* __restrict__ pacc, float* __restrict__ pml,
    uint32_t* __restrict__ cnt, const DecodeShape& sh, SplitWork wk,
    DecodeSmem<D, NW>& sm, Resolve&& resolve, AfterIssue&& after_issue) {
  static_assert(D % 16 == 0 && D >= 64 && D <= 256, "head_dim: a multiple of 16 in [64, 256]");
  constexpr int KC = (D + 31) / 32;          // 32-dim k-chunks of one QK product
  constexpr int NT = D / 16;                 // 16-dim output tiles of PV
  constexpr int DG = D / 8;                  // 8-dim groups of a K row
  // With head_dim % 32 == 16 the last k-chunk holds 16 dims: its dim groups
  // 4(KC-1) + g for g >= 2 lie past the row.  Those lanes load the row's last
  // group instead (in bounds) and feed zeros to the MFMA; their query
  // operand is zero as well.
  constexpr bool KPAD = (D % 32) != 0;
  constexpr int PAIRS = D <= 128 ? 2 : 1;    // 32-token pairs per wave iteration
  constexpr int IT = 32 * PAIRS;             // tokens per wave iteration
  constexpr int ESZ = I8 ? 1 : 2;            // bytes per cache element
  using LVec = typename std::conditional<I8, uint2, uint4>::type;   // 8 elements
  // INT8 with head_dim <= 128 uses 16-byte loads throughout (W8): a K load
  // holds one dim group of two adjacent tokens (t, t + 1), which feed the
  // same row of the two QK MFMAs of a pair, and a V load holds 16 tokens of
  // one dim, which feed both pairs.  Each lane loads the scales of 4 tokens
  // and the others reach the lanes that need them by quad DPP broadcasts.
  constexpr bool W8 = I8 && D <= 128;

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
  const int r = lane & 15, g = lane >> 4;
  const int head0 = kvh * sh.group + chunk * gt;
  const int unit = (seq * sh.num_kv_heads + kvh) * sh.nchunk + chunk;
  const int* btrow = bt + (size_t)seq * sh.max_blocks;
  const int bs = sh.block_size, bsl = sh.bs_log2;
  const int hkv = sh.num_kv_heads;

  float m_run = kNegInf, l_part = 0.f;
  f4_t acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = (f4_t){0.f, 0.f, 0.f, 0.f};
  int e_cur = I8 ? 0 : 14;
  const float c = sh.scale_log2;

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
  // ---- query operand: lane (r, g) holds q[head r][32kk + 8g .. +7]
  h8_t qreg[KC];
  {
    const bool hv = r < gt;
    const half_t* qrow = q + ((size_t)seq * sh.num_heads + head0 + (hv ? r : 0)) * D + 8 * g;
#pragma unroll
    for (int kk = 0; kk < KC; ++kk) {
      const bool dv = !KPAD || kk < KC - 1 || 4 * kk + g < DG;
      const uint4 v = (hv && dv) ? *reinterpret_cast<const uint4*>(qrow + 32 * kk)
                                 : make_uint4(0, 0, 0, 0);
      qreg[kk] = __builtin_bit_cast(h8_t, v);
    }
  }
  float qbias = 0.f;
  if constexpr (I8) {
    float s = 0.f;
#pragma unroll
    for (int kk = 0; kk < KC; ++kk) {
      const uint4 v = __builtin_bit_cast(uint4, qreg[kk]);
      s = dot2(v.x, 0x3C003C00u, s);
      s = dot2(v.y, 0x3C003C00u, s);
      s = dot2(v.z, 0x3C003C00u, s);
      s = dot2(v.w, 0x3C003C00u, s);
    }
    qbias = 1152.f * head_sum(s);
  }

  if (!resolve(wk.ctx, wk.ns)) return;   // work-group uniform, before any barrier
  const int ns_eff = wk.ns;
  const int t_end = min(wk.ctx, t_begin + wk.partition);
  const int n_it = t_end > t_begin ? (t_end - t_begin + IT - 1) / IT : 0;
  const int nblk = t_end > t_begin ? min(((t_end - 1) >> bsl) - b_first + 1, nstage) : 0;
#pragma unroll
  for (int k = 0; k < kStageRegs; ++k) {
    const int i = tid + k * NW * kWave;
    if (i < nstage) sm.blk[i] = staged[k];
  }
  // LDS-only barrier: the writes above are complete (lgkmcnt 0) before it,
  // and no vector-memory wait is implied.
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __builtin_amdgcn_s_barrier();

  // ---- software-pipelined token loop: wave w takes iterations w, w + NW, ...
  // Once the K rows of its current iteration have fed the QK MFMAs it issues
  // the K rows of its next iteration; the V rows (plus INT8 scales) follow
  // once the PV MFMAs have consumed the V registers.  HBM traffic of the next
  // iteration overlaps this iteration's math.
  struct Blocks {
    int kb[PAIRS];
    int vb[PAIRS];
  };
  LVec kx[PAIRS][KC], ky[PAIRS][KC], vr[PAIRS][NT];
  float ksv[PAIRS][8], vsv[PAIRS][8];   // INT8 scales of this lane's 8 tokens
  int nvalid[PAIRS];                    // valid tokens among this lane's 8
  // W8: K rows of tokens (t, t + 1), and the V side of an iteration: V rows
  // of 16 tokens, the scales of the 4 tokens tok0 + 16g + 4(r & 3) + i, and the
  // valid tokens among the lane's 8 of each pair.
  uint4 kw[PAIRS][KC];
  uint4 vw[NT];
  // W8: the scales of the 4 tokens tok0 + 16g + 4(r & 3) + i and the valid
  // tokens among the lane's 8 of each pair.  They are loaded one iteration
  // ahead, with the K rows, so the softmax does not wait for the V rows (the
  // memory counter completes in order): `wa` holds the next iteration's, and
  // each iteration copies them out before loading the following ones.
  struct W8Buf {
    float4 ks4, vs4;
    int nvalid[PAIRS];
  };
  W8Buf wa;

  // Dim-group offset (relative to the lane's group g) of k-chunk kk's K row
  // load: 4 kk, or for the padding lanes of a 16-dim last chunk the row's
  // last group.
  auto kgroup = [&](int kk) { return (!KPAD || 4 * kk + g < DG) ? 4 * kk : DG - 1 - g; };
  auto load_blocks = [&](int it_, Blocks& b) {
    const int tok0 = t_begin + it_ * IT;
    if constexpr (W8) {
      // K rows of lane (r, g) lie in the 16-token group tok0 + 16(r >> 2), its V
      // rows and scales in tok0 + 16g; a group never straddles a block
      // (block_size is a multiple of 16).
      const int kg = tok0 + 16 * (r >> 2);
      const int tg = tok0 + 16 * g;
      const int ki = ((kg < t_end ? kg : t_begin) >> bsl) - b_first;
      const int vi = ((tg < t_end ? tg : t_begin) >> bsl) - b_first;
      b.kb[0] = sm.blk[ki < nblk ? ki : 0];
      b.vb[0] = sm.blk[vi < nblk ? vi : 0];
      return;
    }
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
      const int kg = tok0 + 32 * p + 8 * (r >> 2);
      const int tg = tok0 + 32 * p + 8 * g;
      const int ki = ((kg < t_end ? kg : t_begin) >> bsl) - b_first;
      const int vi = ((tg < t_end ? tg : t_begin) >> bsl) - b_first;
      b.kb[p] = sm.blk[ki < nblk ? ki : 0];
      b.vb[p] = sm.blk[vi < nblk ? vi : 0];
    }
  };
  // K rows: token tok0 + 32p + 8(r>>2) + (r&3) (first MFMA) and + 4 (second).
  auto issue_k = [&](int it_, const Blocks& b) {
    const int tok0 = t_begin + it_ * IT;
    if constexpr (W8) {
      // Row r of pair p: tokens tok0 + 16(r >> 2) + 8p + 2(r & 3) and + 1.
      const int kg = tok0 + 16 * (r >> 2);
      const int kgc = kg < t_end ? kg : t_begin;
      const int kb = (unsigned)b.kb[0] < (unsigned)sh.num_blocks ? b.kb[0] : 0;
      const uint8_t* kp = kc + ((((size_t)kb * hkv + kvh) * (D / 8) + g) * bs +
                                (kgc & (bs - 1)) + 2 * (r & 3)) * 8;
#pragma unroll
      for (int p = 0; p < PAIRS; ++p)
#pragma unroll
        for (int kk = 0; kk < KC; ++kk)
          kw[p][kk] = load_tile<uint4, KNT>(kp + (size_t)kgroup(kk) * bs * 8 + 64 * p);
      return;
    }
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
      const int kg = tok0 + 32 * p + 8 * (r >> 2);
      const int kgc = kg < t_end ? kg : t_begin;
      const int kb = (unsigned)b.kb[p] < (unsigned)sh.num_blocks ? b.kb[p] : 0;
      const int koff = (kgc & (bs - 1)) + (r & 3);
      const uint8_t* kp = kc + ((((size_t)kb * hkv + kvh) * (D / 8) + g) * bs + koff) * 8 * ESZ;
#pragma unroll
      for (int kk = 0; kk < KC; ++kk) {
        const uint8_t* p0 = kp + (size_t)kgroup(kk) * bs * 8 * ESZ;
        kx[p][kk] = load_tile<LVec, KNT>(p0);
        ky[p][kk] = load_tile<LVec, KNT>(p0 + 4 * 8 * ESZ);
      }
    }
  };
  // V rows (dims 16t + r) and the lane's score tokens tok0 + 32p + 8g .. +7.
  // W8: the scales and valid counts of an iteration (see W8Buf).
  auto issue_scales = [&](int it_, const Blocks& b, W8Buf& B) {
    const int tg = t_begin + it_ * IT + 16 * g;
    const int tgc = tg < t_end ? tg : t_begin;
    const bool vok = (unsigned)b.vb[0] < (unsigned)sh.num_blocks;
    const int vb = vok ? b.vb[0] : 0;
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
      const int t0 = tg + 8 * p;
      B.nvalid[p] = (vok && t0 < t_end) ? min(8, t_end - t0) : 0;
    }
    const size_t slot = ((size_t)vb * hkv + kvh) * bs + (tgc & (bs - 1)) + 4 * (r & 3);
    // (plain loads: a scale line holds several kv heads' scales)
    B.ks4 = *reinterpret_cast<const float4*>(ksc + slot);
    B.vs4 = *reinterpret_cast<const float4*>(vsc + slot);
  };
  auto issue_v = [&](int it_, const Blocks& b, W8Buf& B) {
    const int tok0 = t_begin + it_ * IT;
    if constexpr (W8) {
      // V rows: dim 16t + r, tokens tok0 + 16g .. + 15 (pair p uses 8p .. 8p + 7).
      const int tg = tok0 + 16 * g;
      const int tgc = tg < t_end ? tg : t_begin;
      const int vb = (unsigned)b.vb[0] < (unsigned)sh.num_blocks ? b.vb[0] : 0;
      const uint8_t* vp = vc + (((size_t)vb * hkv + kvh) * D + r) * bs + (tgc & (bs - 1));
#pragma unroll
      for (int t = 0; t < NT; ++t) vw[t] = load_tile<uint4, NTL>(vp + (size_t)(16 * t) * bs);
      return;
    }
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
      const int tg = tok0 + 32 * p + 8 * g;
      const bool tin = tg < t_end;
      const int tgc = tin ? tg : t_begin;
      const bool vok = (unsigned)b.vb[p] < (unsigned)sh.num_blocks;
      const int vb = vok ? b.vb[p] : 0;
      const int voff = tgc & (bs - 1);
      nvalid[p] = (tin && vok) ? min(8, t_end - tg) : 0;
      const size_t slot = ((size_t)vb * hkv + kvh) * bs + voff;
      const uint8_t* vp = vc + ((((size_t)vb * hkv + kvh) * D + r) * bs + voff) * ESZ;
#pragma unroll
      for (int t = 0; t < NT; ++t)
        vr[p][t] = load_tile<LVec, NTL>(vp + (size_t)(16 * t) * bs * ESZ);
      if constexpr (I8) {
        const float4 a0 = *reinterpret_cast<const float4*>(ksc + slot);
        const float4 a1 = *reinterpret_cast<const float4*>(ksc + slot + 4);
        const float4 b0 = *reinterpret_cast<const float4*>(vsc + slot);
        const float4 b1 = *reinterpret_cast<const float4*>(vsc + slot + 4);
        ksv[p][0] = a0.x; ksv[p][1] = a0.y; ksv[p][2] = a0.z; ksv[p][3] = a0.w;
        ksv[p][4] = a1.x; ksv[p][5] = a1.y; ksv[p][6] = a1.z; ksv[p][7] = a1.w;
        vsv[p][0] = b0.x; vsv[p][1] = b0.y; vsv[p][2] = b0.z; vsv[p][3] = b0.w;
        vsv[p][4] = b1.x; vsv[p][5] = b1.y; vsv[p][6] = b1.z; vsv[p][7] = b1.w;
      }
    }
  };

  // The loop is rotated so that every load inside it is unconditional: the
  // body issues the next K, finishes the current iteration (softmax, PV),
  // issues the next V, then runs QK of the next iteration.  The wait for K inside the body therefore never covers the V rows
  // issued after it; the last iteration's softmax and PV run after the loop.
  if (w < n_it) {
    auto softmax_pv = [&](float (&s)[PAIRS][8], bool need_mask, W8Buf& B) {
      // ---- online softmax (lane-local except the per-head max)
      float mloc = kNegInf;
      // W8: this lane's 4 scales; token 16g + 8p + j of the lane's row is held
      // by quad position 2p + (j >> 2), element j & 3.
      float ksa[4] = {B.ks4.x, B.ks4.y, B.ks4.z, B.ks4.w};
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
            s[p][j] = (s[p][j] - qbias) * (ksj * c);
          }
      } else {
#pragma unroll
        for (int p = 0; p < PAIRS; ++p)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            float v;
            if constexpr (I8) v = (s[p][j] - qbias) * (ksv[p][j] * c);
            else v = s[p][j] * c;
            s[p][j] = v;
          }
      }
      if (need_mask) {
#pragma unroll
        for (int p = 0; p < PAIRS; ++p)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            s[p][j] = j < nval(p) ? s[p][j] : kNegInf;
            if constexpr (I8 && !W8) vsv[p][j] = j < nval(p) ? vsv[p][j] : 0.f;
          }
      }
#pragma unroll
      for (int p = 0; p < PAIRS; ++p)
#pragma unroll
        for (int j = 0; j < 8; ++j) mloc = fmaxf(mloc, s[p][j]);
      const float m_new = fmaxf(m_run, head_max(mloc));
      const float m_use = m_new == kNegInf ? 0.f : m_new;
      const float alpha_m = exp2f_fast(m_run - m_use);   // rescales l
      float alpha_acc = alpha_m;                         // rescales acc (incl. weight exponent)
      m_run = m_new;
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
        // Keep the weight exponent while the largest weight stays in [2^12, 2^15).
        const float top = __builtin_amdgcn_ldexpf(msv, e_cur);
        if (msv > 0.f && (top >= 32768.f || top < 4096.f)) {
          int e_new = 15 - __builtin_amdgcn_frexp_expf(msv);
          e_new = e_new < 0 ? 0 : (e_new > 30 ? 30 : e_new);
          alpha_acc = __builtin_amdgcn_ldexpf(alpha_m, e_new - e_cur);
          e_cur = e_new;
        }
        wsc = __builtin_amdgcn_ldexpf(1.f, e_cur);
      } else {
        wsc = 16384.f;
      }
      float lsum = 0.f;
      h8_t pb[PAIRS];
#pragma unroll
      for (int p = 0; p < PAIRS; ++p) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float pj = exp2f_fast(s[p][j] - m_use);
          lsum += pj;
          float wj;
          if constexpr (W8) wj = pj * quad_bcast(vsa[j & 3], 2 * p + (j >> 2)) * wsc;
          else if constexpr (I8) wj = pj * vsv[p][j] * wsc;
          else wj = pj * wsc;
          pb[p][j] = (half_t)wj;
        }
      }
      l_part = l_part * alpha_m + lsum;
      if (__builtin_amdgcn_ballot_w64(alpha_acc != 1.f) != 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] *= alpha_acc;
      }

      // ---- PV
#pragma unroll
      for (int p = 0; p < PAIRS; ++p) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          h8_t av;
          if constexpr (W8) {
            av = i8x8_exact(p == 0 ? make_uint2(vw[t].x, vw[t].y)
                                   : make_uint2(vw[t].z, vw[t].w));
          } else if constexpr (I8) {
            av = i8x8_exact(vr[p][t]);
          } else {
            uint4 v = vr[p][t];
            if (need_mask) v = keep_first(v, nval(p));
            av = __builtin_bit_cast(h8_t, v);
          }
          acc[t] = mfma16(av, pb[p], acc[t]);
        }
      }
    };
    auto qk = [&](float (&s)[PAIRS][8]) {
      // ---- QK: scores of tokens tok0 + 32p + 8g + j for head r (W8: tok0 + 16g + 8p + j)
#pragma unroll
      for (int p = 0; p < PAIRS; ++p) {
        f4_t sx = {0.f, 0.f, 0.f, 0.f}, sy = {0.f, 0.f, 0.f, 0.f};
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
          sx = mfma16(ax, qreg[kk], sx);
          sy = mfma16(ay, qreg[kk], sy);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (W8) {
            // rows 4g + e: tokens tok0 + 16g + 8p + 2e (sx) and + 1 (sy)
            s[p][2 * e] = sx[e];
            s[p][2 * e + 1] = sy[e];
          } else {
            s[p][e] = sx[e];
            s[p][4 + e] = sy[e];
          }
        }
      }
    };
    auto mask_needed = [&](const W8Buf& B) {
      // Tokens past the end or in invalid blocks exist only in the last
      // iteration of a split (or with a corrupt block table).
      bool short_lane = false;
#pragma unroll
      for (int p = 0; p < PAIRS; ++p) {
        if constexpr (W8) short_lane = short_lane || B.nvalid[p] < 8;
        else short_lane = short_lane || nvalid[p] < 8;
      }
      return __builtin_amdgcn_ballot_w64(short_lane) != 0;
    };
    {
      Blocks b0;
      load_blocks(w, b0);
      if constexpr (W8) issue_scales(w, b0, wa);
      issue_k(w, b0);
      __builtin_amdgcn_sched_barrier(0);
      issue_v(w, b0, wa);
      __builtin_amdgcn_sched_barrier(0);
    }
    after_issue();
    float s[PAIRS][8];
    qk(s);
    __builtin_amdgcn_sched_barrier(0);
    int nxt = w + NW;
    // One iteration: the next iteration's K rows (and, W8, its scales) go out,
    // this iteration's softmax and PV run, then the next V rows go out and
    // the next QK runs.
    while (nxt < n_it) {
      W8Buf cur = wa;   // W8: this iteration's scales, loaded one iteration ago
      Blocks bn;
      load_blocks(nxt, bn);
      if constexpr (W8) issue_scales(nxt, bn, wa);
      issue_k(nxt, bn);
      __builtin_amdgcn_sched_barrier(0);
      softmax_pv(s, mask_needed(cur), cur);
      __builtin_amdgcn_sched_barrier(0);
      issue_v(nxt, bn, wa);
      __builtin_amdgcn_sched_barrier(0);
      qk(s);
      __builtin_amdgcn_sched_barrier(0);
      nxt += NW;
    }
    softmax_pv(s, mask_needed(wa), wa);
  } else {
    after_issue();
  }

  // ---- per-wave results: m (head r), l, acc (dims 16t + 4g + e)
  float l_run = head_sum(l_part);
  const float unscale = __builtin_amdgcn_ldexpf(1.f, -e_cur);
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] *= unscale;

  // ---- every wave's state goes to LDS; then each thread merges the NW
  // states of its (head, 4-dim chunk) items and writes them out: the output
  // when the unit has one split, else this split's partial.
  if (r < gt) {
    if (g == 0) {
      sm.m[w][r] = m_run;
      sm.l[w][r] = l_run;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
      *reinterpret_cast<f4_t*>(&sm.a[w][r][16 * t + 4 * g]) = acc[t];
  }
  __syncthreads();

  constexpr int CH = D / 4;
  const size_t out_base = ((size_t)seq * sh.num_heads + head0) * D;
  const bool final_here = (FUSED || DIRECT1) && ns_eff == 1;
  const size_t slot = wk.slot0 + (size_t)split * wk.stride;
  const auto racc = buf_rsrc(pacc + slot * gt * D, (uint32_t)(gt * D * 4));
  const auto rml = buf_rsrc(pml + slot * gt * 2, (uint32_t)(gt * 8));
  for (int i = tid; i < gt * CH; i += NW * kWave) {
    const int h = i / CH, c = i - h * CH;
    float mw[NW], M = kNegInf;
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      mw[v] = sm.m[v][h];
      M = fmaxf(M, mw[v]);
    }
    f4_t A = {0.f, 0.f, 0.f, 0.f};
    float L = 0.f;
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const float f = mw[v] == kNegInf ? 0.f : exp2f_fast(mw[v] - M);
      L += sm.l[v][h] * f;
      A += *reinterpret_cast<const f4_t*>(&sm.a[v][h][4 * c]) * f;
    }
    if (final_here) {
      const float inv = L > 0.f ? 1.f / L : 0.f;
      const uint2 pk = make_uint2(pack_h2(A[0] * inv, A[1] * inv), pack_h2(A[2] * inv, A[3] * inv));
      *reinterpret_cast<uint2*>(out + out_base + (size_t)h * D + 4 * c) = pk;
    } else {
      // FUSED: device-coherent (write-through) stores, visible to every XCD
      // once this thread's stores are acknowledged.
      constexpr int POL = FUSED ? kPolicyDevice : 0;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4_t, A), racc,
                                             (h * D + 4 * c) * 4, 0, POL);
      if (c == 0) {
        const f2_t ml = {M, L};
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2_t, ml), rml, h * 8, 0, POL);
      }
    }
  }
  if constexpr (FUSED) {
    if (ns_eff > 1) {
      // Wait until this thread's partial stores are acknowledged, then count
      // the arrival; the last work-group of the unit merges every split.
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_waitcnt(0);
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __syncthreads();
      if (threadIdx.x == 0) {
        const uint32_t prev =
            __hip_atomic_fetch_add(cnt + unit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sm.last = prev == (uint32_t)(ns_eff - 1);
      }
      __syncthreads();
      if (sm.last) {
        merge_splits<D, NW * kWave, true>(pacc, pml, out, wk.slot0, wk.stride, gt, out_base,
                                          ns_eff);
        if (threadIdx.x == 0)
          __hip_atomic_store(cnt + unit, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// Grid form: one work-group per (unit, split) slot of the host's plan.
template <int D, int NW, bool I8, bool FUSED, bool NTL, bool KNT>
__global__ void __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(2)))
decode_kernel(const int* __restrict__ bt, const int* __restrict__ ctxl, PA_SHAPE_HEAD_PARAMS,
              DecodeShape sh_tail, const half_t* __restrict__ q, const uint8_t* __restrict__ kc,
              const uint8_t* __restrict__ vc, const float* __restrict__ ksc,
              const float* __restrict__ vsc, half_t* __restrict__ out, float* __restrict__ pacc,
              float* __restrict__ pml, uint32_t* __restrict__ cnt) {
  PA_SHAPE_REBUILD(sh, sh_tail);
  static_assert(sizeof(DecodeSmem<D, NW>) * (kWavesPerCU / NW) <= kLdsPerCU, "LDS budget");
  __shared__ DecodeSmem<D, NW> sm;

  // ---- work item (XCD-aware).  With at least 8 (sequence, split) items, an
  // item's kv heads and head chunks get work-group indices 8 apart, so they
  // share blockIdx % 8 (their XCD under round-robin dispatch), run at about
  // the same time and meet in that XCD's L2: they read the same block-table
  // lines, the head chunks of a kv head the same K/V tiles, and with INT8 all
  // kv heads of a block the same scale lines (the block's scales are
  // adjacent).  With fewer items that would leave XCDs idle, so the kv heads
  // are spread over the XCDs and only the head chunks are grouped.
  const int wg = blockIdx.x;
  const bool by_item = sh.num_items >= 8;
  const int per = by_item ? sh.num_kv_heads * sh.nchunk : sh.nchunk;
  const int grp = wg / (8 * per);
  const int rem = wg - grp * 8 * per;
  const int sub = rem >> 3;
  const int idx = grp * 8 + (rem & 7);
  int seq, kvh, chunk, split;
  if (by_item) {
    if (idx >= sh.num_items) return;
    split = idx % sh.nsplit;
    seq = idx / sh.nsplit;
    kvh = sub / sh.nchunk;
    chunk = sub - kvh * sh.nchunk;
  } else {
    if (idx >= sh.num_items * sh.num_kv_heads) return;
    split = idx % sh.nsplit;
    const int sk = idx / sh.nsplit;
    kvh = sk % sh.num_kv_heads;
    seq = sk / sh.num_kv_heads;
    chunk = sub;
  }

  // Contexts are clamped to what the block table holds and to what the grid's
  // splits cover, so no work-group reads past the table or the partials.
  // The length is used only after the split's block-id loads are issued.  It
  // is read with a vector load at the top: a scalar load would be scheduled
  // next to its first use, after the argument fetches of the query pointer.
  int zero = 0;
  asm volatile("" : "+v"(zero));
  const int ctx_lane = ctxl[seq + zero];
  const int unit = (seq * sh.num_kv_heads + kvh) * sh.nchunk + chunk;
  const SplitWork wk{seq, kvh, chunk, split, 0, sh.partition, 0, (size_t)unit * sh.nsplit, 1};
  auto resolve = [&](int& ctx, int& ns) {
    const int ctx_raw = __builtin_amdgcn_readfirstlane(ctx_lane);
    const int cap = min(sh.max_blocks * sh.block_size, sh.nsplit * sh.partition);
    ctx = ctx_raw < 0 ? 0 : (ctx_raw > cap ? cap : ctx_raw);
    ns = ctx > 0 ? (ctx + sh.partition - 1) / sh.partition : 1;
    return split < ns;
  };
  decode_split<D, NW, I8, FUSED, false, NTL, KNT>(q, kc, vc, ksc, vsc, bt, out, pacc, pml, cnt, sh, wk,
                                             sm, resolve, [] {});
}

// ---------------------------------------------------------------------------
// In-kernel schedule: persistent work-groups over a compact work list.
//
// Every work-group reads the (clamped) context lengths and derives the same
// schedule in LDS.  The partition P is chosen from the total token count:
// about one item per resident work-group when all lengths are equal (the
// grid plan's shape), about kSchedItemsPerGroup items per work-group
// otherwise.  A row is one split of one sequence; rows that hold a full
// partition come first, the shorter last rows of each sequence after them
// (largest items first).  An item is (row, kv head, head chunk).  Items are
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
  int* info;          // [1 + num_seqs]: partition, slot row base per sequence (for the reduce)
  uint32_t* queue;    // 8 claim counters, kSchedQueueStride words apart
  int rows_max;       // slot rows the partial buffers hold
  int pmin, pmax;     // partition bounds (multiples of kIterTokens)
  int pmin_uniform;   // lower bound when all lengths are equal (one item per work-group)
};

struct SchedSmem {
  int full_pre[kSchedMaxSeqs + 1];   // exclusive prefix of full rows per sequence
  int part_pre[kSchedMaxSeqs + 1];   // exclusive prefix of short last rows
  uint16_t rem[kSchedMaxSeqs];       // context length % P (P <= 8192)
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
    // items measured faster: config 4 32k INT8 93.6 -> 91.8 us), about
    // kSchedItemsPerGroup per work-group otherwise; within [pmin, pmax] and
    // no longer than the longest sequence.
    constexpr uint64_t kGroupsPerCU = kWavesPerCU / NWV;
    const uint64_t groups = sc.uniform ? (gridDim.x + kGroupsPerCU - 1) / kGroupsPerCU : gridDim.x;
    const uint64_t k = sc.uniform ? 1 : kSchedItemsPerGroup;
    uint64_t part = ((t << 10) * (uint64_t)sh.num_kv_heads + groups * k - 1) / (groups * k);
    part = (part + kIterTokens - 1) / kIterTokens * kIterTokens;
    // The ragged lower bound keeps items of a few hundred tokens from paying
    // their fixed costs too often; with equal lengths every resident
    // work-group gets one item, so the smaller grid bound applies.
    const uint64_t lo = sc.uniform ? (uint64_t)sa.pmin_uniform : (uint64_t)sa.pmin;
    part = part < lo ? lo : (part > (uint64_t)sa.pmax ? (uint64_t)sa.pmax : part);
    const uint64_t top = ((uint64_t)(b > 0 ? b : 1) + kIterTokens - 1) / kIterTokens * kIterTokens;
    sc.partition = (int)(part < top ? part : top);
  }
  // Exclusive scans of full rows (ctx / P) and short last rows (0 or 1); the
  // partition doubles (rarely) until the rows fit the partial buffers, which
  // hold them at the upper partition bound.
  while (true) {
    const int P = sc.partition;
    int fs = 0, ps = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = tid * E + e;
      fs += i < S ? c[e] / P : 0;
      ps += i < S ? ((c[e] % P != 0 || c[e] == 0) ? 1 : 0) : 0;
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
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = tid * E + e;
      if (i < S) {
        ss.full_pre[i] = fo;
        ss.part_pre[i] = po;
        ss.rem[i] = (uint16_t)(c[e] % P);
        fo += c[e] / P;
        po += (c[e] % P != 0 || c[e] == 0) ? 1 : 0;
      }
    }
    if (tid == 0) {
      ss.full_pre[S] = tf;
      ss.part_pre[S] = tp;
    }
    sc.n_full = tf;
    sc.n_rows = tf + tp;
    break;
  }
  __syncthreads();
  return sc;
}

template <int D, int NW, bool I8, bool FUSED, bool NTL>
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
  const Schedule sc = build_schedule<NW * kWave>(ctxl, sh, sa, ss);

  const int S = sh.num_seqs, hkv = sh.num_kv_heads, nchunk = sh.nchunk;
  const int P = __builtin_amdgcn_readfirstlane(sc.partition);
  const int n_full = __builtin_amdgcn_readfirstlane(sc.n_full);
  // Claim class of this work-group (its XCD under the usual round-robin
  // dispatch): rows r with r % 8 == cls, each followed by its kv heads and
  // head chunks, so every XCD reads every kv head and the chunks of one
  // (row, kv head) run at about the same time on one XCD and share its L2.
  const int n_rows = __builtin_amdgcn_readfirstlane(sc.n_rows);
  const int per_row = hkv * nchunk;
  const int cls = blockIdx.x & 7;
  const int groups_c = ((int)gridDim.x - cls + 7) >> 3;
  const int items_c = (n_rows > cls ? (n_rows - cls + 7) >> 3 : 0) * per_row;
  uint32_t* queue = sa.queue + cls * kSchedQueueStride;
  // Item indices are compared unsigned: whatever a claim counter holds, no
  // work-group leaves its class's item list.
  int idx = blockIdx.x >> 3;   // index within the class: static first item
  // With no more items than work-groups in the class (equal lengths give one
  // item per work-group) the static first items cover the class: no claims,
  // and the counter stays at zero.
  const bool claims = items_c > groups_c;
  while ((uint32_t)idx < (uint32_t)items_c) {
    // The next item is claimed once this item's first loads are out.
    uint32_t old = 0;
    auto claim = [&] {
      if (claims && threadIdx.x == 0)
        old = __hip_atomic_fetch_add(queue, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    const int row = cls + 8 * (idx / per_row);
    const int sub = idx - (idx / per_row) * per_row;
    const int kvh = sub / nchunk, chunk = sub - (sub / nchunk) * nchunk;
    // Item fields are work-group uniform: keep them in scalar registers.
    int seq, split;
    if (row < n_full) {
      seq = prefix_search(ss.full_pre, S, row);
      split = row - ss.full_pre[seq];
    } else {
      seq = prefix_search(ss.part_pre, S, row - n_full);
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
    decode_split<D, NW, I8, FUSED, true, NTL, false>(q, kc, vc, ksc, vsc, bt, out, pacc, pml, cnt, sh,
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
  // The split-K reduce reads the partition and the slot row bases.
  if (!FUSED && blockIdx.x == 0) {
    if (threadIdx.x == 0) sa.info[0] = P;
    for (int i = threadIdx.x; i < S; i += NW * kWave) sa.info[1 + i] = ss.full_pre[i] + ss.part_pre[i];
  }
}

// Split-K reduce over the in-kernel schedule: one work-group per unit; units
// with a single split were written by the partition kernel.
template <int D>
__global__ void __launch_bounds__(kThreads)
sched_reduce_kernel(const float* __restrict__ pacc, const float* __restrict__ pml,
                    const int* __restrict__ ctxl, const int* __restrict__ info,
                    half_t* __restrict__ out, DecodeShape sh, int rows_max) {
  const int unit = blockIdx.x;
  const int chunk = unit % sh.nchunk;
  const int sk = unit / sh.nchunk;
  const int kvh = sk % sh.num_kv_heads;
  const int seq = sk / sh.num_kv_heads;
  const int cap = sh.max_blocks * sh.block_size;
  int ctx = ctxl[seq];
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int P = info[0];
  if (P < kIterTokens) return;   // (the partition kernel always writes it)
  const int ns = ctx > 0 ? (ctx + P - 1) / P : 1;
  if (ns <= 1) return;
  const int rb = info[1 + seq];
  if (rb < 0 || rb > rows_max - ns) return;   // slots stay inside the partial buffers
  const size_t rowbase = (size_t)rb;
  const int head0 = kvh * sh.group + chunk * sh.head_tile;
  merge_splits<D, kThreads, false>(
      pacc, pml, out, (rowbase * sh.num_kv_heads + kvh) * sh.nchunk + chunk,
      sh.num_kv_heads * sh.nchunk, sh.head_tile, ((size_t)seq * sh.num_heads + head0) * D, ns);
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
  merge_splits<D, kThreads, false>(pacc, pml, out, (size_t)unit * sh.nsplit, 1, sh.head_tile,
                                   ((size_t)seq * sh.num_heads + head0) * D, ns_eff);
}

template <int D, int NW, bool I8, bool NTL, bool KNT>
hipError_t launch_decode_grid(const DecodeLaunch& l, int grid) {
  const DecodeShape& sh = l.shape;
  const auto* q = static_cast<const half_t*>(l.q);
  const auto* kc = static_cast<const uint8_t*>(l.k_cache);
  const auto* vc = static_cast<const uint8_t*>(l.v_cache);
  auto* out = static_cast<half_t*>(l.out);
  if (l.fused) {
    decode_kernel<D, NW, I8, true, NTL, KNT><<<grid, NW * kWave, 0, l.stream>>>(
        l.block_table, l.context_lens, PA_SHAPE_HEAD_ARGS(sh), sh, q, kc, vc, l.k_scales, l.v_scales, out, l.part_acc,
        l.part_ml, l.counters);
    return hipGetLastError();
  }
  decode_kernel<D, NW, I8, false, NTL, KNT><<<grid, NW * kWave, 0, l.stream>>>(
      l.block_table, l.context_lens, PA_SHAPE_HEAD_ARGS(sh), sh, q, kc, vc, l.k_scales, l.v_scales, out, l.part_acc,
      l.part_ml, l.counters);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int units = sh.num_seqs * sh.num_kv_heads * sh.nchunk;
  splitk_reduce_kernel<D><<<units, kThreads, 0, l.stream>>>(l.part_acc, l.part_ml, l.context_lens,
                                                            out, sh);
  return hipGetLastError();
}

template <int D, int NW, bool I8, bool NTL>
hipError_t launch_decode_waves(const DecodeLaunch& l) {
  const DecodeShape& sh = l.shape;
  if (l.sched) {
    const SchedArgs sa{l.sched_info, l.queue, l.rows_max, l.pmin, l.pmax, l.pmin_uniform};
    const auto* q = static_cast<const half_t*>(l.q);
    const auto* kc = static_cast<const uint8_t*>(l.k_cache);
    const auto* vc = static_cast<const uint8_t*>(l.v_cache);
    auto* out = static_cast<half_t*>(l.out);
    if (l.fused) {
      decode_sched_kernel<D, NW, I8, true, NTL><<<l.groups, NW * kWave, 0, l.stream>>>(
          l.block_table, l.context_lens, PA_SHAPE_HEAD_ARGS(sh), sh, q, kc, vc, l.k_scales, l.v_scales, out, l.part_acc,
          l.part_ml, l.counters, sa);
      return hipGetLastError();
    }
    decode_sched_kernel<D, NW, I8, false, NTL><<<l.groups, NW * kWave, 0, l.stream>>>(
        l.block_table, l.context_lens, PA_SHAPE_HEAD_ARGS(sh), sh, q, kc, vc, l.k_scales, l.v_scales, out, l.part_acc,
        l.part_ml, l.counters, sa);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int units = sh.num_seqs * sh.num_kv_heads * sh.nchunk;
    sched_reduce_kernel<D><<<units, kThreads, 0, l.stream>>>(
        l.part_acc, l.part_ml, l.context_lens, l.sched_info, out, sh, l.rows_max);
    return hipGetLastError();
  }
  // Groups of 8 items with their kv heads and head chunks, or, below 8 items,
  // of 8 (item, kv head) pairs with their head chunks (see decode_kernel).
  const int grid = sh.num_items >= 8
                       ? (sh.num_items + 7) / 8 * 8 * sh.num_kv_heads * sh.nchunk
                       : (sh.num_items * sh.num_kv_heads + 7) / 8 * 8 * sh.nchunk;
  if constexpr (!I8 && NTL) {
    if (l.k_nt) return launch_decode_grid<D, NW, I8, NTL, true>(l, grid);
  }
  return launch_decode_grid<D, NW, I8, NTL, false>(l, grid);
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

// Resident work-groups of the scheduled kernel for one head_dim (cached per
// device and variant).
template <int D>
int sched_groups_d(int waves, bool int8_kv) {
  static int cache[64][4] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  const int nw = (D <= 128 && waves == 8) ? 8 : 4;
  const int slot = (nw == 8 ? 2 : 0) + (int8_kv ? 1 : 0);
  if (cache[dev][slot] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    hipError_t e;
    if (nw == 8) {
      if constexpr (D <= 128) {
        e = int8_kv ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
                          &per_cu, decode_sched_kernel<D, 8, true, true, true>, 8 * kWave, 0)
                    : hipOccupancyMaxActiveBlocksPerMultiprocessor(
                          &per_cu, decode_sched_kernel<D, 8, false, true, true>, 8 * kWave, 0);
      } else {
        e = hipErrorInvalidValue;
      }
    } else {
      e = int8_kv ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
                        &per_cu, decode_sched_kernel<D, 4, true, true, true>, 4 * kWave, 0)
                  : hipOccupancyMaxActiveBlocksPerMultiprocessor(
                        &per_cu, decode_sched_kernel<D, 4, false, true, true>, 4 * kWave, 0);
    }
    if (e != hipSuccess || per_cu <= 0 || cus <= 0) return 0;
    cache[dev][slot] = cus * per_cu;
  }
  return cache[dev][slot];
}

}  // namespace pa

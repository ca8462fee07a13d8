// Paged-attention decode kernels for gfx950 (FP16 and INT8 KV).
//
// Work decomposition
//   A work item is (sequence, kv_head, split).  A work-group of 4 waves
//   serves one work item for a tile of GT query heads of that kv head, so
//   every K/V byte fetched from HBM feeds GT heads (the reference launches
//   one block per query head and re-reads KV G times,
//   kernels/paged_attention_v3_warp.cu:159).  The split's token range is cut
//   into 64-token iterations dealt round-robin to the 4 waves; each wave
//   keeps its own online-softmax state and the waves merge through LDS.
//
// Inside one wave iteration (64 tokens = 4 slabs of 16 tokens)
//   QK: lane l owns token 16*(l>>4) + (l&15) and reads that token's whole K
//       row: head_dim/8 loads of 16 B (fp16) or 8 B (int8).  The query is
//       wave-uniform and comes from scalar loads, so no cross-lane reduction
//       is needed for the dot product (v_dot2: two fp16 MACs per op).
//   softmax: one wave max per head (DPP + permlane swaps), exp2 with
//       scale*log2(e) folded in, running (m, l) as in the reference
//       (paged_attention_v3_warp.cu:84-99).
//   PV: lane l owns head dims (l>>1) + 32j and the 8 tokens (l&1)*8.. of
//       each slab, i.e. one 16-B (fp16) / 8-B (int8) load of a V row per
//       (slab, j); softmax weights come back from LDS as packed fp16.
//
// INT8: K is converted to fp16 holding 1152 + k (exact), and the bias is
//   removed from the dot product with 1152*sum(q); the per-token K scale
//   multiplies the dot once (paged_attention_v5_warp_int8.cu:80-85).  V is
//   converted exactly to fp16 integers and its per-token scale is folded into
//   the softmax weight (v5:99-108) while l accumulates the unscaled weight.
//   Weights are stored in fp16 multiplied by 2^e with e chosen per iteration
//   from the largest V scale, so they never overflow fp16 and stay normal.
//
// Splits: `fused` (the single-launch warp variant) writes per-split partials
//   and the last work-group to finish a unit merges them in the same launch;
//   otherwise (split-K) a separate reduce kernel merges them
//   (paged_attention_v4_splitk.cu:156-187).
#pragma once

#include <math.h>

#include <type_traits>

#include "pa_device.hpp"
#include "pa_internal.hpp"

namespace pa {

constexpr int kThreads = kWavesPerGroup * kWave;
constexpr float kNegInf = -INFINITY;

__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }

template <int D, int GT>
struct alignas(16) DecodeSmem {
  uint16_t p[kWavesPerGroup][4][GT][16];   // fp16 softmax weights per slab / head / token
  float m[kWavesPerGroup][GT];
  float l[kWavesPerGroup][GT];
  float a[kWavesPerGroup][GT][D];
  int last;
};

// Merge `ns` split partials of one unit and write the fp16 output rows.
template <int D, int GT>
__device__ __forceinline__ void merge_partials(const float* __restrict__ pacc,
                                               const float* __restrict__ pml, half_t* __restrict__ out,
                                               size_t part_base, size_t out_base, int ns) {
  for (int idx = threadIdx.x; idx < GT * D; idx += kThreads) {
    const int hh = idx / D;
    const int d = idx - hh * D;
    float mx = kNegInf;
    for (int s = 0; s < ns; ++s) mx = fmaxf(mx, pml[((part_base + s) * GT + hh) * 2]);
    float a = 0.f, l = 0.f;
    for (int s = 0; s < ns; ++s) {
      const size_t pi = (part_base + s) * GT + hh;
      const float ms = pml[pi * 2];
      const float f = (ms == kNegInf) ? 0.f : exp2f_fast(ms - mx);
      l += pml[pi * 2 + 1] * f;
      a += pacc[pi * D + d] * f;
    }
    out[out_base + (size_t)hh * D + d] = (half_t)(l > 0.f ? a / l : 0.f);
  }
}

template <int D, int GT, bool I8, bool FUSED>
__global__ void __launch_bounds__(kThreads)
decode_kernel(const half_t* __restrict__ q, const uint8_t* __restrict__ kc,
              const uint8_t* __restrict__ vc, const float* __restrict__ ksc,
              const float* __restrict__ vsc, const int* __restrict__ bt,
              const int* __restrict__ ctxl, half_t* __restrict__ out, float* __restrict__ pacc,
              float* __restrict__ pml, uint32_t* __restrict__ cnt, DecodeShape sh) {
  constexpr int NO = D / 8;         // K groups of 8 dims per token
  constexpr int JV = D / 32;        // V rows per lane per slab
  constexpr int ESZ = I8 ? 1 : 2;   // bytes per cache element
  constexpr bool VEARLY = D <= 128; // issue all V loads before the QK math
  using KVec = typename std::conditional<I8, uint2, uint4>::type;

  __shared__ DecodeSmem<D, GT> sm;

  // ---- work item (XCD-aware: the head tiles of one item share blockIdx % 8)
  const int wg = blockIdx.x;
  const int per_grp = 8 * sh.nchunk;
  const int grp = wg / per_grp;
  const int rem = wg - grp * per_grp;
  const int chunk = rem >> 3;
  const int item = grp * 8 + (rem & 7);
  if (item >= sh.num_items) return;
  const int split = item % sh.nsplit;
  const int sk = item / sh.nsplit;
  const int kvh = sk % sh.num_kv_heads;
  const int seq = sk / sh.num_kv_heads;

  // Contexts are clamped to what the block table holds and to what the grid's
  // splits cover, so no work-group reads past the table or the partials.
  const int cap = min(sh.max_blocks * sh.block_size, sh.nsplit * sh.partition);
  int ctx = ctxl[seq];
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int ns_eff = ctx > 0 ? (ctx + sh.partition - 1) / sh.partition : 1;
  if (split >= ns_eff) return;
  const int t_begin = split * sh.partition;
  const int t_end = min(ctx, t_begin + sh.partition);
  const int n_it = t_end > t_begin ? (t_end - t_begin + kIterTokens - 1) / kIterTokens : 0;

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int head0 = kvh * sh.group + chunk * GT;
  const int unit = (seq * sh.num_kv_heads + kvh) * sh.nchunk + chunk;

  const uint32_t* q32 =
      reinterpret_cast<const uint32_t*>(q + ((size_t)seq * sh.num_heads + head0) * D);
  const int* btrow = bt + (size_t)seq * sh.max_blocks;
  const int bs = sh.block_size;
  const int bsl = sh.bs_log2;

  // 1152 * sum(q) per head, removes the fp16 bias of the converted int8 K.
  float qbias[GT];
  if constexpr (I8) {
#pragma unroll
    for (int hh = 0; hh < GT; ++hh) {
      float sacc = 0.f;
      for (int i = lane; i < D / 2; i += kWave) sacc = dot2(q32[hh * (D / 2) + i], 0x3C003C00u, sacc);
      qbias[hh] = 1152.f * wave_sum(sacc);
    }
  }

  float m_run[GT], l_run[GT], acc[GT][JV];
#pragma unroll
  for (int hh = 0; hh < GT; ++hh) {
    m_run[hh] = kNegInf;
    l_run[hh] = 0.f;
#pragma unroll
    for (int j = 0; j < JV; ++j) acc[hh][j] = 0.f;
  }
  int e_cur = I8 ? 0 : 14;

  const int kb = lane >> 4, kt = lane & 15;   // QK lane: slab, token
  const int vd = lane >> 1, vh = lane & 1;    // PV lane: dim row, token half
  const float c = sh.scale_log2;

  for (int it = w; it < n_it; it += kWavesPerGroup) {
    const int tok0 = t_begin + it * kIterTokens;

    // ---- K addressing and loads (one token per lane)
    const int tau = tok0 + kb * 16 + kt;
    bool vk = tau < t_end;
    const int tau_c = vk ? tau : t_begin;
    int blk = btrow[tau_c >> bsl];
    const int off = tau_c & (bs - 1);
    const bool bok = (unsigned)blk < (unsigned)sh.num_blocks;
    vk = vk && bok;
    blk = bok ? blk : 0;
    const size_t kslot = (size_t)blk * sh.num_kv_heads + kvh;
    const uint8_t* kp = kc + (kslot * NO * bs + off) * 8 * ESZ;
    KVec kr[NO];
#pragma unroll
    for (int o = 0; o < NO; ++o) kr[o] = *reinterpret_cast<const KVec*>(kp + (size_t)o * bs * 8 * ESZ);

    float sk = 1.f, sv = 0.f;
    if constexpr (I8) {
      sk = ksc[kslot * bs + off];
      sv = vsc[kslot * bs + off];
    }

    // ---- V addressing (8 tokens x JV rows per lane and slab)
    const uint8_t* vp[4];
    int nval[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int tv = tok0 + b * 16 + vh * 8;
      const bool in = tv < t_end;
      const int tv_c = in ? tv : t_begin;
      int vb = btrow[tv_c >> bsl];
      const int voff = tv_c & (bs - 1);
      const bool vok = (unsigned)vb < (unsigned)sh.num_blocks;
      vb = vok ? vb : 0;
      vp[b] = vc + ((((size_t)vb * sh.num_kv_heads + kvh) * D + vd) * bs + voff) * ESZ;
      const int nv = t_end - tv;
      nval[b] = (in && vok) ? (nv < 8 ? nv : 8) : 0;
    }
    KVec vr[VEARLY ? 4 : 1][JV];
    if constexpr (VEARLY) {
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int j = 0; j < JV; ++j)
          vr[b][j] = *reinterpret_cast<const KVec*>(vp[b] + (size_t)j * 32 * bs * ESZ);
    }

    // ---- QK: q from scalar loads (re-read every iteration from the scalar cache)
    uint32_t zo;
    asm volatile("s_mov_b32 %0, 0" : "=s"(zo));
    const uint32_t* qq = q32 + zo;
    float s[GT];
#pragma unroll
    for (int hh = 0; hh < GT; ++hh) s[hh] = 0.f;
#pragma unroll
    for (int o = 0; o < NO; ++o) {
      uint32_t k0, k1, k2, k3;
      if constexpr (I8) {
        i8x4_to_biased_h2(kr[o].x, k0, k1);
        i8x4_to_biased_h2(kr[o].y, k2, k3);
      } else {
        k0 = kr[o].x; k1 = kr[o].y; k2 = kr[o].z; k3 = kr[o].w;
      }
#pragma unroll
      for (int hh = 0; hh < GT; ++hh) {
        const uint4 qv = *reinterpret_cast<const uint4*>(qq + hh * (D / 2) + o * 4);
        float t = dot2(qv.x, k0, s[hh]);
        t = dot2(qv.y, k1, t);
        t = dot2(qv.z, k2, t);
        s[hh] = dot2(qv.w, k3, t);
      }
    }

    // ---- online softmax, one wave max per head
    float p[GT], fac[GT];
    const float skc = sk * c;
#pragma unroll
    for (int hh = 0; hh < GT; ++hh) {
      float sc;
      if constexpr (I8) sc = (s[hh] - qbias[hh]) * skc;
      else sc = s[hh] * c;
      sc = vk ? sc : kNegInf;
      const float mt = wave_max(sc);
      const float m_new = fmaxf(m_run[hh], mt);
      const float m_use = (m_new == kNegInf) ? 0.f : m_new;
      fac[hh] = exp2f_fast(m_run[hh] - m_use);
      p[hh] = exp2f_fast(sc - m_use);
      l_run[hh] = l_run[hh] * fac[hh] + p[hh];
      m_run[hh] = m_new;
    }

    // ---- weights to fp16 (times 2^e) into LDS
    float wscale;
    if constexpr (I8) {
      const float svm = vk ? sv : 0.f;
      const float msv = wave_max(svm);
      int e_new = 15 - __builtin_amdgcn_frexp_expf(msv);
      e_new = e_new < 0 ? 0 : (e_new > 30 ? 30 : e_new);
      wscale = __builtin_amdgcn_ldexpf(svm, e_new);
#pragma unroll
      for (int hh = 0; hh < GT; ++hh) fac[hh] = __builtin_amdgcn_ldexpf(fac[hh], e_new - e_cur);
      e_cur = e_new;
    } else {
      wscale = 16384.f;
    }
#pragma unroll
    for (int hh = 0; hh < GT; ++hh) {
      const half_t ph = (half_t)(p[hh] * wscale);
      sm.p[w][kb][hh][kt] = __builtin_bit_cast(uint16_t, ph);
#pragma unroll
      for (int j = 0; j < JV; ++j) acc[hh][j] *= fac[hh];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- PV
    const bool need_mask = !I8 && (__builtin_amdgcn_ballot_w64(nval[0] < 8 || nval[1] < 8 ||
                                                               nval[2] < 8 || nval[3] < 8) != 0);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      KVec vraw[JV];
#pragma unroll
      for (int j = 0; j < JV; ++j) {
        if constexpr (VEARLY) vraw[j] = vr[b][j];
        else vraw[j] = *reinterpret_cast<const KVec*>(vp[b] + (size_t)j * 32 * bs * ESZ);
      }
      uint32_t vv[JV][4];
#pragma unroll
      for (int j = 0; j < JV; ++j) {
        if constexpr (I8) {
          i8x4_to_biased_h2(vraw[j].x, vv[j][0], vv[j][1]);
          i8x4_to_biased_h2(vraw[j].y, vv[j][2], vv[j][3]);
#pragma unroll
          for (int k = 0; k < 4; ++k) vv[j][k] = unbias_h2(vv[j][k]);
        } else {
          vv[j][0] = vraw[j].x; vv[j][1] = vraw[j].y; vv[j][2] = vraw[j].z; vv[j][3] = vraw[j].w;
        }
      }
      if (need_mask) {
        // Zero the fp16 V of tokens past the end (they may hold NaN bits).
        const int n = nval[b];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t mk = (2 * k + 1 < n) ? 0xFFFFFFFFu : ((2 * k < n) ? 0x0000FFFFu : 0u);
#pragma unroll
          for (int j = 0; j < JV; ++j) vv[j][k] &= mk;
        }
      }
#pragma unroll
      for (int hh = 0; hh < GT; ++hh) {
        const uint4 pp = *reinterpret_cast<const uint4*>(&sm.p[w][b][hh][vh * 8]);
#pragma unroll
        for (int j = 0; j < JV; ++j) {
          float t = dot2(pp.x, vv[j][0], acc[hh][j]);
          t = dot2(pp.y, vv[j][1], t);
          t = dot2(pp.z, vv[j][2], t);
          acc[hh][j] = dot2(pp.w, vv[j][3], t);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---- per-wave results
  const float unscale = __builtin_amdgcn_ldexpf(1.f, -e_cur);
#pragma unroll
  for (int hh = 0; hh < GT; ++hh) {
    l_run[hh] = wave_sum(l_run[hh]);
#pragma unroll
    for (int j = 0; j < JV; ++j) acc[hh][j] = pair_sum(acc[hh][j]) * unscale;
  }
  if (lane == 0) {
#pragma unroll
    for (int hh = 0; hh < GT; ++hh) {
      sm.m[w][hh] = m_run[hh];
      sm.l[w][hh] = l_run[hh];
    }
  }
  if ((lane & 1) == 0) {
#pragma unroll
    for (int hh = 0; hh < GT; ++hh)
#pragma unroll
      for (int j = 0; j < JV; ++j) sm.a[w][hh][vd + 32 * j] = acc[hh][j];
  }
  __syncthreads();

  // ---- merge the 4 waves
  const bool final_here = FUSED && ns_eff == 1;
  const size_t out_base = ((size_t)seq * sh.num_heads + head0) * D;
  const size_t part_base = (size_t)unit * sh.nsplit;
  for (int idx = threadIdx.x; idx < GT * D; idx += kThreads) {
    const int hh = idx / D;
    const int d = idx - hh * D;
    float mx = kNegInf;
#pragma unroll
    for (int ww = 0; ww < kWavesPerGroup; ++ww) mx = fmaxf(mx, sm.m[ww][hh]);
    float a = 0.f, l = 0.f;
#pragma unroll
    for (int ww = 0; ww < kWavesPerGroup; ++ww) {
      const float mw = sm.m[ww][hh];
      const float f = (mw == kNegInf) ? 0.f : exp2f_fast(mw - mx);
      a += sm.a[ww][hh][d] * f;
      l += sm.l[ww][hh] * f;
    }
    if (final_here) {
      out[out_base + idx] = (half_t)(l > 0.f ? a / l : 0.f);
    } else {
      const size_t pi = (part_base + split) * GT + hh;
      pacc[pi * D + d] = a;
      if (d == 0) {
        pml[pi * 2] = mx;
        pml[pi * 2 + 1] = l;
      }
    }
  }
  if constexpr (FUSED) {
    if (ns_eff > 1) {
      // Release this split's partial, count arrivals; the last one merges.
      __threadfence();
      __syncthreads();
      if (threadIdx.x == 0) {
        const uint32_t prev =
            __hip_atomic_fetch_add(cnt + unit, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        sm.last = prev == (uint32_t)(ns_eff - 1);
      }
      __syncthreads();
      if (sm.last) {
        __threadfence();
        merge_partials<D, GT>(pacc, pml, out, part_base, out_base, ns_eff);
        if (threadIdx.x == 0)
          __hip_atomic_store(cnt + unit, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// Split-K reduce: one work-group per (seq, kv_head, head tile).
template <int D, int GT>
__global__ void __launch_bounds__(kThreads)
splitk_reduce_kernel(const float* __restrict__ pacc, const float* __restrict__ pml,
                     const int* __restrict__ ctxl, half_t* __restrict__ out, DecodeShape sh) {
  const int unit = blockIdx.x;
  const int chunk = unit % sh.nchunk;
  const int sk = unit / sh.nchunk;
  const int kvh = sk % sh.num_kv_heads;
  const int seq = sk / sh.num_kv_heads;
  // Contexts are clamped to what the block table holds and to what the grid's
  // splits cover, so no work-group reads past the table or the partials.
  const int cap = min(sh.max_blocks * sh.block_size, sh.nsplit * sh.partition);
  int ctx = ctxl[seq];
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int ns_eff = ctx > 0 ? (ctx + sh.partition - 1) / sh.partition : 1;
  const int head0 = kvh * sh.group + chunk * GT;
  merge_partials<D, GT>(pacc, pml, out, (size_t)unit * sh.nsplit,
                        ((size_t)seq * sh.num_heads + head0) * D, ns_eff);
}

template <int D, int GT, bool I8>
hipError_t launch_decode_tile(const DecodeLaunch& l) {
  const DecodeShape& sh = l.shape;
  const int grid = ((sh.num_items + 7) / 8) * 8 * sh.nchunk;
  const auto* q = static_cast<const half_t*>(l.q);
  const auto* kc = static_cast<const uint8_t*>(l.k_cache);
  const auto* vc = static_cast<const uint8_t*>(l.v_cache);
  auto* out = static_cast<half_t*>(l.out);
  if (l.fused) {
    decode_kernel<D, GT, I8, true><<<grid, kThreads, 0, l.stream>>>(
        q, kc, vc, l.k_scales, l.v_scales, l.block_table, l.context_lens, out, l.part_acc,
        l.part_ml, l.counters, sh);
    return hipGetLastError();
  }
  decode_kernel<D, GT, I8, false><<<grid, kThreads, 0, l.stream>>>(
      q, kc, vc, l.k_scales, l.v_scales, l.block_table, l.context_lens, out, l.part_acc, l.part_ml,
      l.counters, sh);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int units = sh.num_seqs * sh.num_kv_heads * sh.nchunk;
  splitk_reduce_kernel<D, GT><<<units, kThreads, 0, l.stream>>>(l.part_acc, l.part_ml,
                                                                l.context_lens, out, sh);
  return hipGetLastError();
}

template <int D, bool I8>
hipError_t launch_decode_dtype(const DecodeLaunch& l) {
  switch (l.head_tile) {
    case 1: return launch_decode_tile<D, 1, I8>(l);
    case 2: return launch_decode_tile<D, 2, I8>(l);
    case 3: return launch_decode_tile<D, 3, I8>(l);
    case 4: return launch_decode_tile<D, 4, I8>(l);
    case 5: return launch_decode_tile<D, 5, I8>(l);
    case 6: return launch_decode_tile<D, 6, I8>(l);
    case 7: return launch_decode_tile<D, 7, I8>(l);
    case 8: return launch_decode_tile<D, 8, I8>(l);
    default: return hipErrorInvalidValue;
  }
}

template <int D>
hipError_t launch_decode_d(const DecodeLaunch& l) {
  return l.int8_kv ? launch_decode_dtype<D, true>(l) : launch_decode_dtype<D, false>(l);
}

}  // namespace pa

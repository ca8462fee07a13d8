// Thin torch extension over libpa_mi355x.so.  Replaces the reference's
// pybind module (kernels/bindings.cpp:45-58): the same op names, argument
// order and error behaviour (TORCH_CHECK -> RuntimeError), launching on the
// caller's current stream.  No device code lives here; every op ends in a
// C-ABI call declared in include/pa_mi355x.h.
#include <torch/extension.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "pa_mi355x.h"

namespace {

constexpr int64_t kRefTile = 128;

// Device memory of a decode call (include/pa_mi355x.h):
//
// * Counters: one buffer per (device, stream), zeroed when it is made; every
//   call leaves its counters zero again, so calls of any shape share it.  It
//   only grows, and a superseded buffer is kept until the process ends: a HIP
//   graph captured earlier may still hold its address.  A buffer first made
//   while the stream is being captured is zeroed by the captured fill only
//   when the graph replays, so the next call outside a capture zeroes it once
//   more before using it.
// * Workspace (split partials, schedule record): plain scratch, allocated per
//   call from the stream-ordered caching allocator as the reference does for
//   its partials (kernels/paged_attention_v4_splitk.cu:216-219).  Under graph
//   capture it comes from the graph's private pool and stays valid for every
//   replay; graphs never share it.
struct Counters {
  at::Tensor buf;
  bool zeroed_eagerly = false;
  std::vector<at::Tensor> retired;
};
std::mutex g_counters_mu;
std::map<std::pair<int, void*>, Counters> g_counters;
// 256 KB: the 1 KB claim-counter block, then 20 bytes per unit (one arrival
// counter and four merge-group counters), about 13k units; grows only for huge batches.
constexpr size_t kMinCounterBytes = 256 << 10;

bool stream_capturing(hipStream_t stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  TORCH_CHECK(hipStreamIsCapturing(stream, &st) == hipSuccess, "hipStreamIsCapturing failed");
  return st != hipStreamCaptureStatusNone;
}

at::Tensor counters_for(const at::Tensor& like, hipStream_t stream, size_t bytes) {
  std::lock_guard<std::mutex> lk(g_counters_mu);
  Counters& c = g_counters[std::make_pair((int)like.get_device(), (void*)stream)];
  const bool capturing = stream_capturing(stream);
  if (!c.buf.defined() || (size_t)c.buf.numel() < bytes) {
    size_t want = std::max(bytes, kMinCounterBytes);
    if (c.buf.defined()) {
      want = std::max(want, 2 * (size_t)c.buf.numel());
      c.retired.push_back(c.buf);
    }
    c.buf = at::zeros({(int64_t)want}, like.options().dtype(at::kByte));
    c.zeroed_eagerly = !capturing;
  } else if (!c.zeroed_eagerly && !capturing) {
    c.buf.zero_();
    c.zeroed_eagerly = true;
  }
  return c.buf;
}

void check_status(pa_status_t st) { TORCH_CHECK(st == PA_OK, pa_status_string(st)); }

// Which reference launcher's block_size rule an op repeats: the naive stage
// checks none (paged_attention_naive.cu:135-140), the vectorised stage only a
// multiple of 8 (paged_attention_v1_vectorized.cu:124), the later ones also
// that it divides the 128-token tile (v2_online.cu:157, v3_warp.cu:149-150).
// The library's own rule (pa_validate_decode) applies to every op after it.
enum class BlockRule { kNone, kMultipleOf8, kTile };

void run_decode(pa_decode_kind_t kind, at::Tensor& out, const at::Tensor& q,
                const at::Tensor& k_cache, const at::Tensor& v_cache,
                const at::Tensor* k_scales, const at::Tensor* v_scales,
                const at::Tensor& block_table, const at::Tensor& context_lens, double scale,
                int64_t block_size, bool check_context, int64_t partition_tokens,
                BlockRule rule = BlockRule::kTile) {
  const bool int8 = kind == PA_DECODE_WARP_I8 || kind == PA_DECODE_SPLITK_I8;
  // The reference launchers' checks, in their order (paged_attention_v3_warp.cu:143-150,
  // paged_attention_v5_warp_int8.cu:159-168).
  TORCH_CHECK(q.is_cuda() && out.is_cuda(), "tensors must be on CUDA");
  TORCH_CHECK(q.scalar_type() == at::kHalf, "q must be fp16");
  if (int8) {
    TORCH_CHECK(k_cache.scalar_type() == at::kChar, "k_cache must be int8");
    TORCH_CHECK(v_cache.scalar_type() == at::kChar, "v_cache must be int8");
    TORCH_CHECK(k_scales->scalar_type() == at::kFloat, "k_scales must be fp32");
    TORCH_CHECK(v_scales->scalar_type() == at::kFloat, "v_scales must be fp32");
  } else {
    TORCH_CHECK(k_cache.scalar_type() == at::kHalf, "k_cache must be fp16");
    TORCH_CHECK(v_cache.scalar_type() == at::kHalf, "v_cache must be fp16");
  }
  TORCH_CHECK(block_table.scalar_type() == at::kInt, "block_table must be int32");
  TORCH_CHECK(context_lens.scalar_type() == at::kInt, "context_lens must be int32");
  int32_t max_ctx = 0;
  bool equal_lens = false;
  if (check_context && context_lens.numel() > 0) {
    // One device->host copy for both the reference's `min >= 1` rule
    // (v3:147-148) and the split count (v4:213-214).
    const auto mnmx = at::aminmax(context_lens);
    const at::Tensor mm = at::stack({std::get<0>(mnmx), std::get<1>(mnmx)}).cpu();
    const int32_t mn = mm[0].item<int32_t>();
    max_ctx = mm[1].item<int32_t>();
    TORCH_CHECK(mn >= 1, "context_lens must be >= 1 (empty sequences unsupported)");
    equal_lens = mn == max_ctx;
  }
  if (int8) {
    TORCH_CHECK(block_size % 16 == 0 && kRefTile % block_size == 0,
                "block_size must divide TILE and be a multiple of 16");
  } else if (rule == BlockRule::kTile) {
    TORCH_CHECK(block_size % 8 == 0 && kRefTile % block_size == 0,
                "block_size must divide TILE and be a multiple of 8");
  } else if (rule == BlockRule::kMultipleOf8) {
    TORCH_CHECK(block_size % 8 == 0, "block_size must be a multiple of 8 for vectorized V");
  }
  // Layout checks the reference leaves implicit.
  TORCH_CHECK(q.dim() == 3 && out.sizes() == q.sizes() && out.scalar_type() == at::kHalf,
              "q and out must be [num_seqs, num_heads, head_dim] fp16");
  TORCH_CHECK(k_cache.dim() == 5 && v_cache.dim() == 4,
              "k_cache must be [blocks, kv_heads, D/x, block_size, x], v_cache [blocks, kv_heads, D, block_size]");
  TORCH_CHECK(block_table.dim() == 2 && context_lens.dim() == 1 &&
                  block_table.size(0) == q.size(0) && context_lens.size(0) == q.size(0),
              "block_table must be [num_seqs, max_blocks] and context_lens [num_seqs]");
  const int64_t x = k_cache.size(4);
  if (int8) TORCH_CHECK(x == 8, "int8 K cache requires x == 8");
  TORCH_CHECK(k_cache.size(3) == block_size && v_cache.size(3) == block_size,
              "cache block dimension must equal block_size");
  TORCH_CHECK(k_cache.size(2) * x == q.size(2) && v_cache.size(2) == q.size(2),
              "cache head_dim does not match q");
  TORCH_CHECK(v_cache.size(0) == k_cache.size(0) && v_cache.size(1) == k_cache.size(1),
              "k_cache and v_cache disagree on blocks / kv_heads");
  const at::Tensor* all[] = {&out, &q, &k_cache, &v_cache, &block_table, &context_lens};
  for (const at::Tensor* t : all) {
    TORCH_CHECK(t->is_cuda() && t->get_device() == q.get_device(), "all tensors must be on q's device");
    TORCH_CHECK(t->is_contiguous(), "all tensors must be contiguous");
  }
  if (int8) {
    for (const at::Tensor* t : {k_scales, v_scales}) {
      TORCH_CHECK(t->is_cuda() && t->get_device() == q.get_device() && t->is_contiguous(),
                  "scales must be contiguous and on q's device");
      TORCH_CHECK(t->dim() == 3 && t->size(0) == k_cache.size(0) && t->size(1) == k_cache.size(1) &&
                      t->size(2) == block_size,
                  "scales must be [blocks, kv_heads, block_size]");
    }
  }

  const int32_t S = (int32_t)q.size(0), H = (int32_t)q.size(1), D = (int32_t)q.size(2);
  const int32_t Hkv = (int32_t)k_cache.size(1), NB = (int32_t)k_cache.size(0);
  const int32_t MB = (int32_t)block_table.size(1);
  check_status(pa_validate_decode(kind, S, H, D, Hkv, NB, (int32_t)block_size, (int32_t)x, MB));
  if (S == 0) return;

  // Split-K with equal lengths, known from the check above: the single-launch
  // plan (host grid, splits merged in the launch) has no empty work-groups to
  // avoid and no schedule to build first.  Same box, alternating, schedule ->
  // grid: config 2's shape 27.25 -> 24.79 us; Llama 32/8 8 x 32k FP16 165.2 ->
  // 157.8 (INT8 91.8 -> 89.8), 64k 320.8 -> 315.6 (174.3 -> 171.5), 128k INT8
  // 343.3 -> 341.0; only 128k FP16 (4 GiB) turns, 656.1 -> 672.7.
  if (equal_lens && (kind == PA_DECODE_SPLITK_F16 || kind == PA_DECODE_SPLITK_I8) &&
      (int64_t)S * Hkv * max_ctx * D * (int8 ? 2 : 4) <= (int64_t(2) << 30))
    kind = int8 ? PA_DECODE_WARP_I8 : PA_DECODE_WARP_F16;

  const at::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  hipStream_t stream = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.get_device()).stream();
  const size_t need = pa_decode_workspace_bytes(kind, S, H, D, Hkv, (int32_t)block_size, MB,
                                                max_ctx, (int32_t)partition_tokens);
  const size_t cneed = pa_decode_counter_bytes(S, H, Hkv);
  at::Tensor cnt = counters_for(q, stream, cneed);
  at::Tensor ws = at::empty({(int64_t)std::max<size_t>(need, 256)}, q.options().dtype(at::kByte));
  const float sc = (float)scale;
  auto ps = reinterpret_cast<pa_stream_t>(stream);
  void* o = out.data_ptr();
  const void *qp = q.data_ptr(), *kp = k_cache.data_ptr(), *vp = v_cache.data_ptr();
  const int32_t* bt = block_table.data_ptr<int32_t>();
  const int32_t* cl = context_lens.data_ptr<int32_t>();
  const int32_t bs = (int32_t)block_size, xx = (int32_t)x, pt = (int32_t)partition_tokens;
  void *cp = cnt.data_ptr(), *wp = ws.data_ptr();
  const size_t cb = cnt.numel(), wb = ws.numel();
  pa_status_t st;
  switch (kind) {
    case PA_DECODE_WARP_F16:
      st = pa_paged_decode_attn_warp(o, qp, kp, vp, bt, cl, sc, bs, S, H, D, Hkv, NB, xx, MB,
                                     max_ctx, pt, cp, cb, wp, wb, ps);
      break;
    case PA_DECODE_SPLITK_F16:
      st = pa_paged_decode_attn_splitk(o, qp, kp, vp, bt, cl, sc, bs, S, H, D, Hkv, NB, xx, MB,
                                       max_ctx, pt, cp, cb, wp, wb, ps);
      break;
    case PA_DECODE_WARP_I8:
      st = pa_paged_decode_attn_warp_int8(o, qp, kp, vp, k_scales->data_ptr<float>(),
                                          v_scales->data_ptr<float>(), bt, cl, sc, bs, S, H, D,
                                          Hkv, NB, xx, MB, max_ctx, pt, cp, cb, wp, wb, ps);
      break;
    default:
      st = pa_paged_decode_attn_splitk_int8(o, qp, kp, vp, k_scales->data_ptr<float>(),
                                            v_scales->data_ptr<float>(), bt, cl, sc, bs, S, H, D,
                                            Hkv, NB, xx, MB, max_ctx, pt, cp, cb, wp, wb, ps);
      break;
  }
  check_status(st);
}

// ---- the reference's six-op surface (kernels/bindings.cpp:7-43) and the naive
// ---- op of its second module (paged_attention_naive.cu:169-172).  The ladder
// ---- stages naive / vec / online compute the same function as warp; on gfx950
// ---- one single-launch kernel serves all four, behind each stage's own checks.

void paged_decode_attention(at::Tensor out, at::Tensor q, at::Tensor k_cache, at::Tensor v_cache,
                            at::Tensor block_table, at::Tensor context_lens, double scale,
                            int64_t block_size) {
  run_decode(PA_DECODE_WARP_F16, out, q, k_cache, v_cache, nullptr, nullptr, block_table,
             context_lens, scale, block_size, true, 0, BlockRule::kNone);
}

void paged_decode_attn_vec(at::Tensor out, at::Tensor q, at::Tensor k_cache, at::Tensor v_cache,
                           at::Tensor block_table, at::Tensor context_lens, double scale,
                           int64_t block_size) {
  run_decode(PA_DECODE_WARP_F16, out, q, k_cache, v_cache, nullptr, nullptr, block_table,
             context_lens, scale, block_size, true, 0, BlockRule::kMultipleOf8);
}

void paged_decode_attn_online(at::Tensor out, at::Tensor q, at::Tensor k_cache,
                              at::Tensor v_cache, at::Tensor block_table,
                              at::Tensor context_lens, double scale, int64_t block_size) {
  run_decode(PA_DECODE_WARP_F16, out, q, k_cache, v_cache, nullptr, nullptr, block_table,
             context_lens, scale, block_size, true, 0, BlockRule::kTile);
}

void paged_decode_attn_warp(at::Tensor out, at::Tensor q, at::Tensor k_cache, at::Tensor v_cache,
                            at::Tensor block_table, at::Tensor context_lens, double scale,
                            int64_t block_size) {
  run_decode(PA_DECODE_WARP_F16, out, q, k_cache, v_cache, nullptr, nullptr, block_table,
             context_lens, scale, block_size, true, 0);
}

void paged_decode_attn_splitk(at::Tensor out, at::Tensor q, at::Tensor k_cache,
                              at::Tensor v_cache, at::Tensor block_table, at::Tensor context_lens,
                              double scale, int64_t block_size) {
  run_decode(PA_DECODE_SPLITK_F16, out, q, k_cache, v_cache, nullptr, nullptr, block_table,
             context_lens, scale, block_size, true, 0);
}

void paged_decode_attn_warp_int8(at::Tensor out, at::Tensor q, at::Tensor k_cache,
                                 at::Tensor v_cache, at::Tensor k_scales, at::Tensor v_scales,
                                 at::Tensor block_table, at::Tensor context_lens, double scale,
                                 int64_t block_size) {
  run_decode(PA_DECODE_WARP_I8, out, q, k_cache, v_cache, &k_scales, &v_scales, block_table,
             context_lens, scale, block_size, true, 0);
}

void paged_decode_attn_splitk_int8(at::Tensor out, at::Tensor q, at::Tensor k_cache,
                                   at::Tensor v_cache, at::Tensor k_scales, at::Tensor v_scales,
                                   at::Tensor block_table, at::Tensor context_lens, double scale,
                                   int64_t block_size) {
  run_decode(PA_DECODE_SPLITK_I8, out, q, k_cache, v_cache, &k_scales, &v_scales, block_table,
             context_lens, scale, block_size, true, 0);
}

// ---- extensions: no host sync (for timing and serving loops) and a forced
// ---- partition size (tests of the multi-split merge, tuning sweeps)

void paged_decode_ex(int64_t kind, at::Tensor out, at::Tensor q, at::Tensor k_cache,
                     at::Tensor v_cache, c10::optional<at::Tensor> k_scales,
                     c10::optional<at::Tensor> v_scales, at::Tensor block_table,
                     at::Tensor context_lens, double scale, int64_t block_size,
                     bool check_context, int64_t partition_tokens) {
  TORCH_CHECK(kind >= 0 && kind <= 3, "kind must be 0..3");
  const auto k = static_cast<pa_decode_kind_t>(kind);
  const bool int8 = k == PA_DECODE_WARP_I8 || k == PA_DECODE_SPLITK_I8;
  TORCH_CHECK(!int8 || (k_scales.has_value() && v_scales.has_value()), "int8 kinds need scales");
  run_decode(k, out, q, k_cache, v_cache, int8 ? &*k_scales : nullptr,
             int8 ? &*v_scales : nullptr, block_table, context_lens, scale, block_size,
             check_context, partition_tokens);
}

std::pair<int64_t, int64_t> decode_plan(int64_t kind, int64_t num_seqs, int64_t num_heads,
                                        int64_t head_dim, int64_t num_kv_heads,
                                        int64_t block_size, int64_t max_blocks,
                                        int64_t max_context_len, int64_t partition_tokens) {
  int32_t part = 0, ns = 0;
  check_status(pa_decode_plan(static_cast<pa_decode_kind_t>(kind), (int32_t)num_seqs,
                              (int32_t)num_heads, (int32_t)head_dim, (int32_t)num_kv_heads,
                              (int32_t)block_size, (int32_t)max_blocks, (int32_t)max_context_len,
                              (int32_t)partition_tokens, &part, &ns));
  return {part, ns};
}

// Checks shared by the cache-write ops; `int8` selects the cache dtypes and
// whether scale tensors are passed.
void check_write(const at::Tensor& key, const at::Tensor& value, const at::Tensor& k_cache,
                 const at::Tensor& v_cache, const at::Tensor* k_scales,
                 const at::Tensor* v_scales, const at::Tensor& slot_mapping, bool int8) {
  TORCH_CHECK(key.is_cuda() && value.is_cuda(), "tensors must be on CUDA");
  if (int8) {
    TORCH_CHECK((key.scalar_type() == at::kHalf || key.scalar_type() == at::kBFloat16) &&
                    value.scalar_type() == key.scalar_type(),
                "key and value must be fp16 or bf16 (the same)");
  } else {
    TORCH_CHECK(key.scalar_type() == at::kHalf && value.scalar_type() == at::kHalf,
                "key and value must be fp16");
  }
  if (int8) {
    TORCH_CHECK(k_cache.scalar_type() == at::kChar && v_cache.scalar_type() == at::kChar,
                "k_cache and v_cache must be int8");
    TORCH_CHECK(k_scales->scalar_type() == at::kFloat && v_scales->scalar_type() == at::kFloat,
                "scales must be fp32");
  } else {
    TORCH_CHECK(k_cache.scalar_type() == at::kHalf && v_cache.scalar_type() == at::kHalf,
                "k_cache and v_cache must be fp16");
  }
  TORCH_CHECK(slot_mapping.scalar_type() == at::kLong, "slot_mapping must be int64");
  TORCH_CHECK(key.dim() == 3 && value.sizes() == key.sizes(),
              "key and value must be [num_tokens, num_kv_heads, head_dim]");
  TORCH_CHECK(key.stride(2) == 1 && value.stride(2) == 1, "head_dim must be the innermost dim");
  TORCH_CHECK(k_cache.dim() == 5 && v_cache.dim() == 4, "cache tensors have the wrong rank");
  const int64_t T = key.size(0), Hkv = key.size(1), D = key.size(2);
  const int64_t NB = k_cache.size(0), bs = k_cache.size(3), x = k_cache.size(4);
  TORCH_CHECK(k_cache.size(1) == Hkv && k_cache.size(2) * x == D && v_cache.size(0) == NB &&
                  v_cache.size(1) == Hkv && v_cache.size(2) == D && v_cache.size(3) == bs,
              "cache shapes do not match key/value");
  TORCH_CHECK(slot_mapping.dim() == 1 && slot_mapping.size(0) == T,
              "slot_mapping must be [num_tokens]");
  for (const at::Tensor* t : {&k_cache, &v_cache, &slot_mapping})
    TORCH_CHECK(t->is_contiguous() && t->is_cuda() && t->get_device() == key.get_device(),
                "cache tensors must be contiguous and on key's device");
  if (int8) {
    TORCH_CHECK(k_scales->dim() == 3 && k_scales->size(0) == NB && k_scales->size(1) == Hkv &&
                    k_scales->size(2) == bs && v_scales->sizes() == k_scales->sizes(),
                "scales must be [blocks, kv_heads, block_size]");
    for (const at::Tensor* t : {k_scales, v_scales})
      TORCH_CHECK(t->is_contiguous() && t->is_cuda() && t->get_device() == key.get_device(),
                  "cache tensors must be contiguous and on key's device");
  }
}

// NEW op (no reference counterpart): per-token INT8 quantize + paged write
// of fp16 or bf16 key / value.
void reshape_and_cache_int8(at::Tensor key, at::Tensor value, at::Tensor k_cache,
                            at::Tensor v_cache, at::Tensor k_scales, at::Tensor v_scales,
                            at::Tensor slot_mapping) {
  check_write(key, value, k_cache, v_cache, &k_scales, &v_scales, slot_mapping, true);
  const at::hip::HIPGuardMasqueradingAsCUDA guard(key.device());
  hipStream_t stream = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(key.get_device()).stream();
  const bool bf = key.scalar_type() == at::kBFloat16;
  check_status((bf ? pa_reshape_and_cache_int8_bf16 : pa_reshape_and_cache_int8)(
      key.data_ptr(), value.data_ptr(), key.stride(0), key.stride(1), value.stride(0),
      value.stride(1), slot_mapping.data_ptr<int64_t>(), (int32_t)key.size(0),
      (int32_t)key.size(1), (int32_t)key.size(2), k_cache.data_ptr(), v_cache.data_ptr(),
      k_scales.data_ptr<float>(), v_scales.data_ptr<float>(), (int32_t)k_cache.size(0),
      (int32_t)k_cache.size(3), (int32_t)k_cache.size(4), reinterpret_cast<pa_stream_t>(stream)));
}

// NEW op: INT8 write with one given scale for all K and one for all V
// (PagedKVCache's per-tensor mode); k_scale / v_scale are 1-element fp32
// tensors on key's device, read by the kernel (no host sync).
void reshape_and_cache_int8_static(at::Tensor key, at::Tensor value, at::Tensor k_cache,
                                   at::Tensor v_cache, at::Tensor k_scales, at::Tensor v_scales,
                                   at::Tensor slot_mapping, at::Tensor k_scale,
                                   at::Tensor v_scale) {
  check_write(key, value, k_cache, v_cache, &k_scales, &v_scales, slot_mapping, true);
  for (const at::Tensor* t : {&k_scale, &v_scale})
    TORCH_CHECK(t->numel() == 1 && t->scalar_type() == at::kFloat && t->is_cuda() &&
                    t->get_device() == key.get_device(),
                "k_scale and v_scale must be one fp32 value each on key's device");
  const at::hip::HIPGuardMasqueradingAsCUDA guard(key.device());
  hipStream_t stream = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(key.get_device()).stream();
  const bool bf = key.scalar_type() == at::kBFloat16;
  check_status((bf ? pa_reshape_and_cache_int8_static_bf16 : pa_reshape_and_cache_int8_static)(
      key.data_ptr(), value.data_ptr(), key.stride(0), key.stride(1), value.stride(0),
      value.stride(1), slot_mapping.data_ptr<int64_t>(), (int32_t)key.size(0),
      (int32_t)key.size(1), (int32_t)key.size(2), k_cache.data_ptr(), v_cache.data_ptr(),
      k_scales.data_ptr<float>(), v_scales.data_ptr<float>(), k_scale.data_ptr<float>(),
      v_scale.data_ptr<float>(), (int32_t)k_cache.size(0), (int32_t)k_cache.size(3),
      (int32_t)k_cache.size(4), reinterpret_cast<pa_stream_t>(stream)));
}

// NEW op: fp16 paged write (PagedKVCache's fp16 mode), vLLM's reshape_and_cache.
void reshape_and_cache(at::Tensor key, at::Tensor value, at::Tensor k_cache, at::Tensor v_cache,
                       at::Tensor slot_mapping) {
  check_write(key, value, k_cache, v_cache, nullptr, nullptr, slot_mapping, false);
  const at::hip::HIPGuardMasqueradingAsCUDA guard(key.device());
  hipStream_t stream = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(key.get_device()).stream();
  check_status(pa_reshape_and_cache_f16(
      key.data_ptr(), value.data_ptr(), key.stride(0), key.stride(1), value.stride(0),
      value.stride(1), slot_mapping.data_ptr<int64_t>(), (int32_t)key.size(0),
      (int32_t)key.size(1), (int32_t)key.size(2), k_cache.data_ptr(), v_cache.data_ptr(),
      (int32_t)k_cache.size(0), (int32_t)k_cache.size(3), (int32_t)k_cache.size(4),
      reinterpret_cast<pa_stream_t>(stream)));
}

}  // namespace

PYBIND11_MODULE(paged_attn_opt, m) {
  m.def("paged_decode_attention", &paged_decode_attention,
        "paged decode (FP16 KV), the naive stage's entry name; single-launch kernel, gfx950");
  m.def("paged_decode_attn_vec", &paged_decode_attn_vec,
        "paged decode (FP16 KV), the vectorized stage's entry name; single-launch kernel, gfx950");
  m.def("paged_decode_attn_online", &paged_decode_attn_online,
        "paged decode (FP16 KV), the online-softmax stage's entry name; single-launch kernel, "
        "gfx950");
  m.def("paged_decode_attn_warp", &paged_decode_attn_warp,
        "single-launch paged decode (FP16 KV), gfx950");
  m.def("paged_decode_attn_splitk", &paged_decode_attn_splitk,
        "split-K paged decode: partition + reduce (FP16 KV), gfx950");
  m.def("paged_decode_attn_warp_int8", &paged_decode_attn_warp_int8,
        "single-launch paged decode (INT8 KV, per-token scales), gfx950");
  m.def("paged_decode_attn_splitk_int8", &paged_decode_attn_splitk_int8,
        "split-K paged decode (INT8 KV, per-token scales), gfx950");
  m.def("paged_decode_ex", &paged_decode_ex,
        "decode with kind 0..3 (warp, splitk, warp_int8, splitk_int8), optional host check "
        "and forced partition size");
  m.def("decode_plan", &decode_plan, "(partition_tokens, num_splits) the launcher would use");
  m.def("reshape_and_cache_int8", &reshape_and_cache_int8,
        "per-token INT8 quantize + paged cache write (new op)");
  m.def("reshape_and_cache_int8_static", &reshape_and_cache_int8_static,
        "INT8 quantize with one given scale per K / V tensor + paged cache write (new op)");
  m.def("reshape_and_cache", &reshape_and_cache, "fp16 paged cache write (new op)");
  m.def("version", []() { return std::string(pa_version()); });
}

// The reference builds its naive stage as a module of its own,
// paged_attn_naive (kernels/paged_attention_naive.cu:169-172).  The same
// shared object also initialises under that name, with that one op.
PYBIND11_MODULE(paged_attn_naive, m) {
  m.def("paged_decode_attention", &paged_decode_attention,
        "paged decode (FP16 KV), the naive stage's module and entry name; single-launch kernel, "
        "gfx950");
}

/*
 * pa_mi355x.h -- C ABI of the MI355X (gfx950) paged-attention decode path.
 *
 * Plain pointers and sizes only: no torch types cross this boundary.  All
 * device pointers refer to memory on the device that is current when the
 * call is made; every launch goes to `stream` (a hipStream_t, 0 = the null
 * stream).  Calls are asynchronous: a PA_OK return means the work was
 * enqueued, not that it finished.
 *
 * Memory layouts (identical to the reference's, kernels/paged_attention_naive.cu:7-9):
 *   q, out        [num_seqs, num_heads, head_dim]                      fp16
 *   k_cache       [num_blocks, num_kv_heads, head_dim/x, block_size, x] fp16 or int8, x = 8
 *   v_cache       [num_blocks, num_kv_heads, head_dim, block_size]      fp16 or int8
 *   k_scales,
 *   v_scales      [num_blocks, num_kv_heads, block_size]               fp32 (int8 only)
 *   block_table   [num_seqs, max_blocks_per_seq]                       int32
 *   context_lens  [num_seqs]                                           int32
 * All arrays are dense and row-major.  kv_head of query head h is
 * h / (num_heads / num_kv_heads).  head_dim is a multiple of 8 in [8, 256]
 * (the reference takes any multiple of 8, kernels/paged_attention_v3_warp.cu:48-58).
 *
 * Behaviour on data the host cannot see (the caller owns these guarantees;
 * the kernels stay memory-safe when they are broken):
 *   - context_lens[s] <= 0 gives out[s] = 0 (the torch shim rejects it first,
 *     as the reference does);
 *   - context_lens[s] is clamped to max_blocks_per_seq * block_size and, when
 *     max_context_len > 0 is passed, to the split plan made for it (pass an
 *     upper bound of every length, or <= 0);
 *   - a block id outside [0, num_blocks) contributes no tokens.
 *
 * Device memory of a decode call, both supplied by the caller:
 *   counters   pa_decode_counter_bytes(...) bytes (or more), 256-byte
 *              aligned: arrival and claim counters.  They must be zero when a
 *              call starts, and every call leaves them zero when its kernels
 *              finish.  Zero them once (pa_decode_counters_reset, or any fill)
 *              and keep them: calls of any shape may share one counter buffer
 *              as long as they run one after another (one stream, or replays
 *              of HIP graphs captured on it that do not overlap).
 *   workspace  pa_decode_workspace_bytes(...) bytes, 256-byte aligned:
 *              scratch for split partials and the schedule record.  No
 *              initial contents are required and nothing is kept between
 *              calls, so it may come from a stream-ordered allocator per call.
 * Two calls that may run at the same time need separate counters and
 * separate workspaces.
 */
#ifndef PA_MI355X_H
#define PA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* pa_stream_t; /* == hipStream_t */

typedef enum pa_status {
  PA_OK = 0,
  PA_ERR_NULL_POINTER = 1,     /* a required pointer is NULL */
  PA_ERR_BAD_SHAPE = 2,        /* sizes inconsistent or out of range */
  PA_ERR_BAD_BLOCK_SIZE = 3,   /* block_size rejected (same rule as the reference) */
  PA_ERR_UNSUPPORTED = 4,      /* head_dim / x not built into this library */
  PA_ERR_WORKSPACE = 5,        /* counters / workspace NULL, misaligned or too small */
  PA_ERR_LAUNCH = 6,           /* the HIP runtime refused the launch */
  PA_ERR_EMPTY_CONTEXT = 7,    /* a context length < 1 (host-side check) */
  PA_ERR_SCRATCH_LIMIT = 8     /* beyond the no-alloc entry point's static scratch */
} pa_status_t;

/* Decode kinds for the planning / workspace queries. */
typedef enum pa_decode_kind {
  PA_DECODE_WARP_F16 = 0,
  PA_DECODE_SPLITK_F16 = 1,
  PA_DECODE_WARP_I8 = 2,
  PA_DECODE_SPLITK_I8 = 3
} pa_decode_kind_t;

const char* pa_status_string(pa_status_t status);
const char* pa_version(void);

/* Host-only shape validation: the checks the reference launchers make with
 * TORCH_CHECK (kernels/paged_attention_v3_warp.cu:143-150,
 * paged_attention_v4_splitk.cu:203-205, paged_attention_v5_warp_int8.cu:159-176),
 * plus the shape rules of this library.  No device access. */
pa_status_t pa_validate_decode(pa_decode_kind_t kind, int32_t num_seqs, int32_t num_heads,
                               int32_t head_dim, int32_t num_kv_heads, int32_t num_blocks,
                               int32_t block_size, int32_t x, int32_t max_blocks_per_seq);

/* Host-only check of context lengths already copied to the host
 * (the reference's `context_lens.min().item() >= 1`, paged_attention_v3_warp.cu:147-148).
 * Writes the maximum to *max_len when max_len != NULL. */
pa_status_t pa_check_context_lens(const int32_t* host_context_lens, int32_t num_seqs,
                                  int32_t* max_len);

/* Split plan of the grid form: how many tokens each work-group covers (a
 * multiple of 64) and how many splits the longest sequence needs.  (Under the
 * in-kernel schedule the kernel picks the partition on the device from the
 * actual lengths; a forced partition_tokens is used as given by both.)  `max_context_len` <= 0
 * means "use max_blocks_per_seq * block_size".  `partition_tokens` > 0
 * forces the partition size (rounded up to a multiple of 64 and capped at
 * 2048 tokens per wave of the work-group for head_dim <= 128, 8192 with 4
 * waves and 16384 with 8, and at 1024 per wave, 4096, for head_dim 256). */
pa_status_t pa_decode_plan(pa_decode_kind_t kind, int32_t num_seqs, int32_t num_heads,
                           int32_t head_dim, int32_t num_kv_heads, int32_t block_size,
                           int32_t max_blocks_per_seq, int32_t max_context_len,
                           int32_t partition_tokens, int32_t* out_partition_tokens,
                           int32_t* out_num_splits);

/* Scratch bytes of one decode call (the `workspace` argument); 0 for an
 * invalid shape. */
size_t pa_decode_workspace_bytes(pa_decode_kind_t kind, int32_t num_seqs, int32_t num_heads,
                                 int32_t head_dim, int32_t num_kv_heads, int32_t block_size,
                                 int32_t max_blocks_per_seq, int32_t max_context_len,
                                 int32_t partition_tokens);
/* Counter bytes of one decode call (the `counters` argument), the same for
 * every kind; 0 for an invalid shape. */
size_t pa_decode_counter_bytes(int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads);

/* Zeroes `bytes` (a multiple of 4) of a counter buffer on `stream` with a
 * fill kernel (no memset node, so a HIP graph may capture it).  For a new
 * buffer, or one whose last call did not run to completion. */
pa_status_t pa_decode_counters_reset(void* counters, size_t bytes, pa_stream_t stream);

/* FP16 KV, single launch.  Replaces paged_decode_attn_warp
 * (kernels/paged_attention_v3_warp.cu:137-176; bound at kernels/bindings.cpp:50-51).
 * When the (seq, kv-head group) units alone cannot fill the GPU the launch
 * also splits the context and the last work-group of each unit merges the
 * partial results in the same launch. */
pa_status_t pa_paged_decode_attn_warp(
    void* out, const void* q, const void* k_cache, const void* v_cache,
    const int32_t* block_table, const int32_t* context_lens, float scale, int32_t block_size,
    int32_t num_seqs, int32_t num_heads, int32_t head_dim, int32_t num_kv_heads,
    int32_t num_blocks, int32_t x, int32_t max_blocks_per_seq, int32_t max_context_len,
    int32_t partition_tokens, void* counters, size_t counter_bytes, void* workspace,
    size_t workspace_bytes, pa_stream_t stream);

/* FP16 KV, split-K: a partition kernel writes per-split (acc, max, sum)
 * partials and a separate reduce kernel merges them.  Replaces
 * paged_decode_attn_splitk (kernels/paged_attention_v4_splitk.cu:191-248;
 * bindings.cpp:52-53). */
pa_status_t pa_paged_decode_attn_splitk(
    void* out, const void* q, const void* k_cache, const void* v_cache,
    const int32_t* block_table, const int32_t* context_lens, float scale, int32_t block_size,
    int32_t num_seqs, int32_t num_heads, int32_t head_dim, int32_t num_kv_heads,
    int32_t num_blocks, int32_t x, int32_t max_blocks_per_seq, int32_t max_context_len,
    int32_t partition_tokens, void* counters, size_t counter_bytes, void* workspace,
    size_t workspace_bytes, pa_stream_t stream);

/* INT8 KV with per-(token, kv_head) fp32 scales, single launch.  Replaces
 * paged_decode_attn_warp_int8 (kernels/paged_attention_v5_warp_int8.cu:150-197;
 * bindings.cpp:54-55). */
pa_status_t pa_paged_decode_attn_warp_int8(
    void* out, const void* q, const void* k_cache, const void* v_cache,
    const float* k_scales, const float* v_scales,
    const int32_t* block_table, const int32_t* context_lens, float scale, int32_t block_size,
    int32_t num_seqs, int32_t num_heads, int32_t head_dim, int32_t num_kv_heads,
    int32_t num_blocks, int32_t x, int32_t max_blocks_per_seq, int32_t max_context_len,
    int32_t partition_tokens, void* counters, size_t counter_bytes, void* workspace,
    size_t workspace_bytes, pa_stream_t stream);

/* INT8 KV, split-K partition + reduce.  Replaces paged_decode_attn_splitk_int8
 * (kernels/paged_attention_v6_splitk_int8.cu:194-259; bindings.cpp:56-57). */
pa_status_t pa_paged_decode_attn_splitk_int8(
    void* out, const void* q, const void* k_cache, const void* v_cache,
    const float* k_scales, const float* v_scales,
    const int32_t* block_table, const int32_t* context_lens, float scale, int32_t block_size,
    int32_t num_seqs, int32_t num_heads, int32_t head_dim, int32_t num_kv_heads,
    int32_t num_blocks, int32_t x, int32_t max_blocks_per_seq, int32_t max_context_len,
    int32_t partition_tokens, void* counters, size_t counter_bytes, void* workspace,
    size_t workspace_bytes, pa_stream_t stream);

/* Decode that allocates nothing.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The same call as
 * the decode entry point of `kind` (pa_paged_decode_attn_warp, _splitk,
 * _warp_int8 or _splitk_int8; k_scales / v_scales are ignored for the FP16
 * kinds), minus the counters and workspace: those live in one static device
 * array of PA_NOALLOC_SCRATCH_BYTES per GPU (the first
 * PA_NOALLOC_COUNTER_BYTES hold the counters, the rest the split partials),
 * which the library keeps until the process ends.  Each call clears the
 * counters it uses with a fill kernel on `stream` before the decode; it calls
 * no hipMalloc, hipFree or allocating library routine.  A call whose counters
 * or partials do not fit gets PA_ERR_SCRATCH_LIMIT before anything is
 * launched (the in-kernel schedule's split capacity shrinks to fit first, so
 * only very large batches are refused).  Every call on a GPU shares that
 * GPU's array: two calls that may overlap on one GPU (different streams, or
 * concurrently replayed graphs) race and give wrong results. */
#define PA_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
#define PA_NOALLOC_COUNTER_BYTES ((size_t)1 << 20)
pa_status_t pa_paged_decode_attn_noalloc(
    pa_decode_kind_t kind, void* out, const void* q, const void* k_cache, const void* v_cache,
    const float* k_scales, const float* v_scales,
    const int32_t* block_table, const int32_t* context_lens, float scale, int32_t block_size,
    int32_t num_seqs, int32_t num_heads, int32_t head_dim, int32_t num_kv_heads,
    int32_t num_blocks, int32_t x, int32_t max_blocks_per_seq, int32_t max_context_len,
    int32_t partition_tokens, pa_stream_t stream);

/* Per-token INT8 quantize + paged-cache write.  NEW API: the reference has
 * no kernel for it; its semantics are those of quantize_per_token
 * (tests/paged_decode_attn.py:106-112) placed as in build_paged_kv_cache_int8
 * (:190-197) and PagedKVCache.decode_append
 * (benchmarks/int8_bridge/paged_cache.py:132-156).  Argument convention of
 * vLLM's reshape_and_cache: key/value [num_tokens, num_kv_heads, head_dim]
 * fp16 with the given element strides (head_dim stride 1), slot_mapping[t] =
 * block * block_size + offset; a slot < 0 or >= num_blocks * block_size
 * skips that token.  Two tokens with the same slot give an unspecified
 * winner.  block_size must be a multiple of 16 dividing 128; x must be 8. */
pa_status_t pa_reshape_and_cache_int8(
    const void* key, const void* value, int64_t key_token_stride, int64_t key_head_stride,
    int64_t value_token_stride, int64_t value_head_stride, const int64_t* slot_mapping,
    int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
    void* k_cache, void* v_cache, float* k_scales, float* v_scales,
    int32_t num_blocks, int32_t block_size, int32_t x, pa_stream_t stream);

/* Per-tensor INT8 quantize + paged-cache write.  NEW API (the reference
 * quantizes with torch): the "int8_per_tensor" write path of PagedKVCache
 * (benchmarks/int8_bridge/paged_cache.py:99-106 prefill, :140-142
 * decode_append).  Every K element is quantized with *k_scale and every V
 * element with *v_scale (one fp32 each, read on the device), as
 * int8(clamp(rne(fp32(x) / scale), -127, 127)), and the scale is stored in
 * each written slot of k_scales / v_scales.  Other arguments and rules as
 * pa_reshape_and_cache_int8. */
pa_status_t pa_reshape_and_cache_int8_static(
    const void* key, const void* value, int64_t key_token_stride, int64_t key_head_stride,
    int64_t value_token_stride, int64_t value_head_stride, const int64_t* slot_mapping,
    int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
    void* k_cache, void* v_cache, float* k_scales, float* v_scales,
    const float* k_scale, const float* v_scale,
    int32_t num_blocks, int32_t block_size, int32_t x, pa_stream_t stream);

/* The two writes above with bfloat16 key / value (bit patterns, same shapes
 * and strides).  NEW API: the reference's quantize_per_token on a bf16 tensor
 * (tests/paged_decode_attn.py:106-112, the dtype its bridge runs Qwen in,
 * benchmarks/int8_bridge/run_bridge.py:99): amax and clamp_min(1e-8) in bf16,
 * scale = fp32(bf16(amax / 127)), q = int8(clamp(rne(fp32(x) / scale), -127,
 * 127)).  The per-tensor form takes the caller's fp32 scales as
 * pa_reshape_and_cache_int8_static does. */
pa_status_t pa_reshape_and_cache_int8_bf16(
    const void* key, const void* value, int64_t key_token_stride, int64_t key_head_stride,
    int64_t value_token_stride, int64_t value_head_stride, const int64_t* slot_mapping,
    int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
    void* k_cache, void* v_cache, float* k_scales, float* v_scales,
    int32_t num_blocks, int32_t block_size, int32_t x, pa_stream_t stream);
pa_status_t pa_reshape_and_cache_int8_static_bf16(
    const void* key, const void* value, int64_t key_token_stride, int64_t key_head_stride,
    int64_t value_token_stride, int64_t value_head_stride, const int64_t* slot_mapping,
    int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
    void* k_cache, void* v_cache, float* k_scales, float* v_scales,
    const float* k_scale, const float* v_scale,
    int32_t num_blocks, int32_t block_size, int32_t x, pa_stream_t stream);

/* FP16 paged-cache write (no quantization).  NEW API (the reference scatters
 * with torch indexing): the "fp16" write path of PagedKVCache
 * (benchmarks/int8_bridge/paged_cache.py:116-130 prefill, :148-150
 * decode_append) and the placement of build_paged_kv_cache
 * (tests/paged_decode_attn.py:85-99): k_cache[blk, h, :, off, :] =
 * key[t, h].view(D/8, 8), v_cache[blk, h, :, off] = value[t, h], with
 * slot_mapping[t] = blk * block_size + off.  block_size must be a multiple
 * of 8 dividing 128; x must be 8; other rules as pa_reshape_and_cache_int8. */
pa_status_t pa_reshape_and_cache_f16(
    const void* key, const void* value, int64_t key_token_stride, int64_t key_head_stride,
    int64_t value_token_stride, int64_t value_head_stride, const int64_t* slot_mapping,
    int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
    void* k_cache, void* v_cache, int32_t num_blocks, int32_t block_size, int32_t x,
    pa_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PA_MI355X_H */

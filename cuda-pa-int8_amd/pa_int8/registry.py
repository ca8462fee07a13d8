"""Python registry of the decode variants, mirroring the reference loader.

Same names and call shapes as ``tests/cuda_ext.py`` (:104-141) of the
reference:

* ``VARIANTS[name](out, q, k_cache, v_cache, block_table, context_lens,
  scale, block_size=16) -> out`` for ``"warp"`` (single launch) and
  ``"splitk"`` (partition + reduce);
* ``VARIANTS_INT8[name](out, q, k_cache, v_cache, k_scales, v_scales,
  block_table, context_lens, scale, block_size=16) -> out`` for
  ``"warp_int8"`` and ``"splitk_int8"``.

The ladder stages ``naive``, ``vec`` and ``online`` (the reference's
optimisation history of the same function) are registered under their names
too, each with its launcher's block_size rule; on gfx950 the single-launch
kernel serves them.

Additions: ``decode`` (any variant, optional host check, forced partition
size), ``decode_plan`` and ``reshape_and_cache_int8`` (the new quantize +
cache-write op).
"""

from __future__ import annotations

from . import _loader

KIND = {"warp": 0, "splitk": 1, "warp_int8": 2, "splitk_int8": 3}


def _ext():
    return _loader.ext()


def _make_variant(op_name):
    def run(out, q, k_cache, v_cache, block_table, context_lens, scale, block_size=16):
        getattr(_ext(), op_name)(out, q, k_cache, v_cache, block_table, context_lens,
                                 float(scale), int(block_size))
        return out
    run.__name__ = op_name
    return run


def _make_variant_int8(op_name):
    def run(out, q, k_cache, v_cache, k_scales, v_scales, block_table, context_lens, scale,
            block_size=16):
        getattr(_ext(), op_name)(out, q, k_cache, v_cache, k_scales, v_scales, block_table,
                                 context_lens, float(scale), int(block_size))
        return out
    run.__name__ = op_name
    return run


def paged_decode_attention(out, q, k_cache, v_cache, block_table, context_lens, scale,
                           block_size=16):
    """The reference's top-level entry name (tests/cuda_ext.py:104-109, the
    naive stage of paged_attention_naive.cu:125-167), served by the
    single-launch kernel."""
    _ext().paged_decode_attention(out, q, k_cache, v_cache, block_table, context_lens,
                                  float(scale), int(block_size))
    return out


VARIANTS = {
    "naive": paged_decode_attention,
    "vec": _make_variant("paged_decode_attn_vec"),
    "online": _make_variant("paged_decode_attn_online"),
    "warp": _make_variant("paged_decode_attn_warp"),
    "splitk": _make_variant("paged_decode_attn_splitk"),
}
VARIANTS_INT8 = {
    "warp_int8": _make_variant_int8("paged_decode_attn_warp_int8"),
    "splitk_int8": _make_variant_int8("paged_decode_attn_splitk_int8"),
}


def decode(variant, out, q, k_cache, v_cache, block_table, context_lens, scale, block_size=16,
           k_scales=None, v_scales=None, check=True, partition_tokens=0):
    """Any variant by name; ``check=False`` skips the host-side context-length
    check (no device->host sync); ``partition_tokens`` > 0 forces the split size."""
    _ext().paged_decode_ex(KIND[variant], out, q, k_cache, v_cache, k_scales, v_scales,
                           block_table, context_lens, float(scale), int(block_size), bool(check),
                           int(partition_tokens))
    return out


def decode_plan(variant, num_seqs, num_heads, head_dim, num_kv_heads, block_size, max_blocks,
                max_context_len=0, partition_tokens=0):
    """``(partition_tokens, num_splits)`` the launcher picks for a shape."""
    return tuple(_ext().decode_plan(KIND[variant], num_seqs, num_heads, head_dim, num_kv_heads,
                                    block_size, max_blocks, max_context_len, partition_tokens))


def reshape_and_cache_int8(key, value, k_cache, v_cache, k_scales, v_scales, slot_mapping):
    """Quantize ``key/value [T, Hkv, D]`` fp16 per token and write them into the
    INT8 paged cache at ``slot_mapping`` (int64, ``block * block_size + off``)."""
    _ext().reshape_and_cache_int8(key, value, k_cache, v_cache, k_scales, v_scales, slot_mapping)


def reshape_and_cache_int8_static(key, value, k_cache, v_cache, k_scales, v_scales, slot_mapping,
                                  k_scale, v_scale):
    """INT8 write with one fp32 scale for all of ``key`` and one for all of
    ``value`` (1-element device tensors, read by the kernel): the per-tensor
    mode of PagedKVCache (benchmarks/int8_bridge/paged_cache.py:99-106,140-142)."""
    _ext().reshape_and_cache_int8_static(key, value, k_cache, v_cache, k_scales, v_scales,
                                         slot_mapping, k_scale, v_scale)


def reshape_and_cache(key, value, k_cache, v_cache, slot_mapping):
    """fp16 write of ``key/value [T, Hkv, D]`` into the paged fp16 cache at
    ``slot_mapping`` (the fp16 mode of PagedKVCache, paged_cache.py:116-130,148-150)."""
    _ext().reshape_and_cache(key, value, k_cache, v_cache, slot_mapping)

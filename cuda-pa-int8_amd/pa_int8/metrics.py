"""Algorithmic byte and flop models of the decode path.

``decode_bytes`` counts what one decode call must move at minimum: K and V
of every live token once (padding inside the last block is not counted),
the per-token fp32 scales for INT8, q and out (fp16), the block-table
entries read and the context lengths.  Split partials are implementation
overhead and are not counted.  ``decode_kv_bytes`` is the reference's
narrower "K+V read once" figure (benchmarks/bench_paged_decode.py:148-152).
"""

from __future__ import annotations

MI355X_HBM_PEAK_GBS = 8000.0        # AMD's published HBM3E peak, GB/s
MI355X_FP32_VECTOR_TFLOPS = 157.3   # published dense fp32 vector peak


def _lens(context_lens):
    return [int(c) for c in context_lens]


def decode_bytes(context_lens, num_heads, num_kv_heads, head_dim, block_size=16,
                 kv_elem_bytes=2, scales=False):
    ctx = _lens(context_lens)
    s = len(ctx)
    tok = sum(ctx)
    b = tok * num_kv_heads * head_dim * 2 * kv_elem_bytes
    if scales:
        b += tok * num_kv_heads * 2 * 4
    b += 2 * s * num_heads * head_dim * 2
    b += 4 * sum((c + block_size - 1) // block_size for c in ctx)
    b += 4 * s
    return b


def decode_kv_bytes(context_lens, num_kv_heads, head_dim, kv_elem_bytes=2):
    return sum(_lens(context_lens)) * num_kv_heads * head_dim * 2 * kv_elem_bytes


def decode_flops(context_lens, num_heads, head_dim):
    """QK and PV multiply-adds, 2 flops each."""
    return 4 * head_dim * num_heads * sum(_lens(context_lens))


def quant_write_bytes(num_tokens, num_kv_heads, head_dim):
    """Read K and V fp16, write int8 K and V plus two fp32 scales, read the slots."""
    t = num_tokens * num_kv_heads
    return t * head_dim * 2 * 2 + t * head_dim * 2 + t * 2 * 4 + 8 * num_tokens

"""CPU oracle for the paged-attention decode path (numpy restatement).

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the torch
extension, the ``pa_int8`` package) imports this module.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
use it, and only as the checker or the timed CPU baseline.

Each function restates the reference's algorithm (file:line under
Yevsquant/cuda-PA-INT8) in vectorised numpy:

* ``paged_decode_attention``     tests/paged_decode_attn.py:4-49
* ``build_paged_kv_cache``       tests/paged_decode_attn.py:52-101
* ``quantize_per_token``         tests/paged_decode_attn.py:106-112
* ``quantize_per_token_bf16``    the same on bfloat16 input (bit patterns;
                                 numpy has no bfloat16)
* ``quantize_per_tensor``        tests/paged_decode_attn.py:115-121
* ``build_paged_kv_cache_int8``  tests/paged_decode_attn.py:124-199
* ``dequantize_kv``              tests/paged_decode_attn.py:202-216
* ``reshape_and_cache_int8``     placement of tests/paged_decode_attn.py:190-197
                                 and benchmarks/int8_bridge/paged_cache.py:132-156
                                 (slot = block * block_size + offset)
* ``reshape_and_cache_int8_static``  the per-tensor write of
                                 benchmarks/int8_bridge/paged_cache.py:99-106,140-142
* ``reshape_and_cache_int8_bf16``, ``reshape_and_cache_int8_static_bf16``
                                 the two writes on bfloat16 input (bit patterns)
* ``reshape_and_cache_f16``      the fp16 write of paged_cache.py:116-130,148-150
                                 (placement of tests/paged_decode_attn.py:85-99)
* ``paged_cache_tensor_scale``   benchmarks/int8_bridge/paged_cache.py:101-102
                                 (``paged_cache_tensor_scale_bf16`` on bfloat16 input)
* ``dense_attention``            tests/test_paged_decode_attn.py:37-52

How each one is pinned (checked against something other than itself) is
listed in tests/test_oracle.py; every function above has at least one such
check.

Deliberate differences from the reference oracle:

* ``paged_decode_attention`` takes ``scale`` explicitly (the reference
  hard-codes ``1/sqrt(head_dim)`` at paged_decode_attn.py:45 and ignores the
  kernel's ``scale`` argument).  ``scale=None`` gives the reference behaviour.
* The cache builders take a ``numpy.random.Generator`` instead of drawing
  ``torch.randperm``; the layout and the block-assignment order are the same
  (``num_blocks = sum(ceil(ctx/bs)) + 1`` physical blocks, shuffled, handed
  out in sequence order), only the random stream differs.
* Quantization of a (token, kv_head) vector whose fp16 ``amax`` is 0 follows
  torch's CPU result: the scale is 0, ``0/0`` is NaN and NaN converts to
  int8 0; a non-zero element over a zero scale is +-inf and clamps to +-127.
"""

from __future__ import annotations

import math

import numpy as np

__all__ = [
    "paged_decode_attention",
    "dense_attention",
    "build_paged_kv_cache",
    "quantize_per_token",
    "quantize_per_token_bf16",
    "bf16_bits_to_f32",
    "f32_to_bf16_bits",
    "quantize_per_tensor",
    "build_paged_kv_cache_int8",
    "dequantize_kv",
    "reshape_and_cache_int8",
    "reshape_and_cache_int8_static",
    "reshape_and_cache_f16",
    "paged_cache_tensor_scale",
    "gather_kv",
]


# --------------------------------------------------------------------------
# gather + attention
# --------------------------------------------------------------------------

def gather_kv(k_cache, v_cache, block_table, ctx, seq, block_size):
    """Contiguous K, V of one sequence from the paged layout.

    K cache ``[NB, Hkv, D/x, bs, x]`` -> ``[ctx, Hkv, D]``;
    V cache ``[NB, Hkv, D, bs]``      -> ``[ctx, Hkv, D]``.
    Same index arithmetic as tests/paged_decode_attn.py:22-33 (block
    ``t // bs``, offset ``t % bs``), done a block at a time.
    """
    nb, hkv, dx, bs, x = k_cache.shape
    assert bs == block_size
    nblk = (ctx + bs - 1) // bs
    blocks = np.asarray(block_table[seq, :nblk], dtype=np.int64)
    kb = k_cache[blocks]                       # [nblk, Hkv, D/x, bs, x]
    kb = kb.transpose(0, 3, 1, 2, 4).reshape(nblk * bs, hkv, dx * x)
    vb = v_cache[blocks]                       # [nblk, Hkv, D, bs]
    vb = vb.transpose(0, 3, 1, 2).reshape(nblk * bs, hkv, -1)
    return kb[:ctx], vb[:ctx]


def paged_decode_attention(q, k_cache, v_cache, block_table, context_lens,
                           scale=None, block_size=16):
    """fp32 paged decode attention (tests/paged_decode_attn.py:4-49).

    ``out[s, h] = softmax_t(scale * K_t . q[s, h]) @ V`` over ``t < ctx_s``
    with ``kv_head = h // (H // Hkv)`` (paged_decode_attn.py:40).  Inputs may
    be any float dtype; they are widened to float32 first, as the reference
    tests do with ``.float()`` (tests/test_paged_decode_attn.py:110-112).
    A sequence with ``ctx == 0`` yields zeros (the product kernels do the
    same on their no-check entry).
    """
    q = np.asarray(q, dtype=np.float32)
    k_cache = np.asarray(k_cache, dtype=np.float32)
    v_cache = np.asarray(v_cache, dtype=np.float32)
    s_, h_, d_ = q.shape
    hkv = k_cache.shape[1]
    g = h_ // hkv
    if scale is None:
        scale = 1.0 / math.sqrt(d_)
    out = np.zeros_like(q)
    for s in range(s_):
        ctx = int(context_lens[s])
        if ctx <= 0:
            continue
        k, v = gather_kv(k_cache, v_cache, block_table, ctx, s, block_size)
        # [Hkv, G, D] x [Hkv, D, ctx] -> [Hkv, G, ctx]
        qs = q[s].reshape(hkv, g, d_)
        sc = np.matmul(qs, k.transpose(1, 2, 0)) * np.float32(scale)
        sc = sc - sc.max(axis=-1, keepdims=True)
        p = np.exp(sc)
        p /= p.sum(axis=-1, keepdims=True)
        o = np.matmul(p, v.transpose(1, 0, 2))  # [Hkv, G, D]
        out[s] = o.reshape(h_, d_)
    return out


def dense_attention(q, k, v, context_lens, num_kv_heads, scale=None):
    """Independent dense oracle on contiguous K/V ``[S, L, Hkv, D]``, float64.

    Same loop structure as tests/test_paged_decode_attn.py:37-52, computed
    head by head in float64 with the textbook softmax.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    s_, h_, d_ = q.shape
    g = h_ // num_kv_heads
    if scale is None:
        scale = 1.0 / math.sqrt(d_)
    out = np.zeros_like(q)
    for b in range(s_):
        clen = int(context_lens[b])
        for h in range(h_):
            kvh = h // g
            scores = (k[b, :clen, kvh, :] @ q[b, h]) * scale
            w = np.exp(scores - scores.max())
            w /= w.sum()
            out[b, h] = (w[:, None] * v[b, :clen, kvh, :]).sum(axis=0)
    return out


# --------------------------------------------------------------------------
# cache builders
# --------------------------------------------------------------------------

def _assign_blocks(context_lens, max_len, block_size, rng):
    """Block table + shuffled pool, following tests/paged_decode_attn.py:65-92."""
    num_seqs = len(context_lens)
    max_blocks = (max_len + block_size - 1) // block_size
    per_seq = [(int(c) + block_size - 1) // block_size for c in context_lens]
    num_blocks = sum(per_seq) + 1          # one spare block (:73)
    perm = rng.permutation(num_blocks).astype(np.int32)
    block_table = np.zeros((num_seqs, max_blocks), dtype=np.int32)
    nxt = 0
    for b in range(num_seqs):
        block_table[b, :per_seq[b]] = perm[nxt:nxt + per_seq[b]]
        nxt += per_seq[b]
    return block_table, num_blocks, per_seq


def _scatter_tokens(dst_k, dst_v, k, v, context_lens, block_table, block_size, x):
    """Write contiguous ``k, v [S, L, Hkv, D]`` into the paged layouts."""
    s_, _, hkv, d_ = k.shape
    for b in range(s_):
        clen = int(context_lens[b])
        if clen == 0:
            continue
        t = np.arange(clen)
        phys = block_table[b, t // block_size].astype(np.int64)
        off = t % block_size
        # K[phys, h, o, off, :] = k[b, t, h, o*x:(o+1)*x]
        kk = k[b, :clen].reshape(clen, hkv, d_ // x, x)
        dst_k[phys, :, :, off, :] = kk
        # V[phys, h, :, off] = v[b, t, h, :]
        dst_v[phys, :, :, off] = v[b, :clen]


def build_paged_kv_cache(k, v, context_lens, block_size=16, x=8, rng=None):
    """Paged fp cache from contiguous K/V (tests/paged_decode_attn.py:52-101).

    Returns ``(k_cache [NB,Hkv,D/x,bs,x], v_cache [NB,Hkv,D,bs], block_table)``
    in the dtype of ``k``; unused slots are zero (:76-81).
    """
    k = np.asarray(k)
    v = np.asarray(v)
    s_, max_len, hkv, d_ = k.shape
    assert d_ % x == 0
    rng = np.random.default_rng(0) if rng is None else rng
    block_table, nb, _ = _assign_blocks(context_lens, max_len, block_size, rng)
    k_cache = np.zeros((nb, hkv, d_ // x, block_size, x), dtype=k.dtype)
    v_cache = np.zeros((nb, hkv, d_, block_size), dtype=v.dtype)
    _scatter_tokens(k_cache, v_cache, k, v, context_lens, block_table, block_size, x)
    return k_cache, v_cache, block_table


# --------------------------------------------------------------------------
# INT8 quantization (bit-exact restatement of tests/paged_decode_attn.py:106-121)
# --------------------------------------------------------------------------

def _scale_from_amax(amax):
    """``(amax.clamp_min(1e-8) / 127.0).to(float32)`` evaluated in amax's dtype.

    fp16: torch evaluates the half division in float32 and rounds once to
    fp16 (round-to-nearest-even); ``clamp_min(1e-8)`` only touches
    ``amax == 0`` and the result stays 0 after the fp16 rounding.
    float32: ``clamp_min`` then a correctly rounded float32 division.
    """
    if amax.dtype == np.float16:
        a = np.maximum(amax.astype(np.float32), np.float32(1e-8))
        s16 = (a / np.float32(127.0)).astype(np.float16)
        return s16.astype(np.float32)
    a = np.maximum(amax.astype(np.float32), np.float32(1e-8))
    return (a / np.float32(127.0)).astype(np.float32)


def _quantize_with_scale(x, scale):
    """``round(x.float() / scale).clamp(-127, 127).to(int8)`` (:111, :120).

    Division is IEEE float32, ``np.rint`` is round-half-even like
    ``torch.round``; NaN (0/0) converts to 0 and +-inf clamps to +-127, as in
    torch's CPU conversion.
    """
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.rint(x.astype(np.float32) / scale)
    r = np.where(np.isnan(r), np.float32(0), r)
    return np.clip(r, -127, 127).astype(np.int8)


def quantize_per_token(x, axis=-1):
    """Per-token symmetric INT8 (tests/paged_decode_attn.py:106-112).

    Returns ``(q int8 like x, scale float32 with ``axis`` reduced)``.
    ``amax`` is taken in x's own dtype (exact for fp16).
    """
    x = np.asarray(x)
    amax = np.abs(x).max(axis=axis, keepdims=True)
    scale = _scale_from_amax(amax)
    q = _quantize_with_scale(x, scale)
    return q, np.squeeze(scale, axis=axis)


def bf16_bits_to_f32(bits):
    """bfloat16 bit patterns (uint16) -> float32 values (exact)."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return b.view(np.float32)


def f32_to_bf16_bits(x):
    """float32 -> bfloat16 bit patterns, round to nearest even (NaN stays NaN)."""
    b = np.asarray(x, dtype=np.float32).view(np.uint32)
    rounded = (b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    return np.where(nan, (b >> np.uint32(16)) | np.uint32(0x40), rounded).astype(np.uint16)


def quantize_per_token_bf16(bits, axis=-1):
    """quantize_per_token (tests/paged_decode_attn.py:106-112) on a bfloat16
    tensor given as bit patterns.  ``amax``, ``clamp_min(1e-8)`` and the
    division by 127 happen in bfloat16: torch widens to float32, computes, and
    rounds once to bfloat16 (for the quotient a correctly rounded float32
    division rounded again to bfloat16, which equals one rounding since
    24 >= 2 * 8 + 2); 1e-8 itself becomes the nearest bfloat16 value."""
    x = bf16_bits_to_f32(bits)
    amax = np.abs(x).max(axis=axis, keepdims=True)
    lo = bf16_bits_to_f32(f32_to_bf16_bits(np.float32(1e-8)))
    a = np.where(np.isnan(amax), amax, np.maximum(amax, lo))
    scale = bf16_bits_to_f32(f32_to_bf16_bits(a / np.float32(127.0)))
    q = _quantize_with_scale(x, scale)
    return q, np.squeeze(scale, axis=axis).astype(np.float32)


def quantize_per_tensor(x):
    """One scale for the whole tensor (tests/paged_decode_attn.py:115-121)."""
    x = np.asarray(x)
    amax = np.abs(x).max()
    scale = _scale_from_amax(np.asarray(amax, dtype=x.dtype))
    q = _quantize_with_scale(x, scale)
    return q, np.float32(scale)


def build_paged_kv_cache_int8(k, v, context_lens, block_size=16, x=8,
                              mode="per_token", rng=None):
    """INT8 paged cache (tests/paged_decode_attn.py:124-199).

    Returns ``(k_cache int8, v_cache int8, k_scales f32 [NB,Hkv,bs],
    v_scales f32, block_table)``.  ``per_token`` quantizes the dense
    ``[S, L, Hkv, D]`` tensors per (seq, token, kv_head) (:175-176);
    ``per_tensor`` uses one scalar per tensor broadcast into every slot
    (:167-172, :191-193).
    """
    assert mode in ("per_token", "per_tensor")
    k = np.asarray(k)
    v = np.asarray(v)
    s_, max_len, hkv, d_ = k.shape
    assert d_ % x == 0
    rng = np.random.default_rng(0) if rng is None else rng
    block_table, nb, _ = _assign_blocks(context_lens, max_len, block_size, rng)
    if mode == "per_tensor":
        kq, ks = quantize_per_tensor(k)
        vq, vs = quantize_per_tensor(v)
        ks_tok = np.full(k.shape[:3], ks, dtype=np.float32)
        vs_tok = np.full(v.shape[:3], vs, dtype=np.float32)
    else:
        kq, ks_tok = quantize_per_token(k, axis=-1)
        vq, vs_tok = quantize_per_token(v, axis=-1)
    k_cache = np.zeros((nb, hkv, d_ // x, block_size, x), dtype=np.int8)
    v_cache = np.zeros((nb, hkv, d_, block_size), dtype=np.int8)
    k_scales = np.zeros((nb, hkv, block_size), dtype=np.float32)
    v_scales = np.zeros((nb, hkv, block_size), dtype=np.float32)
    _scatter_tokens(k_cache, v_cache, kq, vq, context_lens, block_table, block_size, x)
    for b in range(s_):
        clen = int(context_lens[b])
        if clen == 0:
            continue
        t = np.arange(clen)
        phys = block_table[b, t // block_size].astype(np.int64)
        off = t % block_size
        k_scales[phys, :, off] = ks_tok[b, :clen]
        v_scales[phys, :, off] = vs_tok[b, :clen]
    return k_cache, v_cache, k_scales, v_scales, block_table


def dequantize_kv(k_cache, v_cache, k_scales, v_scales):
    """fp32 K/V from int8 + per-slot scales (tests/paged_decode_attn.py:202-216)."""
    k = k_cache.astype(np.float32) * k_scales[:, :, None, :, None]
    v = v_cache.astype(np.float32) * v_scales[:, :, None, :]
    return k, v


def _place(slot_mapping, k_cache, v_cache, kq, vq, k_scales=None, v_scales=None, ks=None,
           vs=None):
    """Write per-token rows at their slots: K to ``k_cache[phys, h, :, off, :]``
    as ``row.view(D/x, x)``, V to ``v_cache[phys, h, :, off]``, scales to
    ``[phys, h, off]``; slots outside ``[0, NB * bs)`` are skipped."""
    nb, hkv, dx, bs, x = k_cache.shape
    slots = np.asarray(slot_mapping, dtype=np.int64)
    ok = (slots >= 0) & (slots < nb * bs)
    idx = np.nonzero(ok)[0]
    phys = slots[idx] // bs
    off = slots[idx] % bs
    k_cache[phys, :, :, off, :] = kq[idx].reshape(len(idx), hkv, dx, x)
    v_cache[phys, :, :, off] = vq[idx]
    if k_scales is not None:
        k_scales[phys, :, off] = ks[idx]
        v_scales[phys, :, off] = vs[idx]


def reshape_and_cache_int8(key, value, slot_mapping, k_cache, v_cache,
                           k_scales, v_scales):
    """Quantize ``key/value [T, Hkv, D]`` per token and write them in place.

    Placement: ``slot = phys_block * bs + off``; K goes to
    ``k_cache[phys, h, :, off, :]`` as ``q.view(D/8, 8)``, V to
    ``v_cache[phys, h, :, off]``, scales to ``[phys, h, off]``
    (tests/paged_decode_attn.py:190-197; the single-token form is
    benchmarks/int8_bridge/paged_cache.py:145-154).  A negative slot, or one
    past the pool, leaves the cache untouched for that token.
    Quantization is ``quantize_per_token`` over D in key's dtype.
    """
    key = np.asarray(key)
    value = np.asarray(value)
    nb, hkv, dx, bs, x = k_cache.shape
    t_, hk, d_ = key.shape
    assert hk == hkv and dx * x == d_
    kq, ks = quantize_per_token(key, axis=-1)
    vq, vs = quantize_per_token(value, axis=-1)
    _place(slot_mapping, k_cache, v_cache, kq, vq, k_scales, v_scales, ks, vs)


def paged_cache_tensor_scale(x):
    """Per-tensor scale of PagedKVCache.prefill (benchmarks/int8_bridge/paged_cache.py:101-102):
    ``(x.abs().amax() / 127.0).to(float32).clamp_min(1e-8)``.

    The division runs in x's dtype (fp16: one rounding to fp16), the clamp
    after the conversion to float32, so ``amax = 0`` gives ``float32(1e-8)``
    (``quantize_per_tensor`` clamps before dividing and gives 0 there).
    """
    x = np.asarray(x)
    amax = np.abs(x).max()
    if x.dtype == np.float16:
        s = (np.float32(amax) / np.float32(127.0)).astype(np.float16).astype(np.float32)
    else:
        s = np.float32(np.float32(amax) / np.float32(127.0))
    return np.float32(max(s, np.float32(1e-8)))


def reshape_and_cache_int8_static(key, value, slot_mapping, k_cache, v_cache, k_scales,
                                  v_scales, k_scale, v_scale):
    """INT8 write with one given fp32 scale for all of K and one for V
    (PagedKVCache "int8_per_tensor": ``_quantize_with_scale``,
    benchmarks/int8_bridge/paged_cache.py:34-38,103-106,140-142); the scale is
    stored in every written slot (``sk.expand``, :105-106)."""
    key = np.asarray(key)
    value = np.asarray(value)
    t_ = key.shape[0]
    kq = _quantize_with_scale(key, np.float32(k_scale))
    vq = _quantize_with_scale(value, np.float32(v_scale))
    hkv = key.shape[1]
    ks = np.full((t_, hkv), np.float32(k_scale), np.float32)
    vs = np.full((t_, hkv), np.float32(v_scale), np.float32)
    _place(slot_mapping, k_cache, v_cache, kq, vq, k_scales, v_scales, ks, vs)


def reshape_and_cache_int8_bf16(key_bits, value_bits, slot_mapping, k_cache, v_cache,
                                k_scales, v_scales):
    """``reshape_and_cache_int8`` on bfloat16 ``key/value [T, Hkv, D]`` given as
    bit patterns: ``quantize_per_token_bf16`` per (token, kv head), the same
    placement."""
    kq, ks = quantize_per_token_bf16(key_bits, axis=-1)
    vq, vs = quantize_per_token_bf16(value_bits, axis=-1)
    _place(slot_mapping, k_cache, v_cache, kq, vq, k_scales, v_scales, ks, vs)


def reshape_and_cache_int8_static_bf16(key_bits, value_bits, slot_mapping, k_cache, v_cache,
                                       k_scales, v_scales, k_scale, v_scale):
    """``reshape_and_cache_int8_static`` on bfloat16 input (bit patterns): the
    values widen exactly to float32 before the division."""
    reshape_and_cache_int8_static(bf16_bits_to_f32(key_bits), bf16_bits_to_f32(value_bits),
                                  slot_mapping, k_cache, v_cache, k_scales, v_scales, k_scale,
                                  v_scale)


def paged_cache_tensor_scale_bf16(bits):
    """``paged_cache_tensor_scale`` on a bfloat16 tensor (bit patterns): amax
    exact, the division by 127 rounded once to bfloat16 (as torch computes a
    bfloat16 quotient), then float32 and the clamp."""
    amax = np.abs(bf16_bits_to_f32(bits)).max()
    s = bf16_bits_to_f32(f32_to_bf16_bits(np.float32(amax) / np.float32(127.0)))
    return np.float32(max(np.float32(s), np.float32(1e-8)))


def reshape_and_cache_f16(key, value, slot_mapping, k_cache, v_cache):
    """fp16 write of ``key/value [T, Hkv, D]`` at their slots (PagedKVCache
    "fp16", benchmarks/int8_bridge/paged_cache.py:116-130,148-150; the layout of
    tests/paged_decode_attn.py:94-97)."""
    _place(slot_mapping, k_cache, v_cache, np.asarray(key).astype(k_cache.dtype),
           np.asarray(value).astype(v_cache.dtype))

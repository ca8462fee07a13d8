"""GPU tests of the cache write path: PagedKVCache and the write ops.

Mirrors gate 1 of the reference's bridge tests (tests/test_int8_bridge.py:66-128):
prefill / decode_append through ``PagedKVCache`` at the Qwen2.5-1.5B head
shape (12 query / 2 kv heads, head_dim 128), then the split-K kernels must
match the oracle over the (dequantized) cache contents.  The tolerance is
the build target's (atol 2e-3, rtol 1e-2; the reference uses 2e-2).  On top
of that every written cache is compared byte for byte with the oracle's
write (oracle/paged_decode_ref.py), and the write ops are checked directly
on scattered slots, odd token counts, other head dims and block sizes, and
special values.
"""

import math

import numpy as np
import pytest
import torch

from _cases import HEAD_DIMS, assert_close
from oracle import paged_decode_ref as ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
HEAD_DIM, BLOCK_SIZE, X = 128, 16, 8
NUM_Q_HEADS, NUM_KV_HEADS = 12, 2
CACHE_VARIANTS = ["fp16", "int8_per_token", "int8_per_tensor"]


@pytest.fixture(scope="module", autouse=True)
def _lib(built):
    import pa_int8

    pa_int8.ext()


def _np(t):
    return t.detach().cpu().numpy()


def _oracle_cache(variant, k, v, lens_written, nb, tensor_scales=None):
    """The cache bytes the reference's PagedKVCache holds after writing
    k/v [L, H, D] (numpy fp16) at slots 0..L-1 of a zeroed layer."""
    L = k.shape[0]
    slots = np.arange(L, dtype=np.int64)
    dt = np.float16 if variant == "fp16" else np.int8
    kc = np.zeros((nb, NUM_KV_HEADS, HEAD_DIM // X, BLOCK_SIZE, X), dt)
    vc = np.zeros((nb, NUM_KV_HEADS, HEAD_DIM, BLOCK_SIZE), dt)
    ks = np.zeros((nb, NUM_KV_HEADS, BLOCK_SIZE), np.float32)
    vs = np.zeros_like(ks)
    if variant == "fp16":
        ref.reshape_and_cache_f16(k, v, slots, kc, vc)
    elif variant == "int8_per_token":
        ref.reshape_and_cache_int8(k, v, slots, kc, vc, ks, vs)
    else:
        sk, sv = tensor_scales
        ref.reshape_and_cache_int8_static(k, v, slots, kc, vc, ks, vs, sk, sv)
    return kc, vc, ks, vs


def _kernel_out(cache, q, scale):
    """tests/test_int8_bridge.py:37-51: the split-K kernel of the cache's kind."""
    import pa_int8

    out = torch.empty_like(q)
    ctx = cache.context_lens(0)
    if cache.is_int8:
        pa_int8.VARIANTS_INT8["splitk_int8"](out, q, cache.k_cache[0], cache.v_cache[0],
                                             cache.k_scales[0], cache.v_scales[0],
                                             cache.block_table, ctx, scale, BLOCK_SIZE)
    else:
        pa_int8.VARIANTS["splitk"](out, q, cache.k_cache[0], cache.v_cache[0], cache.block_table,
                                   ctx, scale, BLOCK_SIZE)
    torch.cuda.synchronize()
    return _np(out.float())


def _reference_out(cache, q, scale):
    """tests/test_int8_bridge.py:54-63: the oracle over the cache contents."""
    if cache.is_int8:
        kd, vd = ref.dequantize_kv(_np(cache.k_cache[0]), _np(cache.v_cache[0]),
                                   _np(cache.k_scales[0]), _np(cache.v_scales[0]))
    else:
        kd, vd = _np(cache.k_cache[0]), _np(cache.v_cache[0])
    return ref.paged_decode_attention(_np(q), kd, vd, _np(cache.block_table),
                                      _np(cache.context_lens(0)), scale=scale,
                                      block_size=BLOCK_SIZE)


def _inputs(clen, seed=0):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((clen, NUM_KV_HEADS, HEAD_DIM), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((clen, NUM_KV_HEADS, HEAD_DIM), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((1, NUM_Q_HEADS, HEAD_DIM), dtype=np.float32).astype(np.float16)
    return k, v, q


def _assert_cache_bytes(cache, variant, k_np, v_np, tensor_scales=None):
    kc, vc, ks, vs = _oracle_cache(variant, k_np, v_np, k_np.shape[0], cache.num_blocks,
                                   tensor_scales)
    assert np.array_equal(_np(cache.k_cache[0]).view(np.uint8), kc.view(np.uint8)), "k_cache"
    assert np.array_equal(_np(cache.v_cache[0]).view(np.uint8), vc.view(np.uint8)), "v_cache"
    if cache.is_int8:
        assert np.array_equal(_np(cache.k_scales[0]).view(np.uint32), ks.view(np.uint32))
        assert np.array_equal(_np(cache.v_scales[0]).view(np.uint32), vs.view(np.uint32))


def _tensor_scales(variant, k_np, v_np):
    if variant != "int8_per_tensor":
        return None
    return ref.paged_cache_tensor_scale(k_np), ref.paged_cache_tensor_scale(v_np)


@pytest.mark.parametrize("variant", CACHE_VARIANTS)
@pytest.mark.parametrize("clen", [1, 16, 17, 31, 128, 500])
def test_prefill_path_matches_reference(variant, clen):
    import pa_int8

    k, v, q = _inputs(clen)
    scale = 1.0 / math.sqrt(HEAD_DIM)
    cache = pa_int8.PagedKVCache(num_layers=1, num_kv_heads=NUM_KV_HEADS, head_dim=HEAD_DIM,
                                 max_len=clen, block_size=BLOCK_SIZE, x=X, variant=variant,
                                 device=DEV)
    cache.prefill(0, torch.from_numpy(k).to(DEV), torch.from_numpy(v).to(DEV))
    torch.cuda.synchronize()
    _assert_cache_bytes(cache, variant, k, v, _tensor_scales(variant, k, v))
    qd = torch.from_numpy(q).to(DEV)
    assert_close(_kernel_out(cache, qd, scale), _reference_out(cache, qd, scale), what=variant)


@pytest.mark.parametrize("variant", CACHE_VARIANTS)
@pytest.mark.parametrize("clen", [17, 31, 128, 500])
def test_decode_append_path_matches_reference(variant, clen):
    import pa_int8

    k, v, q = _inputs(clen, seed=1)
    scale = 1.0 / math.sqrt(HEAD_DIM)
    cache = pa_int8.PagedKVCache(num_layers=1, num_kv_heads=NUM_KV_HEADS, head_dim=HEAD_DIM,
                                 max_len=clen, block_size=BLOCK_SIZE, x=X, variant=variant,
                                 device=DEV)
    kd, vd = torch.from_numpy(k).to(DEV), torch.from_numpy(v).to(DEV)
    cache.prefill(0, kd[:-1], vd[:-1])
    assert cache.decode_append(0, kd[-1], vd[-1]) == clen
    torch.cuda.synchronize()
    # per-tensor scales come from the prefilled part only (paged_cache.py:101-102,140)
    ts = _tensor_scales(variant, k[:-1], v[:-1])
    _assert_cache_bytes(cache, variant, k, v, ts)
    qd = torch.from_numpy(q).to(DEV)
    assert_close(_kernel_out(cache, qd, scale), _reference_out(cache, qd, scale), what=variant)


@pytest.mark.parametrize("variant", CACHE_VARIANTS)
def test_many_appends_across_blocks_and_layers(variant):
    """Prefill 37 tokens, append 60 one at a time (crossing 4 block
    boundaries), on layer 1 of 3; the other layers stay untouched."""
    import pa_int8

    k, v, q = _inputs(97, seed=2)
    cache = pa_int8.PagedKVCache(num_layers=3, num_kv_heads=NUM_KV_HEADS, head_dim=HEAD_DIM,
                                 max_len=100, variant=variant, device=DEV)
    kd, vd = torch.from_numpy(k).to(DEV), torch.from_numpy(v).to(DEV)
    cache.prefill(1, kd[:37], vd[:37])
    for t in range(37, 97):
        assert cache.decode_append(1, kd[t], vd[t]) == t + 1
    torch.cuda.synchronize()
    assert cache.lengths == [0, 97, 0]
    ts = _tensor_scales(variant, k[:37], v[:37])
    kc, vc, ks, vs = _oracle_cache(variant, k, v, 97, cache.num_blocks, ts)
    assert np.array_equal(_np(cache.k_cache[1]).view(np.uint8), kc.view(np.uint8))
    assert np.array_equal(_np(cache.v_cache[1]).view(np.uint8), vc.view(np.uint8))
    for other in (0, 2):
        assert not _np(cache.k_cache[other]).any() and not _np(cache.v_cache[other]).any()
    if cache.is_int8:
        assert np.array_equal(_np(cache.k_scales[1]), ks) and np.array_equal(
            _np(cache.v_scales[1]), vs)


@pytest.mark.parametrize("variant", CACHE_VARIANTS)
def test_reset_and_shorter_prefill_clears_block_tail(variant):
    """A second, shorter prefill leaves zeros after it in its last block, as
    the reference's zero-padded copy does (paged_cache.py:116-128)."""
    import pa_int8

    k, v, _ = _inputs(64, seed=3)
    cache = pa_int8.PagedKVCache(num_layers=1, num_kv_heads=NUM_KV_HEADS, head_dim=HEAD_DIM,
                                 max_len=64, variant=variant, device=DEV)
    kd, vd = torch.from_numpy(k).to(DEV), torch.from_numpy(v).to(DEV)
    cache.prefill(0, kd, vd)
    cache.reset()
    cache.prefill(0, kd[:21], vd[:21])
    torch.cuda.synchronize()
    assert cache.lengths == [21]
    blk = _np(cache.k_cache[0])[1]           # block 1 holds tokens 16..31
    assert not blk[:, :, 5:, :].any() and blk[:, :, :5, :].any()
    assert not _np(cache.v_cache[0])[1][:, :, 5:].any()
    if cache.is_int8:
        assert not _np(cache.k_scales[0])[1][:, 5:].any()


def test_writes_reject_cpu_and_non_fp16_inputs():
    import pa_int8

    cache = pa_int8.PagedKVCache(1, NUM_KV_HEADS, HEAD_DIM, 32, variant="int8_per_token",
                                 device=DEV)
    with pytest.raises(TypeError, match="fp16"):
        cache.prefill(0, torch.zeros(4, 2, 128, device=DEV), torch.zeros(4, 2, 128, device=DEV))
    with pytest.raises(RuntimeError, match="CUDA"):
        pa_int8.reshape_and_cache_int8(torch.zeros(4, 2, 128, dtype=torch.float16),
                                       torch.zeros(4, 2, 128, dtype=torch.float16),
                                       cache.k_cache[0], cache.v_cache[0], cache.k_scales[0],
                                       cache.v_scales[0], torch.arange(4))
    pt = pa_int8.PagedKVCache(1, NUM_KV_HEADS, HEAD_DIM, 32, variant="int8_per_tensor",
                              device=DEV)
    with pytest.raises(RuntimeError, match="prefill"):
        pt.decode_append(0, torch.zeros(2, 128, dtype=torch.float16, device=DEV),
                         torch.zeros(2, 128, dtype=torch.float16, device=DEV))


# ---------------------------------------------------------------- write ops

def _scattered_slots(rng, T, nb, bs, holes=True):
    slots = rng.permutation(nb * bs)[:T].astype(np.int64)
    if holes and T >= 4:
        slots[1] = -1                      # skipped
        slots[T // 2] = nb * bs            # past the pool: skipped
    return slots


@pytest.mark.parametrize("head_dim", HEAD_DIMS)
@pytest.mark.parametrize("block_size", [8, 16, 32, 128])
@pytest.mark.parametrize("num_tokens", [1, 37, 300])
def test_f16_write_op_matches_oracle(head_dim, block_size, num_tokens):
    import pa_int8

    rng = np.random.default_rng(head_dim + block_size + num_tokens)
    hkv, nb = 3, (num_tokens + block_size - 1) // block_size + 4
    key = rng.standard_normal((num_tokens, hkv, head_dim), dtype=np.float32).astype(np.float16)
    val = rng.standard_normal((num_tokens, hkv, head_dim), dtype=np.float32).astype(np.float16)
    for slots in (_scattered_slots(rng, num_tokens, nb, block_size),
                  np.arange(num_tokens, dtype=np.int64) + block_size):   # prefill runs
        kc0 = rng.standard_normal((nb, hkv, head_dim // 8, block_size, 8)).astype(np.float16)
        vc0 = rng.standard_normal((nb, hkv, head_dim, block_size)).astype(np.float16)
        kc, vc = torch.from_numpy(kc0).to(DEV), torch.from_numpy(vc0).to(DEV)
        pa_int8.reshape_and_cache(torch.from_numpy(key).to(DEV), torch.from_numpy(val).to(DEV),
                                  kc, vc, torch.from_numpy(slots).to(DEV))
        torch.cuda.synchronize()
        ek, ev = kc0.copy(), vc0.copy()
        ref.reshape_and_cache_f16(key, val, slots, ek, ev)
        assert np.array_equal(_np(kc).view(np.uint16), ek.view(np.uint16))
        assert np.array_equal(_np(vc).view(np.uint16), ev.view(np.uint16))


@pytest.mark.parametrize("head_dim", HEAD_DIMS)
@pytest.mark.parametrize("block_size", [16, 64])
@pytest.mark.parametrize("num_tokens", [1, 45, 512])
def test_static_int8_write_op_matches_oracle(head_dim, block_size, num_tokens):
    """Bit-exact bytes and stored scales, with scales that put part of the
    values past +-127 (saturation) and special inputs (NaN, inf, 0)."""
    import pa_int8

    rng = np.random.default_rng(7 * head_dim + block_size + num_tokens)
    hkv, nb = 2, (num_tokens + block_size - 1) // block_size + 3
    key = (rng.standard_normal((num_tokens, hkv, head_dim)) * 4).astype(np.float16)
    val = (rng.standard_normal((num_tokens, hkv, head_dim)) * 4).astype(np.float16)
    key.reshape(-1)[:4] = [np.nan, np.inf, -np.inf, 0.0]
    for sk, sv in ((np.float32(0.0234), np.float32(0.1)),      # part of K saturates
                   (np.float32(1e-8), np.float32(3.0)),        # amax = 0 style clamp scale
                   (ref.paged_cache_tensor_scale(key[np.isfinite(key)]),
                    ref.paged_cache_tensor_scale(val))):
        for slots in (_scattered_slots(rng, num_tokens, nb, block_size),
                      np.arange(num_tokens, dtype=np.int64)):
            kc = torch.zeros((nb, hkv, head_dim // 8, block_size, 8), dtype=torch.int8, device=DEV)
            vc = torch.zeros((nb, hkv, head_dim, block_size), dtype=torch.int8, device=DEV)
            ks = torch.zeros((nb, hkv, block_size), dtype=torch.float32, device=DEV)
            vs = torch.zeros_like(ks)
            pa_int8.reshape_and_cache_int8_static(
                torch.from_numpy(key).to(DEV), torch.from_numpy(val).to(DEV), kc, vc, ks, vs,
                torch.from_numpy(slots).to(DEV), torch.tensor([sk], device=DEV),
                torch.tensor([sv], device=DEV))
            torch.cuda.synchronize()
            ek, ev = np.zeros(kc.shape, np.int8), np.zeros(vc.shape, np.int8)
            eks, evs = np.zeros(ks.shape, np.float32), np.zeros(vs.shape, np.float32)
            ref.reshape_and_cache_int8_static(key, val, slots, ek, ev, eks, evs, sk, sv)
            assert np.array_equal(_np(kc), ek) and np.array_equal(_np(vc), ev), (sk, sv)
            assert np.array_equal(_np(ks).view(np.uint32), eks.view(np.uint32))
            assert np.array_equal(_np(vs).view(np.uint32), evs.view(np.uint32))


def test_static_int8_write_near_ties():
    """Values whose quotient lies within the fast path's guard of a
    half-integer take the exact division."""
    import pa_int8

    s = np.float32(0.0123)
    n = np.arange(-126, 127, dtype=np.float64) + 0.5
    # and quotients around the clamp: 126.5 .. 128.5 (rne gives 127 or 128 -> 127)
    edge = np.array([126.4, 126.5, 126.6, 126.99, 127.0, 127.2, 127.5, 127.6, 127.9, 128.0,
                     128.5, 300.0])
    n = np.concatenate([n, edge, -edge])
    cand = (n * float(s)).astype(np.float16)
    key = np.resize(cand, (16, 1, 128)).astype(np.float16)
    val = np.resize(cand[::-1], (16, 1, 128)).astype(np.float16)
    slots = np.arange(16, dtype=np.int64)
    kc = torch.zeros((1, 1, 16, 16, 8), dtype=torch.int8, device=DEV)
    vc = torch.zeros((1, 1, 128, 16), dtype=torch.int8, device=DEV)
    ks = torch.zeros((1, 1, 16), dtype=torch.float32, device=DEV)
    vs = torch.zeros_like(ks)
    pa_int8.reshape_and_cache_int8_static(torch.from_numpy(key).to(DEV),
                                          torch.from_numpy(val).to(DEV), kc, vc, ks, vs,
                                          torch.from_numpy(slots).to(DEV),
                                          torch.tensor([s], device=DEV),
                                          torch.tensor([s], device=DEV))
    torch.cuda.synchronize()
    ek, ev = np.zeros(kc.shape, np.int8), np.zeros(vc.shape, np.int8)
    eks, evs = np.zeros(ks.shape, np.float32), np.zeros(vs.shape, np.float32)
    ref.reshape_and_cache_int8_static(key, val, slots, ek, ev, eks, evs, s, s)
    assert np.array_equal(_np(kc), ek) and np.array_equal(_np(vc), ev)

"""GPU tests of the INT8 quantize + paged-cache write on bfloat16 input.

The reference quantizes its bridge's bf16 K/V directly (quantize_per_token,
tests/paged_decode_attn.py:106-112, on the bf16 model of
benchmarks/int8_bridge/run_bridge.py:99).  Expected caches come from the
oracle's ``reshape_and_cache_int8_bf16`` (``quantize_per_token_bf16``, pinned
to the reference-written golden rows, placed as for fp16), and every byte and
scale bit must match, including slots the kernel must leave untouched.
"""

import ctypes
import os

import numpy as np
import pytest
import torch

from _cases import HEAD_DIMS
from oracle import paged_decode_ref as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _lib(built):
    import pa_int8

    pa_int8.ext()


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _bf16(bits):
    """uint16 bit patterns -> a bf16 tensor on the device."""
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


_BF16 = ref.bf16_bits_to_f32(np.arange(1 << 16, dtype=np.uint16))
_BF16 = _BF16[np.isfinite(_BF16)]


def bf16_rows(d, n, rng):
    """n rows of bf16 bit patterns: normal data, corner cases and rows whose
    quotients x / scale lie close to a half-integer."""
    rows = []
    for _ in range(n // 2):
        rows.append(rng.standard_normal(d).astype(np.float32) * np.float32(rng.choice([1e-3, 1, 40])))
    rows.append(np.zeros(d, np.float32))                                   # amax 0 -> clamp
    r = np.zeros(d, np.float32); r[:3] = [1e-9, -4e-10, 2e-9]; rows.append(r)  # below the clamp
    r = rng.standard_normal(d).astype(np.float32); r[5] = 3e38; rows.append(r)  # near bf16 max
    r = rng.standard_normal(d).astype(np.float32) * 1e-36; rows.append(r)     # tiny scale
    while len(rows) < n:                                                    # near-tie rows
        amax = np.float32(ref.bf16_bits_to_f32(ref.f32_to_bf16_bits(np.float32(rng.uniform(0.05, 3e3)))))
        s = ref.bf16_bits_to_f32(ref.f32_to_bf16_bits(amax / np.float32(127)))
        pool = _BF16[np.abs(_BF16) <= amax]
        qf = pool / s
        near = pool[np.abs(np.abs(qf - np.floor(qf)) - np.float32(0.5)) < 4e-3]
        if near.size < 4:
            continue
        row = rng.choice(near, d).astype(np.float32)
        row[0] = amax
        rows.append(row)
    return ref.f32_to_bf16_bits(np.stack(rows[:n]))


def _slots(pattern, T, nb, bs, rng):
    if pattern == "prefill":
        need = (T + bs - 1) // bs
        blocks = rng.permutation(nb)[:need]
        t = np.arange(T)
        return (blocks[t // bs] * bs + t % bs).astype(np.int64)
    s = rng.permutation(nb * bs)[:T].astype(np.int64)
    if pattern == "padding":
        s[rng.random(T) < 0.2] = -1
    return s


def _compare(got, want):
    for name, g, e in zip(("k_cache", "v_cache", "k_scales", "v_scales"), got, want):
        gb = g.view(np.uint8) if g.dtype == np.int8 else g.view(np.uint32)
        eb = e.view(np.uint8) if e.dtype == np.int8 else e.view(np.uint32)
        bad = np.argwhere(gb != eb)
        assert bad.size == 0, f"{name}: {len(bad)} mismatches, first at {bad[0].tolist()}"


def _caches(rng, nb, hkv, d, bs):
    kc = rng.integers(-128, 128, size=(nb, hkv, d // 8, bs, 8)).astype(np.int8)
    vc = rng.integers(-128, 128, size=(nb, hkv, d, bs)).astype(np.int8)
    ks = rng.standard_normal((nb, hkv, bs)).astype(np.float32)
    vs = rng.standard_normal((nb, hkv, bs)).astype(np.float32)
    return kc, vc, ks, vs


@pytest.mark.parametrize("head_dim", HEAD_DIMS)
@pytest.mark.parametrize("pattern", ["prefill", "scattered", "padding"])
def test_quant_write_bf16_matches_oracle(head_dim, pattern):
    """Per-token bf16 write, every supported head_dim, three slot patterns."""
    import pa_int8

    rng = np.random.default_rng(head_dim * 7 + len(pattern))
    T, hkv, bs = 80, 2, 16
    k = bf16_rows(head_dim, T * hkv, rng).reshape(T, hkv, head_dim)
    v = bf16_rows(head_dim, T * hkv, rng).reshape(T, hkv, head_dim)
    nb = (T + bs - 1) // bs * 2 + 3
    slots = _slots(pattern, T, nb, bs, rng)
    base = _caches(rng, nb, hkv, head_dim, bs)
    want = [a.copy() for a in base]
    ref.reshape_and_cache_int8_bf16(k, v, slots, *want)
    g = [_t(a) for a in base]
    pa_int8.reshape_and_cache_int8(_bf16(k), _bf16(v), *g, _t(slots))
    torch.cuda.synchronize()
    _compare([a.cpu().numpy() for a in g], want)


@pytest.mark.parametrize("pattern", ["prefill", "scattered"])
def test_quant_write_bf16_golden_rows(pattern):
    """Every bf16 row of the golden fixture (written by the reference's own
    quantize_per_token on bf16 input, tests/golden/make_quant_golden.py),
    with the NaN / +-inf rows: the kernel's bytes and scales equal the
    reference's (NaN where the reference's scale is NaN)."""
    import pa_int8

    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz"))
    x, q, sc = z["xb16_bits"], z["qb16"], z["sb16"]
    R, d = x.shape
    rng = np.random.default_rng(len(pattern) + 40)
    bs, nb = 16, R + 4
    slots = _slots(pattern, R, nb, bs, rng)
    kc = torch.zeros((nb, 1, d // 8, bs, 8), dtype=torch.int8, device=DEV)
    vc = torch.zeros((nb, 1, d, bs), dtype=torch.int8, device=DEV)
    ks = torch.zeros((nb, 1, bs), dtype=torch.float32, device=DEV)
    vs = torch.zeros_like(ks)
    pa_int8.reshape_and_cache_int8(_bf16(x[:, None]), _bf16(x[::-1, None]), kc, vc, ks, vs,
                                   _t(slots))
    torch.cuda.synchronize()
    blk, off = slots // bs, slots % bs
    assert np.array_equal(kc.cpu().numpy()[blk, 0, :, off, :].reshape(R, d), q)
    assert np.array_equal(vc.cpu().numpy()[blk, 0, :, off], q[::-1])
    for got, want in ((ks.cpu().numpy()[blk, 0, off], sc), (vs.cpu().numpy()[blk, 0, off], sc[::-1])):
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_quant_write_bf16_through_c_abi():
    """The C entry point itself (pa_reshape_and_cache_int8_bf16), strided input:
    key and value are views of a fused [T, 3, Hkv, D] buffer."""
    import pa_int8

    lib = pa_int8.capi()
    rng = np.random.default_rng(5)
    T, hkv, d, bs, nb = 70, 2, 128, 16, 12
    qkv = bf16_rows(d, T * 3 * hkv, rng).reshape(T, 3, hkv, d)
    tq = _bf16(qkv)
    key, value = tq[:, 1], tq[:, 2]
    slots = rng.permutation(nb * bs)[:T].astype(np.int64)
    base = _caches(rng, nb, hkv, d, bs)
    want = [a.copy() for a in base]
    ref.reshape_and_cache_int8_bf16(qkv[:, 1], qkv[:, 2], slots, *want)
    g = [_t(a) for a in base]
    ts = _t(slots)
    st = lib.pa_reshape_and_cache_int8_bf16(
        key.data_ptr(), value.data_ptr(), key.stride(0), key.stride(1), value.stride(0),
        value.stride(1), ts.data_ptr(), T, hkv, d, g[0].data_ptr(), g[1].data_ptr(),
        g[2].data_ptr(), g[3].data_ptr(), nb, bs, 8, ctypes.c_void_p(0))
    assert st == 0, lib.pa_status_string(st)
    torch.cuda.synchronize()
    _compare([a.cpu().numpy() for a in g], want)


@pytest.mark.parametrize("head_dim", [64, 128])
def test_quant_write_static_bf16(head_dim):
    """Per-tensor mode on bf16 input: the caller's scales, including one so
    small that most quotients saturate at +-127."""
    import pa_int8

    rng = np.random.default_rng(head_dim)
    T, hkv, bs = 48, 2, 16
    k = bf16_rows(head_dim, T * hkv, rng).reshape(T, hkv, head_dim)
    v = bf16_rows(head_dim, T * hkv, rng).reshape(T, hkv, head_dim)
    nb = 8
    slots = _slots("scattered", T, nb, bs, rng)
    for k_scale, v_scale in ((ref.paged_cache_tensor_scale_bf16(k),
                              ref.paged_cache_tensor_scale_bf16(v)),
                             (np.float32(1e-3), np.float32(0.37))):
        base = _caches(rng, nb, hkv, head_dim, bs)
        want = [a.copy() for a in base]
        ref.reshape_and_cache_int8_static_bf16(k, v, slots, *want, k_scale, v_scale)
        g = [_t(a) for a in base]
        pa_int8.reshape_and_cache_int8_static(
            _bf16(k), _bf16(v), *g, _t(slots), _t(np.array([k_scale], np.float32)),
            _t(np.array([v_scale], np.float32)))
        torch.cuda.synchronize()
        _compare([a.cpu().numpy() for a in g], want)


@pytest.mark.parametrize("variant", ["int8_per_token", "int8_per_tensor"])
def test_paged_cache_bf16_prefill_and_append(variant):
    """PagedKVCache on bf16 K/V, as the reference's bridge feeds it: prefill
    then appends, every cache byte and scale as the oracle writes them."""
    from pa_int8 import PagedKVCache

    rng = np.random.default_rng(11)
    hkv, d, L, n_app = 2, 128, 37, 5
    cache = PagedKVCache(num_layers=1, num_kv_heads=hkv, head_dim=d, max_len=64,
                         variant=variant, device=DEV)
    k = bf16_rows(d, (L + n_app) * hkv, rng).reshape(L + n_app, hkv, d)
    v = bf16_rows(d, (L + n_app) * hkv, rng).reshape(L + n_app, hkv, d)
    cache.prefill(0, _bf16(k[:L]), _bf16(v[:L]))
    for t in range(L, L + n_app):
        cache.decode_append(0, _bf16(k[t]), _bf16(v[t]))
    torch.cuda.synchronize()
    nb, bs = cache.num_blocks, cache.block_size
    want = [np.zeros((nb, hkv, d // 8, bs, 8), np.int8), np.zeros((nb, hkv, d, bs), np.int8),
            np.zeros((nb, hkv, bs), np.float32), np.zeros((nb, hkv, bs), np.float32)]
    slots = np.arange(L + n_app, dtype=np.int64)
    if variant == "int8_per_token":
        ref.reshape_and_cache_int8_bf16(k, v, slots, *want)
    else:
        ref.reshape_and_cache_int8_static_bf16(k, v, slots, *want,
                                               ref.paged_cache_tensor_scale_bf16(k[:L]),
                                               ref.paged_cache_tensor_scale_bf16(v[:L]))
    got = [cache.k_cache[0].cpu().numpy(), cache.v_cache[0].cpu().numpy(),
           cache.k_scales[0].cpu().numpy(), cache.v_scales[0].cpu().numpy()]
    _compare(got, want)

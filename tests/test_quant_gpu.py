"""GPU tests of the INT8 quantize + paged-cache write kernel (bit-exact).

The expected caches come from the oracle's ``reshape_and_cache_int8``
(quantize_per_token of tests/paged_decode_attn.py:106-112 placed as at
:190-197).  Every byte of k_cache/v_cache and every scale bit must match,
including slots the kernel must leave untouched.
"""

import numpy as np
import pytest
import torch

from _cases import HEAD_DIMS, assert_close, make_lens, record_headroom
from oracle import paged_decode_ref as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _lib(built):
    import pa_int8

    pa_int8.ext()


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def special_rows(d, rng):
    """Rows that pin the corner cases of the quantizer."""
    rows = []
    rows.append(np.zeros(d, np.float32))                                   # amax = 0
    r = np.zeros(d, np.float32); r[:4] = [1e-7, -3e-7, 6e-8, 0]; rows.append(r)  # scale -> 0
    r = rng.standard_normal(d).astype(np.float32) * 2e-3; rows.append(r)  # subnormal fp16 scale
    r = np.zeros(d, np.float32)
    ties = [127, 2.5, 3.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -126.5, 63.5, -0.49]
    r[:min(12, d)] = ties[:min(12, d)]
    rows.append(r)                                                          # exact ties, scale 1
    r = rng.standard_normal(d).astype(np.float32); r[0] = 1000.0; rows.append(r)  # outlier
    r = np.full(d, -65504.0, np.float32); r[1::2] = 65504.0; rows.append(r)     # fp16 max
    return np.stack(rows)


_FP16 = np.arange(1 << 16, dtype=np.uint16).view(np.float16)
_FP16 = _FP16[np.isfinite(_FP16)].astype(np.float32)


def near_tie_rows(d, n, rng):
    """Rows whose quotients x / scale lie within 2e-4 of a half-integer: the
    inputs where x * (1/scale) and the IEEE quotient can round differently."""
    rows = []
    while len(rows) < n:
        amax = np.float32(np.float16(rng.uniform(0.05, 3000.0)))
        s = np.float32(np.float16(max(amax, np.float32(1e-8)) / np.float32(127)))
        x = _FP16[np.abs(_FP16) <= amax]
        qf = x / s
        near = x[np.abs(np.abs(qf - np.floor(qf)) - np.float32(0.5)) < 2e-4]
        if near.size < 4:
            continue
        row = rng.choice(near, size=d)
        row[0] = amax                     # pins the scale
        rows.append(row)
    return np.stack(rows).astype(np.float16)


def make_kv(T, hkv, d, rng):
    k = rng.standard_normal((T, hkv, d)).astype(np.float32)
    v = rng.standard_normal((T, hkv, d)).astype(np.float32) * 3.0
    sp = special_rows(d, rng)
    n = min(len(sp), T)
    k[:n, 0] = sp[:n]
    v[:n, -1] = sp[::-1][:n]
    return k.astype(np.float16), v.astype(np.float16)


def slots_for(pattern, T, num_blocks, bs, rng):
    if pattern == "prefill":
        # sequences of ragged length filling their own blocks in order
        lens = []
        left = T
        while left > 0:
            l = int(min(left, rng.integers(1, 200)))
            lens.append(l)
            left -= l
        need = sum((l + bs - 1) // bs for l in lens)
        assert need <= num_blocks
        perm = rng.permutation(num_blocks)[:need]
        out, nb = [], 0
        for l in lens:
            nblk = (l + bs - 1) // bs
            blocks = perm[nb:nb + nblk]
            nb += nblk
            t = np.arange(l)
            out.append(blocks[t // bs] * bs + t % bs)
        return np.concatenate(out).astype(np.int64)
    if pattern == "scattered":
        return rng.permutation(num_blocks * bs)[:T].astype(np.int64)
    if pattern == "padding":
        s = rng.permutation(num_blocks * bs)[:T].astype(np.int64)
        s[rng.random(T) < 0.2] = -1
        s[3] = num_blocks * bs + 7          # past the pool: skipped
        return s
    raise ValueError(pattern)


def run_case(T, hkv, d, bs, pattern, seed, kv=None):
    rng = np.random.default_rng(seed)
    k, v = make_kv(T, hkv, d, rng) if kv is None else kv(T, hkv, d, rng)
    num_blocks = (T + bs - 1) // bs * 2 + 3
    slots = slots_for(pattern, T, num_blocks, bs, rng)
    kc = rng.integers(-128, 128, size=(num_blocks, hkv, d // 8, bs, 8)).astype(np.int8)
    vc = rng.integers(-128, 128, size=(num_blocks, hkv, d, bs)).astype(np.int8)
    ks = rng.standard_normal((num_blocks, hkv, bs)).astype(np.float32)
    vs = rng.standard_normal((num_blocks, hkv, bs)).astype(np.float32)
    ekc, evc, eks, evs = kc.copy(), vc.copy(), ks.copy(), vs.copy()
    ref.reshape_and_cache_int8(k, v, slots, ekc, evc, eks, evs)

    import pa_int8

    tkc, tvc, tks, tvs = _t(kc), _t(vc), _t(ks), _t(vs)
    pa_int8.reshape_and_cache_int8(_t(k), _t(v), tkc, tvc, tks, tvs, _t(slots))
    torch.cuda.synchronize()
    got = [x.cpu().numpy() for x in (tkc, tvc, tks, tvs)]
    for name, g, e in zip(("k_cache", "v_cache", "k_scales", "v_scales"), got,
                          (ekc, evc, eks, evs)):
        gb = g.view(np.uint8) if g.dtype == np.int8 else g.view(np.uint32)
        eb = e.view(np.uint8) if e.dtype == np.int8 else e.view(np.uint32)
        bad = np.argwhere(gb != eb)
        assert bad.size == 0, f"{name}: {len(bad)} mismatches, first at {bad[0].tolist()}: " \
                              f"got {g[tuple(bad[0])]} want {e[tuple(bad[0])]}"


@pytest.mark.parametrize("head_dim", HEAD_DIMS)
@pytest.mark.parametrize("block_size", [16, 32, 64, 128])
@pytest.mark.parametrize("pattern", ["prefill", "scattered", "padding"])
def test_quant_write_bitexact(head_dim, block_size, pattern):
    run_case(T=301, hkv=2, d=head_dim, bs=block_size, pattern=pattern, seed=head_dim + block_size)


@pytest.mark.parametrize("head_dim", HEAD_DIMS)
@pytest.mark.parametrize("pattern", ["prefill", "scattered"])
def test_quant_write_near_ties(head_dim, pattern):
    """Every element near a rounding tie: the kernel's reciprocal fast path must
    hand these to the exact division (bit-exact with the IEEE quotient)."""
    def kv(T, hkv, d, rng):
        k = near_tie_rows(d, T * hkv, rng).reshape(T, hkv, d)
        v = near_tie_rows(d, T * hkv, rng).reshape(T, hkv, d)
        return k, v
    run_case(T=96, hkv=2, d=head_dim, bs=16, pattern=pattern, seed=head_dim + 5, kv=kv)


@pytest.mark.parametrize("pattern", ["prefill", "scattered"])
def test_quant_write_matches_reference_golden_rows(pattern):
    """Every fp16 row of the golden fixture (written by the reference's own
    quantize_per_token, tests/golden/make_quant_golden.py), including the rows
    with NaN and +-inf, goes through the write kernel: each token's int8
    bytes must equal the reference's, and its scale too (bit for bit where
    finite; NaN where the reference's is NaN)."""
    import os

    import pa_int8

    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz"))
    x = np.concatenate([z["x16"], z["xnf"]])                     # [R, 128]
    q = np.concatenate([z["q16"], z["qnf"]])
    sc = np.concatenate([z["s16"], z["snf"]])
    R, d = x.shape
    rng = np.random.default_rng(len(pattern))
    T = R                                     # one token per row; K and V get the rows
    k = x[:, None, :]                         # [T, 1, D]
    v = x[::-1][:, None, :].copy()            # reversed order for V
    bs, nb = 16, R + 4                        # room for one block per token
    slots = slots_for(pattern, T, nb, bs, rng)
    kc = torch.zeros((nb, 1, d // 8, bs, 8), dtype=torch.int8, device=DEV)
    vc = torch.zeros((nb, 1, d, bs), dtype=torch.int8, device=DEV)
    ks = torch.zeros((nb, 1, bs), dtype=torch.float32, device=DEV)
    vs = torch.zeros_like(ks)
    pa_int8.reshape_and_cache_int8(_t(k), _t(v), kc, vc, ks, vs, _t(slots))
    torch.cuda.synchronize()
    blk, off = slots // bs, slots % bs
    gk = kc.cpu().numpy()[blk, 0, :, off, :].reshape(T, d)
    gv = vc.cpu().numpy()[blk, 0, :, off]
    assert np.array_equal(gk, q) and np.array_equal(gv, q[::-1])
    for got, want in ((ks.cpu().numpy()[blk, 0, off], sc), (vs.cpu().numpy()[blk, 0, off], sc[::-1])):
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_quant_write_single_token_append():
    """decode_append pattern (benchmarks/int8_bridge/paged_cache.py:132-156): T=batch."""
    run_case(T=5, hkv=4, d=128, bs=16, pattern="scattered", seed=3)


def test_quant_write_strided_input():
    """key/value as views of a fused [T, 3, Hkv, D] qkv buffer."""
    rng = np.random.default_rng(9)
    T, hkv, d, bs = 70, 2, 128, 16
    qkv = rng.standard_normal((T, 3, hkv, d)).astype(np.float16)
    tq = _t(qkv)
    key, value = tq[:, 1], tq[:, 2]
    nb = 12
    slots = rng.permutation(nb * bs)[:T].astype(np.int64)
    kc = np.zeros((nb, hkv, d // 8, bs, 8), np.int8); vc = np.zeros((nb, hkv, d, bs), np.int8)
    ks = np.zeros((nb, hkv, bs), np.float32); vs = np.zeros_like(ks)
    ekc, evc, eks, evs = kc.copy(), vc.copy(), ks.copy(), vs.copy()
    ref.reshape_and_cache_int8(qkv[:, 1], qkv[:, 2], slots, ekc, evc, eks, evs)
    import pa_int8

    g = [_t(a) for a in (kc, vc, ks, vs)]
    pa_int8.reshape_and_cache_int8(key, value, *g, _t(slots))
    torch.cuda.synchronize()
    for a, e in zip(g, (ekc, evc, eks, evs)):
        assert np.array_equal(a.cpu().numpy().view(np.uint8), e.view(np.uint8))


def test_quant_write_full_size_then_decode():
    """BASELINE config 3 write: 64 x 8192 tokens x 2 kv heads, then INT8 decode of it."""
    import pa_int8

    rng = np.random.default_rng(77)
    S, L, hkv, H, d, bs = 64, 8192, 2, 12, 128, 16
    nblk = S * L // bs
    perm = rng.permutation(nblk + 1).astype(np.int32)
    bt = perm[:nblk].reshape(S, L // bs)
    t = np.arange(L)
    slots = (bt[:, t // bs].astype(np.int64) * bs + t % bs).reshape(-1)
    T = S * L
    k = rng.standard_normal((T, hkv, d), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((T, hkv, d), dtype=np.float32).astype(np.float16)
    kc = torch.zeros((nblk + 1, hkv, d // 8, bs, 8), dtype=torch.int8, device=DEV)
    vc = torch.zeros((nblk + 1, hkv, d, bs), dtype=torch.int8, device=DEV)
    ks = torch.zeros((nblk + 1, hkv, bs), dtype=torch.float32, device=DEV)
    vs = torch.zeros_like(ks)
    pa_int8.reshape_and_cache_int8(_t(k), _t(v), kc, vc, ks, vs, _t(slots))
    torch.cuda.synchronize()
    # bit-exact against the oracle quantizer on every token
    kq, ksc = ref.quantize_per_token(k, axis=-1)
    vq, vsc = ref.quantize_per_token(v, axis=-1)
    phys = slots // bs
    off = slots % bs
    gk = kc.cpu().numpy()[phys, :, :, off, :].reshape(T, hkv, d)
    assert np.array_equal(gk, kq)
    gv = vc.cpu().numpy()[phys, :, :, off]
    assert np.array_equal(gv, vq)
    assert np.array_equal(ks.cpu().numpy()[phys, :, off].view(np.uint32), ksc.view(np.uint32))
    assert np.array_equal(vs.cpu().numpy()[phys, :, off].view(np.uint32), vsc.view(np.uint32))
    # decode over the kernel-written cache (first 4 sequences checked against the oracle)
    q = rng.standard_normal((S, H, d), dtype=np.float32).astype(np.float16)
    lens = np.full(S, L, np.int32)
    out = torch.empty((S, H, d), dtype=torch.float16, device=DEV)
    pa_int8.VARIANTS_INT8["warp_int8"](out, _t(q), kc, vc, ks, vs, _t(bt), _t(lens),
                                       1.0 / np.sqrt(d), bs)
    torch.cuda.synchronize()
    kd, vd = ref.dequantize_kv(kc.cpu().numpy(), vc.cpu().numpy(), ks.cpu().numpy(),
                               vs.cpu().numpy())
    want = ref.paged_decode_attention(q[:4], kd, vd, bt[:4], lens[:4], scale=1.0 / np.sqrt(d))
    ratio = assert_close(out[:4].float().cpu().numpy(), want, what="decode after write")
    record_headroom("cfg3", "warp_int8 64 x 8192 12/2 over the kernel-written cache", ratio,
                    variant="warp_int8", seqs_checked=4)


@pytest.mark.parametrize("block_size", [16, 32])
@pytest.mark.parametrize("pattern", ["prefill", "scattered", "padding"])
def test_write_stream_probe_stores_where_the_kernel_does(block_size, pattern):
    """The benchmark's write-stream probe (pa_probe_quant_write, the write
    kernel's template in its PROBE form) stores each element's high byte and a
    scale of 1 at exactly the cache positions the write op fills, and leaves
    every other byte alone: its address stream is the kernel's."""
    from pa_int8 import _loader

    lib = _loader.probe_capi()
    rng = np.random.default_rng(block_size + len(pattern))
    T, hkv, d, bs = 80, 2, 128, block_size
    k, v = make_kv(T, hkv, d, rng)
    nb = (T + bs - 1) // bs * 2 + 3
    slots = slots_for(pattern, T, nb, bs, rng)
    kc = rng.integers(-128, 128, size=(nb, hkv, d // 8, bs, 8)).astype(np.int8)
    vc = rng.integers(-128, 128, size=(nb, hkv, d, bs)).astype(np.int8)
    ks = rng.standard_normal((nb, hkv, bs)).astype(np.float32)
    vs = rng.standard_normal((nb, hkv, bs)).astype(np.float32)
    want = [a.copy() for a in (kc, vc, ks, vs)]
    hi = lambda x: (x.view(np.uint16) >> 8).astype(np.uint8).view(np.int8)
    for t, s in enumerate(slots):
        if not 0 <= s < nb * bs:
            continue
        blk, off = s // bs, s % bs
        want[0][blk, :, :, off, :] = hi(k[t]).reshape(hkv, d // 8, 8)
        want[1][blk, :, :, off] = hi(v[t])
        want[2][blk, :, off] = 1.0
        want[3][blk, :, off] = 1.0
    tk, tv, ts = _t(k), _t(v), _t(slots)
    g = [_t(a) for a in (kc, vc, ks, vs)]
    st = lib.pa_probe_quant_write(tk.data_ptr(), tv.data_ptr(), tk.stride(0), tk.stride(1),
                                  tv.stride(0), tv.stride(1), ts.data_ptr(), T, hkv,
                                  g[0].data_ptr(), g[1].data_ptr(), g[2].data_ptr(),
                                  g[3].data_ptr(), nb, bs, None)
    assert st == 0
    torch.cuda.synchronize()
    for name, got, exp in zip(("k_cache", "v_cache", "k_scales", "v_scales"), g, want):
        got = got.cpu().numpy()
        gb = got.view(np.uint8) if got.dtype == np.int8 else got.view(np.uint32)
        eb = exp.view(np.uint8) if exp.dtype == np.int8 else exp.view(np.uint32)
        bad = np.argwhere(gb != eb)
        assert bad.size == 0, f"{name}: {len(bad)} mismatches, first at {bad[0].tolist()}"

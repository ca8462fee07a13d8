"""CPU tests that pin the oracle (oracle/paged_decode_ref.py).

Each oracle function is checked against something other than itself:

* paged_decode_attention -- an independent float64 dense oracle on the
  reference's own grid (tests/test_paged_decode_attn.py:55-77), invariants
  (ctx=1, constant K, convex-hull bounds, physical-block permutation, scale)
  and a planted mistake that the grid must catch.
* quantize_per_token / quantize_per_tensor -- golden vectors written by the
  reference's own functions (tests/golden/quant_golden.npz), an exact-rational
  restatement of the arithmetic, and the reference's unit tests
  (tests/test_quant.py:17-105).
* build_paged_kv_cache(_int8), dequantize_kv, reshape_and_cache_int8 --
  gather round trips, the golden dequant vectors and cross-agreement of the
  two placement routes.
"""

import math
import os
from fractions import Fraction

import numpy as np
import pytest

from _cases import CONTEXT_LENS, GQA, NUM_SEQS, fp16_case, make_lens
from oracle import paged_decode_ref as ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz")


# ------------------------------------------------------------------ attention

def _f32_case(num_seqs, lens, h, hkv, d=128, seed=0):
    return fp16_case(num_seqs, lens, h, hkv, head_dim=d, seed=seed, dtype=np.float32)


@pytest.mark.parametrize("clen", CONTEXT_LENS)
@pytest.mark.parametrize("num_heads,num_kv_heads", GQA)
@pytest.mark.parametrize("num_seqs", NUM_SEQS)
def test_paged_oracle_matches_dense(clen, num_heads, num_kv_heads, num_seqs):
    c = _f32_case(num_seqs, make_lens(clen, num_seqs), num_heads, num_kv_heads)
    got = ref.paged_decode_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"],
                                     c["lens"])
    want = ref.dense_attention(c["q"], c["k"], c["v"], c["lens"], num_kv_heads)
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-5)


def test_dense_oracle_against_textbook_formula():
    """The float64 dense oracle equals softmax attention written out by hand."""
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 2, 4))
    k = rng.standard_normal((1, 3, 1, 4))
    v = rng.standard_normal((1, 3, 1, 4))
    got = ref.dense_attention(q, k, v, [3], 1, scale=0.5)
    for h in range(2):
        w = [math.exp(0.5 * sum(q[0, h, i] * k[0, t, 0, i] for i in range(4))) for t in range(3)]
        z = sum(w)
        o = [sum(w[t] * v[0, t, 0, i] for t in range(3)) / z for i in range(4)]
        np.testing.assert_allclose(got[0, h], o, rtol=1e-12)


def test_planted_gqa_mistake_is_caught():
    """A kv_head = h % Hkv mapping (instead of h // G) must fail the dense check."""
    c = _f32_case(2, make_lens(40, 2), 8, 2)
    good = ref.paged_decode_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"],
                                      c["lens"])
    perm = np.arange(8).reshape(2, 4).T.reshape(-1)     # h -> head order of h % Hkv
    bad = ref.paged_decode_attention(c["q"][:, perm], c["k_cache"], c["v_cache"],
                                     c["block_table"], c["lens"])[:, np.argsort(perm)]
    want = ref.dense_attention(c["q"], c["k"], c["v"], c["lens"], 2)
    assert np.allclose(good, want, atol=1e-5)
    assert not np.allclose(bad, want, atol=1e-3)


def test_ctx_one_returns_first_value():
    c = _f32_case(3, np.array([1, 1, 1], np.int32), 8, 2)
    got = ref.paged_decode_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"],
                                     c["lens"])
    for s in range(3):
        for h in range(8):
            np.testing.assert_allclose(got[s, h], c["v"][s, 0, h // 4], rtol=1e-6)


def test_constant_keys_give_mean_of_values():
    c = _f32_case(2, np.array([37, 90], np.int32), 8, 4)
    k = np.broadcast_to(c["k"][:, :1], c["k"].shape).copy()
    kc, vc, bt = ref.build_paged_kv_cache(k, c["v"], c["lens"], rng=np.random.default_rng(3))
    got = ref.paged_decode_attention(c["q"], kc, vc, bt, c["lens"])
    for s, n in enumerate(c["lens"]):
        for h in range(8):
            np.testing.assert_allclose(got[s, h], c["v"][s, :n, h // 2].mean(0), atol=1e-5)


def test_output_within_value_hull():
    c = _f32_case(3, make_lens(300, 3), 12, 2)
    got = ref.paged_decode_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"],
                                     c["lens"])
    for s, n in enumerate(c["lens"]):
        for h in range(12):
            vv = c["v"][s, :n, h // 6]
            assert (got[s, h] <= vv.max(0) + 1e-5).all() and (got[s, h] >= vv.min(0) - 1e-5).all()


def test_block_permutation_invariance():
    c = _f32_case(3, make_lens(200, 3), 8, 2)
    nb = c["k_cache"].shape[0]
    perm = np.random.default_rng(9).permutation(nb)     # new id of old block b is perm[b]
    kc = np.empty_like(c["k_cache"]); kc[perm] = c["k_cache"]
    vc = np.empty_like(c["v_cache"]); vc[perm] = c["v_cache"]
    bt = perm[c["block_table"]].astype(np.int32)
    a = ref.paged_decode_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"], c["lens"])
    b = ref.paged_decode_attention(c["q"], kc, vc, bt, c["lens"])
    np.testing.assert_allclose(a, b, atol=1e-6)


def test_explicit_scale_equals_scaled_query():
    c = _f32_case(2, make_lens(50, 2), 8, 8)
    a = ref.paged_decode_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"],
                                   c["lens"], scale=0.3)
    b = ref.paged_decode_attention(c["q"] * np.float32(0.3 * math.sqrt(128)), c["k_cache"],
                                   c["v_cache"], c["block_table"], c["lens"])
    np.testing.assert_allclose(a, b, atol=1e-5)


def test_zero_context_gives_zero():
    c = _f32_case(2, np.array([5, 5], np.int32), 8, 2)
    out = ref.paged_decode_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"],
                                     np.array([0, 5], np.int32))
    assert np.all(out[0] == 0) and np.any(out[1] != 0)


# ------------------------------------------------------------------ quantization

def _golden():
    if not os.path.exists(GOLDEN):
        pytest.skip("golden vectors missing")
    return np.load(GOLDEN)


def test_quant_per_token_matches_reference_golden_fp16():
    z = _golden()
    q, s = ref.quantize_per_token(z["x16"], axis=-1)
    assert np.array_equal(q, z["q16"])
    assert np.array_equal(s.view(np.uint32), z["s16"].view(np.uint32))


def test_quant_per_token_matches_reference_golden_fp32():
    z = _golden()
    q, s = ref.quantize_per_token(z["x32"], axis=-1)
    assert np.array_equal(q, z["q32"])
    assert np.array_equal(s.view(np.uint32), z["s32"].view(np.uint32))


def test_quant_per_token_matches_reference_golden_nonfinite():
    """Rows holding NaN or +-inf: amax propagates them into the scale (NaN or
    inf) and every element converts to 0 (x / inf = 0, NaN -> 0)."""
    z = _golden()
    q, s = ref.quantize_per_token(z["xnf"], axis=-1)
    assert np.array_equal(q, z["qnf"])
    assert np.array_equal(np.isnan(s), np.isnan(z["snf"]))
    fin = ~np.isnan(z["snf"])
    assert np.array_equal(s[fin], z["snf"][fin])
    assert not q.any() and np.isnan(z["snf"]).any() and np.isinf(z["snf"]).any()


def test_quant_per_token_matches_reference_golden_bf16():
    z = _golden()
    q, s = ref.quantize_per_token_bf16(z["xb16_bits"], axis=-1)
    assert np.array_equal(q, z["qb16"])
    fin = ~np.isnan(z["sb16"])
    assert np.array_equal(np.isnan(s), ~fin)
    assert np.array_equal(s[fin].view(np.uint32), z["sb16"][fin].view(np.uint32))


def test_paged_cache_tensor_scale_bf16_matches_torch():
    """The per-tensor scale of PagedKVCache.prefill on bf16 K/V
    (benchmarks/int8_bridge/paged_cache.py:101-102) evaluated by torch's own
    bfloat16 arithmetic on the CPU: amax, the bf16 quotient, float32, clamp."""
    rng = np.random.default_rng(21)
    cases = [rng.standard_normal((7, 2, 64)).astype(np.float32) * sc for sc in (1e-12, 3e-9, 1.0, 3e4)]
    cases.append(np.zeros((3, 2, 64), np.float32))
    import torch

    for x in cases:
        bits = ref.f32_to_bf16_bits(x)
        t = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
        want = (t.abs().amax() / 127.0).to(torch.float32).clamp_min(1e-8).item()
        got = ref.paged_cache_tensor_scale_bf16(bits)
        assert np.float32(want).view(np.uint32) == np.float32(got).view(np.uint32)


def test_reshape_and_cache_int8_bf16_places_golden_rows():
    """The bf16 write places quantize_per_token_bf16's rows of the golden
    fixture (reference-written) at their slots; untouched slots keep their
    bytes."""
    z = _golden()
    x = z["xb16_bits"]                                  # [R, 128] bf16 bits
    R, d = x.shape
    bs, nb = 16, 4
    rng = np.random.default_rng(3)
    slots = rng.permutation(nb * bs)[:R].astype(np.int64)
    kc = np.full((nb, 1, d // 8, bs, 8), 5, np.int8); vc = np.full((nb, 1, d, bs), 5, np.int8)
    ks = np.full((nb, 1, bs), 7.0, np.float32); vs = ks.copy()
    ref.reshape_and_cache_int8_bf16(x[:, None], x[::-1, None].copy(), slots, kc, vc, ks, vs)
    blk, off = slots // bs, slots % bs
    assert np.array_equal(kc[blk, 0, :, off, :].reshape(R, d), z["qb16"])
    assert np.array_equal(vc[blk, 0, :, off], z["qb16"][::-1])
    got = ks[blk, 0, off]
    fin = ~np.isnan(z["sb16"])
    assert np.array_equal(got[fin].view(np.uint32), z["sb16"][fin].view(np.uint32))
    free = np.setdiff1d(np.arange(nb * bs), slots)
    assert (kc[free // bs, 0, :, free % bs, :] == 5).all() and (ks[free // bs, 0, free % bs] == 7).all()


def test_bf16_rounding_helpers():
    """f32 -> bf16 bit rounding agrees with torch's conversion on every bf16
    neighbourhood we can name: exact values, midpoints (ties to even), and
    random floats; NaN stays NaN."""
    import torch

    rng = np.random.default_rng(11)
    base = rng.integers(0, 1 << 16, size=4096, dtype=np.uint32).astype(np.uint16)
    f = ref.bf16_bits_to_f32(base)
    f = f[np.isfinite(f)]
    mids = (f.view(np.uint32) + np.uint32(0x8000)).view(np.float32)     # exact midpoints
    rnd = rng.standard_normal(4096).astype(np.float32) * np.float32(1e3)
    for x in (f, mids[np.isfinite(mids)], rnd, np.array([np.nan, np.inf, -np.inf], np.float32)):
        want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        got = ref.f32_to_bf16_bits(x)
        nan = np.isnan(x)
        assert np.array_equal(got[~nan], want[~nan])
        assert np.isnan(ref.bf16_bits_to_f32(got[nan])).all()


def test_quant_per_tensor_matches_reference_golden():
    z = _golden()
    q, s = ref.quantize_per_tensor(z["xt"])
    assert np.array_equal(q, z["qt"]) and np.float32(s) == z["st"]
    q, s = ref.quantize_per_tensor(np.zeros((1, 2, 1, 128), np.float16))
    assert np.array_equal(q, z["qz"]) and np.float32(s) == z["sz"]


def test_dequantize_matches_reference_golden():
    z = _golden()
    kd, vd = ref.dequantize_kv(z["kc"], z["vc"], z["ks"], z["vs"])
    assert np.array_equal(kd, z["kd"]) and np.array_equal(vd, z["vd"])


def _fp16_rne(fr):
    """Exact rational -> nearest fp16 value (ties to even), as a Fraction."""
    if fr == 0:
        return Fraction(0)
    e = math.floor(math.log2(fr))
    while Fraction(2) ** e > fr:
        e -= 1
    while Fraction(2) ** (e + 1) <= fr:
        e += 1
    e = max(e, -14)                       # subnormal spacing below 2^-14
    ulp = Fraction(2) ** (e - 10)
    n = fr / ulp
    fl = math.floor(n)
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return fl * ulp


def _rne_int(fr):
    fl = math.floor(fr)
    rem = fr - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return fl


def _quant_rational(row16):
    """Per-token quant from exact rationals (independent of numpy's float ops)."""
    vals = [Fraction(float(v)) for v in row16]
    amax = max(abs(v) for v in vals)
    s = _fp16_rne(amax / 127)
    if s == 0:
        return [0 if v == 0 else (127 if v > 0 else -127) for v in vals], 0.0
    return [max(-127, min(127, _rne_int(v / s))) for v in vals], float(s)


def test_quant_matches_exact_rational_arithmetic():
    rng = np.random.default_rng(5)
    rows = [rng.standard_normal(64) * 10 ** rng.uniform(-4, 3) for _ in range(60)]
    rows += [np.array([127, 2.5, 3.5, -2.5, 0.5, -0.5, 1.5, 126.5] * 8),
             np.zeros(64), np.full(64, 1e-7)]
    x = np.stack(rows).astype(np.float16)
    q, s = ref.quantize_per_token(x, axis=-1)
    for i, row in enumerate(x):
        qe, se = _quant_rational(row)
        assert q[i].tolist() == qe, i
        assert float(s[i]) == se, i


def test_quant_round_half_even_and_saturation():
    x = np.zeros((1, 16), np.float16)
    x[0, :9] = [127, 2.5, 3.5, -2.5, 0.5, -0.5, 1.5, 126.5, -126.5]
    q, s = ref.quantize_per_token(x)
    assert float(s[0]) == 1.0
    assert q[0, :9].tolist() == [127, 2, 4, -2, 0, 0, 2, 126, -126]
    y = np.random.default_rng(0).standard_normal((2, 64)).astype(np.float32)
    y[0, 0] = 1000.0
    q, s = ref.quantize_per_token(y)
    assert q[0, 0] == 127 and np.abs(q).max() <= 127 and s[0] > s[1]


# tests/test_quant.py:17-105 restated against the oracle
def test_per_token_scale_formula_and_range():
    x = np.random.default_rng(0).standard_normal((4, 7, 128)).astype(np.float32)
    q, s = ref.quantize_per_token(x)
    np.testing.assert_allclose(s, np.maximum(np.abs(x).max(-1), 1e-8) / 127.0, rtol=1e-6)
    assert s.shape == (4, 7) and q.dtype == np.int8 and np.abs(q.astype(int)).max() <= 127


def test_per_token_roundtrip_bound():
    x = np.random.default_rng(0).standard_normal((8, 256)).astype(np.float32)
    q, s = ref.quantize_per_token(x)
    dq = q.astype(np.float32) * s[:, None]
    assert np.linalg.norm(dq - x) / np.linalg.norm(x) < 0.02


def test_int8_builder_dequant_roundtrip():
    rng = np.random.default_rng(0)
    lens = np.array([40, 33], np.int32)
    k = rng.standard_normal((2, 40, 2, 128)).astype(np.float32)
    v = rng.standard_normal((2, 40, 2, 128)).astype(np.float32)
    kc, vc, ks, vs, bt = ref.build_paged_kv_cache_int8(k, v, lens)
    kd, vd = ref.dequantize_kv(kc, vc, ks, vs)
    for s in range(2):
        kk, vv = ref.gather_kv(kd, vd, bt, int(lens[s]), s, 16)
        tol_k = np.abs(k[s, :lens[s]]).max(-1, keepdims=True) / 127 / 2 + 1e-6
        tol_v = np.abs(v[s, :lens[s]]).max(-1, keepdims=True) / 127 / 2 + 1e-6
        assert (np.abs(kk - k[s, :lens[s]]) <= tol_k).all()
        assert (np.abs(vv - v[s, :lens[s]]) <= tol_v).all()


def test_fp16_builder_gather_roundtrip_and_layout():
    c = fp16_case(3, make_lens(70, 3), 8, 2)
    for s, n in enumerate(c["lens"]):
        kk, vv = ref.gather_kv(c["k_cache"], c["v_cache"], c["block_table"], int(n), s, 16)
        assert np.array_equal(kk, c["k"][s, :n]) and np.array_equal(vv, c["v"][s, :n])
    # one element by the explicit layout formula of tests/paged_decode_attn.py:94-97
    s, t, h, dd = 1, 37, 1, 93
    blk = c["block_table"][s, t // 16]
    assert c["k_cache"][blk, h, dd // 8, t % 16, dd % 8] == c["k"][s, t, h, dd]
    assert c["v_cache"][blk, h, dd, t % 16] == c["v"][s, t, h, dd]
    # pool size and spare block (paged_decode_attn.py:73)
    assert c["k_cache"].shape[0] == sum((int(n) + 15) // 16 for n in c["lens"]) + 1


def test_reshape_and_cache_matches_builder_placement():
    """Writing token by token through slots equals the int8 builder's layout."""
    rng = np.random.default_rng(4)
    lens = np.array([50, 17, 33], np.int32)
    k = rng.standard_normal((3, 50, 2, 64)).astype(np.float16)
    v = rng.standard_normal((3, 50, 2, 64)).astype(np.float16)
    kc, vc, ks, vs, bt = ref.build_paged_kv_cache_int8(k, v, lens, rng=np.random.default_rng(1))
    ekc, evc = np.zeros_like(kc), np.zeros_like(vc)
    eks, evs = np.zeros_like(ks), np.zeros_like(vs)
    seq = np.repeat(np.arange(3), lens)
    tok = np.concatenate([np.arange(n) for n in lens])
    slots = bt[seq, tok // 16].astype(np.int64) * 16 + tok % 16
    ref.reshape_and_cache_int8(k[seq, tok], v[seq, tok], slots, ekc, evc, eks, evs)
    assert np.array_equal(ekc, kc) and np.array_equal(evc, vc)
    assert np.array_equal(eks, ks) and np.array_equal(evs, vs)
    # negative / out-of-pool slots write nothing
    before = ekc.copy()
    ref.reshape_and_cache_int8(k[:1, 0], v[:1, 0], np.array([-1]), ekc, evc, eks, evs)
    ref.reshape_and_cache_int8(k[:1, 0], v[:1, 0], np.array([ekc.shape[0] * 16]), ekc, evc, eks,
                               evs)
    assert np.array_equal(before, ekc)


# ------------------------------------------- PagedKVCache write modes (oracle)

def _float_rne(fr, mant_bits, emin):
    """Exact rational -> nearest binary float with `mant_bits` fraction bits and
    minimum normal exponent `emin` (ties to even), as a Fraction; no overflow."""
    if fr == 0:
        return Fraction(0)
    sign = 1 if fr > 0 else -1
    a = abs(fr)
    e = math.floor(math.log2(a))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = Fraction(2) ** (max(e, emin) - mant_bits)
    return sign * _rne_int(a / ulp) * ulp


def test_paged_cache_tensor_scale_closed_form():
    """(amax / 127) rounded in the input dtype, then widened, then clamped at
    1e-8 (paged_cache.py:101-102), from exact rationals."""
    amaxes = [0.0, 6e-8, 1e-6, 1.2e-5, 6.1e-5, 0.0077, 0.5, 1.0, 3.14159, 127.0, 1000.0, 65504.0]
    for a in amaxes:
        x = np.array([a, -a / 2, 0.0], np.float16)
        a16 = Fraction(float(np.float16(a)))
        s = _float_rne(a16 / 127, 10, -14)                 # fp16 division
        want = max(float(s), float(np.float32(1e-8)))
        got = ref.paged_cache_tensor_scale(x)
        assert got.dtype == np.float32 and float(got) == float(np.float32(want)), a
        y = np.array([a, -a / 3], np.float32)             # fp32 input: one fp32 rounding
        s32 = _float_rne(Fraction(float(np.float32(a))) / 127, 23, -126)
        want32 = max(float(s32), float(np.float32(1e-8)))
        assert float(ref.paged_cache_tensor_scale(y)) == float(np.float32(want32)), a
    # the clamp order differs from quantize_per_tensor at amax = 0
    z = np.zeros(8, np.float16)
    assert float(ref.paged_cache_tensor_scale(z)) == float(np.float32(1e-8))
    assert float(ref.quantize_per_tensor(z)[1]) == 0.0


def test_static_quant_matches_exact_rational_arithmetic():
    """q = clamp(rne(fp32(x / s)), -127, 127) from exact rationals, including
    saturation far beyond the scale, NaN -> 0 and inf -> +-127."""
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(512) * 40).astype(np.float16)
    x[:6] = [np.inf, -np.inf, np.nan, 0.0, 65504.0, -65504.0]
    for s in (np.float32(1e-8), np.float32(0.0078125), np.float32(0.3), np.float32(2.7e-3)):
        q = ref._quantize_with_scale(x, s)
        for xi, qi in zip(x, q):
            if np.isnan(xi):
                want = 0
            elif np.isinf(xi):
                want = 127 if xi > 0 else -127
            else:
                quo = _float_rne(Fraction(float(xi)) / Fraction(float(s)), 23, -126)
                want = max(-127, min(127, _rne_int(quo)))
            assert int(qi) == want, (float(xi), float(s))


def test_static_write_matches_per_tensor_builder():
    """Writing with quantize_per_tensor's scales through slots equals the
    per-tensor int8 builder (tests/paged_decode_attn.py:167-172,190-197)."""
    rng = np.random.default_rng(6)
    lens = np.array([40, 23], np.int32)
    k = rng.standard_normal((2, 40, 2, 128)).astype(np.float16)
    v = (rng.standard_normal((2, 40, 2, 128)) * 3).astype(np.float16)
    kc, vc, ks, vs, bt = ref.build_paged_kv_cache_int8(k, v, lens, mode="per_tensor",
                                                       rng=np.random.default_rng(2))
    _, sk = ref.quantize_per_tensor(k)
    _, sv = ref.quantize_per_tensor(v)
    ekc, evc = np.zeros_like(kc), np.zeros_like(vc)
    eks, evs = np.zeros_like(ks), np.zeros_like(vs)
    seq = np.repeat(np.arange(2), lens)
    tok = np.concatenate([np.arange(n) for n in lens])
    slots = bt[seq, tok // 16].astype(np.int64) * 16 + tok % 16
    ref.reshape_and_cache_int8_static(k[seq, tok], v[seq, tok], slots, ekc, evc, eks, evs, sk, sv)
    assert np.array_equal(ekc, kc) and np.array_equal(evc, vc)
    assert np.array_equal(eks, ks) and np.array_equal(evs, vs)


def test_f16_write_matches_builder_placement():
    c = fp16_case(3, make_lens(45, 3), 8, 2, seed=8)
    kc = np.zeros_like(c["k_cache"])
    vc = np.zeros_like(c["v_cache"])
    lens, bt = c["lens"], c["block_table"]
    seq = np.repeat(np.arange(3), lens)
    tok = np.concatenate([np.arange(n) for n in lens])
    slots = bt[seq, tok // 16].astype(np.int64) * 16 + tok % 16
    ref.reshape_and_cache_f16(c["k"][seq, tok], c["v"][seq, tok], slots, kc, vc)
    assert np.array_equal(kc, c["k_cache"]) and np.array_equal(vc, c["v_cache"])

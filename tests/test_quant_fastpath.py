"""CPU check of the arithmetic the quantize kernel uses (no GPU needed).

The kernel (cuda-pa-int8_amd/csrc/pa_quant.hip) computes the per-token scale
as fp16(fl(a * fl(1/127))) and q = rne(x / s) through y = x * r, where r is
the hardware reciprocal of s (within 1 ulp of 1/s), and falls back to the
IEEE division when y lies within 4e-5 of a half-integer.  The reference
computes fp16(a / 127) and rne(fp32(x) / scale) with IEEE divisions
(tests/paged_decode_attn.py:106-112).  This test checks the scale form for
every fp16 value, and replays the fast path in numpy float32 arithmetic for
every finite fp16 x against many scales and every reciprocal within 1 ulp of
1/s, asserting that whenever the fast path is taken its integer equals the
reference's.  Both product forms the compiler may emit are covered: the
rounded product fl(x * r), and the exact product x * r (FMA-contracted).
"""

import numpy as np

GUARD = np.float32(4.0e-5)
HALF = np.float32(0.5) - GUARD
LIMIT = np.float32(127.5) - GUARD


def _all_fp16():
    x = np.arange(1 << 16, dtype=np.uint16).view(np.float16)
    return x[np.isfinite(x)].astype(np.float32)


def _scales(rng):
    # s = fp32(fp16(a / 127)) for amax values spread over the fp16 range, plus
    # subnormal fp16 scales and the scale 1 (exact ties).
    amax = np.concatenate([
        rng.uniform(1e-3, 60000.0, 120).astype(np.float16),
        (2.0 ** rng.uniform(-14, 15, 40)).astype(np.float16),
        np.array([127.0, 1.0, 6e-8, 1e-5, 65504.0], np.float16),
    ]).astype(np.float32)
    s = (np.maximum(amax, np.float32(1e-8)) / np.float32(127)).astype(np.float16).astype(np.float32)
    return np.unique(s[s > 0])


def test_fast_path_matches_ieee_quotient():
    rng = np.random.default_rng(0)
    xs = _all_fp16()
    taken = 0
    for s in _scales(rng):
        s = np.float32(s)
        amax = np.float32(127) * s * np.float32(1.01)        # inputs the row can hold
        x = xs[np.abs(xs) <= amax]
        want = np.rint(x / s)                                 # float32 IEEE quotient, RNE
        r0 = np.float32(1) / s
        for r in (r0, np.nextafter(r0, np.float32(np.inf)), np.nextafter(r0, np.float32(0))):
            y = (x * r).astype(np.float32)                    # rounded product
            y_exact = x.astype(np.float64) * np.float64(r)    # FMA-contracted product
            for yy in (y, y_exact):
                q = np.rint(yy)
                ok = (np.abs(yy - q) < HALF) & (np.abs(yy) < LIMIT)
                # the kernel takes the fast byte from the rounded product: it must
                # agree with the reference wherever either form passes the test
                for fast in (np.rint(y), np.rint(y_exact)):
                    bad = ok & (fast != want)
                    assert not bad.any(), (float(s), x[bad][:4], fast[bad][:4], want[bad][:4])
                taken += int(ok.sum())
    assert taken > 1_000_000


def test_scale_by_multiplication_equals_division():
    """fp16(fl(a * fl(1/127))) == fp16(fl(a / 127)) for every fp16 a >= 0 and the
    clamp value 1e-8 (the kernel's form against the reference's)."""
    a = np.arange(1 << 15, dtype=np.uint16).view(np.float16).astype(np.float32)   # +0 .. +inf, NaN
    a = np.concatenate([a[np.isfinite(a)], np.array([1e-8], np.float32)])
    inv = np.float32(1) / np.float32(127)
    by_mul = (a * inv).astype(np.float32).astype(np.float16)
    by_div = (a / np.float32(127)).astype(np.float32).astype(np.float16)
    assert np.array_equal(by_mul.view(np.uint16), by_div.view(np.uint16))


def test_group_max_equals_per_element_test():
    """The kernel tests the largest |y - rint(y)| of a group once; on finite
    values that is the per-element test taken over the group."""
    rng = np.random.default_rng(2)
    y = (rng.uniform(-127, 127, (4096, 8))).astype(np.float32)
    y[::7, 3] = np.float32(5.5) + rng.uniform(-1e-5, 1e-5, y[::7, 3].shape).astype(np.float32)
    d = np.abs(y - np.rint(y))
    per_elem = (d < HALF).all(axis=1)
    grouped = d.max(axis=1) < HALF
    assert np.array_equal(per_elem, grouped) and (~grouped).any()


def test_guard_is_needed():
    # A planted mistake: without the guard the rounded product disagrees with
    # the IEEE quotient for some fp16 inputs, so the fallback is not dead code.
    rng = np.random.default_rng(1)
    xs = _all_fp16()
    mismatches = 0
    for s in _scales(rng):
        s = np.float32(s)
        x = xs[np.abs(xs) <= np.float32(127) * s]
        r = np.float32(1) / s
        y = (x * r).astype(np.float32)
        mismatches += int((np.rint(y) != np.rint(x / s)).sum())
    assert mismatches > 0

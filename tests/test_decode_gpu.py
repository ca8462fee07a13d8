"""GPU parity tests of the decode kernels against the CPU oracle.

Mirrors the reference's matrix (tests/test_paged_decode_attn.py:80-464):
every variant over CONTEXT_LENS x GQA x NUM_SEQS, long contexts across split
boundaries, INT8 against the dequantized-cache oracle, finiteness, ctx=0
rejection and the precision / outlier checks.  Tolerance is the build
target's atol 2e-3 / rtol 1e-2 on fp16 outputs (the reference tests use
2e-2).  Extra cases: forced small partitions (multi-split merges of both the
single-launch and the split-K path), head_dim 64/256, every block size,
group sizes 1..32, masked/invalid inputs on the no-check entry, a direct
C-ABI call and HIP-graph replay.
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from _cases import (ATOL, CONTEXT_LENS, GQA, HEAD_DIMS, LONG_CONTEXT_LENS, NUM_SEQS, RTOL,
                    assert_close, fp16_case, int8_case, make_lens, oracle_fp16, oracle_int8,
                    record_headroom)

pytestmark = pytest.mark.gpu

DEV = "cuda"
F16_VARIANTS = ["warp", "splitk"]
I8_VARIANTS = ["warp_int8", "splitk_int8"]


@pytest.fixture(scope="module", autouse=True)
def _lib(built):
    import pa_int8

    pa_int8.ext()
    return pa_int8


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def run_fp16(c, variant, check=True, partition=0, lens=None):
    import pa_int8

    q = _t(c["q"])
    out = torch.empty_like(q)
    pa_int8.decode(variant, out, q, _t(c["k_cache"]), _t(c["v_cache"]), _t(c["block_table"]),
                   _t(c["lens"] if lens is None else lens), c["scale"], c["block_size"],
                   check=check, partition_tokens=partition)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def run_int8(c, variant, check=True, partition=0):
    import pa_int8

    q = _t(c["q"])
    out = torch.empty_like(q)
    pa_int8.decode(variant, out, q, _t(c["k_cache8"]), _t(c["v_cache8"]), _t(c["block_table8"]),
                   _t(c["lens"]), c["scale"], c["block_size"], k_scales=_t(c["k_scales"]),
                   v_scales=_t(c["v_scales"]), check=check, partition_tokens=partition)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


# ---------------------------------------------------------------- FP16 matrix

@pytest.mark.parametrize("name", ["naive", "vec", "online", "warp", "splitk"])
@pytest.mark.parametrize("clen", CONTEXT_LENS)
@pytest.mark.parametrize("num_heads,num_kv_heads", GQA)
def test_registry_variant_matches_oracle(name, clen, num_heads, num_kv_heads):
    """Every name of the reference registry (tests/cuda_ext.py:112-125), called
    with its own signature, as tests/test_paged_decode_attn.py:80-119 does."""
    import pa_int8

    c = fp16_case(3, make_lens(clen, 3), num_heads, num_kv_heads, seed=21)
    q = _t(c["q"])
    out = torch.empty_like(q)
    ret = pa_int8.VARIANTS[name](out, q, _t(c["k_cache"]), _t(c["v_cache"]),
                                 _t(c["block_table"]), _t(c["lens"]), c["scale"],
                                 c["block_size"])
    assert ret is out
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), oracle_fp16(c), what=name)


def test_registry_block_size_rules():
    """vec accepts any multiple of 8 the library builds (paged_attention_v1_vectorized.cu:124);
    online / warp / splitk also require it to divide the 128-token tile
    (v2_online.cu:157); sizes outside the library's set raise RuntimeError."""
    import pa_int8

    c = fp16_case(2, make_lens(100, 2), 8, 2, block_size=8, seed=4)
    args = lambda: (torch.empty_like(_t(c["q"])), _t(c["q"]), _t(c["k_cache"]),  # noqa: E731
                    _t(c["v_cache"]), _t(c["block_table"]), _t(c["lens"]), c["scale"])
    for name in ("naive", "vec", "online", "warp", "splitk"):
        out = pa_int8.VARIANTS[name](*args(), 8)
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), oracle_fp16(c), what=name)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        pa_int8.VARIANTS["vec"](*args(), 12)
    with pytest.raises(RuntimeError, match="divide TILE"):
        pa_int8.VARIANTS["online"](*args(), 24)
    with pytest.raises(RuntimeError):
        pa_int8.VARIANTS["naive"](*args(), 12)


@pytest.mark.parametrize("variant", F16_VARIANTS)
@pytest.mark.parametrize("clen", CONTEXT_LENS)
@pytest.mark.parametrize("num_heads,num_kv_heads", GQA)
@pytest.mark.parametrize("num_seqs", NUM_SEQS)
def test_fp16_matches_oracle(variant, clen, num_heads, num_kv_heads, num_seqs):
    c = fp16_case(num_seqs, make_lens(clen, num_seqs), num_heads, num_kv_heads)
    assert_close(run_fp16(c, variant), oracle_fp16(c), what=variant)


@pytest.mark.parametrize("variant", F16_VARIANTS)
@pytest.mark.parametrize("clen", LONG_CONTEXT_LENS)
@pytest.mark.parametrize("num_heads,num_kv_heads", [(8, 8), (8, 2)])
def test_fp16_long(variant, clen, num_heads, num_kv_heads):
    c = fp16_case(2, make_lens(clen, 2), num_heads, num_kv_heads)
    assert_close(run_fp16(c, variant), oracle_fp16(c), what=variant)


@pytest.mark.parametrize("variant", F16_VARIANTS)
@pytest.mark.parametrize("partition", [64, 128, 320])
@pytest.mark.parametrize("clen", [65, 300, 1000, 2049])
def test_fp16_forced_partition(variant, partition, clen):
    """Many splits per sequence: exercises the LSE merge of both paths."""
    c = fp16_case(3, make_lens(clen, 3), 12, 2, seed=3)
    assert_close(run_fp16(c, variant, partition=partition), oracle_fp16(c), what=variant)


@pytest.mark.parametrize("variant", F16_VARIANTS)
@pytest.mark.parametrize("head_dim", HEAD_DIMS)
@pytest.mark.parametrize("clen", [17, 700])
@pytest.mark.parametrize("num_heads,num_kv_heads", [(8, 2), (32, 1)])
def test_fp16_head_dims(variant, head_dim, clen, num_heads, num_kv_heads):
    c = fp16_case(2, make_lens(clen, 2), num_heads, num_kv_heads, head_dim=head_dim, seed=5)
    assert_close(run_fp16(c, variant), oracle_fp16(c), what=f"{variant} D={head_dim}")


@pytest.mark.parametrize("variant", F16_VARIANTS)
@pytest.mark.parametrize("head_dim", [24, 40, 72, 80, 96, 112, 136, 200])
def test_fp16_head_dims_forced_splits(variant, head_dim):
    """Head dims that are not a multiple of 32 (masked last QK chunk of 8,
    16 or 24 dims; with head_dim % 16 == 8 also a half last output tile)
    across many splits, both work distributions."""
    import pa_int8

    lib = pa_int8.capi()
    c = fp16_case(3, make_lens(2100, 3), 12, 2, head_dim=head_dim, seed=6)
    want = oracle_fp16(c)
    try:
        for mode in (1, 2):
            assert lib.pa_decode_set_schedule(mode) == 0
            assert_close(run_fp16(c, variant, partition=256), want,
                         what=f"{variant} D={head_dim} schedule={mode}")
    finally:
        lib.pa_decode_set_schedule(0)


@pytest.mark.parametrize("variant", F16_VARIANTS)
@pytest.mark.parametrize("block_size", [8, 32, 64, 128])
def test_fp16_block_sizes(variant, block_size):
    c = fp16_case(3, make_lens(333, 3), 8, 2, block_size=block_size, seed=7)
    assert_close(run_fp16(c, variant), oracle_fp16(c), what=f"{variant} bs={block_size}")


@pytest.mark.parametrize("variant", F16_VARIANTS)
@pytest.mark.parametrize("num_heads,num_kv_heads", [(3, 1), (12, 2), (24, 2), (32, 1), (14, 2),
                                                    (10, 2), (32, 8)])
def test_fp16_group_sizes(variant, num_heads, num_kv_heads):
    c = fp16_case(2, make_lens(250, 2), num_heads, num_kv_heads, seed=11)
    assert_close(run_fp16(c, variant), oracle_fp16(c), what=f"{variant} {num_heads}/{num_kv_heads}")


@pytest.mark.parametrize("variant", F16_VARIANTS + I8_VARIANTS)
@pytest.mark.parametrize("num_heads,num_kv_heads", [(32, 1), (17, 1), (40, 2), (24, 1),
                                                    (64, 1), (96, 2)])
@pytest.mark.parametrize("mode", [1, 2, 3])
def test_two_column_tiles(variant, num_heads, num_kv_heads, mode):
    """Group sizes of 17..32 query heads run in one work-group per kv head with
    two MFMA column tiles (64/1 and 96/2: two such chunks of 32 and 48 = 24+24);
    ragged lengths, grid (mode 1), in-kernel schedule (mode 2; 16-head tiles)
    and stream partition (mode 3), default and
    forced short partitions (many-split merges)."""
    import pa_int8

    lib = pa_int8.capi()
    lens = np.array([1, 333, 2100, 17], np.int32)
    int8 = variant.endswith("int8")
    c = (int8_case if int8 else fp16_case)(4, lens, num_heads, num_kv_heads, seed=num_heads)
    want = oracle_int8(c) if int8 else oracle_fp16(c)
    run = run_int8 if int8 else run_fp16
    try:
        assert lib.pa_decode_set_schedule(mode) == 0
        for part in (0, 128):
            assert_close(run(c, variant, partition=part), want,
                         what=f"{variant} {num_heads}/{num_kv_heads} mode {mode} P={part}")
    finally:
        lib.pa_decode_set_schedule(0)


@pytest.mark.parametrize("head_dim", [64, 80, 96, 112, 256])
@pytest.mark.parametrize("variant", ["warp", "splitk_int8"])
def test_two_column_tiles_head_dims(head_dim, variant):
    """MQA 32/1 at every head_dim: two column tiles up to 128, two 16-head
    chunks at 256."""
    int8 = variant.endswith("int8")
    c = (int8_case if int8 else fp16_case)(3, make_lens(900, 3), 32, 1, head_dim=head_dim,
                                           seed=head_dim)
    got = run_int8(c, variant) if int8 else run_fp16(c, variant)
    assert_close(got, oracle_int8(c) if int8 else oracle_fp16(c),
                 what=f"{variant} 32/1 D={head_dim}")


def test_fp16_qwen_config_full_size():
    """BASELINE config 2 at its real size: 32 seqs x 4096, 12/2 heads, D=128."""
    c = fp16_case(32, np.full(32, 4096, dtype=np.int32), 12, 2, seed=2)
    ref = oracle_fp16(c)
    for variant in F16_VARIANTS:
        ratio = assert_close(run_fp16(c, variant), ref, what=variant)
        record_headroom("cfg2", f"{variant} 32 x 4096 12/2, all sequences", ratio,
                        variant=variant, seqs_checked=32)


@pytest.mark.parametrize("variant", F16_VARIANTS)
@pytest.mark.parametrize("clen", [1, 17, 4096])
def test_outputs_finite(variant, clen):
    c = fp16_case(2, make_lens(clen, 2), 8, 2)
    assert np.isfinite(run_fp16(c, variant)).all()


@pytest.mark.parametrize("variant", F16_VARIANTS)
def test_empty_context_rejected(variant):
    """ctx=0 must raise RuntimeError (tests/test_paged_decode_attn.py:337-361)."""
    import pa_int8

    c = fp16_case(2, np.array([8, 1], dtype=np.int32), 8, 2)
    q = _t(c["q"])
    out = torch.empty_like(q)
    with pytest.raises(RuntimeError):
        pa_int8.VARIANTS[variant](out, q, _t(c["k_cache"]), _t(c["v_cache"]),
                                  _t(c["block_table"]), _t(np.array([8, 0], np.int32)),
                                  c["scale"], 16)


@pytest.mark.parametrize("variant", F16_VARIANTS)
def test_nocheck_zero_and_clamped_context(variant):
    """No-check entry: ctx<=0 gives zeros; ctx beyond the table is clamped."""
    c = fp16_case(3, np.array([40, 20, 33], dtype=np.int32), 8, 2, seed=4)
    lens = np.array([0, 20, 10_000], dtype=np.int32)
    got = run_fp16(c, variant, check=False, lens=lens)
    assert np.all(got[0] == 0)
    cap = c["block_table"].shape[1] * c["block_size"]
    c2 = dict(c, lens=np.array([1, 20, cap], dtype=np.int32))
    want = oracle_fp16(c2)
    assert_close(got[1:], want[1:], what="clamped")


@pytest.mark.parametrize("variant", F16_VARIANTS)
def test_invalid_block_ids_are_skipped(variant):
    c = fp16_case(2, np.array([64, 64], dtype=np.int32), 8, 2, seed=8)
    bt = c["block_table"].copy()
    bt[0, 1] = 10_000_000   # block 1 of seq 0 -> outside the pool
    bt[1, 3] = -5
    c2 = dict(c, block_table=bt)
    got = run_fp16(c2, variant, check=False)
    # oracle: drop those 16-token blocks
    keep0 = [0, 2, 3]
    keep1 = [0, 1, 2]
    from oracle import paged_decode_ref as ref
    for s, keep in ((0, keep0), (1, keep1)):
        sub = dict(c, q=c["q"][s:s + 1], block_table=c["block_table"][s:s + 1, keep],
                   lens=np.array([16 * len(keep)], dtype=np.int32))
        assert_close(got[s:s + 1], oracle_fp16(sub), what=f"seq {s}")


def test_warp_equals_splitk_randomized():
    """Two different merge paths must agree on ragged batches."""
    rng = np.random.default_rng(123)
    lens = rng.integers(1, 3000, size=7).astype(np.int32)
    c = fp16_case(7, lens, 24, 4, seed=9)
    a = run_fp16(c, "warp")
    b = run_fp16(c, "splitk")
    assert_close(a, b, what="warp vs splitk")
    assert_close(a, oracle_fp16(c), what="warp vs oracle")


# ---------------------------------------------------------------- INT8 matrix

@pytest.mark.parametrize("variant", I8_VARIANTS)
@pytest.mark.parametrize("mode", ["per_token", "per_tensor"])
@pytest.mark.parametrize("clen", CONTEXT_LENS)
@pytest.mark.parametrize("num_heads,num_kv_heads", GQA)
@pytest.mark.parametrize("num_seqs", NUM_SEQS)
def test_int8_matches_dequant_oracle(variant, mode, clen, num_heads, num_kv_heads, num_seqs):
    c = int8_case(num_seqs, make_lens(clen, num_seqs), num_heads, num_kv_heads, mode=mode)
    assert_close(run_int8(c, variant), oracle_int8(c), what=variant)


@pytest.mark.parametrize("variant", I8_VARIANTS)
@pytest.mark.parametrize("mode", ["per_token", "per_tensor"])
@pytest.mark.parametrize("clen", LONG_CONTEXT_LENS)
@pytest.mark.parametrize("num_heads,num_kv_heads", [(8, 8), (8, 2)])
def test_int8_long(variant, mode, clen, num_heads, num_kv_heads):
    c = int8_case(2, make_lens(clen, 2), num_heads, num_kv_heads, mode=mode)
    assert_close(run_int8(c, variant), oracle_int8(c), what=variant)


@pytest.mark.parametrize("variant", I8_VARIANTS)
@pytest.mark.parametrize("partition", [64, 192])
@pytest.mark.parametrize("clen", [300, 2049])
def test_int8_forced_partition(variant, partition, clen):
    c = int8_case(3, make_lens(clen, 3), 12, 2, seed=13)
    assert_close(run_int8(c, variant, partition=partition), oracle_int8(c), what=variant)


@pytest.mark.parametrize("variant", I8_VARIANTS)
@pytest.mark.parametrize("head_dim", HEAD_DIMS)
@pytest.mark.parametrize("num_heads,num_kv_heads", [(8, 2), (32, 1)])
def test_int8_head_dims(variant, head_dim, num_heads, num_kv_heads):
    c = int8_case(2, make_lens(600, 2), num_heads, num_kv_heads, head_dim=head_dim, seed=17)
    assert_close(run_int8(c, variant), oracle_int8(c), what=f"{variant} D={head_dim}")
    assert_close(run_int8(c, variant, partition=128), oracle_int8(c),
                 what=f"{variant} D={head_dim} P=128")


@pytest.mark.parametrize("variant", I8_VARIANTS)
@pytest.mark.parametrize("block_size", [32, 64, 128])
def test_int8_block_sizes(variant, block_size):
    c = int8_case(3, make_lens(333, 3), 8, 2, block_size=block_size, seed=19)
    assert_close(run_int8(c, variant), oracle_int8(c), what=f"{variant} bs={block_size}")


@pytest.mark.parametrize("variant", I8_VARIANTS)
@pytest.mark.parametrize("num_heads,num_kv_heads", [(12, 2), (32, 1), (32, 8), (6, 2)])
def test_int8_group_sizes(variant, num_heads, num_kv_heads):
    c = int8_case(2, make_lens(400, 2), num_heads, num_kv_heads, seed=23)
    assert_close(run_int8(c, variant), oracle_int8(c), what=f"{variant} {num_heads}/{num_kv_heads}")


@pytest.mark.parametrize("variant", I8_VARIANTS)
def test_int8_large_and_tiny_scales(variant):
    """V scales spanning many binades (per-iteration fp16 weight exponent)."""
    c = int8_case(2, make_lens(700, 2), 8, 2, seed=29)
    rng = np.random.default_rng(5)
    mul = np.exp2(rng.integers(-20, 9, size=c["v_scales"].shape)).astype(np.float32)
    c["v_scales"] = (c["v_scales"] * mul).astype(np.float32)
    c["k_scales"] = (c["k_scales"] * np.float32(3.0)).astype(np.float32)
    want = oracle_int8(c)
    atol = ATOL * float(np.abs(want).max() + 1)
    assert_close(run_int8(c, variant), want, atol=atol, what=variant)


@pytest.mark.parametrize("variant", I8_VARIANTS)
@pytest.mark.parametrize("clen", [1, 17, 4096])
def test_int8_outputs_finite(variant, clen):
    c = int8_case(2, make_lens(clen, 2), 8, 2)
    assert np.isfinite(run_int8(c, variant)).all()


@pytest.mark.parametrize("variant", I8_VARIANTS)
def test_int8_empty_context_rejected(variant):
    import pa_int8

    c = int8_case(2, np.array([8, 1], dtype=np.int32), 8, 2)
    q = _t(c["q"])
    out = torch.empty_like(q)
    with pytest.raises(RuntimeError):
        pa_int8.VARIANTS_INT8[variant](out, q, _t(c["k_cache8"]), _t(c["v_cache8"]),
                                       _t(c["k_scales"]), _t(c["v_scales"]),
                                       _t(c["block_table8"]), _t(np.array([8, 0], np.int32)),
                                       c["scale"], 16)


def test_int8_unit_scales_match_fp16():
    """All scales 1 and small-integer K/V: the INT8 path equals the FP16 path."""
    rng = np.random.default_rng(31)
    lens = np.array([500, 260], dtype=np.int32)
    c = fp16_case(2, lens, 8, 2, seed=31)
    ki = rng.integers(-3, 4, size=c["k_cache"].shape).astype(np.int8)
    vi = rng.integers(-100, 101, size=c["v_cache"].shape).astype(np.int8)
    c["k_cache"] = ki.astype(np.float16)
    c["v_cache"] = vi.astype(np.float16)
    c8 = dict(c, k_cache8=ki, v_cache8=vi, block_table8=c["block_table"],
              k_scales=np.ones(ki.shape[:2] + (16,), np.float32),
              v_scales=np.ones(ki.shape[:2] + (16,), np.float32))
    for v16, v8 in (("warp", "warp_int8"), ("splitk", "splitk_int8")):
        a = run_fp16(c, v16)
        b = run_int8(c8, v8)
        assert_close(b, a, atol=ATOL * 50, rtol=RTOL, what=v8)


def _rel_err(out, ref_):
    d = np.abs(out - ref_)
    return (d / np.maximum(np.abs(ref_), 1e-3)).mean()


@pytest.mark.parametrize("variant", I8_VARIANTS)
@pytest.mark.parametrize("clen", [128, 500])
@pytest.mark.parametrize("num_heads,num_kv_heads", [(8, 8), (8, 2)])
def test_int8_precision_metric(variant, clen, num_heads, num_kv_heads):
    """Per-token quant error vs FP16 (tests/test_paged_decode_attn.py:256-306)."""
    lens = make_lens(clen, 2)
    pt = int8_case(2, lens, num_heads, num_kv_heads, mode="per_token")
    ptn = int8_case(2, lens, num_heads, num_kv_heads, mode="per_tensor")
    fp = run_fp16(pt, "warp")
    e_pt = _rel_err(run_int8(pt, variant), fp)
    e_ptn = _rel_err(run_int8(ptn, variant), fp)
    assert e_pt < 0.2
    assert e_pt <= e_ptn + 1e-3


@pytest.mark.parametrize("variant", I8_VARIANTS)
def test_int8_precision_outlier_distribution(variant):
    """Outlier K channels {3, 50, 97} x20 (tests/test_paged_decode_attn.py:419-464)."""
    mul = np.ones(128, dtype=np.float32)
    mul[[3, 50, 97]] = 20.0
    lens = make_lens(500, 2)
    pt = int8_case(2, lens, 8, 2, mode="per_token", k_mul=mul)
    ptn = int8_case(2, lens, 8, 2, mode="per_tensor", k_mul=mul)
    fp = run_fp16(pt, "warp").reshape(-1)

    def cos(a):
        a = a.reshape(-1)
        return float(a @ fp / (np.linalg.norm(a) * np.linalg.norm(fp) + 1e-12))

    c_pt = cos(run_int8(pt, variant))
    c_ptn = cos(run_int8(ptn, variant))
    assert c_pt > 0.99
    assert c_pt >= c_ptn - 1e-4


@pytest.mark.parametrize("variant", ["splitk", "splitk_int8"])
def test_long_context_element_outliers(variant):
    """Config 4's data at its context length: K/V ~ N(0,1) with a Bernoulli(0.01)
    mask x20, 32 768 tokens, Llama-3-8B heads 32/8, against the oracle."""
    from oracle import paged_decode_ref as ref

    rng = np.random.default_rng(44)
    s, ctx, h, hkv, d = 2, 32768, 32, 8, 128
    lens = np.array([ctx, ctx - 1000], dtype=np.int32)

    def draw(shape):
        x = rng.standard_normal(shape, dtype=np.float32)
        x[rng.random(shape) < 0.01] *= 20.0
        return x.astype(np.float16)

    q = rng.standard_normal((s, h, d), dtype=np.float32).astype(np.float16)
    k, v = draw((s, ctx, hkv, d)), draw((s, ctx, hkv, d))
    c = dict(q=q, lens=lens, scale=1.0 / math.sqrt(d), block_size=16)
    if variant == "splitk":
        kc, vc, bt = ref.build_paged_kv_cache(k, v, lens, block_size=16, x=8, rng=rng)
        c.update(k_cache=kc, v_cache=vc, block_table=bt)
        out, want = run_fp16(c, variant), oracle_fp16(c)
    else:
        kc, vc, ks, vs, bt = ref.build_paged_kv_cache_int8(k, v, lens, block_size=16, x=8,
                                                           rng=rng)
        c.update(k_cache8=kc, v_cache8=vc, k_scales=ks, v_scales=vs, block_table8=bt)
        out, want = run_int8(c, variant), oracle_int8(c)
    ratio = assert_close(out, want, what=f"{variant} 32k outliers")
    record_headroom("cfg4", f"{variant} 2 x 32768 32/8 outliers (numpy-drawn)", ratio,
                    variant=variant, seqs_checked=2)


# ---------------------------------------------------------------- boundary / runtime

def test_capi_direct_call():
    """The C ABI called through ctypes, counters and workspace owned by the caller;
    one counter buffer serves both kinds and stays zero after each call."""
    import pa_int8

    lib = pa_int8.capi()
    c = fp16_case(3, make_lens(900, 3), 12, 2, seed=37)
    q = _t(c["q"])
    out = torch.zeros_like(q)
    kc, vc, bt, ln = _t(c["k_cache"]), _t(c["v_cache"]), _t(c["block_table"]), _t(c["lens"])
    S, H, D = c["q"].shape
    NB, Hkv = c["k_cache"].shape[:2]
    MB = c["block_table"].shape[1]
    stream = torch.cuda.current_stream().cuda_stream
    cb = lib.pa_decode_counter_bytes(S, H, Hkv)
    counters = torch.full((cb,), 0x5A, dtype=torch.uint8, device=DEV)
    assert lib.pa_decode_counters_reset(counters.data_ptr(), cb, stream) == 0
    for fn, kind in ((lib.pa_paged_decode_attn_warp, 0), (lib.pa_paged_decode_attn_splitk, 1)):
        need = lib.pa_decode_workspace_bytes(kind, S, H, D, Hkv, 16, MB, 0, 64)
        # scratch with arbitrary contents
        ws = torch.full((need + 256,), 0xFF, dtype=torch.uint8, device=DEV)
        aligned = (ws.data_ptr() + 255) // 256 * 256
        out.zero_()
        st = fn(out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(),
                ln.data_ptr(), ctypes.c_float(c["scale"]), 16, S, H, D, Hkv, NB, 8, MB, 0, 64,
                counters.data_ptr(), cb, aligned, need, stream)
        assert st == 0, lib.pa_status_string(st)
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), oracle_fp16(c), what=f"capi kind {kind}")
        assert int(counters.count_nonzero()) == 0
        # too-small workspace / counters are refused before any launch
        st = fn(out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(),
                ln.data_ptr(), ctypes.c_float(c["scale"]), 16, S, H, D, Hkv, NB, 8, MB, 0, 64,
                counters.data_ptr(), cb, aligned, 16, stream)
        assert st == 5
        st = fn(out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(),
                ln.data_ptr(), ctypes.c_float(c["scale"]), 16, S, H, D, Hkv, NB, 8, MB, 0, 64,
                counters.data_ptr(), cb - 256, aligned, need, stream)
        assert st == 5


@pytest.mark.parametrize("variant", ["warp", "warp_int8", "splitk"])
def test_graph_replay_matches_eager(variant):
    """Capture the no-check entry in a HIP graph; every replay equals eager."""
    import pa_int8

    int8 = variant.endswith("int8")
    c = int8_case(4, make_lens(1500, 4), 12, 2, seed=41) if int8 else \
        fp16_case(4, make_lens(1500, 4), 12, 2, seed=41)
    q = _t(c["q"])
    kw = {}
    if int8:
        kc, vc, bt = _t(c["k_cache8"]), _t(c["v_cache8"]), _t(c["block_table8"])
        kw = dict(k_scales=_t(c["k_scales"]), v_scales=_t(c["v_scales"]))
    else:
        kc, vc, bt = _t(c["k_cache"]), _t(c["v_cache"]), _t(c["block_table"])
    ln = _t(c["lens"])
    out = torch.empty_like(q)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pa_int8.decode(variant, out, q, kc, vc, bt, ln, c["scale"], 16, check=False, **kw)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        pa_int8.decode(variant, out, q, kc, vc, bt, ln, c["scale"], 16, check=False, **kw)
    for _ in range(4):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("policy", [0, 1, 2])
def test_load_policies_agree(head_dim, policy):
    """Every cache-load hint gives the oracle's result: plain (1), non-temporal
    V (2; FP16 grid launches with splits of >= 1024 tokens then load K
    non-temporally too) and automatic (0), on the grid and the scheduled forms,
    with two splits of 4096 tokens per sequence."""
    import pa_int8

    lib = pa_int8.capi()
    lens = np.array([8192, 5000], np.int32)
    c = fp16_case(2, lens, 8, 2, head_dim=head_dim, seed=40 + policy)
    want = oracle_fp16(c)
    try:
        assert lib.pa_decode_set_load_policy(policy) == 0
        for mode in (0, 1):
            assert lib.pa_decode_set_schedule(mode) == 0
            for variant in F16_VARIANTS:
                assert_close(run_fp16(c, variant, partition=4096), want,
                             what=f"{variant} D={head_dim} policy={policy} schedule={mode}")
    finally:
        lib.pa_decode_set_load_policy(0)
        lib.pa_decode_set_schedule(0)

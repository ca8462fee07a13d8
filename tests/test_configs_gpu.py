"""Parity at the BASELINE configs' real sizes, on the benchmark's own inputs.

Each test builds the inputs exactly as bench.py does for that config
(``bench.make_case``: fp16 N(0,1) q/K/V drawn on the device, 1% outliers x20
for config 4, INT8 caches written by the quantize + write kernel from fp16
tokens, randomly permuted block tables), runs the launch the benchmark times
(the no-check entry), and compares a sample of sequences with the CPU oracle
(tests/paged_decode_attn.py:4-49 restated in oracle/paged_decode_ref.py); INT8
against the oracle on the dequantized cache (:202-216).  Tolerance: atol 2e-3
/ rtol 1e-2 on the fp16 outputs.  Every comparison also records its headroom
ratio max|err| / (atol + rtol |ref|) (to the file named by PA_PARITY_LOG).
"""

import numpy as np
import pytest
import torch

from _cases import assert_close, record_headroom, subset_oracle
from oracle import paged_decode_ref as ref

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _lib(built):
    import pa_int8

    pa_int8.ext()
    yield
    pa_int8.capi().pa_decode_set_schedule(0)


def _bench():
    import bench

    return bench


def make_case(lens, h, hkv, d=128, int8=False, outliers=False, seed=0):
    return _bench().make_case(torch, list(lens), h, hkv, d, 16, DEV, seed, int8, outliers, 1)


def run(case, variant, check=False):
    import pa_int8

    kc, vc, ks, vs = case["caches"][0]
    kw = {} if ks is None else dict(k_scales=ks, v_scales=vs)
    out = torch.empty_like(case["q"])
    pa_int8.decode(variant, out, case["q"], kc, vc, case["bt"], case["ctx"], case["scale"],
                   case["bs"], check=check, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def check(case, variant, seqs, config, what, **extra):
    got = run(case, variant)
    ratio = assert_close(got[list(seqs)], subset_oracle(case, seqs), what=f"{config} {what}")
    assert np.isfinite(got).all()
    record_headroom(config, what, ratio, variant=variant, seqs_checked=len(seqs), **extra)
    return got


# ------------------------------------------------------------------ config 1

def test_config1_exact_shape():
    """Config 1 as BASELINE states it: 4 sequences, 8 q = 8 kv heads, D=64,
    lengths uniform in [100, 512] (numpy seed 0, as bench.py), 128 physical
    blocks handed out by a random permutation, scale 1/8; every registry name,
    and both INT8 names on the cache quantized from it."""
    import pa_int8

    rng = np.random.default_rng(0)
    lens = rng.integers(100, 513, size=4).astype(np.int32)
    S, H, D, bs = 4, 8, 64, 16
    perm = rng.permutation(128).astype(np.int32)
    bt = perm.reshape(S, 32)                                  # 32 blocks = 512 tokens each
    kc = rng.standard_normal((128, H, D // 8, bs, 8), dtype=np.float32).astype(np.float16)
    vc = rng.standard_normal((128, H, D, bs), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((S, H, D), dtype=np.float32).astype(np.float16)
    want = ref.paged_decode_attention(q, kc, vc, bt, lens, scale=0.125, block_size=bs)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    worst = 0.0
    for name, fn in pa_int8.VARIANTS.items():
        out = torch.empty((S, H, D), dtype=torch.float16, device=DEV)
        fn(out, t(q), t(kc), t(vc), t(bt), t(lens), 0.125, bs)
        torch.cuda.synchronize()
        worst = max(worst, assert_close(out.float().cpu().numpy(), want, what=f"config 1 {name}"))
    record_headroom("cfg1", "fp16, all five registry names", worst)
    # INT8: quantize every token's K/V (per token) into the same slots, decode
    kq, ksc = ref.quantize_per_token(kc.transpose(0, 1, 3, 2, 4).reshape(128, H, bs, D), axis=-1)
    vq, vsc = ref.quantize_per_token(vc.transpose(0, 1, 3, 2), axis=-1)
    k8 = kq.reshape(128, H, bs, D // 8, 8).transpose(0, 1, 3, 2, 4)
    v8 = vq.transpose(0, 1, 3, 2)
    kd, vd = ref.dequantize_kv(k8, v8, ksc, vsc)
    want8 = ref.paged_decode_attention(q, kd, vd, bt, lens, scale=0.125, block_size=bs)
    worst = 0.0
    for name, fn in pa_int8.VARIANTS_INT8.items():
        out = torch.empty((S, H, D), dtype=torch.float16, device=DEV)
        fn(out, t(q), t(k8), t(v8), t(ksc), t(vsc), t(bt), t(lens), 0.125, bs)
        torch.cuda.synchronize()
        worst = max(worst, assert_close(out.float().cpu().numpy(), want8,
                                        what=f"config 1 {name}"))
    record_headroom("cfg1", "int8 per token, both names", worst)


# ------------------------------------------------------------------ config 2 / 3

@pytest.mark.parametrize("variant", ["warp", "splitk"])
def test_config2_bench_inputs(variant):
    case = make_case([4096] * 32, 12, 2)
    check(case, variant, [0, 13, 31], "cfg2", f"{variant} 32 x 4096 12/2")


@pytest.mark.parametrize("variant", ["warp", "warp_int8", "splitk", "splitk_int8"])
def test_config3_full_size(variant):
    """Config 3: 64 x 8192, 12/2, D=128; the INT8 cache is the write kernel's
    per-token quantization of N(0,1) tokens; the FP16 leg is the same shape."""
    int8 = variant.endswith("int8")
    case = make_case([8192] * 64, 12, 2, int8=int8)
    check(case, variant, [0, 21, 42, 63], "cfg3", f"{variant} 64 x 8192 12/2")


# ------------------------------------------------------------------ config 4

@pytest.mark.parametrize("ctx", [32768, 65536, 131072])
@pytest.mark.parametrize("variant", ["splitk", "splitk_int8"])
def test_config4_long_context(ctx, variant):
    """Config 4: 8 sequences x ctx, Llama-3-8B heads 32/8, N(0,1) K/V with a
    Bernoulli(0.01) mask x20; the first and last sequence checked."""
    int8 = variant.endswith("int8")
    case = make_case([ctx] * 8, 32, 8, int8=int8, outliers=True, seed=4)
    check(case, variant, [0, 7], "cfg4", f"{variant} 8 x {ctx} 32/8 outliers", ctx=ctx)


@pytest.mark.parametrize("variant", ["splitk", "splitk_int8"])
@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_config4_reference_partition(variant, mode):
    """Config 4 as BASELINE states it, with the reference's partition size
    (PARTITION_SIZE 512, kernels/paged_attention_v4_splitk.cu:24): 8 x 32768,
    32/8 heads, 1% outliers x20, 64 splits per sequence, under the automatic
    choice (0), the host grid with its reduce launch (1), the in-kernel
    schedule with the two-level in-launch merge (2) and the stream partition
    (3); the first and last sequence checked."""
    import pa_int8

    int8 = variant.endswith("int8")
    case = make_case([32768] * 8, 32, 8, int8=int8, outliers=True, seed=4)
    part, ns = pa_int8.decode_plan(variant, 8, 32, 128, 8, 16, case["bt"].shape[1], 0, 512)
    assert (part, ns) == (512, 64)
    kc, vc, ks, vs = case["caches"][0]
    kw = {} if ks is None else dict(k_scales=ks, v_scales=vs)
    out = torch.empty_like(case["q"])
    assert pa_int8.capi().pa_decode_set_schedule(mode) == 0
    try:
        pa_int8.decode(variant, out, case["q"], kc, vc, case["bt"], case["ctx"], case["scale"],
                       case["bs"], check=False, partition_tokens=512, **kw)
        torch.cuda.synchronize()
    finally:
        pa_int8.capi().pa_decode_set_schedule(0)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    ratio = assert_close(got[[0, 7]], subset_oracle(case, [0, 7]),
                         what=f"cfg4 {variant} P=512 schedule {mode}")
    record_headroom("cfg4", f"{variant} 8 x 32768 32/8 outliers P=512 schedule {mode}", ratio,
                    variant=variant, seqs_checked=2, ctx=32768, partition=512, schedule=mode)


@pytest.mark.parametrize("head_dim", [128, 72, 200])
@pytest.mark.parametrize("bs", [8, 16, 32])
@pytest.mark.parametrize("variant,mode", [("warp", 0), ("splitk", 1)])
def test_group_mapping_large_fp16(bs, variant, mode, head_dim):
    """FP16 grid launches that read more than 32 MB take the group mapping
    (16-token groups per MFMA row tile, each group half at its own block):
    block sizes 8 (a group spans two blocks), 16 and 32, lengths that end
    inside a group and inside a block, on the single launch and the grid
    form of split-K (its reduce launch); head_dim 72 and 200 add a short
    last QK chunk and a half last output tile; every sequence checked."""
    import pa_int8

    lens = [8192 - 37 * i for i in range(8)]
    case = _bench().make_case(torch, lens, 12, 2, head_dim, bs, DEV, 7, False, False, 1)
    kc, vc = case["caches"][0][0], case["caches"][0][1]
    assert kc.numel() * 2 * 2 > 32 << 20          # a non-temporal (group-mapped) launch
    out = torch.empty_like(case["q"])
    assert pa_int8.capi().pa_decode_set_schedule(mode) == 0
    try:
        pa_int8.decode(variant, out, case["q"], kc, vc, case["bt"], case["ctx"], case["scale"], bs,
                       check=False)
        torch.cuda.synchronize()
    finally:
        pa_int8.capi().pa_decode_set_schedule(0)
    seqs = list(range(8))
    ratio = assert_close(out.float().cpu().numpy(), subset_oracle(case, seqs),
                         what=f"{variant} block_size {bs} D={head_dim}")
    record_headroom("group-mapping", f"{variant} 8 ragged x ~8192 12/2 D={head_dim} block_size {bs}",
                    ratio)


@pytest.mark.parametrize("variant", ["warp", "warp_int8"])
def test_config4_single_launch(variant):
    """The single-launch kinds on config 4's 64k shape (in-launch split merge)."""
    int8 = variant.endswith("int8")
    case = make_case([65536] * 8, 32, 8, int8=int8, outliers=True, seed=5)
    check(case, variant, [3], "cfg4", f"{variant} 8 x 65536 32/8 outliers", ctx=65536)


# ------------------------------------------------------------------ config 5

@pytest.mark.parametrize("hkv", [8, 1])
@pytest.mark.parametrize("variant", ["splitk", "splitk_int8"])
@pytest.mark.parametrize("mode", [1, 2, 3])
def test_config5_ragged_mix(hkv, variant, mode):
    """Config 5: 256 sequences, lognormal(ln 1024, 1.0) lengths clipped to
    [16, 32768] (seed 5, as bench.py), 32 q heads over 8 kv heads or MQA 32/1,
    on the host grid (mode 1), the in-kernel schedule (mode 2) and the stream
    partition (mode 3); 24
    sequences checked, the longest and the shortest among them."""
    import pa_int8

    lens = _bench().lognormal_lens(256, seed=5)
    int8 = variant.endswith("int8")
    case = make_case(lens, 32, hkv, int8=int8, seed=6)
    order = np.argsort(lens)
    rng = np.random.default_rng(hkv * 10 + mode)
    seqs = sorted({int(order[0]), int(order[-1]), *rng.choice(256, size=22, replace=False)})
    assert pa_int8.capi().pa_decode_set_schedule(mode) == 0
    try:
        check(case, variant, seqs, "cfg5", f"{variant} 256 ragged 32/{hkv} schedule {mode}",
              schedule=mode)
    finally:
        pa_int8.capi().pa_decode_set_schedule(0)

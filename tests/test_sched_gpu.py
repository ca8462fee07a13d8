"""GPU tests of the three work distributions of the decode kernels.

``pa_decode_set_schedule`` selects the grid form (one work-group per
(unit, split) slot of the host plan), the in-kernel schedule (persistent
work-groups over a compact work list built from context_lens on the device)
or the stream partition (split-K kinds: every resident work-group takes an
equal contiguous range of all streams' chunks; the single-launch kinds run
the grid under it).  All must give the oracle's result on ragged batches,
capacity-sized block tables, many sequences and zero-length sequences; the
schedule's claim counters must return to zero after every launch (checked by
running different shapes back to back); results are bitwise reproducible.
"""

import math

import numpy as np
import pytest
import torch

from _cases import assert_close, fp16_case, int8_case, oracle_fp16, oracle_int8

pytestmark = pytest.mark.gpu
DEV = "cuda"
GRID, SCHED, STREAM = 1, 2, 3


@pytest.fixture(scope="module", autouse=True)
def _lib(built):
    import pa_int8

    pa_int8.ext()
    yield
    pa_int8.capi().pa_decode_set_schedule(0)


def _mode(m):
    import pa_int8

    assert pa_int8.capi().pa_decode_set_schedule(m) == 0


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def ragged_lens(n, seed, lo=1, hi=3000):
    rng = np.random.default_rng(seed)
    x = np.exp(rng.normal(math.log(300), 1.2, n))
    return np.clip(np.round(x), lo, hi).astype(np.int32)


def run(c, variant, lens=None, bt=None, check=True, int8=False, partition=0):
    import pa_int8

    q = _t(c["q"])
    out = torch.empty_like(q)
    kw = {}
    if int8:
        kc, vc, table = c["k_cache8"], c["v_cache8"], c["block_table8"]
        kw = dict(k_scales=_t(c["k_scales"]), v_scales=_t(c["v_scales"]))
    else:
        kc, vc, table = c["k_cache"], c["v_cache"], c["block_table"]
    pa_int8.decode(variant, out, q, _t(kc), _t(vc), _t(table if bt is None else bt),
                   _t(c["lens"] if lens is None else lens), c["scale"], c["block_size"],
                   check=check, partition_tokens=partition, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("mode", [GRID, SCHED, STREAM])
@pytest.mark.parametrize("variant", ["warp", "splitk"])
@pytest.mark.parametrize("heads", [(16, 8), (12, 2), (32, 1)])
def test_ragged_fp16(mode, variant, heads):
    _mode(mode)
    lens = ragged_lens(37, seed=heads[1])
    c = fp16_case(len(lens), lens, heads[0], heads[1], seed=11)
    assert_close(run(c, variant), oracle_fp16(c), what=f"mode {mode} {variant} {heads}")


@pytest.mark.parametrize("mode", [GRID, SCHED, STREAM])
@pytest.mark.parametrize("variant", ["warp", "splitk"])
@pytest.mark.parametrize("partition", [0, 64])
def test_ragged_fp16_head_dim_256(mode, variant, partition):
    """FP16 at head_dim 256 reads its query operand from a tile staged in LDS
    over the wave-merge slots.  Many work items per work-group (the schedule,
    small forced partitions) and many stream parts per work-group (the stream
    partition) check that no item's query tile meets another item's merge."""
    _mode(mode)
    lens = ragged_lens(41, seed=7)
    c = fp16_case(len(lens), lens, 8, 2, head_dim=256, seed=21)
    assert_close(run(c, variant, partition=partition), oracle_fp16(c),
                 what=f"mode {mode} {variant} partition {partition}")


# Two-level merge bound per head_dim: a unit folds in two levels from
# max(12, 65536 / (heads per tile * head_dim)) splits.  With 32 query heads on
# one kv head and 64-token splits, the lengths below give units of 70, 47, 33,
# 19, 11 and 1 splits.  Per tile: FP16 at head_dim <= 128 serves 32 heads
# (two levels from 32 splits at 64 dims, 26 at 80, 16 at 128); INT8 serves 32
# in the grid form and 16 under the schedule (64, 52 and 32 splits); head_dim
# 256 serves 16 (16 splits) and reads its query from LDS.
TWO_LEVEL_LENS = [4480, 2100, 700, 3000, 1, 1200]


@pytest.mark.parametrize("mode,head_dim", [(m, d) for m in (GRID, SCHED)
                                            for d in (64, 72, 80, 128, 200, 256)] +
                         [(STREAM, 128), (STREAM, 72)])
@pytest.mark.parametrize("variant", ["warp", "splitk", "warp_int8", "splitk_int8"])
def test_two_level_split_merge(mode, head_dim, variant):
    """A unit whose split partials hold at least 256 KB of accumulators is
    merged in two levels: the last split of each of four groups folds its
    group, the last group folds the four.  Units of one and two levels meet
    in one launch (TWO_LEVEL_LENS); the second run checks that every counter
    came back to zero.  The stream partition merges the split-K kinds in its
    reduce launch (and runs the single-launch kinds on the grid), so it is
    run at head_dim 128 only."""
    _mode(mode)
    lens = np.array(TWO_LEVEL_LENS, dtype=np.int32)
    int8 = variant.endswith("int8")
    c = (int8_case if int8 else fp16_case)(len(lens), lens, 32, 1, head_dim=head_dim, seed=23)
    ref = (oracle_int8 if int8 else oracle_fp16)(c)
    for i in range(2):
        assert_close(run(c, variant, int8=int8, partition=64), ref,
                     what=f"mode {mode} {variant} D={head_dim} run {i}")


@pytest.mark.parametrize("mode", [GRID, SCHED])
@pytest.mark.parametrize("variant,head_dim", [("warp", 128), ("splitk", 128), ("warp", 256),
                                              ("warp_int8", 128), ("splitk_int8", 128)])
@pytest.mark.parametrize("scale", [-0.09, 0.0])
def test_nonpositive_scale(mode, variant, head_dim, scale):
    """The softmax scale may be zero (equal weights over the valid tokens) or
    negative (the scores' order reverses); masked tails in the last chunks of
    ragged lengths must still get zero weight (32 query heads per kv head:
    32-head tiles FP16 at 128 dims)."""
    _mode(mode)
    lens = np.array([1, 37, 300, 1000, 77], dtype=np.int32)
    int8 = variant.endswith("int8")
    c = (int8_case if int8 else fp16_case)(len(lens), lens, 32, 1, head_dim=head_dim, seed=29)
    c = dict(c, scale=scale)
    ref = (oracle_int8 if int8 else oracle_fp16)(c)
    assert_close(run(c, variant, int8=int8), ref, what=f"mode {mode} {variant} D={head_dim}")


@pytest.mark.parametrize("mode", [GRID, SCHED, STREAM])
@pytest.mark.parametrize("variant", ["warp_int8", "splitk_int8"])
@pytest.mark.parametrize("heads", [(16, 8), (32, 1)])
def test_ragged_int8(mode, variant, heads):
    _mode(mode)
    lens = ragged_lens(29, seed=heads[1] + 3)
    c = int8_case(len(lens), lens, heads[0], heads[1], seed=12)
    assert_close(run(c, variant, int8=True), oracle_int8(c), what=f"mode {mode} {variant}")


@pytest.mark.parametrize("mode", [GRID, SCHED, STREAM])
@pytest.mark.parametrize("variant", ["warp", "splitk"])
def test_capacity_sized_block_table(mode, variant):
    """A block table sized for a long maximum length with short sequences in it
    (the serving layout): the grid plans many empty splits, the schedule none."""
    _mode(mode)
    lens = ragged_lens(20, seed=5, hi=900)
    c = fp16_case(len(lens), lens, 8, 2, seed=13)
    bt = np.zeros((len(lens), c["block_table"].shape[1] * 6), np.int32)
    bt[:, :c["block_table"].shape[1]] = c["block_table"]
    assert_close(run(c, variant, bt=bt), oracle_fp16(c), what=f"mode {mode} {variant}")


@pytest.mark.parametrize("num_seqs", [1024, 1025])
@pytest.mark.parametrize("variant", ["warp", "splitk"])
def test_many_sequences(num_seqs, variant):
    """The in-kernel schedule holds up to 1024 sequences; 1025 falls back to the grid."""
    _mode(0)
    rng = np.random.default_rng(num_seqs)
    lens = rng.integers(1, 80, size=num_seqs).astype(np.int32)
    c = fp16_case(num_seqs, lens, 4, 1, head_dim=64, seed=14)
    assert_close(run(c, variant), oracle_fp16(c), what=f"{num_seqs} seqs")
    _mode(SCHED)
    assert_close(run(c, variant), oracle_fp16(c), what=f"{num_seqs} seqs, schedule forced")
    _mode(STREAM)
    assert_close(run(c, variant), oracle_fp16(c), what=f"{num_seqs} seqs, stream partition")


@pytest.mark.parametrize("mode", [SCHED, STREAM])
@pytest.mark.parametrize("variant", ["warp", "splitk", "warp_int8", "splitk_int8"])
def test_schedule_is_reproducible(variant, mode):
    _mode(mode)
    lens = ragged_lens(33, seed=21)
    int8 = variant.endswith("int8")
    c = (int8_case if int8 else fp16_case)(len(lens), lens, 16, 4, seed=15)
    a = run(c, variant, int8=int8)
    for _ in range(3):
        assert np.array_equal(run(c, variant, int8=int8), a)


@pytest.mark.parametrize("mode", [SCHED, STREAM])
def test_claim_counters_reset_between_shapes(mode):
    """Different shapes and lengths back to back on one stream: every launch
    must see zeroed claim and arrival counters (and, under the stream
    partition, scratch that the previous shape left)."""
    _mode(mode)
    for i, (n, heads, hi) in enumerate([(9, (8, 2), 4000), (40, (16, 8), 600),
                                        (3, (32, 1), 9000), (64, (8, 2), 200)]):
        lens = ragged_lens(n, seed=40 + i, hi=hi)
        c = fp16_case(n, lens, heads[0], heads[1], seed=16 + i)
        for variant in ("warp", "splitk"):
            assert_close(run(c, variant), oracle_fp16(c), what=f"shape {i} {variant}")


@pytest.mark.parametrize("mode", [SCHED, STREAM])
@pytest.mark.parametrize("variant", ["warp", "splitk", "splitk_int8"])
def test_schedule_zero_and_clamped_context(variant, mode):
    """No-check entry under the schedule and the stream partition: ctx <= 0
    gives zeros, ctx beyond the block table is clamped to it."""
    _mode(mode)
    if variant.endswith("int8"):
        c = int8_case(4, np.array([40, 20, 33, 500], dtype=np.int32), 8, 2, seed=17)
        lens = np.array([0, 20, 10_000, -3], dtype=np.int32)
        got = run(c, variant, lens=lens, check=False, int8=True)
        assert np.all(got[0] == 0) and np.all(got[3] == 0)
        cap = c["block_table8"].shape[1] * c["block_size"]
        c2 = dict(c, lens=np.array([1, 20, cap, 1], dtype=np.int32))
        assert_close(got[1:3], oracle_int8(c2)[1:3], what="clamped")
        return
    c = fp16_case(4, np.array([40, 20, 33, 500], dtype=np.int32), 8, 2, seed=17)
    lens = np.array([0, 20, 10_000, -3], dtype=np.int32)
    got = run(c, variant, lens=lens, check=False)
    assert np.all(got[0] == 0) and np.all(got[3] == 0)
    cap = c["block_table"].shape[1] * c["block_size"]
    c2 = dict(c, lens=np.array([1, 20, cap, 1], dtype=np.int32))
    assert_close(got[1:3], oracle_fp16(c2)[1:3], what="clamped")


@pytest.mark.parametrize("num_seqs", [1, 63, 64, 65, 130])
@pytest.mark.parametrize("variant", ["splitk", "splitk_int8"])
def test_schedule_small_batch_boundary(num_seqs, variant):
    """Batches of at most 64 sequences take the one-wave schedule build, larger
    ones the work-group build: both sides of the boundary with ragged lengths,
    zero lengths, lengths at whole partitions (no short row) and a forced
    partition that puts short rows in every band."""
    _mode(SCHED)
    lens = ragged_lens(num_seqs, seed=num_seqs + 50, hi=4000)
    if num_seqs > 3:
        lens[1] = 0
        lens[2] = 1024
        lens[3] = 2048
    int8 = variant.endswith("int8")
    c = (int8_case if int8 else fp16_case)(num_seqs, np.maximum(lens, 1), 8, 2, seed=19)
    want = (oracle_int8 if int8 else oracle_fp16)(c)
    got = run(c, variant, lens=lens, check=False, int8=int8)
    nz = lens > 0
    assert np.all(got[~nz] == 0)
    assert_close(got[nz], want[nz], what=f"{num_seqs} seqs")
    for p in (256, 1024):
        got = run(c, variant, lens=lens, check=False, int8=int8, partition=p)
        assert_close(got[nz], want[nz], what=f"{num_seqs} seqs P={p}")


@pytest.mark.parametrize("partition", [64, 320, 2048])
def test_schedule_forced_partition(partition):
    _mode(SCHED)
    lens = ragged_lens(12, seed=partition, hi=5000)
    c = fp16_case(len(lens), lens, 12, 2, seed=18)
    for variant in ("warp", "splitk"):
        assert_close(run(c, variant, partition=partition), oracle_fp16(c),
                     what=f"P={partition} {variant}")


def _distribution(c, variant, mb, ctx=0):
    """The planner's work distribution (1 grid, 2 schedule) for case `c`."""
    import ctypes

    import pa_int8

    kind = {"warp": 0, "splitk": 1, "warp_int8": 2, "splitk_int8": 3}[variant]
    info = (ctypes.c_int32 * 7)()
    S, H, D = c["q"].shape
    Hkv = c["k_cache"].shape[1]
    assert pa_int8.capi().pa_decode_plan_detail(kind, S, H, D, Hkv, c["block_size"], mb, ctx,
                                                0, info, 7) == 0
    return info[4]


@pytest.mark.parametrize("variant", ["splitk", "splitk_int8"])
@pytest.mark.parametrize("extra_blocks", [0, 1])
def test_split_k_small_launch_boundary(variant, extra_blocks):
    """Split-K calls reading at most 64 MiB of K/V (bound: the table's
    capacity for the no-check entry) take the single-launch plan; one block
    more of capacity and they keep the in-kernel schedule.  Both sides give
    the oracle's result, with short ragged sequences in a capacity-sized table."""
    _mode(0)
    int8 = variant.endswith("int8")
    lens = ragged_lens(4, seed=31, hi=2500)
    c = (int8_case if int8 else fp16_case)(len(lens), lens, 8, 8, seed=31)
    # FP16 K/V of 4 sequences x 8 kv heads x 4096 tokens x 128 dims is 64 MiB; INT8 at 8192
    cap_blocks = (512 if int8 else 256) + extra_blocks
    table = c["block_table8"] if int8 else c["block_table"]
    bt = np.zeros((len(lens), cap_blocks), np.int32)
    bt[:, :table.shape[1]] = table
    assert _distribution(c, variant, cap_blocks) == (2 if extra_blocks else 1)
    want = (oracle_int8 if int8 else oracle_fp16)(c)
    assert_close(run(c, variant, bt=bt, check=False, int8=int8), want,
                 what=f"{variant} capacity {cap_blocks} blocks")


@pytest.mark.parametrize("variant", ["splitk", "splitk_int8"])
@pytest.mark.parametrize("heads", [(12, 2), (32, 1)])
def test_ragged_floor_below_one_item_per_cu(variant, heads):
    """A ragged launch with less work than one floor-sized item per CU (16
    sequences of median 2048 tokens) runs items of about one per CU; the
    result is the oracle's, and bitwise equal to the forced-schedule run
    at the same partition choice."""
    _mode(0)
    int8 = variant.endswith("int8")
    rng = np.random.default_rng(41)
    lens = np.clip(np.round(np.exp(rng.normal(math.log(2048), 1.0, 16))), 16, 12000).astype(np.int32)
    h, hkv = heads
    c = (int8_case if int8 else fp16_case)(len(lens), lens, h, hkv, seed=41)
    table = c["block_table8"] if int8 else c["block_table"]
    # a table sized for 32k tokens: past the 64 MiB bound of the single-launch plan
    bt = np.zeros((len(lens), 2048), np.int32)
    bt[:, :table.shape[1]] = table
    assert _distribution(c, variant, bt.shape[1]) == 2
    want = (oracle_int8 if int8 else oracle_fp16)(c)
    got = run(c, variant, bt=bt, check=False, int8=int8)
    assert_close(got, want, what=f"{variant} {h}/{hkv}")
    _mode(SCHED)
    again = run(c, variant, bt=bt, check=False, int8=int8)
    assert np.array_equal(got, again)


@pytest.mark.parametrize("int8", [False, True])
def test_checked_equal_lengths_take_the_single_launch_plan(int8):
    """The reference-named split-K ops read the lengths for their `min >= 1`
    check; with equal lengths they run the single-launch plan, so their output
    is bitwise the single-launch op's, and the oracle's within tolerance.
    Ragged lengths keep the split-K plan."""
    from pa_int8 import registry

    _mode(0)
    for lens, equal in ((np.full(6, 3000, np.int32), True),
                        (np.array([3000, 2999, 3000, 100, 3000, 3000], np.int32), False)):
        c = (int8_case if int8 else fp16_case)(len(lens), lens, 12, 2, seed=43)
        want = (oracle_int8 if int8 else oracle_fp16)(c)
        q = _t(c["q"])
        outs = {}
        for name in (("warp_int8", "splitk_int8") if int8 else ("warp", "splitk")):
            out = torch.empty_like(q)
            if int8:
                registry.VARIANTS_INT8[name](out, q, _t(c["k_cache8"]), _t(c["v_cache8"]),
                                             _t(c["k_scales"]), _t(c["v_scales"]),
                                             _t(c["block_table8"]), _t(lens), c["scale"],
                                             c["block_size"])
            else:
                registry.VARIANTS[name](out, q, _t(c["k_cache"]), _t(c["v_cache"]),
                                        _t(c["block_table"]), _t(lens), c["scale"],
                                        c["block_size"])
            torch.cuda.synchronize()
            outs[name] = out.float().cpu().numpy()
            assert_close(outs[name], want, what=f"{name} equal={equal}")
        a, b = outs.values()
        if equal:
            assert np.array_equal(a, b)

"""CPU tests of the host side: the C-ABI library, its validation and planning
logic, the torch shim's error paths and the byte model.  No GPU needed."""

import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("pa_mi355x.h", "pa_mi355x_tuning.h")]
PROBE_HEADER = os.path.join(ROOT, "cuda-pa-int8_amd", "csrc", "bench", "pa_probe.h")


@pytest.fixture(scope="module")
def lib(built):
    import pa_int8

    return pa_int8.capi()


def declared_functions(headers=HEADERS):
    names = set()
    for h in headers:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(pa_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol(built):
    lib_path, _ = built
    so = ctypes.CDLL(lib_path)
    names = declared_functions()
    assert len(names) >= 16
    missing = [n for n in names if not hasattr(so, n)]
    assert not missing, missing


def test_prototypes_cover_the_header(built):
    from pa_int8 import _loader

    assert set(declared_functions()) == set(_loader.PROTOTYPES)


def test_probes_live_outside_the_product_library(built):
    """The benchmark's probes are declared and exported by their own library only."""
    from pa_int8 import _loader

    probe_names = declared_functions([PROBE_HEADER])
    assert set(probe_names) == set(_loader.PROBE_PROTOTYPES)
    product = ctypes.CDLL(built[0])
    probes = _loader.probe_capi()
    for n in probe_names:
        assert hasattr(probes, n) and not hasattr(product, n), n


def test_version_and_status_strings(lib):
    assert b"gfx950" in lib.pa_version()
    for code in range(9):
        assert lib.pa_status_string(code)
    assert lib.pa_status_string(99) == b"unknown status"


# validate: the reference's TORCH_CHECK rules (v3:149-150, v5:167-168, v5:176)
@pytest.mark.parametrize("bs,f16_ok,i8_ok", [(8, True, False), (16, True, True), (32, True, True),
                                             (64, True, True), (128, True, True), (24, False, False),
                                             (256, False, False), (0, False, False), (4, False, False)])
def test_validate_block_size_rule(lib, bs, f16_ok, i8_ok):
    f16 = lib.pa_validate_decode(0, 2, 8, 128, 2, 10, bs, 8, 4)
    i8 = lib.pa_validate_decode(2, 2, 8, 128, 2, 10, bs, 8, 4)
    assert (f16 == 0) == f16_ok and (i8 == 0) == i8_ok
    if not f16_ok:
        assert f16 == 3


def test_validate_shape_rules(lib):
    assert lib.pa_validate_decode(0, 2, 8, 128, 2, 10, 16, 4, 4) == 4      # x != 8
    for d in (0, 4, 12, 100, 264, 512):                                    # head_dim not built
        assert lib.pa_validate_decode(0, 2, 8, d, 2, 10, 16, 8, 4) == 4
    assert lib.pa_validate_decode(0, 2, 8, 128, 3, 10, 16, 8, 4) == 2      # H % Hkv
    assert lib.pa_validate_decode(0, 2, 8, 128, 2, 0, 16, 8, 4) == 2       # no blocks
    assert lib.pa_validate_decode(0, 0, 8, 128, 2, 0, 16, 8, 0) == 0       # empty batch is fine
    for d in range(8, 257, 8):
        for kind in range(4):
            assert lib.pa_validate_decode(kind, 1, 32, d, 1, 1, 16, 8, 1) == 0


def test_check_context_lens(lib):
    mx = ctypes.c_int32(0)
    a = (ctypes.c_int32 * 3)(5, 9, 2)
    assert lib.pa_check_context_lens(ctypes.cast(a, ctypes.c_void_p), 3, ctypes.byref(mx)) == 0
    assert mx.value == 9
    b = (ctypes.c_int32 * 2)(8, 0)
    assert lib.pa_check_context_lens(ctypes.cast(b, ctypes.c_void_p), 2, None) == 7


@pytest.mark.parametrize("s,h,hkv,ctx", [(32, 12, 2, 4096), (64, 12, 2, 8192), (8, 32, 8, 131072),
                                         (256, 32, 1, 32768), (4, 8, 8, 512), (1, 8, 1, 1)])
def test_plan_invariants(lib, s, h, hkv, ctx):
    part, ns = ctypes.c_int32(), ctypes.c_int32()
    mb = (ctx + 15) // 16
    for kind in range(4):
        assert lib.pa_decode_plan(kind, s, h, 128, hkv, 16, mb, ctx, 0, ctypes.byref(part),
                                  ctypes.byref(ns)) == 0
        assert part.value % 64 == 0 and part.value >= 64
        assert ns.value >= 1 and part.value * ns.value >= ctx
        assert part.value * (ns.value - 1) < ctx
        need = lib.pa_decode_workspace_bytes(kind, s, h, 128, hkv, 16, mb, ctx, 0)
        assert need % 256 == 0 and need > 0
    # counters: the 8 claim counters (1 KB), then one arrival counter per
    # (sequence, kv head, head chunk of <= 16 query heads) and four per unit
    # for the groups of a two-level merge
    chunks = -(-(h // hkv) // 16)
    units = s * hkv * chunks
    assert lib.pa_decode_counter_bytes(s, h, hkv) == 1024 + -(-units * 5 * 4 // 256) * 256
    # forced partition sizes are rounded up to 64 tokens
    assert lib.pa_decode_plan(0, s, h, 128, hkv, 16, mb, ctx, 100, ctypes.byref(part),
                              ctypes.byref(ns)) == 0
    assert part.value == min(128, (ctx + 63) // 64 * 64)


def test_forced_partition_is_capped(lib):
    # a split holds at most 2048 tokens per wave of the work-group for
    # head_dim <= 128 and 1024 for head_dim 256 (its block ids are staged in
    # LDS): FP16 split-K with one head chunk runs 8 waves (16384 tokens),
    # head_dim 256 and INT8 split-K run 4 (4096 / 8192)
    part, ns = ctypes.c_int32(), ctypes.c_int32()
    for kind, d, cap in ((1, 128, 16384), (1, 64, 16384), (1, 256, 4096), (3, 128, 8192)):
        assert lib.pa_decode_plan(kind, 8, 32, d, 8, 16, 8192, 131072, 100000, ctypes.byref(part),
                                  ctypes.byref(ns)) == 0
        assert part.value == cap and ns.value == 131072 // cap, (kind, d, part.value)
    lib.pa_decode_set_waves_per_group(4)
    try:
        assert lib.pa_decode_plan(1, 8, 32, 128, 8, 16, 8192, 131072, 100000, ctypes.byref(part),
                                  ctypes.byref(ns)) == 0
        assert part.value == 8192
    finally:
        lib.pa_decode_set_waves_per_group(0)


def test_probe_host_checks(built):
    from pa_int8 import _loader

    lib = _loader.probe_capi()
    # rejected before any device access: chunk sizes outside {1, 2, 4k*n} KB
    for chunk in (0, 512, 3072, 6144):
        assert lib.pa_probe_read_chunks(16, 1 << 20, 16, 4, chunk, 16, 64, None) == 2
    assert lib.pa_probe_read_chunks(None, 1 << 20, 16, 4, 4096, 16, 64, None) == 1
    assert lib.pa_probe_read_contiguous(16, 1 << 20, 16, 0, None) == 2
    assert lib.pa_probe_read_write(None, 1 << 20, 16, 64, None) == 1
    assert lib.pa_probe_read_write(16, 1 << 20, 16, 0, None) == 2
    assert lib.pa_probe_read_write(16, 1 << 34, 16, 64, None) == 2     # output past 4 GiB
    # the write-stream probe: the write op's argument rules, checked on the host
    args = [16, 16, 512, 256, 512, 256, 16, 64, 2, 16, 16, 16, 16, 100]
    assert lib.pa_probe_quant_write(None, *args[1:], 16, None) == 1
    for bs in (8, 24, 256):
        assert lib.pa_probe_quant_write(*args, bs, None) == 3
    assert lib.pa_probe_quant_write(16, 16, 512, 256, 512, 260, *args[6:], 16, None) == 2
    assert lib.pa_probe_quant_write(24, *args[1:], 16, None) == 2      # unaligned key


def test_single_launch_group_sizes(lib):
    """The single-launch kinds run one 4-wave work-group per CU (256 of them
    at configs 2 and 3) with a 16-head tile on launches over 32 MB; the
    32-head tile (MQA) and small, latency-bound launches keep 8 waves."""
    info = (ctypes.c_int32 * 8)()

    def plan(kind, s, h, d, hkv, ctx):
        assert lib.pa_decode_plan_detail(kind, s, h, d, hkv, 16, (ctx + 15) // 16, ctx, 0, info,
                                         8) == 0
        return dict(partition=info[0], splits=info[1], waves=info[2], tile=info[3])

    for kind in (0, 2):                                   # warp, warp_int8
        p = plan(kind, 32, 12, 128, 2, 4096)              # config 2: 64 units x 4 splits
        assert (p["waves"], p["partition"], p["splits"]) == (4, 1024, 4), (kind, p)
        p = plan(kind, 64, 12, 128, 2, 8192)              # config 3: 128 units x 2 splits
        assert (p["waves"], p["partition"], p["splits"]) == (4, 4096, 2), (kind, p)
        p = plan(kind, 8, 32, 128, 1, 32768)              # MQA: one 32-head tile per kv head
        assert p["tile"] == 32 and p["waves"] == 8, (kind, p)
    p = plan(0, 4, 8, 64, 8, 512)                         # config 1: tiny, latency-bound
    assert p["waves"] == 8, p
    p = plan(0, 1, 8, 128, 8, 4096)                       # 16.8 MB, below the 32 MB threshold
    assert p["waves"] == 8, p


def test_small_split_k_launches_take_the_grid(lib):
    """Split-K launches that read at most 64 MB (bound: every sequence at the
    checked maximum, else at the table's capacity) take the single-launch
    plan: the host grid with the splits merged in the launch, as warp /
    warp_int8 plan the same shape; larger ones keep the in-kernel schedule.
    Forced modes (grid = 1, schedule = 2) are left alone."""
    info = (ctypes.c_int32 * 7)()

    def plan(kind, s, h, hkv, mb, ctx):
        assert lib.pa_decode_plan_detail(kind, s, h, 128, hkv, 16, mb, ctx, 0, info, 7) == 0
        return tuple(info)

    for splitk, warp in ((1, 0), (3, 2)):
        for s, h, hkv, ctx in ((1, 12, 2, 1024), (1, 12, 2, 16384), (1, 8, 8, 4096),
                               (8, 8, 1, 4096), (4, 12, 2, 9008)):
            p = plan(splitk, s, h, hkv, (ctx + 15) // 16, ctx)
            assert p[4] == 1 and p[6] == 1, (splitk, s, ctx, p)          # grid, merged in launch
            assert p == plan(warp, s, h, hkv, (ctx + 15) // 16, ctx)
        # the bound follows the checked maximum, else the table's capacity
        assert plan(splitk, 64, 12, 2, 2048, 1024)[4] == 1               # 1024 tokens checked
        assert plan(splitk, 64, 12, 2, 2048, 0)[4] == 2                  # 32768-token capacity
        for s, h, hkv, ctx in ((64, 12, 2, 8192), (8, 32, 8, 32768), (256, 32, 1, 16401)):
            assert plan(splitk, s, h, hkv, (ctx + 15) // 16, ctx)[4] == 2, (splitk, s, ctx)
    # config 2: 128 MiB of FP16 K/V keeps the schedule; its INT8 cache is 64 MiB
    assert plan(1, 32, 12, 2, 256, 4096)[4] == 2 and plan(3, 32, 12, 2, 256, 4096)[4] == 1
    # exactly 64 MiB of FP16 K/V takes the grid, one block more the schedule
    assert plan(1, 1, 8, 8, 1024, 16384)[4] == 1
    assert plan(1, 1, 8, 8, 1025, 16400)[4] == 2
    for mode, want in ((1, 1), (2, 2)):
        assert lib.pa_decode_set_schedule(mode) == 0
        try:
            assert plan(1, 1, 12, 2, 64, 1024)[4] == want
            assert plan(1, 1, 12, 2, 64, 1024)[6] == (1 if mode == 2 else 0)
        finally:
            lib.pa_decode_set_schedule(0)


def test_waves_override_hook(lib):
    assert lib.pa_decode_set_waves_per_group(3) == 2
    for w in (4, 8, 0):
        assert lib.pa_decode_set_waves_per_group(w) == 0


def test_tuning_hooks_are_per_thread(lib):
    """A hook set on one thread leaves the plans of other threads alone."""
    import threading

    part, ns = ctypes.c_int32(), ctypes.c_int32()

    def plan():
        assert lib.pa_decode_plan(1, 8, 32, 128, 8, 16, 8192, 131072, 100000, ctypes.byref(part),
                                  ctypes.byref(ns)) == 0
        return part.value

    base = plan()
    seen = []
    t = threading.Thread(target=lambda: (lib.pa_decode_set_waves_per_group(4), seen.append(plan()),
                                         lib.pa_decode_set_waves_per_group(0)))
    t.start()
    t.join()
    assert seen == [base // 2] and plan() == base


def test_decode_rejects_missing_workspace(lib):
    # host-side refusal before any device access: NULL counters or workspace
    f = ctypes.c_float(0.1)
    st = lib.pa_paged_decode_attn_warp(1, 1, 1, 1, 1, 1, f, 16, 2, 8, 128, 2, 10, 8, 4, 0, 0,
                                       None, 0, None, 0, None)
    assert st == 5
    st = lib.pa_paged_decode_attn_warp(1, 1, 1, 1, 1, 1, f, 16, 2, 8, 128, 2, 10, 8, 4, 0, 0,
                                       256, 1 << 20, None, 0, None)
    assert st == 5
    st = lib.pa_paged_decode_attn_warp(1, 1, 1, 1, 1, 1, f, 16, 2, 8, 128, 2, 10, 8, 4, 0, 0,
                                       256, 16, 512, 1 << 20, None)       # counters too small
    assert st == 5
    st = lib.pa_paged_decode_attn_warp(1, 1, 1, 1, 1, 1, f, 16, 2, 8, 128, 2, 10, 8, 4, 0, 0,
                                       260, 1 << 20, 512, 1 << 20, None)  # misaligned counters
    assert st == 5
    st = lib.pa_paged_decode_attn_warp(None, 1, 1, 1, 1, 1, f, 16, 2, 8, 128, 2, 10, 8, 4, 0, 0,
                                       None, 0, None, 0, None)
    assert st == 1


def test_counters_reset_host_checks(lib):
    assert lib.pa_decode_counters_reset(None, 0, None) == 0       # nothing to do
    assert lib.pa_decode_counters_reset(None, 64, None) == 1
    assert lib.pa_decode_counters_reset(256, 6, None) == 2        # not whole words


def test_quant_write_host_checks(lib):
    args = [16, 16, 1024, 512, 1024, 512, 16, 4, 2, 128, 16, 16, 16, 16, 10]
    assert lib.pa_reshape_and_cache_int8(*args, 8, 8, None) == 3          # block_size 8
    assert lib.pa_reshape_and_cache_int8(*args, 16, 4, None) == 4         # x = 4
    bad = list(args)
    bad[2] = 1001                                                         # unaligned stride
    assert lib.pa_reshape_and_cache_int8(*bad, 16, 8, None) == 2


def test_torch_shim_rejects_cpu_tensors(built):
    import torch

    import pa_int8

    q = torch.zeros(2, 8, 128, dtype=torch.float16)
    kc = torch.zeros(4, 2, 16, 16, 8, dtype=torch.float16)
    vc = torch.zeros(4, 2, 128, 16, dtype=torch.float16)
    bt = torch.zeros(2, 2, dtype=torch.int32)
    ln = torch.ones(2, dtype=torch.int32)
    for name, fn in pa_int8.VARIANTS.items():
        with pytest.raises(RuntimeError, match="CUDA"):
            fn(torch.empty_like(q), q, kc, vc, bt, ln, 0.1, 16)
    for name, fn in pa_int8.VARIANTS_INT8.items():
        with pytest.raises(RuntimeError, match="CUDA"):
            fn(torch.empty_like(q), q, kc.to(torch.int8), vc.to(torch.int8),
               torch.ones(4, 2, 16), torch.ones(4, 2, 16), bt, ln, 0.1, 16)


def test_registry_mirrors_reference_names(built):
    import inspect

    import cuda_ext
    import pa_int8

    # tests/cuda_ext.py:38-49,112-141
    assert set(cuda_ext.VARIANTS) == {"naive", "vec", "online", "warp", "splitk"}
    assert set(cuda_ext.VARIANTS_INT8) == {"warp_int8", "splitk_int8"}
    for name, fn in pa_int8.VARIANTS.items():
        p16 = list(inspect.signature(fn).parameters)
        assert p16 == ["out", "q", "k_cache", "v_cache", "block_table", "context_lens", "scale",
                       "block_size"], name
    assert cuda_ext.paged_decode_attention is pa_int8.VARIANTS["naive"]
    p8 = list(inspect.signature(pa_int8.VARIANTS_INT8["splitk_int8"]).parameters)
    assert p8 == ["out", "q", "k_cache", "v_cache", "k_scales", "v_scales", "block_table",
                  "context_lens", "scale", "block_size"]


def test_byte_model_closed_forms():
    from pa_int8 import metrics

    assert metrics.decode_bytes([4096] * 32, 12, 2, 128) == 134_447_232
    assert metrics.decode_bytes([8192] * 64, 12, 2, 128, kv_elem_bytes=1,
                                scales=True) == 277_348_608
    assert metrics.decode_bytes([8192] * 64, 12, 2, 128) == 537_395_456
    assert metrics.decode_bytes([32768] * 8, 32, 8, 128) == 1_073_938_464
    assert metrics.decode_bytes([131072] * 8, 32, 8, 128) == 4_295_360_544
    assert metrics.decode_bytes([131072] * 8, 32, 8, 128, kv_elem_bytes=1,
                                scales=True) == 2_214_985_760
    assert metrics.quant_write_bytes(64 * 8192, 2, 128) == 817_889_280
    assert metrics.decode_kv_bytes([4096] * 32, 2, 128) == 134_217_728


def test_extension_exports_reference_op_names(built):
    """The six ops of kernels/bindings.cpp:45-58 plus the naive module's
    paged_decode_attention (paged_attention_naive.cu:169-172)."""
    import pa_int8

    ext = pa_int8.ext()
    for op in ("paged_decode_attn_vec", "paged_decode_attn_online", "paged_decode_attn_warp",
               "paged_decode_attn_splitk", "paged_decode_attn_warp_int8",
               "paged_decode_attn_splitk_int8", "paged_decode_attention"):
        assert callable(getattr(ext, op)), op


def test_naive_module_under_its_own_name(built):
    """The reference builds its naive op as the module paged_attn_naive
    (kernels/paged_attention_naive.cu:169-172); after loading, both module
    names import, as the reference's JIT-built modules do."""
    import importlib

    from pa_int8 import _loader

    naive = _loader.naive_ext()
    assert callable(naive.paged_decode_attention)
    assert importlib.import_module("paged_attn_naive") is naive
    assert importlib.import_module("paged_attn_opt") is _loader.ext()


def test_paged_cache_class_host_logic():
    """PagedKVCache's shapes, identity table and byte accounting
    (benchmarks/int8_bridge/paged_cache.py:41-86,158-182; the size gate of
    tests/test_int8_bridge.py:98-108), constructed on the CPU: no kernel runs."""
    import torch

    import pa_int8

    kw = dict(num_layers=28, num_kv_heads=2, head_dim=128, max_len=2048, block_size=16, x=8,
              device="cpu")
    fp16 = pa_int8.PagedKVCache(variant="fp16", **kw)
    i8 = pa_int8.PagedKVCache(variant="int8_per_token", **kw)
    assert fp16.k_cache.shape == (28, 128, 2, 16, 16, 8) and fp16.k_cache.dtype == torch.float16
    assert i8.v_cache.shape == (28, 128, 2, 128, 16) and i8.v_cache.dtype == torch.int8
    assert i8.k_scales.shape == (28, 128, 2, 16)
    assert fp16.block_table.tolist() == [list(range(128))]
    assert i8.kv_bytes() < fp16.kv_bytes() and i8.kv_bytes() / fp16.kv_bytes() < 0.6
    assert fp16.kv_bytes_for_len(2048) == fp16.kv_bytes()
    assert i8.kv_bytes_for_len(2048) == i8.kv_bytes()
    assert i8.kv_bytes_for_len(17) == 2 * 28 * (2 * 2 * 128 * 16 + 2 * 2 * 16 * 4)
    # every figure follows the allocated tensors' per-block sizes
    for cache in (fp16, i8):
        per_block = sum(t[0, 0].numel() * t.element_size()
                        for t in (cache.k_cache, cache.v_cache) +
                        ((cache.k_scales, cache.v_scales) if cache.is_int8 else ()))
        assert cache.layout.block_bytes() == per_block
        assert cache.kv_bytes_for_len(1) == per_block * 28
        assert cache.kv_bytes_for_len(0) == 0
        assert cache.kv_bytes_for_len(33) == 3 * per_block * 28
    with pytest.raises(AssertionError):
        pa_int8.PagedKVCache(variant="int4", **kw)
    with pytest.raises(AssertionError):
        pa_int8.PagedKVCache(variant="fp16", **dict(kw, head_dim=100))
    c = pa_int8.PagedKVCache(variant="int8_per_tensor", **kw)
    assert c.context_lens(3).tolist() == [0] and c.lengths == [0] * 28
    with pytest.raises(RuntimeError, match="CUDA"):
        c.prefill(0, torch.zeros(5, 2, 128, dtype=torch.float16),
                  torch.zeros(5, 2, 128, dtype=torch.float16))
    # the device-slot append of a captured decode step, and its host bookkeeping
    tok = torch.zeros(2, 128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="prefill sets"):
        c.append_at(1, tok, tok, torch.zeros(1, dtype=torch.int64))
    with pytest.raises(TypeError, match="one-element int64"):
        fp16.append_at(0, tok, tok, torch.zeros(1, dtype=torch.int32))
    with pytest.raises(TypeError, match="one-element int64"):
        fp16.append_at(0, tok, tok, torch.zeros(2, dtype=torch.int64))
    assert fp16.capacity == 2048
    fp16.advance(2047)
    assert fp16.lengths == [2047] * 28 and fp16.context_lens(5).tolist() == [2047]
    with pytest.raises(AssertionError, match="full"):
        fp16.advance(2)
    fp16.advance(1)
    assert fp16.lengths == [2048] * 28
    fp16.reset()
    assert fp16.lengths == [0] * 28


@pytest.mark.parametrize("int8", [False, True])
def test_bench_gate_reference_matches_oracle(int8):
    """bench.dense_reference (the correctness gate the benchmark runs before
    timing each config) agrees with the oracle on the CPU, FP16 and INT8."""
    import sys

    import torch

    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench
    from _cases import fp16_case, int8_case, oracle_fp16, oracle_int8

    lens = np.array([300, 17, 1000], np.int32)
    c = (int8_case if int8 else fp16_case)(3, lens, 12, 2, seed=5)
    t = torch.from_numpy
    if int8:
        caches = [(t(c["k_cache8"]), t(c["v_cache8"]), t(c["k_scales"]), t(c["v_scales"]))]
        bt, want = c["block_table8"], oracle_int8(c)
    else:
        caches = [(t(c["k_cache"]), t(c["v_cache"]), None, None)]
        bt, want = c["block_table"], oracle_fp16(c)
    case = dict(caches=caches, bt=t(bt), bs=16, lens=[int(x) for x in lens], head_dim=128,
                q=t(c["q"]), scale=c["scale"])
    for s in range(3):
        got = bench.dense_reference(torch, case, s).numpy()
        np.testing.assert_allclose(got, want[s], atol=1e-5, rtol=1e-5)
    assert bench.gate_seqs([5, 9, 1, 7, 3, 2, 8]) == [0, 1, 2, 3, 4, 5, 6]
    assert bench.gate_seqs([4] * 100, 2) == [0, 50, 99]


def test_bench_dense_gather_inverts_the_paged_layout():
    """bench.gather_dense (the dense baseline's input) recovers the contiguous
    K/V that the oracle's builder scattered into the paged layout, repeated
    over the GQA group."""
    import sys

    import torch

    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench
    from oracle import paged_decode_ref as ref

    rng = np.random.default_rng(3)
    s, ctx, hkv, h, d, bs = 3, 40, 2, 6, 16, 16
    k = rng.standard_normal((s, ctx, hkv, d)).astype(np.float16)
    v = rng.standard_normal((s, ctx, hkv, d)).astype(np.float16)
    kc, vc, bt = ref.build_paged_kv_cache(k, v, np.full(s, ctx), block_size=bs, rng=rng)
    case = dict(caches=[(torch.from_numpy(kc), torch.from_numpy(vc), None, None)],
                bt=torch.from_numpy(bt.astype(np.int32)), bs=bs)
    kd, vd = bench.gather_dense(torch, case, [ctx] * s, h)
    assert kd.shape == (s, h, ctx, d) and vd.shape == (s, h, ctx, d)
    want_k = np.repeat(k.transpose(0, 2, 1, 3), h // hkv, axis=1)
    want_v = np.repeat(v.transpose(0, 2, 1, 3), h // hkv, axis=1)
    assert np.array_equal(kd.numpy(), want_k) and np.array_equal(vd.numpy(), want_v)


def test_bench_rotation_outruns_the_infinity_cache():
    """Decode caches rotate over at least 4x the 256 MB Infinity Cache (2x let
    K lines hit in it on MI355X) unless the 8-copy cap binds, which only
    happens for caches far smaller than it (launch-bound configs)."""
    import sys

    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench

    mall = 256 << 20
    for nbytes in (4_203_024, 134_447_232, 277_348_608, 537_395_456, 553_844_768,
                   1_073_938_464, 4_295_360_544):
        n = bench.copies_for(nbytes)
        assert 1 <= n <= 8
        assert n * nbytes >= 4 * mall or n == 8, (nbytes, n)
    assert bench.copies_for(134_447_232) == 8          # config 2: 1.08 GB cycled
    assert bench.copies_for(537_395_456) == 2          # config 3 FP16: 1.07 GB

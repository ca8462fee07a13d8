#!/usr/bin/env python3
"""Benchmark of the gfx950 paged-attention decode path on one MI355X.

A step is one decode call over one batch (all sequences, all heads).  The
headline workload is BASELINE config 2: Qwen2.5-1.5B-shape GQA 12/2,
head_dim 128, 32 sequences x 4096 tokens, FP16 KV, single-launch kernel.
``value`` is its algorithmic HBM bytes per step / time per step (GB/s).
The other BASELINE configs are measured the same way (INT8 vs FP16,
long-context split-K, ragged serving mix, quantize + cache-write, the tiny
CPU-runnable case), next to a dense baseline (SDPA over K/V gathered into
contiguous tensors, as the reference's bench_paged_decode.py:131-145 does).
The stdout line carries the headline, its roofline, the CPU baseline and a
[us, fraction of peak] summary per measurement; the full per-config record
(plans, correctness gates, address-stream probes, read ceilings) goes to
--detail-out and to the stderr lines.

Timing: W eager warm-up steps, then the K steps are captured in one HIP
graph (each step reads a different copy of the cache when one copy would
fit in the 256 MB Infinity Cache) and replayed untimed for at least 300 ms
of GPU time, so that the clocks have settled as in a serving loop; a timed region
is one replay of exactly K steps, bracketed by synchronize() and HIP events
on the stream the kernels run on, and a measurement is the median of three
such replays (five for the headline).  The no-sync entry is timed (the
reference's ``context_lens.min().item()`` host check is skipped).

    python bench.py [--steps K] [--warmup W] [--configs cfg2,cfg3,...]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.join(ROOT, "cuda-pa-int8_amd")
for _p in (ROOT, PKG_ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "decode µs + achieved HBM GB/s (% of peak), FP16 vs INT8 KV, GQA 12/2 d128"
MALL_BYTES = 256 << 20
ALL_CONFIGS = ["cfg2", "cfg1", "cfg3", "cfg3w", "cfg4", "cfg5", "refshapes", "dense", "e2e",
               "ceiling"]

# The reference's published A100 rows (head_dim 128, block_size 16, fp16 q/K/V
# ~ N(0,1)), measured here at the same shapes: (batch, ctx, q heads, kv heads,
# variant, A100 us, source under the reference checkout).
REF_SHAPES = [
    (1, 4096, 8, 8, "splitk", 86.0, "report/kernel_optimization.md:231"),
    (32, 4096, 8, 8, "splitk", 403.0, "report/kernel_optimization.md:257"),
    (64, 4096, 8, 8, "warp", 674.7, "report/kernel_optimization.md:269"),
    (64, 4096, 8, 8, "splitk", 699.8, "report/kernel_optimization.md:270"),
    (64, 4096, 8, 1, "warp", 458.0, "report/kernel_optimization.md:529"),
    (64, 4096, 8, 1, "splitk", 398.1, "report/kernel_optimization.md:530"),
    (32, 4096, 16, 4, "warp", 521.7, "report/kernel_optimization.md:776"),
    (32, 4096, 16, 4, "splitk", 415.4, "report/kernel_optimization.md:777"),
    (32, 2048, 8, 8, "warp", 277.7, "report/int8_quant.md:26"),
    (32, 2048, 8, 8, "splitk", 254.8, "report/int8_quant.md:27"),
    (32, 2048, 8, 8, "warp_int8", 269.0, "report/int8_quant.md:28"),
    (32, 2048, 8, 8, "splitk_int8", 199.6, "report/int8_quant.md:29"),
    (8, 4096, 8, 1, "splitk", 102.6, "report/int8_quant.md:36"),
    (8, 4096, 8, 1, "splitk_int8", 104.9, "report/int8_quant.md:38"),
    (32, 4096, 16, 4, "splitk", 438.6, "report/int8_quant.md:45"),
    (32, 4096, 16, 4, "splitk_int8", 393.6, "report/int8_quant.md:47"),
]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# --------------------------------------------------------------------------- inputs

def _block_table(torch, lens, bs, dev, gen):
    nblk = [(int(n) + bs - 1) // bs for n in lens]
    nb = sum(nblk) + 1
    perm = torch.randperm(nb, device=dev, generator=gen).to(torch.int32)
    bt = torch.zeros((len(lens), max(nblk)), dtype=torch.int32, device=dev)
    off = 0
    for s, k in enumerate(nblk):
        bt[s, :k] = perm[off:off + k]
        off += k
    return bt, nb


def _randn(torch, shape, dev, gen, outliers):
    t = torch.randn(shape, dtype=torch.float16, device=dev, generator=gen)
    if outliers:
        m = torch.rand(shape, device=dev, generator=gen) < 0.01
        t = torch.where(m, t * 20, t)
    return t


def make_case(torch, lens, num_heads, num_kv_heads, head_dim, bs, dev, seed, int8, outliers,
              copies):
    """Paged caches of N(0,1) fp16 K/V (optionally 1% outliers x20).

    FP16 caches are filled in their layout directly.  INT8 caches are
    produced by the quantize + write kernel from fp16 tokens, one sequence at
    a time, so they hold real per-token quantized data.
    """
    import pa_int8

    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    bt, nb = _block_table(torch, lens, bs, dev, gen)
    s = len(lens)
    q = torch.randn((s, num_heads, head_dim), dtype=torch.float16, device=dev, generator=gen)
    ctx = torch.tensor(lens, dtype=torch.int32, device=dev)
    caches = []
    for _ in range(copies):
        if not int8:
            kc = _randn(torch, (nb, num_kv_heads, head_dim // 8, bs, 8), dev, gen, outliers)
            vc = _randn(torch, (nb, num_kv_heads, head_dim, bs), dev, gen, outliers)
            caches.append((kc, vc, None, None))
            continue
        kc = torch.zeros((nb, num_kv_heads, head_dim // 8, bs, 8), dtype=torch.int8, device=dev)
        vc = torch.zeros((nb, num_kv_heads, head_dim, bs), dtype=torch.int8, device=dev)
        ks = torch.zeros((nb, num_kv_heads, bs), dtype=torch.float32, device=dev)
        vs = torch.zeros_like(ks)
        for si, n in enumerate(lens):
            t = torch.arange(n, device=dev)
            slots = bt[si, t // bs].to(torch.int64) * bs + t % bs
            k = _randn(torch, (n, num_kv_heads, head_dim), dev, gen, outliers)
            v = _randn(torch, (n, num_kv_heads, head_dim), dev, gen, outliers)
            pa_int8.reshape_and_cache_int8(k, v, kc, vc, ks, vs, slots)
        caches.append((kc, vc, ks, vs))
    torch.cuda.synchronize()
    return dict(q=q, bt=bt, ctx=ctx, caches=caches, lens=list(lens), bs=bs, nb=nb,
                scale=1.0 / math.sqrt(head_dim), heads=num_heads, kv_heads=num_kv_heads,
                head_dim=head_dim)


def copies_for(bytes_per_copy):
    """Enough distinct cache copies that the rotation outruns the Infinity Cache:
    at least 4x its size in total (the V tiles are read non-temporally, so the
    lines that can stay in it are K's, half of each copy)."""
    return max(1, min(8, math.ceil(4 * MALL_BYTES / max(1, bytes_per_copy))))


# --------------------------------------------------------------------------- timing

EAGER_ONLY = False   # --eager: every measurement uses plain launches
WARM_MS = 300.0      # untimed graph replays before each measurement, in ms of GPU time
WARM_MAX_REPLAYS = 5000


def time_steps(torch, step_fns, steps, warmup, replays=1):
    """Median ms per step over `replays` timed graph replays of `steps` steps
    (with --eager: `steps` plain launches after `warmup` ones)."""
    n = len(step_fns)
    for i in range(warmup):
        step_fns[i % n]()
    if EAGER_ONLY:
        return time_eager(torch, step_fns, steps)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):            # warm the side stream's workspace
        for i in range(min(n, 2)):
            step_fns[i]()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(steps):
            step_fns[i % n]()
    with torch.cuda.stream(stream):
        # one untimed replay, timed to size the warm-up: the GPU's clocks settle only
        # after 100-300 ms of sustained work (config 4 INT8 runs 3-4% slower before)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        g.replay()
        b.record(stream)
        torch.cuda.synchronize()
        for _ in range(min(WARM_MAX_REPLAYS, math.ceil(WARM_MS / max(a.elapsed_time(b), 1e-3)))):
            g.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(replays):
        with torch.cuda.stream(stream):
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            start.record(stream)
            g.replay()
            end.record(stream)
            torch.cuda.synchronize()
        times.append(start.elapsed_time(end) / steps)
    del g
    times.sort()
    return times[len(times) // 2]


def time_eager(torch, step_fns, steps):
    n = len(step_fns)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        step_fns[i % n]()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def decode_steps(torch, case, variant, partition=0):
    import pa_int8

    out = torch.empty_like(case["q"])
    fns = []
    for kc, vc, ks, vs in case["caches"]:
        kw = {} if ks is None else dict(k_scales=ks, v_scales=vs)

        def fn(kc=kc, vc=vc, kw=kw):
            pa_int8.decode(variant, out, case["q"], kc, vc, case["bt"], case["ctx"],
                           case["scale"], case["bs"], check=False, partition_tokens=partition,
                           **kw)
        fns.append(fn)
    return fns, out


def dense_reference(torch, case, seq):
    """fp32 dense attention of one sequence in torch on the device: its K/V
    gathered from the first cache copy through the block table (INT8 values
    times their scales), softmax(scale * K q) V per query head."""
    kc, vc, ks, vs = case["caches"][0]
    bs, n = case["bs"], case["lens"][seq]
    nblk = (n + bs - 1) // bs
    ids = case["bt"][seq, :nblk].long()
    hkv, d = kc.shape[1], case["head_dim"]
    k = kc[ids].permute(0, 3, 1, 2, 4).reshape(nblk * bs, hkv, d).float()   # [t, Hkv, D]
    v = vc[ids].permute(0, 3, 1, 2).reshape(nblk * bs, hkv, d).float()
    if ks is not None:
        k = k * ks[ids].permute(0, 2, 1).reshape(nblk * bs, hkv, 1)
        v = v * vs[ids].permute(0, 2, 1).reshape(nblk * bs, hkv, 1)
    k, v = k[:n].permute(1, 2, 0).contiguous(), v[:n].permute(1, 0, 2).contiguous()
    q = case["q"][seq].float().view(hkv, -1, d)                              # [Hkv, G, D]
    p = torch.softmax(torch.bmm(q, k) * case["scale"], dim=-1)               # [Hkv, G, t]
    return torch.bmm(p, v).reshape(-1, d)                                   # [H, D]


def gate(torch, case, fns, out, seqs, atol=2e-3, rtol=1e-2):
    """The correctness gate before timing (as bench_paged_decode.py:180-188 checks
    every variant first): one call of the timed step, its outputs for `seqs`
    against dense torch attention in fp32.  Returns {ok, headroom, seqs}."""
    fns[0]()
    torch.cuda.synchronize()
    worst = 0.0
    for s in seqs:
        want = dense_reference(torch, case, s)
        err = (out[s].float() - want).abs()
        worst = max(worst, float((err / (atol + rtol * want.abs())).max()))
    return dict(ok=bool(worst <= 1.0), headroom=round(worst, 4), seqs_checked=len(seqs),
                tolerance=f"atol {atol} rtol {rtol}, fp32 dense torch attention")


def gate_seqs(lens, n=6):
    """Sequences the gate checks: the first, the last, the longest, the shortest
    and a few between."""
    S = len(lens)
    picks = {0, S - 1, int(max(range(S), key=lambda i: lens[i])),
             int(min(range(S), key=lambda i: lens[i]))}
    picks |= {i * S // n for i in range(n)}
    return sorted(picks)


# --------------------------------------------------------------------------- configs

PLAN_FIELDS = ("partition_tokens", "splits", "waves", "head_tile", "distribution", "load_hints",
               "merged_in_launch")


def plan_detail(variant, case, partition=0):
    """The plan the library runs `variant` under for this case
    (pa_decode_plan_detail of the tuning header), as a dict."""
    import ctypes

    import pa_int8

    kind = pa_int8.registry.KIND[variant]
    q, bt = case["q"], case["bt"]
    info = (ctypes.c_int32 * 7)()
    st = pa_int8.capi().pa_decode_plan_detail(kind, q.shape[0], q.shape[1], q.shape[2],
                                              case["kv_heads"], case["bs"], bt.shape[1], 0,
                                              partition, info, 7)
    if st != 0:
        raise RuntimeError(f"pa_decode_plan_detail: status {st}")
    return dict(zip(PLAN_FIELDS, list(info)))


def probe_decode_stream(torch, case, variant, steps, warmup, replays=3):
    """Time of the exact-address-stream probe (libpa_bench_probe.so): the
    decode launch's own loads over the same caches, block table and plan, with
    the attention math replaced by a checksum.  Grid-form plans only (the
    single-launch kinds at up to 16 query heads per kv head, head_dim 128);
    None otherwise."""
    from pa_int8._loader import probe_capi

    plan = plan_detail(variant, case)
    q = case["q"]
    if plan["distribution"] != 1 or plan["head_tile"] != case["heads"] // case["kv_heads"] \
            or q.shape[2] != 128:
        return None
    lib = probe_capi()
    sink = torch.zeros(1024, dtype=torch.int32, device="cuda")
    int8 = variant.endswith("int8")
    fns = []
    for kc, vc, ks, vs in case["caches"]:
        def fn(kc=kc, vc=vc, ks=ks, vs=vs):
            st = lib.pa_probe_decode_stream(
                1 if int8 else 0, q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                ks.data_ptr() if int8 else None, vs.data_ptr() if int8 else None,
                case["bt"].data_ptr(), case["ctx"].data_ptr(), q.shape[0], q.shape[1],
                case["kv_heads"], case["bs"], kc.shape[0], case["bt"].shape[1], 0,
                plan["partition_tokens"], plan["waves"], plan["load_hints"], sink.data_ptr(),
                torch.cuda.current_stream().cuda_stream)
            if st != 0:
                raise RuntimeError(f"pa_probe_decode_stream: status {st}")
        fns.append(fn)
    return time_steps(torch, fns, steps, warmup, replays)


def run_decode_cfg(torch, name, lens, h, hkv, d, variant, steps, warmup, seed=0, outliers=False,
                   replays=3, eager=False, partition=0, eager_only=False, probe=False):
    from pa_int8 import metrics

    int8 = variant.endswith("int8")
    per_copy = metrics.decode_kv_bytes(lens, hkv, d, 1 if int8 else 2)
    case = make_case(torch, lens, h, hkv, d, 16, "cuda", seed, int8, outliers,
                     copies_for(per_copy))
    fns, out = decode_steps(torch, case, variant, partition)
    checked = gate(torch, case, fns, out, gate_seqs(lens, 2 if sum(lens) > 2 ** 20 else 6))
    if not checked["ok"]:
        log(f"[bench] GATE FAILED {name} {variant}: headroom {checked['headroom']} > 1")
    if eager_only:
        for i in range(warmup):
            fns[i % len(fns)]()
        ms = time_eager(torch, fns, steps)
    else:
        ms = time_steps(torch, fns, steps, warmup, replays)
    nbytes = metrics.decode_bytes(lens, h, hkv, d, kv_elem_bytes=1 if int8 else 2, scales=int8)
    import pa_int8

    part, ns = pa_int8.decode_plan(variant, len(lens), h, d, hkv, 16, case["bt"].shape[1], 0,
                                   partition)
    res = dict(variant=variant, us=round(ms * 1e3, 2), algo_bytes=nbytes,
               gbs=round(nbytes / (ms * 1e-3) / 1e9, 1),
               frac_peak=round(nbytes / (ms * 1e-3) / 1e9 / metrics.MI355X_HBM_PEAK_GBS, 4),
               kv_only_gbs=round(metrics.decode_kv_bytes(lens, hkv, d, 1 if int8 else 2)
                                 / (ms * 1e-3) / 1e9, 1),
               seqs=len(lens), heads=f"{h}/{hkv}", head_dim=d, total_tokens=int(sum(lens)),
               partition_tokens=part, splits=ns, cache_copies=len(case["caches"]),
               steps=steps, ok=checked["ok"], gate=checked)
    if eager:
        res["eager_us"] = round(time_eager(torch, fns, steps) * 1e3, 2)
    if probe and not eager_only:
        pms = probe_decode_stream(torch, case, variant, steps, warmup, replays)
        if pms is not None:
            res["address_stream_probe"] = dict(
                us=round(pms * 1e3, 2), gbs=round(nbytes / (pms * 1e-3) / 1e9, 1),
                decode_over_probe=round(ms / pms, 4),
                what="the decode launch's own loads (same plan, caches and block table) with "
                     "the attention math replaced by a checksum")
            log(f"[bench] {name} {variant} address-stream probe: {res['address_stream_probe']['us']} "
                f"us (decode / probe = {ms / pms:.3f})")
    del case, fns
    torch.cuda.empty_cache()
    log(f"[bench] {name} {variant}: {res['us']} us, {res['gbs']} GB/s "
        f"({100 * res['frac_peak']:.1f}% of peak)")
    return res


def probe_quant_write(torch, k, v, slots, dests, steps, warmup, replays=3):
    """Time of the write kernel's address-stream probe (libpa_bench_probe.so):
    the same launch, loads and stores over the same inputs, slots and
    destination caches, with the quantization replaced by a byte pick (it
    overwrites the caches)."""
    from pa_int8._loader import probe_capi

    lib = probe_capi()
    T, hkv, _ = k.shape
    fns = []
    for kc, vc, ks, vs in dests:
        def fn(kc=kc, vc=vc, ks=ks, vs=vs):
            st = lib.pa_probe_quant_write(
                k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
                slots.data_ptr(), T, hkv, kc.data_ptr(), vc.data_ptr(), ks.data_ptr(),
                vs.data_ptr(), kc.shape[0], kc.shape[3], torch.cuda.current_stream().cuda_stream)
            if st != 0:
                raise RuntimeError(f"pa_probe_quant_write: status {st}")
        fns.append(fn)
    return time_steps(torch, fns, steps, warmup, replays)


def run_quant_write(torch, steps, warmup, seed=0):
    import pa_int8
    from pa_int8 import metrics

    S, L, hkv, d, bs = 64, 8192, 2, 128, 16
    dev = "cuda"
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    lens = [L] * S
    bt, nb = _block_table(torch, lens, bs, dev, gen)
    t = torch.arange(L, device=dev)
    slots = (bt[:, t // bs].to(torch.int64) * bs + t % bs).reshape(-1)
    T = S * L
    k = torch.randn((T, hkv, d), dtype=torch.float16, device=dev, generator=gen)
    v = torch.randn((T, hkv, d), dtype=torch.float16, device=dev, generator=gen)
    # Two destination caches, alternating: a step never rewrites lines that the
    # previous step left dirty in the 256 MB Infinity Cache.
    dests = []
    for _ in range(2):
        kc = torch.zeros((nb, hkv, d // 8, bs, 8), dtype=torch.int8, device=dev)
        vc = torch.zeros((nb, hkv, d, bs), dtype=torch.int8, device=dev)
        ks = torch.zeros((nb, hkv, bs), dtype=torch.float32, device=dev)
        dests.append((kc, vc, ks, torch.zeros_like(ks)))

    def mk(kc, vc, ks, vs):
        return lambda: pa_int8.reshape_and_cache_int8(k, v, kc, vc, ks, vs, slots)

    # gate: 4096 sampled tokens against torch's own quantize_per_token on the
    # device (tests/paged_decode_attn.py:106-112), bytes and scale bits
    mk(*dests[0])()
    torch.cuda.synchronize()
    pick = torch.randperm(T, device=dev, generator=gen)[:4096]
    kc, vc, ks, vs = dests[0]
    blk, off = slots[pick] // bs, slots[pick] % bs
    ok = True
    for x, cache, sc, is_v in ((k, kc, ks, False), (v, vc, vs, True)):
        xs = x[pick]                                                     # [n, Hkv, D] fp16
        amax = xs.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8)
        want_s = (amax / 127.0).to(torch.float32)
        want_q = torch.round(xs.to(torch.float32) / want_s).clamp(-127, 127).to(torch.int8)
        got_q = cache[blk].permute(0, 1, 3, 2) if is_v else \
            cache[blk].permute(0, 1, 3, 2, 4).reshape(len(pick), hkv, bs, d)
        got_q = got_q[torch.arange(len(pick), device=dev), :, off]       # [n, Hkv, D]
        got_s = sc[blk, :, off]
        ok = ok and bool(torch.equal(got_q, want_q)) and bool(
            torch.equal(got_s.view(torch.int32), want_s.squeeze(-1).view(torch.int32)))
    if not ok:
        log("[bench] GATE FAILED cfg3w quant_write")
    ms = time_steps(torch, [mk(*dd) for dd in dests], steps, warmup, 3)
    nbytes = metrics.quant_write_bytes(T, hkv, d)
    res = dict(us=round(ms * 1e3, 2), algo_bytes=nbytes, gbs=round(nbytes / (ms * 1e-3) / 1e9, 1),
               frac_peak=round(nbytes / (ms * 1e-3) / 1e9 / metrics.MI355X_HBM_PEAK_GBS, 4),
               tokens=T, kv_heads=hkv, head_dim=d,
               slot_pattern="per-sequence block runs (prefill), block ids randomly permuted",
               destination_copies=len(dests), steps=steps, ok=ok,
               gate="4096 sampled tokens: int8 bytes and scale bits equal torch's "
                    "quantize_per_token on the device")
    log(f"[bench] cfg3w quant_write: {res['us']} us, {res['gbs']} GB/s")
    # after the gate and the timing: the probe overwrites the caches
    pms = probe_quant_write(torch, k, v, slots, dests, steps, warmup)
    res["write_stream_probe"] = dict(
        us=round(pms * 1e3, 2), gbs=round(nbytes / (pms * 1e-3) / 1e9, 1),
        write_over_probe=round(ms / pms, 3),
        note="the write kernel's own launch, loads and stores with the quantization replaced by "
             "a byte pick (pa_probe_quant_write): its address stream alone")
    log(f"[bench] cfg3w quant_write address-stream probe: {res['write_stream_probe']['us']} us "
        f"({res['write_stream_probe']['gbs']} GB/s; write / probe = "
        f"{res['write_stream_probe']['write_over_probe']})")
    del k, v, dests
    torch.cuda.empty_cache()
    return res


def gather_dense(torch, case, lens, num_heads):
    """Contiguous fp16 K/V [S, H, ctx, D] gathered from the first paged cache
    copy through the block tables, repeated over the GQA group (equal lengths)."""
    kc, vc = case["caches"][0][0], case["caches"][0][1]
    bt = case["bt"]
    S, ctx = len(lens), lens[0]
    nblk = (ctx + case["bs"] - 1) // case["bs"]
    ids = bt[:, :nblk].long()                                    # [S, nblk]
    k = kc[ids]                                                  # [S, nblk, Hkv, D/8, bs, 8]
    k = k.permute(0, 2, 1, 4, 3, 5).reshape(S, kc.shape[1], nblk * case["bs"], -1)
    v = vc[ids]                                                  # [S, nblk, Hkv, D, bs]
    v = v.permute(0, 2, 1, 4, 3).reshape(S, vc.shape[1], nblk * case["bs"], -1)
    k, v = k[:, :, :ctx].contiguous(), v[:, :, :ctx].contiguous()
    rep = num_heads // kc.shape[1]
    if rep > 1:
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
    return k, v


def dense_attention_fn(torch, q, k, v, scale):
    """(fn, impl): fn() computes dense attention of q [S, H, 1, D] over
    contiguous K/V [S, H, ctx, D] in fp16.  SDPA on its flash or
    memory-efficient backend; if neither takes the shape, an fp16 matmul form
    over contiguous operands (softmax in fp32) stands in, and impl names it."""
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel

        def dense():
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                return torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=scale)
        dense()
        torch.cuda.synchronize()
        return dense, "sdpa"
    except RuntimeError:
        kt = k.transpose(-1, -2).contiguous()

        def dense():
            p = torch.softmax(torch.matmul(q, kt).float() * scale, dim=-1).to(torch.float16)
            return torch.matmul(p, v)
        return dense, "fp16 matmul (q k^T, softmax in fp32, p v), contiguous operands"


def run_dense_baseline(torch, name, lens, h, hkv, d, steps, warmup, outliers=False):
    """Dense attention over gathered, GQA-repeated K/V (the reference's SDPA
    ceiling, bench_paged_decode.py:131-145), timed with plain launches next to
    the paged kernel on the same inputs.  SDPA runs on its flash or
    memory-efficient backend; if neither takes the shape, an fp16 matmul form
    over contiguous operands stands in (named in the result)."""
    import pa_int8
    from pa_int8 import metrics

    case = make_case(torch, lens, h, hkv, d, 16, "cuda", 0, False, outliers, 1)
    k, v = gather_dense(torch, case, lens, h)
    q = case["q"].unsqueeze(2)                                   # [S, H, 1, D]
    scale = case["scale"]
    dense, impl = dense_attention_fn(torch, q, k, v, scale)
    ref = dense()
    torch.cuda.synchronize()
    for _ in range(warmup):
        dense()
    ms_dense = time_eager(torch, [dense], steps)
    out = torch.empty_like(case["q"])
    pa_int8.decode("warp", out, case["q"], case["caches"][0][0], case["caches"][0][1],
                   case["bt"], case["ctx"], scale, 16)
    torch.cuda.synchronize()
    diff = (out.float() - ref.squeeze(2).float()).abs().max().item()
    dense_bytes = 2 * k.numel() * k.element_size() + 2 * q.numel() * 2
    paged_bytes = metrics.decode_bytes(lens, h, hkv, d, kv_elem_bytes=2, scales=False)
    res = dict(impl=impl, us=round(ms_dense * 1e3, 2), bytes_read=dense_bytes,
               gbs=round(dense_bytes / (ms_dense * 1e-3) / 1e9, 1),
               paged_algo_bytes=paged_bytes,
               max_abs_diff_vs_paged_warp=round(diff, 6), seqs=len(lens), heads=f"{h}/{hkv}",
               context=lens[0], steps=steps,
               note="K/V gathered and repeated over the GQA group outside the timed region")
    log(f"[bench] {name} dense baseline ({impl}): {res['us']} us "
        f"({res['gbs']} GB/s over {dense_bytes} B read); max |dense - paged| {diff:.2e}")
    del case, k, v, q
    torch.cuda.empty_cache()
    return res


def _bridge_model(torch, seed):
    """The random-init Qwen2.5-1.5B-shape model (fp16, 28 layers, 12 q / 2 kv
    heads, head_dim 128, vocab 151936) on the bridge's attention interface."""
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from pa_int8 import qwen_bridge as br

    cfg = Qwen2Config(vocab_size=151936, hidden_size=1536, intermediate_size=8960,
                      num_hidden_layers=28, num_attention_heads=12, num_key_value_heads=2,
                      max_position_embeddings=32768, rope_theta=1e6, tie_word_embeddings=True)
    torch.manual_seed(seed)
    with torch.device("cuda"):
        model = Qwen2ForCausalLM(cfg).to(torch.float16).eval()
    br.register()
    model.set_attn_implementation(br.ATTN_NAME)
    return model, cfg


def _bridge_cache(variant, n):
    from pa_int8 import PagedKVCache

    return PagedKVCache(num_layers=28, num_kv_heads=2, head_dim=128, max_len=n, variant=variant)


def run_e2e_long(torch, long_len=16384, max_new=64, seed=0):
    """Only the graph-replayed decode after a `long_len`-token prompt, FP16 and
    INT8 (per-token) caches, two passes: the workload of the bridge's kernel
    trace at a long context (`--configs e2elong` under rocprofv3)."""
    from pa_int8 import qwen_bridge as br

    model, cfg = _bridge_model(torch, seed)
    g = torch.Generator().manual_seed(seed + 1)
    prompt = torch.randint(0, cfg.vocab_size, (1, long_len), generator=g).cuda()
    res = {}
    for rep in range(2):
        for variant in ("fp16", "int8_per_token"):
            cache = _bridge_cache(variant, long_len + max_new)
            _, ttft, tpot, _ = br.generate_greedy_graph(model, prompt, max_new, cache)
            res[f"{variant}_pass{rep}"] = dict(ttft_ms=round(ttft * 1e3, 2),
                                               graph_tpot_ms=round(tpot * 1e3, 3))
            log(f"[bench] e2e long {long_len} {variant} pass {rep}: TPOT {tpot * 1e3:.3f} ms graph")
            del cache
    del model
    torch.cuda.empty_cache()
    return res


def run_e2e_bridge(torch, prompt_len=1024, max_new=64, seed=0, long_len=16384):
    """End-to-end greedy decode of a random-init Qwen2.5-1.5B-shape model (fp16,
    28 layers, 12 q / 2 kv heads, head_dim 128, vocab 151936) through the
    transformers bridge: prompt attention by SDPA, every decode step's
    attention by the split-K kernel over the paged cache (reference:
    benchmarks/int8_bridge/run_bridge.py).  Per cache variant: time to first
    token, time per output token with eager launches (the reference's way) and
    with the decode step replayed from a captured HIP graph, KV-cache bytes,
    and agreement with the FP16 variant (greedy match; mean |log p| difference
    on the FP16 continuation, teacher-forced).  A second setup decodes after a
    `long_len`-token prompt, graph replays only, where the cache's bytes are a
    visible share of each token's reads.  No checkpoint is available offline,
    so perplexity itself is not meaningful here and is not reported."""
    from pa_int8 import qwen_bridge as br

    model, cfg = _bridge_model(torch, seed)
    g = torch.Generator().manual_seed(seed)
    prompt = torch.randint(0, cfg.vocab_size, (1, prompt_len), generator=g).cuda()
    variants = ("fp16", "int8_per_token", "int8_per_tensor")
    new_cache = _bridge_cache

    res = {}
    ref_tokens = ref_lp = None
    # two passes over the variants; the first pays one-time costs (kernel loads, clock
    # ramp: a first FP16 pass measured 18.8 ms per token, later passes 13.3 ms)
    for rep in range(2):
        for variant in variants:
            cache = new_cache(variant, prompt_len + max_new)
            gen, ttft, tpot, _ = br.generate_greedy(model, prompt, max_new, cache)
            gen_g, _, tpot_g, _ = br.generate_greedy_graph(model, prompt, max_new, cache)
            if rep == 0:
                continue
            if ref_tokens is None:
                ref_tokens = gen
            lp = torch.tensor(br.teacher_force_logprobs(model, prompt, ref_tokens, cache))
            if ref_lp is None:
                ref_lp = lp
            res[variant] = dict(
                ttft_ms=round(ttft * 1e3, 2), tpot_ms=round(tpot * 1e3, 3),
                graph_tpot_ms=round(tpot_g * 1e3, 3),
                graph_tokens_match_eager=round(float((gen_g == gen).float().mean()), 4),
                kv_bytes=int(cache.kv_bytes_for_len(prompt_len + max_new)),
                greedy_match_vs_fp16=round(float((gen == ref_tokens).float().mean()), 4),
                mean_abs_dlogp_vs_fp16=round(float((lp - ref_lp).abs().mean()), 5))
            log(f"[bench] e2e bridge {variant}: TTFT {res[variant]['ttft_ms']} ms, "
                f"TPOT {res[variant]['tpot_ms']} ms eager, {res[variant]['graph_tpot_ms']} ms "
                f"graph, mean |dlogp| vs fp16 {res[variant]['mean_abs_dlogp_vs_fp16']}")
            del cache
    g = torch.Generator().manual_seed(seed + 1)
    prompt = torch.randint(0, cfg.vocab_size, (1, long_len), generator=g).cuda()
    long = {}
    for variant in ("fp16",) + variants:   # the first FP16 pass warms the long shapes
        cache = new_cache(variant, long_len + max_new)
        _, ttft, tpot_g, _ = br.generate_greedy_graph(model, prompt, max_new, cache)
        long[variant] = dict(ttft_ms=round(ttft * 1e3, 2), graph_tpot_ms=round(tpot_g * 1e3, 3),
                             kv_bytes=int(cache.kv_bytes_for_len(long_len + max_new)))
        del cache
    for variant in variants:
        log(f"[bench] e2e bridge, {long_len}-token prompt, {variant}: TTFT "
            f"{long[variant]['ttft_ms']} ms, TPOT {long[variant]['graph_tpot_ms']} ms graph")
    res[f"prompt_{long_len}"] = long
    res["setup"] = dict(model="random-init Qwen2.5-1.5B shape (no checkpoint offline), fp16",
                        prompt_len=prompt_len, long_prompt_len=long_len, max_new=max_new,
                        batch=1,
                        decode_attention="split-K kernel via transformers AttentionInterface",
                        timing="wall clock, synchronized: TTFT one prompt call; tpot_ms the "
                               "mean eager one-token model call (host launches of 28 layers "
                               "dominate it); graph_tpot_ms the mean per token over replays of "
                               "the captured decode step, each with one argmax and one id copy",
                        agreement="random weights give nearly flat logits, so one early argmax "
                                  "flip changes every later greedy token: greedy_match is "
                                  "informational; mean_abs_dlogp (teacher-forced on the FP16 "
                                  "continuation) measures the quantization error; "
                                  "graph_tokens_match_eager compares the graph replays' greedy "
                                  "tokens with the eager loop's on the same cache variant")
    del model
    torch.cuda.empty_cache()
    return res


def lognormal_lens(n, seed):
    import numpy as np

    rng = np.random.default_rng(seed)
    lens = np.clip(np.round(rng.lognormal(math.log(1024), 1.0, n)), 16, 32768).astype(int)
    return [int(x) for x in lens]


def steps_for(us_est, cap):
    return int(max(10, min(cap, 40_000 // max(1, us_est))))


def run_cfg5_counter_launches(torch, launches=8):
    """Config 5's four decode launches (32/8 and MQA 32/1, FP16 and INT8) for
    counter collection under rocprofv3 --pmc: plain launches, no timing and no
    gate.  The cases are built without torch index kernels: the block table
    and slot mapping are made on the host, and each INT8 cache is written by
    one call of the write kernel."""
    import math

    import numpy as np

    import pa_int8

    dev, bs, d = "cuda", 16, 128
    lens = lognormal_lens(256, seed=5)
    rng = np.random.default_rng(5)
    nblk = [(n + bs - 1) // bs for n in lens]
    nb = sum(nblk) + 1
    perm = rng.permutation(nb).astype(np.int32)
    bt_np = np.zeros((len(lens), max(nblk)), np.int32)
    off = 0
    for s_, k in enumerate(nblk):
        bt_np[s_, :k] = perm[off:off + k]
        off += k
    slots = np.concatenate([bt_np[s_, np.arange(n) // bs].astype(np.int64) * bs + np.arange(n) % bs
                            for s_, n in enumerate(lens)])
    bt, ctx = torch.from_numpy(bt_np).to(dev), torch.tensor(lens, dtype=torch.int32).to(dev)
    slots_t, T = torch.from_numpy(slots).to(dev), int(sum(lens))
    done = []
    for hkv in (8, 1):
        q = torch.randn((len(lens), 32, d), dtype=torch.float16, device=dev)
        out = torch.empty_like(q)
        for int8 in (False, True):
            if int8:
                kc = torch.zeros((nb, hkv, d // 8, bs, 8), dtype=torch.int8, device=dev)
                vc = torch.zeros((nb, hkv, d, bs), dtype=torch.int8, device=dev)
                ks = torch.zeros((nb, hkv, bs), dtype=torch.float32, device=dev)
                vs = torch.zeros_like(ks)
                k = torch.randn((T, hkv, d), dtype=torch.float16, device=dev)
                v = torch.randn((T, hkv, d), dtype=torch.float16, device=dev)
                pa_int8.reshape_and_cache_int8(k, v, kc, vc, ks, vs, slots_t)
                del k, v
                kw, variant = dict(k_scales=ks, v_scales=vs), "splitk_int8"
            else:
                kc = torch.randn((nb, hkv, d // 8, bs, 8), dtype=torch.float16, device=dev)
                vc = torch.randn((nb, hkv, d, bs), dtype=torch.float16, device=dev)
                kw, variant = {}, "splitk"
            torch.cuda.synchronize()
            for _ in range(launches):
                pa_int8.decode(variant, out, q, kc, vc, bt, ctx, 1.0 / math.sqrt(d), bs,
                               check=False, **kw)
            torch.cuda.synchronize()
            done.append(f"32/{hkv} {variant} x{launches}")
            log(f"[bench] cfg5 counter launches: 32/{hkv} {variant} x{launches}")
            del kc, vc, kw
            torch.cuda.empty_cache()
    return dict(launches=done, note="plain launches for rocprofv3 counters; not timed")


def run_counter_launches(torch, launches=8):
    """Plain launches (no timing, no gate) of the decode kernels whose stalls
    the counter summaries break down: config 2 `warp`, config 3 `warp_int8`
    and `warp`, config 4 32k `splitk_int8` and `splitk`, config 4's lengths at
    MQA 32/1 (both kinds), then config 5's four launches
    (run_cfg5_counter_launches)."""
    done = []
    for name, lens, h, hkv, variant, outliers in (
            ("cfg2", [4096] * 32, 12, 2, "warp", False),
            ("cfg3", [8192] * 64, 12, 2, "warp_int8", False),
            ("cfg3", [8192] * 64, 12, 2, "warp", False),
            ("cfg4 32k", [32768] * 8, 32, 8, "splitk_int8", True),
            ("cfg4 32k", [32768] * 8, 32, 8, "splitk", True),
            ("mqa 8x32k", [32768] * 8, 32, 1, "splitk", True),
            ("mqa 8x32k", [32768] * 8, 32, 1, "splitk_int8", True)):
        case = make_case(torch, lens, h, hkv, 128, 16, "cuda", 0, variant.endswith("int8"),
                         outliers, 1)
        fns, _ = decode_steps(torch, case, variant)
        for _ in range(launches):
            fns[0]()
        torch.cuda.synchronize()
        done.append(f"{name} {variant} x{launches}")
        log(f"[bench] counter launches: {done[-1]}")
        del case, fns
        torch.cuda.empty_cache()
    done += run_cfg5_counter_launches(torch, launches)["launches"]
    return dict(launches=done, note="plain launches for rocprofv3 counters; not timed")


def run_configs(torch, names, steps, warmup):
    import numpy as np

    out = {}
    if "cfg1" in names:
        rng = np.random.default_rng(0)
        lens = [int(x) for x in rng.integers(100, 513, size=4)]
        out["cfg1_tiny_mha_fp16"] = run_decode_cfg(torch, "cfg1", lens, 8, 8, 64, "warp",
                                                   steps, warmup)
    if "cfg3" in names:
        lens = [8192] * 64
        r8 = run_decode_cfg(torch, "cfg3", lens, 12, 2, 128, "warp_int8", steps_for(40, steps),
                            warmup, probe=True)
        r16 = run_decode_cfg(torch, "cfg3", lens, 12, 2, 128, "warp", steps_for(80, steps),
                             warmup, probe=True)
        out["cfg3_qwen_int8"] = r8
        out["cfg3_qwen_fp16_same_shape"] = r16
        out["cfg3_int8_over_fp16_latency"] = round(r8["us"] / r16["us"], 3)
    if "cfg3w" in names:
        out["cfg3w_quant_write"] = run_quant_write(torch, steps_for(120, steps), warmup)
    if "cfg4" in names:
        for ctx in (32768, 65536, 131072):
            lens = [ctx] * 8
            for variant in ("splitk", "splitk_int8"):
                est = ctx // 250 if variant == "splitk" else ctx // 500
                out[f"cfg4_llama_{ctx // 1024}k_{variant}"] = run_decode_cfg(
                    torch, f"cfg4 {ctx}", lens, 32, 8, 128, variant, steps_for(est, steps),
                    warmup, outliers=True)
                # the reference's partition size as BASELINE states config 4
                # (kernels/paged_attention_v4_splitk.cu:24), beside the planner's
                out[f"cfg4_llama_{ctx // 1024}k_{variant}_p512"] = run_decode_cfg(
                    torch, f"cfg4 {ctx} P=512", lens, 32, 8, 128, variant,
                    steps_for(est, steps), warmup, outliers=True, partition=512)
        # Config 4's lengths at MQA 32/1 (an extra line, not a BASELINE config):
        # 32 splits of 32 heads per sequence, the shape the two-level split
        # merge is for.
        for variant in ("splitk", "splitk_int8"):
            out[f"cfg4_mqa_32k_{variant}"] = run_decode_cfg(
                torch, "cfg4 MQA 32768", [32768] * 8, 32, 1, 128, variant,
                steps_for(40, steps), warmup, outliers=True)
    if "cfg5" in names:
        lens = lognormal_lens(256, seed=5)
        for hkv in (8, 1):
            for variant in ("splitk", "splitk_int8"):
                out[f"cfg5_ragged_32_{hkv}_{variant}"] = run_decode_cfg(
                    torch, "cfg5", lens, 32, hkv, 128, variant, steps_for(300, steps), warmup)
        out["cfg5_lens"] = dict(n=256, median=int(np.median(lens)), mean=float(np.mean(lens)),
                                max=int(max(lens)), sigma=1.0,
                                distribution="lognormal(ln 1024, 1.0) clipped [16, 32768], seed 5")
    if "cfg5counters" in names:
        out["cfg5_counter_launches"] = run_cfg5_counter_launches(torch)
    if "counters" in names:
        out["counter_launches"] = run_counter_launches(torch)
    if "refshapes" in names:
        rows = []
        for b, ctx, h, hkv, variant, a100_us, src in REF_SHAPES:
            r = run_decode_cfg(torch, f"ref b{b} ctx{ctx} {h}/{hkv}", [ctx] * b, h, hkv, 128,
                               variant, steps_for(max(5, ctx * b * hkv // 50_000), steps), warmup)
            r.update(a100_us=a100_us, a100_source=src,
                     a100_over_mi355x_latency=round(a100_us / r["us"], 2))
            rows.append(r)
        out["reference_shapes"] = dict(
            rows=rows, note="the reference's published A100-SXM4-80GB rows (1555 GB/s peak) at "
                            "the same shapes; kv_only_gbs counts K+V read once, as the "
                            "reference's GB/s does (bench_paged_decode.py:148-152)")
    if "e2e" in names:
        out["e2e_qwen_bridge"] = run_e2e_bridge(torch)
    if "e2elong" in names:
        out["e2e_long_context"] = run_e2e_long(torch)
    if "dense" in names:
        out["dense_cfg2_qwen_fp16"] = run_dense_baseline(torch, "cfg2", [4096] * 32, 12, 2, 128,
                                                         steps_for(150, steps), warmup)
        out["dense_cfg4_llama_32k_fp16"] = run_dense_baseline(
            torch, "cfg4 32768", [32768] * 8, 32, 8, 128, steps_for(700, steps), warmup,
            outliers=True)
    return out


# --------------------------------------------------------------------------- ceiling probes

def read_ceiling(torch, sizes=(134_217_728, 1_073_741_824)):
    """Practical HBM read rates from the benchmark's streaming-read probes: a
    contiguous sweep and chunks in random order -- 4 KB (one FP16 K or V tile
    of a block, D=128) and 2 KB (one INT8 tile) -- at the headline's size and
    at 1 GiB; best grid of a few, MALL-rotated."""
    from pa_int8._loader import probe_capi

    lib = probe_capi()
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    out = {}
    for nbytes in sizes:
        copies = copies_for(nbytes)
        bufs = [torch.ones(nbytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]
        res = {}
        for name, chunk in (("contiguous", 0), ("chunks_4k_random", 4096),
                            ("chunks_2k_random", 2048)):
            nchunk = nbytes // chunk if chunk else 0
            order = (torch.randperm(nchunk, device="cuda").to(torch.int32) if chunk else sink)
            best = 0.0
            for grid in (1024, 2048, 4096):
                def mk(b, grid=grid, chunk=chunk, nchunk=nchunk, order=order):
                    def f():
                        s = torch.cuda.current_stream().cuda_stream
                        if not chunk:
                            st = lib.pa_probe_read_contiguous(b.data_ptr(), nbytes,
                                                              sink.data_ptr(), grid, s)
                        else:
                            st = lib.pa_probe_read_chunks(b.data_ptr(), nbytes, order.data_ptr(),
                                                          nchunk, chunk, sink.data_ptr(), grid, s)
                        assert st == 0, st
                    return f
                steps = 40 if nbytes < (1 << 29) else 10
                ms = time_steps(torch, [mk(b) for b in bufs], steps, 4, 3)
                best = max(best, nbytes / (ms * 1e-3) / 1e9)
            res[name + "_gbs"] = round(best, 1)
        res["copies_rotated"] = copies
        out[str(nbytes)] = res
        del bufs
        torch.cuda.empty_cache()
        log(f"[bench] read ceiling at {nbytes} B: {res}")
    out["read_write_1gib"] = read_write_ceiling(torch)
    return out


def read_write_ceiling(torch, nbytes=1 << 30):
    """Mixed read + write rates (the roof the write kernel shares), in GB/s of
    bytes read plus bytes written: torch's same-dtype copy (1 byte read per
    byte written, about nbytes moved) and the library's read+write probe (2
    bytes read per byte written, the write kernel's ratio; 512 MiB read,
    256 MiB written into one of two alternating buffers, non-temporal loads and
    stores; best grid)."""
    from pa_int8._loader import probe_capi

    res = {}
    n_copy = nbytes // 2
    src = torch.ones(n_copy, dtype=torch.uint8, device="cuda")
    dsts = [torch.empty_like(src) for _ in range(2)]
    ms = time_steps(torch, [lambda dd=dd: dd.copy_(src) for dd in dsts], 20, 4, 3)
    res["copy_1to1_gbs"] = round(2 * n_copy / (ms * 1e-3) / 1e9, 1)
    del src, dsts
    lib = probe_capi()
    rd = 512 << 20
    src = torch.ones(rd, dtype=torch.uint8, device="cuda")
    # two destinations, alternating (as the write kernel's measurement)
    dsts = [torch.empty(rd // 2, dtype=torch.uint8, device="cuda") for _ in range(2)]
    best = 0.0
    for grid in (1024, 2048, 4096):
        def mk(dst, grid=grid):
            def f():
                st = lib.pa_probe_read_write(src.data_ptr(), rd, dst.data_ptr(), grid,
                                             torch.cuda.current_stream().cuda_stream)
                assert st == 0, st
            return f
        ms = time_steps(torch, [mk(dd) for dd in dsts], 20, 4, 3)
        best = max(best, (rd + rd // 2) / (ms * 1e-3) / 1e9)
    res["probe_2to1_gbs"] = round(best, 1)
    del src, dsts
    torch.cuda.empty_cache()
    log(f"[bench] read+write ceiling: {res}")
    return res


# --------------------------------------------------------------------------- CPU baseline

def cpu_baseline(seconds):
    """The numpy oracle on config-2-shaped sequences, for a bounded time."""
    import numpy as np

    from threadpoolctl import threadpool_limits

    from oracle import paged_decode_ref as ref
    from pa_int8 import metrics

    # the host threads this process may use: its CPU affinity, capped by the
    # OMP_NUM_THREADS the box sets (its CPU share)
    threads = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    with threadpool_limits(limits=threads, user_api="blas"):
        return _cpu_baseline_timed(seconds, threads, np, ref, metrics)


def _cpu_baseline_timed(seconds, threads, np, ref, metrics):
    rng = np.random.default_rng(0)
    n_seq, ctx, h, hkv, d = 2, 4096, 12, 2, 128
    lens = np.full(n_seq, ctx, np.int32)
    nblk = ctx // 16
    nb = n_seq * nblk + 1
    kc = rng.standard_normal((nb, hkv, d // 8, 16, 8), dtype=np.float32).astype(np.float16)
    vc = rng.standard_normal((nb, hkv, d, 16), dtype=np.float32).astype(np.float16)
    bt = rng.permutation(nb)[:n_seq * nblk].reshape(n_seq, nblk).astype(np.int32)
    q = rng.standard_normal((n_seq, h, d), dtype=np.float32).astype(np.float16)
    ref.paged_decode_attention(q, kc, vc, bt, lens, scale=1 / math.sqrt(d))   # warm-up
    calls, t0 = [], time.perf_counter()
    while time.perf_counter() - t0 < seconds or len(calls) < 5:
        t1 = time.perf_counter()
        ref.paged_decode_attention(q, kc, vc, bt, lens, scale=1 / math.sqrt(d))
        calls.append(time.perf_counter() - t1)
    dt = time.perf_counter() - t0
    med = float(np.median(calls))                  # seconds per call of n_seq sequences
    nbytes = metrics.decode_bytes([ctx] * n_seq, h, hkv, d)
    seq_ms = med / n_seq * 1e3
    return dict(value=round(nbytes / med / 1e9, 3), unit="GB/s", cores=int(threads),
                kind="port",
                sample=(f"numpy oracle on config-2 sequences (4096 tokens, 12/2 heads, D=128, "
                        f"fp16 widened to fp32), {n_seq} per call, median of {len(calls)} calls "
                        f"in {dt:.1f} s: {seq_ms:.2f} ms per sequence, {seq_ms * 32:.1f} ms "
                        f"per 32-sequence step; BLAS on {threads} threads, gather on one"),
                host_cpus=os.cpu_count(), cpu_model=_cpu_model())


def _cpu_model():
    """The host CPU's model name (lscpu, else /proc/cpuinfo), or None."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


# --------------------------------------------------------------------------- the line

LINE_LIMIT = 4096          # bytes of the final stdout line, kept well inside what the driver reads
HEADLINE_REPLAYS = 5       # the headline is the median of this many K-step graph replays


def _finite(x, nd):
    """x rounded to nd places, or None when it is missing or not finite."""
    if x is None:
        return None
    x = float(x)
    return round(x, nd) if math.isfinite(x) else None


def summarize(configs, peak_gbs=8000.0):
    """{name: [us, fraction of HBM peak]} for every timed decode or write entry
    of `configs`, and {name: INT8 us / FP16 us} for each shape timed both ways.
    Entries without a time (counter launches, length statistics) are left out;
    the end-to-end bridge is summarized by its time per output token."""
    out, ratios = {}, {}
    for name, r in configs.items():
        if not isinstance(r, dict):
            continue
        if "rows" in r:                                       # the reference's A100 shapes
            for row in r["rows"]:
                key = "ref_b{}_{}_{}_{}".format(row["seqs"], row["total_tokens"] // row["seqs"],
                                                row["heads"], row["variant"])
                out[key] = [_finite(row.get("us"), 2), _finite(row.get("frac_peak"), 4)]
            continue
        if "us" in r:
            frac = r.get("frac_peak")
            if frac is None and r.get("gbs") is not None:
                frac = r["gbs"] / peak_gbs
            out[name] = [_finite(r["us"], 2), _finite(frac, 4)]
            continue
        # the bridge: per variant, and per variant of a nested setup (a longer prompt)
        entries = []
        for k, v in r.items():
            if isinstance(v, dict):
                entries.append((f"{name}_{k}", v))
                entries += [(f"{name}_{k}_{k2}", v2) for k2, v2 in v.items() if isinstance(v2, dict)]
        for key, v in entries:
            for field in ("tpot_ms", "graph_tpot_ms"):
                if field in v:
                    out[f"{key}_{field}"] = [_finite(v[field], 3), None]
    for name, r in out.items():
        if "_int8" in name:
            fp_name = name.replace("_int8", "", 1)
            fp = out.get(fp_name)
            if fp and fp[0] and r[0]:
                ratios[fp_name] = round(r[0] / fp[0], 3)
    if configs.get("cfg3_qwen_int8") and configs.get("cfg3_qwen_fp16_same_shape"):
        ratios["cfg3_qwen"] = round(configs["cfg3_qwen_int8"]["us"]
                                    / configs["cfg3_qwen_fp16_same_shape"]["us"], 3)
    return out, ratios


def headline_line(steps, warmup, head, configs, traffic, cpu, peak_gbs=8000.0):
    """The one JSON object bench.py prints on stdout: the headline (config 2,
    single launch, FP16), its roofline, the CPU baseline and a [us, frac]
    summary of every other measurement.  Per-config detail (plans, gates,
    probes, ceilings) goes to the side file and the stderr lines instead, so
    the line stays under LINE_LIMIT bytes."""
    ms = head["us"] / 1e3
    nbytes = head["algo_bytes"]
    achieved = nbytes / (ms * 1e-3) / 1e9
    summary, ratios = summarize(configs, peak_gbs)
    cpu_short = None
    if cpu is not None:
        cpu_short = {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample") if k in cpu}
        if cpu.get("cpu_model"):
            cpu_short["cpu_model"] = cpu["cpu_model"]
    probe = head.get("address_stream_probe") or {}
    line = {
        "metric": METRIC,
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: fp16 N(0,1) q/K/V, random-permuted block tables; INT8 caches "
                "written by the quantize kernel",
        "config": {
            "workload": "BASELINE config 2: Qwen2.5-1.5B-shape GQA 12/2, head_dim 128, "
                        "block_size 16, 32 seqs x 4096 ctx, FP16 KV, single launch "
                        "(paged_decode_attn_warp)",
            "algo_bytes_per_step": nbytes,
            "timing": f"median of {HEADLINE_REPLAYS} replays of a {steps}-step HIP graph "
                      f"after {WARM_MS:g} ms of untimed replays, "
                      f"{head.get('cache_copies')} cache copies rotated, no host sync",
            "gate": {"ok": head.get("ok"),
                     "headroom": _finite((head.get("gate") or {}).get("headroom"), 4)},
            "decode_over_probe": _finite(probe.get("decode_over_probe"), 4),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": peak_gbs,
            "unit": "GB/s",
            "frac": round(achieved / peak_gbs, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu_short,
        "summary_us_frac": summary,
        "int8_over_fp16": ratios,
    }
    # Past the limit, the reference-shape rows go first, then the bridge's times,
    # then the latest entries (all stay in the side file and on stderr).
    for prefix in ("ref_", "e2e"):
        if len(json.dumps(line, allow_nan=False)) <= LINE_LIMIT:
            break
        for d in (summary, ratios):
            for k in [k for k in d if k.startswith(prefix)]:
                del d[k]
    while len(json.dumps(line, allow_nan=False)) > LINE_LIMIT and (summary or ratios):
        (ratios or summary).popitem()
    return line


def write_detail(path, detail):
    """The full per-config record beside the line (plans, gates, probes,
    ceilings); a failure to write it is reported and does not end the run."""
    if not path:
        return
    try:
        os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
        with open(path, "w") as f:
            json.dump(detail, f, indent=1, default=str)
        log(f"[bench] per-config detail written to {path}")
    except OSError as e:
        log(f"[bench] could not write {path}: {e}")


# --------------------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--configs", default="all",
                    help="comma list of " + ",".join(ALL_CONFIGS) + " or 'all'; also "
                    "cfg5counters (config 5's decode launches for rocprofv3 counters, untimed), "
                    "counters (those and the other kernels the counter summaries cover), "
                    "e2elong (the bridge's graph-replayed decode after a 16k prompt only, "
                    "for a kernel trace)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="time every measurement with plain launches instead of a HIP graph "
                         "(used under rocprofv3 counter collection)")
    ap.add_argument("--pmc-copy", action="store_true",
                    help="also run a 256 MiB device copy (calibrates FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--detail-out", default=os.path.join("gpurun_out", "bench_detail.json"),
                    help="file for the full per-config record ('' to skip)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              f"(the decode path runs on a single MI355X; it would shard by sequence or kv head, "
              f"with no communication)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    import pa_int8
    from pa_int8 import metrics

    pa_int8.ext()
    names = ALL_CONFIGS if args.configs == "all" else args.configs.split(",")
    global EAGER_ONLY
    EAGER_ONLY = args.eager

    # ---- headline: config 2, single-launch FP16
    lens = [4096] * 32
    head = run_decode_cfg(torch, "cfg2", lens, 12, 2, 128, "warp", args.steps, args.warmup,
                          replays=HEADLINE_REPLAYS, eager=True, eager_only=args.eager,
                          probe=True)
    head_sk = run_decode_cfg(torch, "cfg2", lens, 12, 2, 128, "splitk", args.steps, args.warmup)

    configs = {"cfg2_qwen_fp16_warp": head, "cfg2_qwen_fp16_splitk": head_sk}
    if args.pmc_copy:
        src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    configs.update(run_configs(torch, [n for n in names if n != "cfg2"], args.steps,
                               args.warmup))

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "pmc_traffic_cfg2_warp.md")
    if os.path.exists(tpath):
        # line "traffic_bytes_per_launch: N" of the committed counter summary
        for line in open(tpath):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = int(line.split(":")[1].strip())

    ceiling = read_ceiling(torch) if "ceiling" in names or args.configs == "all" else None

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline ...")
        cpu = cpu_baseline(args.cpu_seconds)

    line = headline_line(args.steps, args.warmup, head, configs, traffic, cpu)
    write_detail(args.detail_out, dict(line=line, configs=configs, read_ceiling=ceiling,
                                       cpu_baseline_full=cpu))
    print(json.dumps(line, allow_nan=False), flush=True)


if __name__ == "__main__":
    main()

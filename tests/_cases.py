"""Shared input builders for the decode / quant tests.

Inputs are drawn with numpy (seeded) and paged with the oracle's builders,
then copied to the device; the reference draws ``torch.randn`` on the device
instead (tests/test_paged_decode_attn.py:96-103), so the values differ but
the shapes, length patterns and layouts are the same.
"""

from __future__ import annotations

import math

import numpy as np

from oracle import paged_decode_ref as ref

HEAD_DIM = 128
BLOCK_SIZE = 16
X = 8
# every head_dim the library is built for (the reference takes any multiple
# of 8: kernels/paged_attention_v3_warp.cu:48-58; this build takes every
# multiple of 8 in [8, 256])
HEAD_DIMS = list(range(8, 257, 8))

# tests/test_paged_decode_attn.py:19-22
CONTEXT_LENS = [1, 15, 16, 17, 31, 128, 500]
GQA = [(8, 8), (8, 2), (8, 1), (16, 4)]
NUM_SEQS = [1, 3]
# :126
LONG_CONTEXT_LENS = [512, 513, 1024, 2000, 4096]

# tolerance stated by the build target (decode output in fp16)
ATOL = 2e-3
RTOL = 1e-2


def make_lens(clen, num_seqs):
    """Per-seq lengths varied within a batch, >= 1 (tests/test_paged_decode_attn.py:25-28)."""
    return np.array([max(1, clen - 5 * b) for b in range(num_seqs)], dtype=np.int32)


def fp16_case(num_seqs, lens, num_heads, num_kv_heads, head_dim=HEAD_DIM, block_size=BLOCK_SIZE,
              seed=0, k_mul=None, dtype=np.float16):
    """q, contiguous k/v and the paged fp16 cache built from them."""
    rng = np.random.default_rng(seed)
    max_len = int(max(lens))
    q = rng.standard_normal((num_seqs, num_heads, head_dim), dtype=np.float32).astype(dtype)
    k = rng.standard_normal((num_seqs, max_len, num_kv_heads, head_dim), dtype=np.float32)
    v = rng.standard_normal((num_seqs, max_len, num_kv_heads, head_dim), dtype=np.float32)
    if k_mul is not None:
        k = k * k_mul
    k = k.astype(dtype)
    v = v.astype(dtype)
    kc, vc, bt = ref.build_paged_kv_cache(k, v, lens, block_size=block_size, x=X, rng=rng)
    return dict(q=q, k=k, v=v, lens=np.asarray(lens, dtype=np.int32), k_cache=kc, v_cache=vc,
                block_table=bt, scale=1.0 / math.sqrt(head_dim), block_size=block_size)


def int8_case(num_seqs, lens, num_heads, num_kv_heads, mode="per_token", head_dim=HEAD_DIM,
              block_size=BLOCK_SIZE, seed=0, k_mul=None):
    c = fp16_case(num_seqs, lens, num_heads, num_kv_heads, head_dim, block_size, seed, k_mul)
    rng = np.random.default_rng(seed + 1)
    kc, vc, ks, vs, bt = ref.build_paged_kv_cache_int8(c["k"], c["v"], c["lens"],
                                                       block_size=block_size, x=X, mode=mode,
                                                       rng=rng)
    c.update(k_cache8=kc, v_cache8=vc, k_scales=ks, v_scales=vs, block_table8=bt)
    return c


def oracle_fp16(c):
    return ref.paged_decode_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"],
                                      c["lens"], scale=c["scale"], block_size=c["block_size"])


def oracle_int8(c):
    kd, vd = ref.dequantize_kv(c["k_cache8"], c["v_cache8"], c["k_scales"], c["v_scales"])
    return ref.paged_decode_attention(c["q"], kd, vd, c["block_table8"], c["lens"],
                                      scale=c["scale"], block_size=c["block_size"])


def subset_oracle(case, seqs):
    """The oracle's output for sequences `seqs` of a device case built by
    bench.make_case: their blocks are gathered on the device, copied to the
    host and renumbered, so the oracle sees only what it needs."""
    import torch

    bs, lens = case["bs"], case["lens"]
    kc, vc, ks, vs = case["caches"][0]
    nblk = [(lens[s] + bs - 1) // bs for s in seqs]
    ids = torch.cat([case["bt"][s, :n].long() for s, n in zip(seqs, nblk)])
    bt = np.zeros((len(seqs), max(nblk)), np.int32)
    off = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = np.arange(off, off + n)
        off += n
    k = kc.index_select(0, ids).cpu().numpy()
    v = vc.index_select(0, ids).cpu().numpy()
    if ks is not None:
        k, v = ref.dequantize_kv(k, v, ks.index_select(0, ids).cpu().numpy(),
                                 vs.index_select(0, ids).cpu().numpy())
    q = case["q"].cpu().numpy()[list(seqs)]
    sub_lens = np.array([lens[s] for s in seqs], np.int32)
    return ref.paged_decode_attention(q, k, v, bt, sub_lens, scale=case["scale"], block_size=bs)


def assert_close(out, expect, atol=ATOL, rtol=RTOL, what=""):
    """Elementwise |out - expect| <= atol + rtol * |expect|.  Returns the
    headroom ratio max(|out - expect| / (atol + rtol * |expect|)): 1.0 is the
    edge of the tolerance, small values mean a wide margin."""
    out = np.asarray(out, dtype=np.float32)
    expect = np.asarray(expect, dtype=np.float32)
    err = np.abs(out - expect)
    bound = atol + rtol * np.abs(expect)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - rtol * np.abs(expect)), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.size} elements outside atol={atol} rtol={rtol}; "
            f"worst at {i}: got {out[i]}, want {expect[i]}, max|err|={err.max():.3e}")
    return float((err / bound).max()) if err.size else 0.0


def record_headroom(config, what, ratio, **extra):
    """Appends one line of JSON (config, case, headroom ratio) to the file named
    by PA_PARITY_LOG, when it is set; the full-size parity tests call it."""
    import json
    import os

    path = os.environ.get("PA_PARITY_LOG")
    line = dict(config=config, case=what, headroom=round(ratio, 4), **extra)
    print("[parity]", json.dumps(line), flush=True)
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(line) + "\n")

"""Write golden vectors of the reference's INT8 quantizers.

Runs ONLY in the development container, where the reference checkout exists
at /root/reference.  It imports ``quantize_per_token``, ``quantize_per_tensor``
and ``dequantize_kv`` from the reference's tests/paged_decode_attn.py
(:106-121, :202-216) and stores inputs and outputs as data in
``quant_golden.npz`` next to this script.  The GPU box never runs this file;
the tests read only the .npz.

Why an import: the degenerate cases (amax == 0, an fp16 scale that is
subnormal or rounds to 0, NaN from 0/0 cast to int8, rows holding NaN or
+-inf, whose amax propagates the NaN or infinity) are decided by torch's own
arithmetic and casts, which no closed form fixes.  The ordinary rows are
stored alongside them so the same fixture also pins the common path.  The
bfloat16 rows (stored as their uint16 bit patterns) pin the quantizer on
bf16 input, where the clamp at 1e-8 and the scale's rounding happen in
bfloat16.

    python tests/golden/make_quant_golden.py [--reference /root/reference]
"""

from __future__ import annotations

import argparse
import importlib.util
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def load_reference(root):
    path = os.path.join(root, "tests", "paged_decode_attn.py")
    spec = importlib.util.spec_from_file_location("reference_paged_decode_attn", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def fp16_rows(rng, d):
    rows = [rng.standard_normal(d) for _ in range(24)]
    rows.append(np.zeros(d))                                      # amax = 0
    r = np.zeros(d); r[:3] = [1e-7, -3e-7, 6e-8]; rows.append(r)  # scale rounds to 0
    rows.append(rng.standard_normal(d) * 2e-3)                    # subnormal fp16 scale
    rows.append(rng.standard_normal(d) * 5e-5)
    r = np.zeros(d)
    r[:12] = [127, 2.5, 3.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -126.5, 63.5, -0.49]
    rows.append(r)                                                # exact ties, scale 1
    r = rng.standard_normal(d); r[0] = 1000.0; rows.append(r)    # outlier saturates
    r = np.full(d, -65504.0); r[1::2] = 65504.0; rows.append(r)   # fp16 max
    rows.append(rng.standard_normal(d) * 300.0)
    r = rng.standard_normal(d); r[5] = -7.0; rows.append(r)      # negative amax
    return np.stack(rows).astype(np.float16)


def nonfinite_rows(rng, d):
    """Rows holding NaN or +-inf among ordinary values (appended after the
    rows above, from their own generator, so the other arrays are unchanged)."""
    rows = []
    r = rng.standard_normal(d); r[7] = np.nan; rows.append(r)
    r = rng.standard_normal(d); r[0] = np.inf; rows.append(r)
    r = rng.standard_normal(d); r[d - 1] = -np.inf; rows.append(r)
    r = rng.standard_normal(d); r[3], r[9] = np.inf, np.nan; rows.append(r)
    rows.append(np.full(d, np.nan))
    r = np.zeros(d); r[11] = -np.inf; rows.append(r)
    return np.stack(rows)


def bf16_bits(x):
    """float32 -> bfloat16 bit patterns (uint16), through torch's own rounding."""
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def bf16_rows(rng, d):
    rows = [rng.standard_normal(d) for _ in range(16)]
    rows.append(np.zeros(d))                                      # amax = 0 -> clamp 1e-8
    rows.append(rng.standard_normal(d) * 1e-10)                   # amax below the clamp
    rows.append(rng.standard_normal(d) * 3e-9)
    rows.append(rng.standard_normal(d) * 1e30)                    # huge scales
    r = np.zeros(d)
    r[:12] = [127, 2.5, 3.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -126.5, 63.5, -0.49]
    rows.append(r)                                                # ties at scale 1
    r = rng.standard_normal(d); r[0] = 1000.0; rows.append(r)
    rows.append(rng.standard_normal(d) * 300.0)
    return np.concatenate([np.stack(rows), nonfinite_rows(rng, d)])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--out", default=os.path.join(HERE, "quant_golden.npz"))
    args = ap.parse_args()
    ref = load_reference(args.reference)
    rng = np.random.default_rng(2024)
    d = 128

    x16 = fp16_rows(rng, d)                                   # [R, D] fp16
    q16, s16 = ref.quantize_per_token(torch.from_numpy(x16), dim=-1)
    x32 = (rng.standard_normal((8, d)) * np.array([1, 1e-3, 50, 1, 1, 1, 1e-30, 1])[:, None])
    x32 = x32.astype(np.float32)
    x32[4] = 0.0
    q32, s32 = ref.quantize_per_token(torch.from_numpy(x32), dim=-1)
    # per-tensor on a small [S, L, H, D] block and on an all-zero block
    xt = (rng.standard_normal((2, 5, 2, d)) * 0.7).astype(np.float16)
    qt, st = ref.quantize_per_tensor(torch.from_numpy(xt))
    qz, sz = ref.quantize_per_tensor(torch.zeros((1, 2, 1, d), dtype=torch.float16))
    # dequantize_kv on a small random cache
    nb, h, bs = 3, 2, 16
    kc = rng.integers(-127, 128, size=(nb, h, d // 8, bs, 8)).astype(np.int8)
    vc = rng.integers(-127, 128, size=(nb, h, d, bs)).astype(np.int8)
    ks = rng.random((nb, h, bs)).astype(np.float32)
    vs = rng.random((nb, h, bs)).astype(np.float32)
    kd, vd = ref.dequantize_kv(torch.from_numpy(kc), torch.from_numpy(vc), torch.from_numpy(ks),
                               torch.from_numpy(vs))
    # rows with NaN / +-inf (fp16), and bf16 rows, from a second generator
    rng2 = np.random.default_rng(2025)
    xnf = nonfinite_rows(rng2, d).astype(np.float16)
    qnf, snf = ref.quantize_per_token(torch.from_numpy(xnf), dim=-1)
    xb = bf16_bits(bf16_rows(rng2, d))
    qb, sb = ref.quantize_per_token(torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16),
                                    dim=-1)

    np.savez_compressed(
        args.out,
        x16=x16, q16=q16.numpy(), s16=s16.numpy(),
        x32=x32, q32=q32.numpy(), s32=s32.numpy(),
        xt=xt, qt=qt.numpy(), st=np.float32(st.item()),
        qz=qz.numpy(), sz=np.float32(sz.item()),
        kc=kc, vc=vc, ks=ks, vs=vs, kd=kd.numpy(), vd=vd.numpy(),
        xnf=xnf, qnf=qnf.numpy(), snf=snf.numpy(),
        xb16_bits=xb, qb16=qb.numpy(), sb16=sb.numpy(),
        torch_version=np.array(torch.__version__),
    )
    print("wrote", args.out)


if __name__ == "__main__":
    main()

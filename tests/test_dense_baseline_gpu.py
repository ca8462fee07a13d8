"""The dense baseline the benchmark times beside the paged kernel computes the
same function.

bench.py times SDPA over K/V gathered out of the paged cache into contiguous
[S, H, ctx, D] tensors and repeated over the GQA group (the reference's dense
ceiling, benchmarks/bench_paged_decode.py:131-145).  Here the same gather
(bench.gather_dense) and the same call (bench.dense_attention_fn) run on a
config-2 slice and a config-4 32k slice; the dense output, the paged
single-launch and split-K outputs and the CPU oracle must agree within
atol 2e-3 / rtol 1e-2 (fp16 outputs).  Each comparison's max |difference| and
headroom are recorded.
"""

import numpy as np
import pytest
import torch

from _cases import assert_close, record_headroom, subset_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _lib(built):
    import pa_int8

    pa_int8.ext()


@pytest.mark.parametrize("config,lens,h,hkv,outliers", [
    ("cfg2", [4096] * 4, 12, 2, False),
    ("cfg4", [32768] * 2, 32, 8, True),
])
def test_dense_baseline_matches_paged_and_oracle(config, lens, h, hkv, outliers):
    import bench
    import pa_int8

    case = bench.make_case(torch, lens, h, hkv, 128, 16, "cuda", 0, False, outliers, 1)
    k, v = bench.gather_dense(torch, case, lens, h)
    assert k.shape == (len(lens), h, lens[0], 128) and v.shape == k.shape
    q = case["q"].unsqueeze(2)
    dense, impl = bench.dense_attention_fn(torch, q, k, v, case["scale"])
    got_dense = dense().squeeze(2).float().cpu().numpy()
    torch.cuda.synchronize()
    assert np.isfinite(got_dense).all()
    seqs = list(range(len(lens)))
    want = subset_oracle(case, seqs)
    r = assert_close(got_dense, want, what=f"{config} dense ({impl}) vs oracle")
    record_headroom(config, f"dense baseline ({impl}) vs oracle", r,
                    max_abs_diff=float(np.abs(got_dense - want).max()))
    kc, vc = case["caches"][0][0], case["caches"][0][1]
    for variant in ("warp", "splitk"):
        out = torch.empty_like(case["q"])
        pa_int8.decode(variant, out, case["q"], kc, vc, case["bt"], case["ctx"], case["scale"],
                       16, check=False)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        r1 = assert_close(got, got_dense, what=f"{config} paged {variant} vs dense")
        r2 = assert_close(got, want, what=f"{config} paged {variant} vs oracle")
        record_headroom(config, f"paged {variant} vs dense baseline", r1,
                        max_abs_diff=float(np.abs(got - got_dense).max()))
        record_headroom(config, f"paged {variant} vs oracle (dense test)", r2)

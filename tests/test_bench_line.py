"""The benchmark's stdout line: one strict-JSON object, small enough for the
driver to read, carrying the headline, its roofline and the CPU baseline
(the reference's bench prints a short table per variant,
benchmarks/bench_paged_decode.py:63-78,148-152)."""

import json
import math

import bench


def _decode_entry(variant, us, algo_bytes, seqs, ctx, heads, probe=True):
    """A result of the shape run_decode_cfg returns, every detail field filled."""
    gbs = algo_bytes / (us * 1e-6) / 1e9
    r = dict(variant=variant, us=us, algo_bytes=algo_bytes, gbs=round(gbs, 1),
             frac_peak=round(gbs / 8000.0, 4), kv_only_gbs=round(gbs * 0.999, 1), seqs=seqs,
             heads=heads, head_dim=128, total_tokens=seqs * ctx, partition_tokens=2048,
             splits=2, cache_copies=8, steps=200, ok=True,
             gate=dict(ok=True, headroom=0.0146, seqs_checked=7,
                       tolerance="atol 0.002 rtol 0.01, fp32 dense torch attention"),
             eager_us=us * 1.2)
    if probe:
        r["address_stream_probe"] = dict(
            us=us / 1.08, gbs=gbs * 1.08, decode_over_probe=1.08,
            what="the decode launch's own loads (same plan, caches and block table) with the "
                 "attention math replaced by a checksum")
    return r


def _full_configs():
    """Every entry a default run records, with long detail fields."""
    c = {"cfg2_qwen_fp16_warp": _decode_entry("warp", 25.31, 134447232, 32, 4096, "12/2"),
         "cfg2_qwen_fp16_splitk": _decode_entry("splitk", 29.56, 134447232, 32, 4096, "12/2"),
         "cfg1_tiny_mha_fp16": _decode_entry("warp", 4.77, 343296, 4, 300, "8/8", False),
         "cfg3_qwen_int8": _decode_entry("warp_int8", 47.43, 277348608, 64, 8192, "12/2"),
         "cfg3_qwen_fp16_same_shape": _decode_entry("warp", 83.97, 537395456, 64, 8192,
                                                    "12/2")}
    c["cfg3_int8_over_fp16_latency"] = 0.565
    c["cfg3w_quant_write"] = dict(
        us=166.4, algo_bytes=817889280, gbs=4915.2, frac_peak=0.6144, tokens=524288, kv_heads=2,
        head_dim=128, slot_pattern="per-sequence block runs (prefill), block ids randomly "
        "permuted", destination_copies=2, steps=200, ok=True, gate="x" * 120,
        write_stream_probe=dict(us=160.0, gbs=5100.0, write_over_probe=1.04, note="y" * 160))
    for ctx in (32, 64, 128):
        for v in ("splitk", "splitk_int8"):
            c[f"cfg4_llama_{ctx}k_{v}"] = _decode_entry(v, 165.0 * ctx / 32, 1 << 30, 8,
                                                        ctx * 1024, "32/8", False)
            c[f"cfg4_llama_{ctx}k_{v}_p512"] = _decode_entry(v, 170.0 * ctx / 32, 1 << 30, 8,
                                                             ctx * 1024, "32/8", False)
    for v in ("splitk", "splitk_int8"):
        c[f"cfg4_mqa_32k_{v}"] = _decode_entry(v, 37.1, 134545664, 8, 32768, "32/1", False)
        for hkv in (8, 1):
            c[f"cfg5_ragged_32_{hkv}_{v}"] = _decode_entry(v, 278.5 / hkv, 211e6 / hkv, 256,
                                                           1700, f"32/{hkv}", False)
    c["cfg5_lens"] = dict(n=256, median=1024, mean=1700.0, max=32768, sigma=1.0,
                          distribution="lognormal(ln 1024, 1.0) clipped [16, 32768], seed 5")
    rows = []
    for b, ctx, h, hkv, v, a100, src in bench.REF_SHAPES:
        r = _decode_entry(v, 50.0, 1 << 28, b, ctx, f"{h}/{hkv}", False)
        r.update(a100_us=a100, a100_source=src, a100_over_mi355x_latency=round(a100 / 50.0, 2))
        rows.append(r)
    c["reference_shapes"] = dict(rows=rows, note="z" * 200)
    c["e2e_qwen_bridge"] = {v: dict(ttft_ms=80.0, tpot_ms=12.1, graph_tpot_ms=0.912,
                                    graph_tokens_match_eager=1.0, kv_bytes=1 << 24,
                                    greedy_match_vs_fp16=1.0, mean_abs_dlogp_vs_fp16=0.001)
                            for v in ("fp16", "int8_per_token", "int8_per_tensor")}
    c["e2e_qwen_bridge"]["prompt_16384"] = {
        v: dict(ttft_ms=900.0, graph_tpot_ms=1.01, kv_bytes=1 << 28)
        for v in ("fp16", "int8_per_token", "int8_per_tensor")}
    c["e2e_qwen_bridge"]["setup"] = dict(model="w" * 300)
    for name in ("dense_cfg2_qwen_fp16", "dense_cfg4_llama_32k_fp16"):
        c[name] = dict(impl="sdpa", us=340.85, bytes_read=806e6, gbs=2363.0,
                       paged_algo_bytes=134447232, max_abs_diff_vs_paged_warp=6.1e-5, seqs=32,
                       heads="12/2", context=4096, steps=200, note="n" * 90)
    return c


def _cpu():
    return dict(value=0.858, unit="GB/s", cores=16, kind="port",
                sample="s" * 260, host_cpus=128, cpu_model="AMD EPYC 9575F 64-Core Processor")


def test_line_is_strict_json_under_the_limit():
    configs = _full_configs()
    full = json.dumps(configs)
    assert len(full) > 4 * bench.LINE_LIMIT          # the detail alone would not fit
    line = bench.headline_line(20, 5, configs["cfg2_qwen_fp16_warp"], configs, 136804814,
                               _cpu())
    s = json.dumps(line, allow_nan=False)
    assert len(s.encode()) <= bench.LINE_LIMIT, len(s)
    back = json.loads(s)
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
              "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
              "roofline", "cpu_baseline"):
        assert k in back, k
    assert back["steps"] == 20 and back["warmup"] == 5 and back["n_gpus"] == 1
    # value is the headline entry's algorithmic bytes over its time
    assert math.isclose(back["value"], 134447232 / 25.31e-6 / 1e9, rel_tol=1e-4)
    assert math.isclose(back["ms_per_step"], 0.02531)
    rf = back["roofline"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert math.isclose(rf["frac"], rf["achieved"] / rf["peak"], rel_tol=1e-3)
    assert rf["traffic"] == 136804814
    assert back["cpu_baseline"]["kind"] == "port" and back["cpu_baseline"]["cores"] == 16
    summ = back["summary_us_frac"]
    for name in ("cfg3_qwen_int8", "cfg3w_quant_write", "cfg4_llama_128k_splitk_int8",
                 "cfg4_llama_32k_splitk_p512", "cfg5_ragged_32_1_splitk_int8",
                 "dense_cfg2_qwen_fp16"):
        assert len(summ[name]) == 2 and summ[name][0] > 0, name
    assert "cfg5_lens" not in summ and "cfg3_int8_over_fp16_latency" not in summ
    e2e = bench.summarize(configs)[0]   # the bridge's times per output token, both setups
    assert e2e["e2e_qwen_bridge_int8_per_token_graph_tpot_ms"] == [0.912, None]
    assert e2e["e2e_qwen_bridge_fp16_tpot_ms"] == [12.1, None]
    assert e2e["e2e_qwen_bridge_prompt_16384_int8_per_tensor_graph_tpot_ms"] == [1.01, None]
    assert not [k for k in e2e if k.startswith("e2e_qwen_bridge_setup")]
    assert back["int8_over_fp16"]["cfg3_qwen"] == 0.565
    assert "cfg4_llama_64k_splitk_p512" in back["int8_over_fp16"]
    assert math.isclose(back["int8_over_fp16"]["cfg4_llama_32k_splitk"],
                        configs["cfg4_llama_32k_splitk_int8"]["us"]
                        / configs["cfg4_llama_32k_splitk"]["us"], rel_tol=1e-3)


def test_line_survives_missing_and_non_finite_values():
    configs = _full_configs()
    head = dict(configs["cfg2_qwen_fp16_warp"])
    head["gate"] = dict(head["gate"], headroom=float("nan"))
    head["address_stream_probe"] = dict(head["address_stream_probe"],
                                        decode_over_probe=float("inf"))
    configs["cfg5_ragged_32_8_splitk"]["us"] = float("nan")
    configs["cfg3w_quant_write"]["frac_peak"] = None
    line = bench.headline_line(20, 5, head, configs, None, None)
    s = json.dumps(line, allow_nan=False)               # raises on any NaN or inf left
    back = json.loads(s)
    assert back["cpu_baseline"] is None and back["roofline"]["traffic"] is None
    assert back["config"]["gate"]["headroom"] is None
    assert back["summary_us_frac"]["cfg5_ragged_32_8_splitk"][0] is None
    assert back["summary_us_frac"]["cfg3w_quant_write"][1] is not None   # from its GB/s


def test_line_drops_reference_rows_first_when_too_long():
    configs = _full_configs()
    for i in range(60):                                  # a run with many extra entries
        configs[f"extra_measurement_with_a_long_name_{i:03d}"] = dict(us=10.0 + i,
                                                                      frac_peak=0.5)
    line = bench.headline_line(20, 5, configs["cfg2_qwen_fp16_warp"], configs, 1, _cpu())
    s = json.dumps(line, allow_nan=False)
    assert len(s.encode()) <= bench.LINE_LIMIT
    keys = line["summary_us_frac"]
    assert not any(k.startswith("ref_") for k in keys)
    assert "cfg2_qwen_fp16_warp" in keys and "cfg4_llama_128k_splitk" in keys
    assert json.loads(s)["value"] == line["value"]

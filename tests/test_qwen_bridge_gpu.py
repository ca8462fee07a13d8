"""The transformers bridge on the GPU (counterpart of the reference's gate 2,
tests/test_int8_bridge.py:131-185, which needs Qwen weights that are not
available offline): a random-init Qwen2 with the Qwen2.5-1.5B attention shape
runs prompt + decode through the paged cache and the split-K kernels, and its
per-token log-probabilities are compared with the same model's dense fp32
attention (``reference_attention``) on the same tokens."""

import numpy as np
import pytest
import torch

from _qwen import LOGP_MAX, tiny_qwen

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")


def _tokens(n, seed, vocab=512):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (1, n), generator=g).cuda()


@pytest.fixture(scope="module")
def model():
    from pa_int8 import qwen_bridge as br

    br.register()
    return tiny_qwen(dtype=torch.float16, device="cuda")


def _bridge_logprobs(model, prompt, cont, variant):
    from pa_int8 import PagedKVCache
    from pa_int8 import qwen_bridge as br

    model.set_attn_implementation(br.ATTN_NAME)
    cfg = model.config
    cache = PagedKVCache(num_layers=cfg.num_hidden_layers, num_kv_heads=cfg.num_key_value_heads,
                         head_dim=cfg.hidden_size // cfg.num_attention_heads,
                         max_len=prompt.shape[1] + cont.shape[1], variant=variant)
    return np.array(br.teacher_force_logprobs(model, prompt, cont, cache)), cache


def _reference_logprobs(model, prompt, cont):
    from pa_int8 import qwen_bridge as br

    model.set_attn_implementation(br.REFERENCE_ATTN_NAME)
    return np.array(br.reference_logprobs(model, prompt, cont))


@pytest.mark.parametrize("plen,n", [(40, 24), (301, 8), (16, 17)])
def test_fp16_bridge_matches_dense_reference(model, plen, n):
    prompt, cont = _tokens(plen, plen), _tokens(n, plen + 1)
    got, cache = _bridge_logprobs(model, prompt, cont, "fp16")
    want = _reference_logprobs(model, prompt, cont)
    err = np.abs(got - want)
    print(f"fp16 bridge, prompt {plen} + {n}: max |dlogp| {err.max():.2e}, mean {err.mean():.2e}")
    assert err.max() < LOGP_MAX
    # every continuation token but the last (whose logits nobody reads) is fed
    assert cache.lengths == [plen + n - 1] * model.config.num_hidden_layers


def test_greedy_generation_follows_the_reference(model):
    """Every token the bridge generates greedily is the reference's argmax at
    that position, wherever the reference's top-2 margin is clear."""
    from pa_int8 import PagedKVCache
    from pa_int8 import qwen_bridge as br

    prompt = _tokens(33, 7)
    model.set_attn_implementation(br.ATTN_NAME)
    cfg = model.config
    cache = PagedKVCache(num_layers=cfg.num_hidden_layers, num_kv_heads=cfg.num_key_value_heads,
                         head_dim=128, max_len=33 + 20, variant="fp16")
    gen, ttft, tpot, steps = br.generate_greedy(model, prompt, 20, cache)
    assert gen.shape == (1, 20) and ttft > 0 and tpot > 0 and len(steps) == 20
    model.set_attn_implementation(br.REFERENCE_ATTN_NAME)
    ids = torch.cat([prompt, gen[:, :-1]], dim=1)
    with torch.no_grad():
        logits = model(input_ids=ids, use_cache=False).logits[0, 32:].float()
    top2 = logits.topk(2, dim=-1)
    clear = (top2.values[:, 0] - top2.values[:, 1]) > 0.05
    agree = top2.indices[:, 0] == gen[0]
    assert bool((agree | ~clear).all()), (agree.cpu().tolist(), clear.cpu().tolist())
    assert int(clear.sum()) >= 10


def test_int8_bridges_track_fp16(model):
    """INT8 caches (per token, per tensor) against the FP16 bridge on the same
    tokens; per-token scales are at least as close as one per-tensor scale."""
    prompt, cont = _tokens(64, 11), _tokens(32, 12)
    fp, _ = _bridge_logprobs(model, prompt, cont, "fp16")
    err = {}
    for variant in ("int8_per_token", "int8_per_tensor"):
        lp, _ = _bridge_logprobs(model, prompt, cont, variant)
        err[variant] = np.abs(lp - fp)
        print(f"{variant}: max |dlogp| vs fp16 {err[variant].max():.3e}, "
              f"mean {err[variant].mean():.3e}")
    assert err["int8_per_token"].max() < 0.5
    assert err["int8_per_token"].mean() < 0.1
    assert err["int8_per_token"].mean() <= err["int8_per_tensor"].mean() * 1.1 + 1e-3


@pytest.fixture(scope="module")
def model_bf16():
    from pa_int8 import qwen_bridge as br

    br.register()
    return tiny_qwen(dtype=torch.bfloat16, device="cuda")


def test_bf16_model_through_the_bridge(model_bf16):
    """The reference's runner loads the model in bfloat16
    (benchmarks/int8_bridge/run_bridge.py:99).  The bridge then hands the
    kernel an fp16 copy of the query; the fp16 cache converts the bf16 K/V
    (exactly), and the INT8 caches quantize them directly, as
    quantize_per_token does on bf16.  The fp16 cache must match the dense fp32
    reference on the same model; the INT8 caches must track the fp16 cache as
    they do on an fp16 model."""
    prompt, cont = _tokens(48, 21), _tokens(16, 22)
    want = _reference_logprobs(model_bf16, prompt, cont)
    fp, cache = _bridge_logprobs(model_bf16, prompt, cont, "fp16")
    err = np.abs(fp - want)
    print(f"bf16 model, fp16 cache: max |dlogp| vs dense fp32 {err.max():.2e}, "
          f"mean {err.mean():.2e}")
    assert cache.lengths == [48 + 16 - 1] * model_bf16.config.num_hidden_layers
    assert err.max() < 2 * LOGP_MAX
    for variant in ("int8_per_token", "int8_per_tensor"):
        lp, cache = _bridge_logprobs(model_bf16, prompt, cont, variant)
        assert cache.k_scales.dtype == torch.float32
        e = np.abs(lp - fp)
        print(f"bf16 model, {variant}: max |dlogp| vs fp16 cache {e.max():.3e}, "
              f"mean {e.mean():.3e}")
        assert e.max() < 0.5
        assert e.mean() < 0.1


@pytest.mark.parametrize("variant", ["fp16", "int8_per_token", "int8_per_tensor"])
def test_graph_decode_matches_eager(model, variant):
    """The captured decode step (DecodeGraph), replayed token after token with
    eager work (argmax, id copy, logits read back) between the replays, gives
    the eager bridge's logits at every step, the same greedy tokens, and the
    same cache contents and lengths."""
    from pa_int8 import PagedKVCache
    from pa_int8 import qwen_bridge as br

    model.set_attn_implementation(br.ATTN_NAME)
    cfg = model.config
    prompt, n = _tokens(37, 3), 14
    caches = [PagedKVCache(num_layers=cfg.num_hidden_layers, num_kv_heads=cfg.num_key_value_heads,
                           head_dim=128, max_len=37 + n + 5, variant=variant) for _ in range(2)]
    gen_e, _, _, seen_e = br.generate_greedy(model, prompt, n, caches[0])
    gen_g, ttft, tpot, seen_g = br.generate_greedy_graph(model, prompt, n, caches[1],
                                                         keep_logits=True)
    assert ttft > 0 and tpot > 0 and len(seen_g) == n
    err = max(float((a - b).abs().max()) for a, b in zip(seen_e, seen_g))
    print(f"{variant}: graph vs eager max |dlogit| over {n} steps {err:.2e}")
    assert err < 1e-2
    assert torch.equal(gen_e, gen_g)
    assert caches[0].lengths == caches[1].lengths == [37 + n - 1] * cfg.num_hidden_layers
    for name in caches[0].layout.tensors():
        a, b = getattr(caches[0], name), getattr(caches[1], name)
        if a.dtype == torch.int8:   # quantized from K/V that may differ in the last bit
            assert int((a.int() - b.int()).abs().max()) <= 1, name
        else:
            assert torch.allclose(a.float(), b.float(), atol=1e-2, rtol=1e-2), name

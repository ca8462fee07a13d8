"""Host-side checks of the transformers bridge (pa_int8.qwen_bridge), no GPU.

The GPU tests compare the bridge (paged cache + decode kernels) with
``reference_attention``, a dense fp32 causal attention over the same
model.  Here that checker is pinned against the oracle's float64 dense
attention, the incremental and whole-sequence reference paths are shown to
agree, and a planted one-position cache mistake is shown to exceed the
tolerance the GPU tests use.  The bridge's own entry checks are covered too.
"""

import numpy as np
import pytest
import torch

from oracle import paged_decode_ref as ref

transformers = pytest.importorskip("transformers")

from _qwen import LOGP_MAX, tiny_qwen  # noqa: E402


@pytest.mark.parametrize("lq,lk", [(1, 37), (20, 20), (5, 33)])
def test_reference_attention_matches_float64_oracle(lq, lk):
    from pa_int8 import qwen_bridge as br

    rng = np.random.default_rng(lq * 100 + lk)
    h, hkv, d = 12, 2, 128
    q = rng.standard_normal((1, h, lq, d)).astype(np.float32)
    k = rng.standard_normal((1, hkv, lk, d)).astype(np.float32)
    v = rng.standard_normal((1, hkv, lk, d)).astype(np.float32)
    out, w = br.reference_attention(None, torch.from_numpy(q), torch.from_numpy(k),
                                    torch.from_numpy(v), None, scaling=d ** -0.5)
    assert w is None and out.shape == (1, lq, h, d)
    # row i sees keys [0, i + lk - lq]
    kk = np.broadcast_to(k[0].transpose(1, 0, 2)[None], (lq, lk, hkv, d))
    vv = np.broadcast_to(v[0].transpose(1, 0, 2)[None], (lq, lk, hkv, d))
    lens = np.arange(lq) + 1 + (lk - lq)
    want = ref.dense_attention(q[0].transpose(1, 0, 2), kk, vv, lens, hkv)   # [lq, H, D]
    np.testing.assert_allclose(out[0].numpy(), want, atol=1e-5, rtol=1e-5)


def _shifted_reference(model_layers_to_break):
    """A reference attention that drops the newest key in the given layers
    (a planted cache mistake)."""
    from pa_int8 import qwen_bridge as br

    def fn(module, query, key, value, attention_mask, scaling=None, **kw):
        if module.layer_idx in model_layers_to_break and query.shape[2] == 1:
            key, value = key[:, :, :-1], value[:, :, :-1]
        return br.reference_attention(module, query, key, value, attention_mask, scaling)
    return fn


def test_incremental_reference_agrees_and_planted_mistake_is_caught():
    from transformers import AttentionInterface, DynamicCache

    from pa_int8 import qwen_bridge as br

    br.register()
    model = tiny_qwen()
    model.set_attn_implementation(br.REFERENCE_ATTN_NAME)
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, 512, (1, 21), generator=g)
    cont = torch.randint(0, 512, (1, 12), generator=g)
    whole = np.array(br.reference_logprobs(model, prompt, cont))

    def incremental():
        with torch.no_grad():
            cache = DynamicCache(config=model.config)
            out = model(input_ids=prompt, past_key_values=cache, use_cache=True)
            lp = []
            for i in range(cont.shape[1]):
                lp.append(torch.log_softmax(out.logits[0, -1].float(), -1)[cont[0, i]].item())
                out = model(input_ids=cont[:, i:i + 1], past_key_values=out.past_key_values,
                            use_cache=True)
        return np.array(lp)

    inc = incremental()
    assert np.abs(inc - whole).max() < 1e-3
    AttentionInterface.register("pa_planted_shift", _shifted_reference({1}))
    model.set_attn_implementation("pa_planted_shift")
    bad = incremental()
    assert np.abs(bad - whole).max() > 4 * LOGP_MAX


def test_bridge_entry_checks():
    from pa_int8 import qwen_bridge as br

    class M:
        layer_idx = 0

    br.set_active_cache(None)
    x = torch.zeros(1, 12, 1, 128)
    kv = torch.zeros(1, 2, 1, 128)
    with pytest.raises(RuntimeError, match="set_active_cache"):
        br.paged_bridge_attention(M(), x, kv, kv, None)

    class Cache:
        pass

    br.set_active_cache(Cache())
    with pytest.raises(RuntimeError, match="batch 1"):
        br.paged_bridge_attention(M(), torch.zeros(2, 12, 1, 128), kv.expand(2, -1, -1, -1),
                                  kv.expand(2, -1, -1, -1), None)
    br.set_active_cache(None)


def test_sessions_are_scoped_to_their_context():
    """A DecodeSession binds its cache only while it is entered, and restores
    whatever was bound before it (nested sessions, set_active_cache)."""
    from pa_int8 import qwen_bridge as br

    class Cache:
        is_int8 = False

        def reset(self):
            self.was_reset = True

    outer, inner = Cache(), Cache()
    br.set_active_cache(outer)
    assert br._SESSION.get().cache is outer
    with br.DecodeSession(None, inner) as s:
        assert br._SESSION.get() is s and inner.was_reset and s.position == 0
    assert br._SESSION.get().cache is outer
    br.set_active_cache(None)
    assert br._SESSION.get() is None


def test_decode_graph_needs_a_prompted_session():
    """A decode step is captured inside a session with a model, after its
    prompt step; nothing is captured otherwise."""
    from pa_int8 import qwen_bridge as br

    class Cache:
        is_int8 = False

        def reset(self):
            pass

    with br.DecodeSession(None, Cache()) as s:
        with pytest.raises(RuntimeError, match="after the prompt step"):
            br.DecodeGraph(s)
    with br.DecodeSession(object(), Cache()) as s:
        with pytest.raises(RuntimeError, match="after the prompt step"):
            br.DecodeGraph(s)
        assert s._graph is None


def test_register_is_idempotent():
    from transformers import AttentionInterface

    from pa_int8 import qwen_bridge as br

    br.register()
    br.register()
    assert br.ATTN_NAME in AttentionInterface._global_mapping
    assert br.REFERENCE_ATTN_NAME in AttentionInterface._global_mapping

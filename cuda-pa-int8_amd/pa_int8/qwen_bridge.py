"""Qwen2 decode-step attention through the paged kernels (transformers bridge).

Counterpart of benchmarks/int8_bridge/qwen_paged_attn.py:1-164.  A
transformers ``AttentionInterface`` function replaces only the attention math
(q/k/v projections, RoPE and o_proj stay in the model; the interface is called
after RoPE, before the GQA repeat):

* a prompt chunk (q_len > 1) is written into the active ``PagedKVCache``
  (quantized for the INT8 variants) and its output is full-precision causal
  attention over the chunk (:47-55);
* a decode step (q_len == 1) appends the token's K/V to the cache and takes its
  output from the split-K decode kernel, FP16 or INT8 (:57-71).

Batch 1, one sequence; the model runs with ``use_cache=False`` and explicit
``position_ids`` so the interface only ever sees the current chunk
(:11-13).  The active cache is module state set per generation call.
"""

from __future__ import annotations

import time

import torch

from .registry import VARIANTS, VARIANTS_INT8

ATTN_NAME = "paged_int8_bridge"          # name of qwen_paged_attn.py:28
REFERENCE_ATTN_NAME = "pa_fp32_reference"

_active = {"cache": None}
_registered = set()


def set_active_cache(cache):
    """The PagedKVCache the interface writes to and reads from (:33-35)."""
    _active["cache"] = cache


def _causal_fp32(query, key, value, scaling):
    """Causal attention in fp32 over contiguous operands, GQA by repetition.

    query [B, H, Lq, D], key/value [B, Hkv, Lk, D]; the last query row sits at
    the last key.  Returns [B, H, Lq, D] in query's dtype."""
    b, h, lq, d = query.shape
    hkv, lk = key.shape[1], key.shape[2]
    q = query.float()
    k = key.float().repeat_interleave(h // hkv, dim=1)
    v = value.float().repeat_interleave(h // hkv, dim=1).contiguous()
    kt = k.transpose(-1, -2).contiguous()
    s = torch.matmul(q, kt) * scaling                             # [B, H, Lq, Lk]
    if lq > 1:
        i = torch.arange(lq, device=q.device).view(lq, 1) + (lk - lq)
        j = torch.arange(lk, device=q.device).view(1, lk)
        s = s.masked_fill(j > i, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v).to(query.dtype)


def _prefill_attention(query, key, value, scaling):
    """Causal attention of a prompt chunk: SDPA on its flash / memory-efficient
    backend (torch's math backend is never used: it issues batched products
    on transposed views), else the fp32 form above."""
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel

        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return torch.nn.functional.scaled_dot_product_attention(
                query, key, value, is_causal=True, scale=scaling, enable_gqa=True)
    except RuntimeError:
        return _causal_fp32(query, key, value, scaling)


def paged_bridge_attention(module, query, key, value, attention_mask, scaling=None,
                           dropout=0.0, **kwargs):
    """Attention interface (shapes as transformers passes them):
    query [1, H, q_len, D], key/value [1, Hkv, q_len, D] (post-RoPE).  Returns
    ``(out [1, q_len, H, D], None)``."""
    cache = _active["cache"]
    if cache is None:
        raise RuntimeError("no active PagedKVCache: call set_active_cache() first")
    b, h, q_len, d = query.shape
    if b != 1:
        raise RuntimeError("the paged bridge decodes one sequence (batch 1)")
    if scaling is None:
        scaling = d ** -0.5
    layer = module.layer_idx

    if q_len > 1:
        cache.prefill(layer, key[0].transpose(0, 1).contiguous(),
                      value[0].transpose(0, 1).contiguous())
        out = _prefill_attention(query, key, value, scaling)
        return out.transpose(1, 2).contiguous(), None

    cache.decode_append(layer, key[0, :, 0, :], value[0, :, 0, :])
    q = query[0].transpose(0, 1).contiguous().to(torch.float16)   # [1, H, D]
    out = torch.empty_like(q)
    ctx = cache.context_lens(layer)
    if cache.is_int8:
        VARIANTS_INT8["splitk_int8"](out, q, cache.k_cache[layer], cache.v_cache[layer],
                                     cache.k_scales[layer], cache.v_scales[layer],
                                     cache.block_table, ctx, scaling, cache.block_size)
    else:
        VARIANTS["splitk"](out, q, cache.k_cache[layer], cache.v_cache[layer],
                           cache.block_table, ctx, scaling, cache.block_size)
    return out.unsqueeze(1).to(query.dtype), None


def reference_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0,
                        **kwargs):
    """Dense causal attention in fp32 over whatever K/V the model passes (its
    own cache, or the whole sequence): the checker the bridge is compared with."""
    if scaling is None:
        scaling = query.shape[-1] ** -0.5
    out = _causal_fp32(query, key, value, scaling)
    return out.transpose(1, 2).contiguous(), None


def register():
    """Register both interfaces once; select one with
    ``model.set_attn_implementation(ATTN_NAME)`` (:77-83)."""
    from transformers import AttentionInterface

    for name, fn in ((ATTN_NAME, paged_bridge_attention),
                     (REFERENCE_ATTN_NAME, reference_attention)):
        if name not in _registered:
            AttentionInterface.register(name, fn)
            _registered.add(name)


def _sync():
    torch.cuda.synchronize()


@torch.no_grad()
def generate_greedy(model, input_ids, max_new_tokens, cache):
    """Greedy decode through the bridge cache (:86-128).  Returns
    ``(ids [1, n], ttft_s, tpot_s, step_logits)``; step_logits are the
    next-token logits (prompt's last position, then every step) as CPU fp32."""
    dev = input_ids.device
    cache.reset()
    set_active_cache(cache)
    n0 = input_ids.shape[1]
    _sync()
    t0 = time.perf_counter()
    logits = model(input_ids=input_ids, position_ids=torch.arange(n0, device=dev)[None],
                   use_cache=False).logits[:, -1, :]
    _sync()
    ttft = time.perf_counter() - t0
    step_logits = [logits[0].float().cpu()]
    tok = logits.argmax(-1, keepdim=True)
    out = [tok]
    times = []
    for i in range(max_new_tokens - 1):
        pos = torch.tensor([[n0 + i]], device=dev)
        _sync()
        t0 = time.perf_counter()
        logits = model(input_ids=tok, position_ids=pos, use_cache=False).logits[:, -1, :]
        _sync()
        times.append(time.perf_counter() - t0)
        step_logits.append(logits[0].float().cpu())
        tok = logits.argmax(-1, keepdim=True)
        out.append(tok)
    tpot = sum(times) / len(times) if times else float("nan")
    return torch.cat(out, dim=1), ttft, tpot, step_logits


@torch.no_grad()
def teacher_force_logprobs(model, prompt_ids, cont_ids, cache):
    """Log-probabilities the cache's variant gives the fixed continuation
    ``cont_ids [1, n]`` after ``prompt_ids``, through the same prompt + decode
    path as generate_greedy (:131-158).  Returns a list of n floats."""
    dev = prompt_ids.device
    cache.reset()
    set_active_cache(cache)
    n0 = prompt_ids.shape[1]
    logits = model(input_ids=prompt_ids, position_ids=torch.arange(n0, device=dev)[None],
                   use_cache=False).logits[:, -1, :]
    logps = []
    for i in range(cont_ids.shape[1]):
        t = cont_ids[0, i]
        logps.append(torch.log_softmax(logits[0].float(), dim=-1)[t].item())
        logits = model(input_ids=t.view(1, 1), position_ids=torch.tensor([[n0 + i]], device=dev),
                       use_cache=False).logits[:, -1, :]
    return logps


def teacher_force_ppl(model, prompt_ids, cont_ids, cache):
    """Perplexity of ``cont_ids`` under the cache's variant (:161-164)."""
    lp = teacher_force_logprobs(model, prompt_ids, cont_ids, cache)
    return float(torch.exp(torch.tensor(-sum(lp) / len(lp))))


@torch.no_grad()
def reference_logprobs(model, prompt_ids, cont_ids):
    """The same log-probabilities from one dense forward over prompt +
    continuation with ``REFERENCE_ATTN_NAME`` (the model must use it)."""
    ids = torch.cat([prompt_ids, cont_ids], dim=1)
    n0, n = prompt_ids.shape[1], cont_ids.shape[1]
    logits = model(input_ids=ids, position_ids=torch.arange(ids.shape[1], device=ids.device)[None],
                   use_cache=False).logits[0, n0 - 1:n0 - 1 + n].float()
    lp = torch.log_softmax(logits, dim=-1)
    return lp.gather(1, cont_ids[0].view(-1, 1)).view(-1).cpu().tolist()

"""Qwen2 decode-step attention on the paged kernels: a transformers bridge.

Behaviour of benchmarks/int8_bridge/qwen_paged_attn.py:1-164 -- the same
interface name, batch 1, a prompt chunk written into the active
``PagedKVCache`` and attended causally in full precision, every one-token
step appended to the cache and answered by the split-K decode kernel over it
-- built around one object instead of module state and parallel loops:

* ``DecodeSession(model, cache)`` owns one pass over one sequence.  Entering
  it binds the cache to the attention interface through a context variable,
  so a bridged model and a reference model (or two threads) never see each
  other's cache.
* ``DecodeSession.step(ids)`` is the only place the model is called: it feeds
  ``ids`` at the next positions (explicit ``position_ids`` and
  ``use_cache=False``, so attention only ever receives the new chunk) and
  returns the last position's logits.
* Greedy generation and teacher forcing are two token-picking policies over
  one loop (``_run``): token i is picked from the logits that precede it and
  fed as the next step.  Teacher forcing skips the forward of its last token,
  whose logits nobody reads, and reads the log-probabilities back once at the
  end instead of once per token.
* A decode step calls the kernel through the no-sync entry: the cache knows
  its length on the host, so no ``context_lens.min()`` device-to-host copy is
  made per layer (the reference's op makes one).
* ``DecodeGraph`` captures the one-token step (all layers: projections, the
  cache write and the decode kernel) as one HIP graph whose position and
  length live on the device; ``generate_greedy_graph`` replays it per token.
  The eager loop's time per token is the host launching 28 layers' kernels;
  the replay's is the device's.
* Every model call computes the logits of its last position only
  (``logits_to_keep=1``): a 1024-token prompt's full logits would be 0.3 GB.
"""

from __future__ import annotations

import contextvars
import math
import time

import torch

from . import registry

ATTN_NAME = "paged_int8_bridge"          # the interface name of qwen_paged_attn.py:28
REFERENCE_ATTN_NAME = "pa_fp32_reference"

_SESSION: contextvars.ContextVar = contextvars.ContextVar("pa_int8_decode_session",
                                                          default=None)
_registered = set()


# --------------------------------------------------------------------------- attention math

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


# --------------------------------------------------------------------------- session

class DecodeSession:
    """One pass of `model` over one sequence with its attention on `cache`.

    Use as a context manager; ``model`` may be None when only the attention
    interface is driven (``set_active_cache``)."""

    def __init__(self, model, cache):
        self.model = model
        self.cache = cache
        self.position = 0
        self._token = None
        self._graph = None         # the DecodeGraph being warmed up or captured
        if getattr(cache, "is_int8", False):
            self._kernel = "splitk_int8"
        else:
            self._kernel = "splitk"

    def __enter__(self):
        self.cache.reset()
        self.position = 0
        self._token = _SESSION.set(self)
        return self

    def __exit__(self, *exc):
        _SESSION.reset(self._token)
        self._token = None
        return False

    @torch.no_grad()
    def step(self, ids):
        """Feeds `ids` ([1, n]) at the next n positions; returns the logits of
        the last one ([1, vocab])."""
        n = ids.shape[1]
        pos = torch.arange(self.position, self.position + n, device=ids.device).unsqueeze(0)
        logits = self.model(input_ids=ids, position_ids=pos, use_cache=False,
                            logits_to_keep=1).logits[:, -1, :]
        self.position += n
        return logits

    def attend(self, layer, query, key, value, scaling):
        """The interface's work for one layer: query [1, H, n, D] and key/value
        [1, Hkv, n, D] after RoPE.  Returns [1, n, H, D]."""
        b, h, n, d = query.shape
        if b != 1:
            raise RuntimeError("the paged bridge decodes one sequence (batch 1)")
        if scaling is None:
            scaling = d ** -0.5
        k_tok = key[0].permute(1, 0, 2)                  # [n, Hkv, D], one row per position
        v_tok = value[0].permute(1, 0, 2)
        c = self.cache
        if n > 1:
            if self._graph is not None:
                raise RuntimeError("a captured decode step feeds one token")
            c.prefill(layer, k_tok.contiguous(), v_tok.contiguous())
            return _prefill_attention(query, key, value, scaling).transpose(1, 2).contiguous()
        if self._graph is None:
            c.decode_append(layer, k_tok[0], v_tok[0])
            ctx = c.context_lens(layer)
        else:   # the position and the length are device buffers the graph advances
            c.append_at(layer, k_tok[0], v_tok[0], self._graph.slot)
            ctx = self._graph.ctx
        q = query.reshape(1, h, d).to(torch.float16)
        out = torch.empty_like(q)
        scales = dict(k_scales=c.k_scales[layer], v_scales=c.v_scales[layer]) if c.is_int8 else {}
        registry.decode(self._kernel, out, q, c.k_cache[layer], c.v_cache[layer], c.block_table,
                        ctx, scaling, c.block_size, check=False, **scales)
        return out.view(1, 1, h, d).to(query.dtype)


class DecodeGraph:
    """A session's one-token decode step, captured once as a HIP graph and
    replayed for every later token.

    The step reads its inputs from device buffers: the token id, its position
    (also the cache slot it is written to: batch 1, identity block table) and
    the context length the decode kernel reads.  The graph advances the
    position and the length itself, so a step is one copy of the id and one
    replay: no per-layer host work, and no host-to-device copy of a length
    (the eager step makes one per layer).  Allocations during capture come
    from torch's graph-private pool; the library's split counters are cleared
    by a fill kernel, which a graph replays correctly.

    Build it inside the session (``with DecodeSession(...) as s``), after the
    prompt step.  It stays valid for that pass only: its buffers hold this
    pass's position, and its kernels this cache's tensors."""

    @torch.no_grad()
    def __init__(self, session):
        s = session
        if s.model is None or s.position == 0:
            raise RuntimeError("capture a decode step after the prompt step of a session "
                               "with a model")
        dev = s.cache.k_cache.device
        self.session = s
        self.ids = torch.zeros((1, 1), dtype=torch.long, device=dev)
        self.pos = torch.full((1, 1), s.position, dtype=torch.long, device=dev)
        self.slot = self.pos.view(1)
        self.ctx = torch.full((1,), s.position + 1, dtype=torch.int32, device=dev)
        self.graph = torch.cuda.CUDAGraph()
        pos0, ctx0 = self.pos.clone(), self.ctx.clone()
        s._graph = self
        try:
            # One eager pass on a side stream first (lazy library set-up stays out
            # of the capture).  It writes token 0's K/V at the next slot; the first
            # replay writes the real token there.
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                self._body()
            torch.cuda.current_stream().wait_stream(side)
            self.pos.copy_(pos0)
            self.ctx.copy_(ctx0)
            with torch.cuda.graph(self.graph):
                self.logits = self._body()
        finally:
            s._graph = None

    def _body(self):
        logits = self.session.model(input_ids=self.ids, position_ids=self.pos, use_cache=False,
                                    logits_to_keep=1).logits[:, -1, :]
        self.pos.add_(1)
        self.ctx.add_(1)
        return logits

    def step(self, ids):
        """Feeds ``ids`` ([1, 1] on the device) at the next position; returns the
        logits of that position ([1, vocab], overwritten by the next step)."""
        s = self.session
        if s.position >= s.cache.capacity:
            raise AssertionError("cache is full")
        self.ids.copy_(ids)
        self.graph.replay()
        s.position += 1
        s.cache.advance(1)
        return self.logits


def set_active_cache(cache):
    """Binds `cache` to the attention interface in the current context without
    a model (the reference's module-level switch, qwen_paged_attn.py:33-35);
    None unbinds.  ``DecodeSession`` does this for a pass of a model."""
    _SESSION.set(DecodeSession(None, cache) if cache is not None else None)


def paged_bridge_attention(module, query, key, value, attention_mask, scaling=None,
                           dropout=0.0, **kwargs):
    """transformers AttentionInterface function of ``ATTN_NAME``: the active
    session's cache takes the chunk's K/V and answers the query.  Returns
    ``(out [1, q_len, H, D], None)``."""
    session = _SESSION.get()
    if session is None:
        raise RuntimeError("no active PagedKVCache: enter a DecodeSession or call "
                           "set_active_cache() first")
    return session.attend(module.layer_idx, query, key, value, scaling), None


def reference_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0,
                        **kwargs):
    """Dense causal attention in fp32 over whatever K/V the model passes (its
    own cache, or the whole sequence): the checker the bridge is compared with."""
    if scaling is None:
        scaling = query.shape[-1] ** -0.5
    out = _causal_fp32(query, key, value, scaling)
    return out.transpose(1, 2).contiguous(), None


def register():
    """Registers both interfaces once; select one with
    ``model.set_attn_implementation(ATTN_NAME)`` (qwen_paged_attn.py:77-83)."""
    from transformers import AttentionInterface

    for name, fn in ((ATTN_NAME, paged_bridge_attention),
                     (REFERENCE_ATTN_NAME, reference_attention)):
        if name not in _registered:
            AttentionInterface.register(name, fn)
            _registered.add(name)


# --------------------------------------------------------------------------- drivers

def _run(model, cache, prompt_ids, n_tokens, pick, timed=False):
    """Prompt, then the picked tokens: token i = pick(i, logits before it) is a
    [1, 1] id tensor, fed as the next step unless it is the last.  Returns the
    wall time of every model call (synchronized) when `timed`."""
    times = []

    def call(session, ids):
        if not timed:
            return session.step(ids)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        logits = session.step(ids)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
        return logits

    with DecodeSession(model, cache) as s:
        logits = call(s, prompt_ids)
        for i in range(n_tokens):
            tok = pick(i, logits)
            if i + 1 < n_tokens:
                logits = call(s, tok)
    return times


def generate_greedy(model, input_ids, max_new_tokens, cache):
    """Greedy decode through the bridge (qwen_paged_attn.py:86-128).  Returns
    ``(ids [1, n], ttft_s, tpot_s, step_logits)``: the time of the prompt call,
    the mean time of the one-token calls, and the next-token logits before
    every generated token (CPU fp32)."""
    chosen, seen = [], []

    def pick(i, logits):
        seen.append(logits[0].float().cpu())
        tok = logits.argmax(-1, keepdim=True)
        chosen.append(tok)
        return tok

    times = _run(model, cache, input_ids, max_new_tokens, pick, timed=True)
    decode = times[1:]
    tpot = sum(decode) / len(decode) if decode else float("nan")
    return torch.cat(chosen, dim=1), times[0], tpot, seen


def generate_greedy_graph(model, input_ids, max_new_tokens, cache, keep_logits=False):
    """generate_greedy with every one-token step replayed from a captured
    ``DecodeGraph``.  Returns ``(ids [1, n], ttft_s, tpot_s, step_logits)``:
    the prompt call's wall time, the mean wall time per token over the
    replays (the capture excluded; each token costs one replay, one argmax and
    one id copy, as in the eager loop), and, with `keep_logits`, the logits
    before every generated token (CPU fp32; reading them back synchronizes)."""
    chosen, seen = [], []
    with DecodeSession(model, cache) as s:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        logits = s.step(input_ids)
        torch.cuda.synchronize()
        ttft = time.perf_counter() - t0
        tpot = float("nan")
        if keep_logits:
            seen.append(logits[0].float().cpu())
        tok = logits.argmax(-1, keepdim=True)
        chosen.append(tok)
        if max_new_tokens > 1:
            g = DecodeGraph(s)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(max_new_tokens - 1):
                logits = g.step(tok)
                if keep_logits:
                    seen.append(logits[0].float().cpu())
                tok = logits.argmax(-1, keepdim=True)
                chosen.append(tok)
            torch.cuda.synchronize()
            tpot = (time.perf_counter() - t0) / (max_new_tokens - 1)
    return torch.cat(chosen, dim=1), ttft, tpot, seen


def teacher_force_logprobs(model, prompt_ids, cont_ids, cache):
    """Natural-log probabilities the cache's variant gives the fixed
    continuation ``cont_ids [1, n]`` after ``prompt_ids``, through the same
    prompt + decode steps as generate_greedy (qwen_paged_attn.py:131-158).
    Returns a list of n floats."""
    cont = cont_ids[0]
    picked = []

    def pick(i, logits):
        picked.append(torch.log_softmax(logits[0].float(), dim=-1)[cont[i]])
        return cont[i].view(1, 1)

    _run(model, cache, prompt_ids, cont.shape[0], pick)
    return torch.stack(picked).cpu().tolist()


def teacher_force_ppl(model, prompt_ids, cont_ids, cache):
    """Perplexity of ``cont_ids`` under the cache's variant (qwen_paged_attn.py:161-164)."""
    lp = teacher_force_logprobs(model, prompt_ids, cont_ids, cache)
    return math.exp(-sum(lp) / len(lp))


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

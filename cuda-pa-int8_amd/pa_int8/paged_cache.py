"""Per-layer paged K/V cache whose writes run on the gfx950 kernels.

Mirrors ``PagedKVCache`` of benchmarks/int8_bridge/paged_cache.py:41-182: the
same constructor, attributes (``k_cache``, ``v_cache``, ``k_scales``,
``v_scales``, ``block_table``, ``lengths``), methods and byte figures, for
batch 1 with an identity block table.  The tensors, their sizes and the tail
clearing all follow one ``PagedLayout`` (per-block shapes of the kernels'
layouts).  The three variants are the reference's:

* ``"fp16"``            -- fp16 cache (write: ``reshape_and_cache``);
* ``"int8_per_token"``  -- int8 cache, one fp32 scale per (token, kv head)
  (write: ``reshape_and_cache_int8``, bit-exact with ``quantize_per_token``);
* ``"int8_per_tensor"`` -- int8 cache, one fp32 scale per layer and tensor,
  taken at prefill as ``(amax / 127).to(float32).clamp_min(1e-8)``
  (paged_cache.py:101-102) and reused by every append
  (write: ``reshape_and_cache_int8_static``).

Where the reference quantizes with several torch ops and scatters with
permuted copies, each write here is one kernel launch; the per-tensor amax
is a torch reduction on the device.  ``prefill`` also clears the unused tail
of the last block, as the reference's zero-padded copy does (:116-128).
Writes take fp16 K/V on a HIP device, and the INT8 variants bf16 too (the
dtype the reference's bridge runs Qwen in, quantized directly as its
quantize_per_token does); the fp16 variant converts other float dtypes first,
as the reference does (:111).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import registry

VARIANTS = ("fp16", "int8_per_token", "int8_per_tensor")


@dataclass(frozen=True)
class PagedLayout:
    """Geometry of one layer's paged tensors, as the write and decode kernels
    address them: per tensor, the shape of one physical block, its dtype and
    the axis (within the block) that runs over the block's token slots.

    K ``[Hkv, D/x, bs, x]`` and V ``[Hkv, D, bs]`` in fp16 or int8; with INT8,
    one fp32 scale per (kv head, slot) for K and for V ``[Hkv, bs]``.  Every
    size the cache reports is read off these per-block shapes."""

    num_kv_heads: int
    head_dim: int
    block_size: int
    x: int
    int8: bool

    def blocks_for(self, tokens):
        return -(-int(tokens) // self.block_size)

    def tensors(self):
        """{name: (per-block shape, dtype, token axis)} in allocation order."""
        h, d, bs, x = self.num_kv_heads, self.head_dim, self.block_size, self.x
        store = torch.int8 if self.int8 else torch.float16
        spec = {"k_cache": ((h, d // x, bs, x), store, 2),
                "v_cache": ((h, d, bs), store, 2)}
        if self.int8:
            spec["k_scales"] = ((h, bs), torch.float32, 1)
            spec["v_scales"] = ((h, bs), torch.float32, 1)
        return spec

    def block_bytes(self):
        """Bytes of one physical block over every tensor of one layer."""
        total = 0
        for shape, dtype, _ in self.tensors().values():
            n = 1
            for e in shape:
                n *= e
            total += n * torch.empty((), dtype=dtype).element_size()
        return total


class PagedKVCache:
    def __init__(self, num_layers, num_kv_heads, head_dim, max_len, block_size=16, x=8,
                 variant="fp16", device="cuda"):
        # (AssertionError, as the reference's constructor raises for these)
        if variant not in VARIANTS:
            raise AssertionError(f"variant must be one of {VARIANTS}, got {variant!r}")
        if head_dim % x:
            raise AssertionError(f"head_dim {head_dim} is not a multiple of x = {x}")
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.x = x
        self.variant = variant
        self.is_int8 = variant != "fp16"
        self.device = device
        self.layout = PagedLayout(num_kv_heads, head_dim, block_size, x, self.is_int8)
        self.num_blocks = self.layout.blocks_for(max_len)
        # k_cache, v_cache (and k_scales, v_scales): [num_layers, num_blocks, *block shape]
        for name, (shape, dtype, _) in self.layout.tensors().items():
            setattr(self, name, torch.zeros((num_layers, self.num_blocks) + shape, dtype=dtype,
                                            device=device))
        # batch 1: sequence block j is physical block j in every layer, so slot t is token t
        self.block_table = torch.arange(self.num_blocks, dtype=torch.int32,
                                        device=device).view(1, -1)
        self._slots = torch.arange(self.num_blocks * block_size, dtype=torch.int64, device=device)
        self.reset()

    def reset(self):
        """Every layer empty again; per-tensor scales are taken anew at the next prefill."""
        self.lengths = [0] * self.num_layers
        if self.is_int8:
            self._k_tensor_scale = [None] * self.num_layers
            self._v_tensor_scale = [None] * self.num_layers

    def _tensors(self):
        return [getattr(self, name) for name in self.layout.tensors()]

    # --- write path ---------------------------------------------------------

    def _kernel_input(self, t):
        if self.variant == "fp16" and t.dtype != torch.float16:
            t = t.to(torch.float16)
        if t.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"PagedKVCache({self.variant!r}) writes fp16 or bf16 K/V; "
                            f"got {t.dtype}")
        if t.stride(-1) != 1 or t.stride(0) % 8 or t.stride(1) % 8 or t.data_ptr() % 16:
            t = t.contiguous()
        return t

    def _write(self, layer_idx, k, v, slots):
        kc, vc = self.k_cache[layer_idx], self.v_cache[layer_idx]
        if self.variant == "fp16":
            registry.reshape_and_cache(k, v, kc, vc, slots)
        elif self.variant == "int8_per_token":
            registry.reshape_and_cache_int8(k, v, kc, vc, self.k_scales[layer_idx],
                                            self.v_scales[layer_idx], slots)
        else:
            registry.reshape_and_cache_int8_static(
                k, v, kc, vc, self.k_scales[layer_idx], self.v_scales[layer_idx], slots,
                self._k_tensor_scale[layer_idx], self._v_tensor_scale[layer_idx])

    def prefill(self, layer_idx, k, v):
        """Write the prompt's K/V ``[L, num_kv_heads, head_dim]`` at positions
        [0, L) of `layer_idx` and set the layer length to L (paged_cache.py:88-130)."""
        L, H, D = k.shape
        assert H == self.num_kv_heads and D == self.head_dim
        assert L <= self.num_blocks * self.block_size
        k, v = self._kernel_input(k), self._kernel_input(v)
        if self.variant == "int8_per_tensor":
            self._k_tensor_scale[layer_idx] = (
                (k.abs().amax() / 127.0).to(torch.float32).clamp_min(1e-8).reshape(1))
            self._v_tensor_scale[layer_idx] = (
                (v.abs().amax() / 127.0).to(torch.float32).clamp_min(1e-8).reshape(1))
        if L > 0:
            self._write(layer_idx, k, v, self._slots[:L])
        # the rest of the last block holds zeros, as after the reference's padded copy
        off = L % self.block_size
        if off:
            blk = L // self.block_size
            for name, (_, _, tok_axis) in self.layout.tensors().items():
                getattr(self, name)[layer_idx, blk].narrow(tok_axis, off,
                                                           self.block_size - off).zero_()
        self.lengths[layer_idx] = L

    def decode_append(self, layer_idx, k, v):
        """Append one token's K/V ``[num_kv_heads, head_dim]`` at the layer's
        current length; returns the new length (paged_cache.py:132-156)."""
        t = self.lengths[layer_idx]
        assert t < self.num_blocks * self.block_size, "cache is full"
        if self.variant == "int8_per_tensor" and self._k_tensor_scale[layer_idx] is None:
            raise RuntimeError("int8_per_tensor: prefill sets the layer's scales before appends")
        k = self._kernel_input(k.reshape(1, self.num_kv_heads, self.head_dim))
        v = self._kernel_input(v.reshape(1, self.num_kv_heads, self.head_dim))
        self._write(layer_idx, k, v, self._slots[t:t + 1])
        self.lengths[layer_idx] = t + 1
        return t + 1

    @property
    def capacity(self):
        """Token slots per layer."""
        return self.num_blocks * self.block_size

    def append_at(self, layer_idx, k, v, slot):
        """Write one token's K/V ``[num_kv_heads, head_dim]`` at the slot that
        the device tensor `slot` (int64, one element) holds.  This is the
        append of a captured decode step, whose position lives on the device;
        the host lengths move with ``advance`` once the step has run."""
        if self.variant == "int8_per_tensor" and self._k_tensor_scale[layer_idx] is None:
            raise RuntimeError("int8_per_tensor: prefill sets the layer's scales before appends")
        if slot.dtype != torch.int64 or slot.numel() != 1 or slot.device != self.k_cache.device:
            raise TypeError("slot must be a one-element int64 tensor on the cache's device")
        k = self._kernel_input(k.reshape(1, self.num_kv_heads, self.head_dim))
        v = self._kernel_input(v.reshape(1, self.num_kv_heads, self.head_dim))
        self._write(layer_idx, k, v, slot.reshape(1))

    def advance(self, n=1):
        """Count `n` tokens appended to every layer by ``append_at``."""
        if any(t + n > self.capacity for t in self.lengths):
            raise AssertionError("cache is full")
        self.lengths = [t + n for t in self.lengths]

    # --- read path ----------------------------------------------------------

    def context_lens(self, layer_idx):
        return torch.tensor([self.lengths[layer_idx]], dtype=torch.int32, device=self.device)

    def kv_bytes(self):
        """Bytes of the whole allocation: K, V and (INT8) their scales, every
        layer and block (paged_cache.py:161-170)."""
        return sum(t.numel() * t.element_size() for t in self._tensors())

    def kv_bytes_for_len(self, n):
        """Bytes that `n` tokens occupy over all layers: whole blocks, each
        with its K, V and scale slots (paged_cache.py:172-182)."""
        return self.layout.blocks_for(n) * self.layout.block_bytes() * self.num_layers

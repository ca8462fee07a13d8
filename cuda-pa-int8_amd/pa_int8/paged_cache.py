"""Per-layer paged K/V cache whose writes run on the gfx950 kernels.

Mirrors ``PagedKVCache`` of benchmarks/int8_bridge/paged_cache.py:41-182: the
same constructor, attributes (``k_cache``, ``v_cache``, ``k_scales``,
``v_scales``, ``block_table``, ``lengths``), methods and byte accounting, for
batch 1 with an identity block table.  The three variants are the
reference's:

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

import torch

from . import registry

VARIANTS = ("fp16", "int8_per_token", "int8_per_tensor")


class PagedKVCache:
    def __init__(self, num_layers, num_kv_heads, head_dim, max_len, block_size=16, x=8,
                 variant="fp16", device="cuda"):
        assert variant in VARIANTS
        assert head_dim % x == 0
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.x = x
        self.variant = variant
        self.is_int8 = variant != "fp16"
        self.device = device

        self.num_blocks = (max_len + block_size - 1) // block_size
        store = torch.int8 if self.is_int8 else torch.float16
        self.k_cache = torch.zeros(num_layers, self.num_blocks, num_kv_heads, head_dim // x,
                                   block_size, x, dtype=store, device=device)
        self.v_cache = torch.zeros(num_layers, self.num_blocks, num_kv_heads, head_dim,
                                   block_size, dtype=store, device=device)
        if self.is_int8:
            self.k_scales = torch.zeros(num_layers, self.num_blocks, num_kv_heads, block_size,
                                        dtype=torch.float32, device=device)
            self.v_scales = torch.zeros(num_layers, self.num_blocks, num_kv_heads, block_size,
                                        dtype=torch.float32, device=device)
            self._k_tensor_scale = [None] * num_layers
            self._v_tensor_scale = [None] * num_layers
        # identity block table (batch 1), shared by every layer
        self.block_table = torch.arange(self.num_blocks, dtype=torch.int32,
                                        device=device).view(1, -1)
        # slot ids 0 .. num_blocks * block_size - 1: slot t is token t
        self._slots = torch.arange(self.num_blocks * block_size, dtype=torch.int64, device=device)
        self.lengths = [0] * num_layers

    def reset(self):
        self.lengths = [0] * self.num_layers
        if self.is_int8:
            self._k_tensor_scale = [None] * self.num_layers
            self._v_tensor_scale = [None] * self.num_layers

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
            self.k_cache[layer_idx, blk, :, :, off:, :].zero_()
            self.v_cache[layer_idx, blk, :, :, off:].zero_()
            if self.is_int8:
                self.k_scales[layer_idx, blk, :, off:].zero_()
                self.v_scales[layer_idx, blk, :, off:].zero_()
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

    # --- read path ----------------------------------------------------------

    def context_lens(self, layer_idx):
        return torch.tensor([self.lengths[layer_idx]], dtype=torch.int32, device=self.device)

    def kv_bytes(self):
        """Bytes of the whole K/V allocation (and scales) (paged_cache.py:161-170)."""
        b = self.k_cache.element_size() * self.k_cache.nelement()
        b += self.v_cache.element_size() * self.v_cache.nelement()
        if self.is_int8:
            b += self.k_scales.element_size() * self.k_scales.nelement()
            b += self.v_scales.element_size() * self.v_scales.nelement()
        return b

    def kv_bytes_for_len(self, n):
        """Bytes K+V (and int8 scales) need for `n` tokens over all layers
        (paged_cache.py:172-182)."""
        blocks = (n + self.block_size - 1) // self.block_size
        elem = 1 if self.is_int8 else 2
        per_blk = 2 * self.num_kv_heads * self.head_dim * self.block_size
        b = blocks * per_blk * elem * self.num_layers
        if self.is_int8:
            b += blocks * 2 * self.num_kv_heads * self.block_size * 4 * self.num_layers
        return b

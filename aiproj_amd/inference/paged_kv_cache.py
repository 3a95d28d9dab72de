"""Per-layer paged K/V storage, reference `src/torch_llm/inference/paged_kv_cache.py:6-79`.

Layout (API, indexed directly by callers and tests):
    k, v              [num_blocks, block_size, num_kv_heads, head_dim]   cache dtype
    k_scales, v_scales [num_blocks, block_size, num_kv_heads]            float32, FP8 only
One float32 scale per (page, slot in page, KV head), i.e. per token per head
(reference `inference/kvcache_config.py:46-47`, handoff decision D12).

`append_kv` validates shapes, dtypes and devices without reading device values,
then calls the HIP quantize-and-scatter kernel (FP8 caches) or the HIP cast-and-
scatter kernel (plain device caches). Plain caches in host memory keep the
reference's indexed store; FP8 storage has no host path, as in the reference.
"""

from __future__ import annotations

import torch as t

from aiproj_amd import _native
from aiproj_amd.kernals.kv_cache.quantized_append import quantize_append_wrapper, store_append


class PagedKVCache:
    """Per-layer paged storage; allocation and lengths belong to PageAllocator."""

    def __init__(
        self,
        num_blocks: int,
        block_size: int,
        num_kv_heads: int,
        head_dim: int,
        device,
        cache_dtype,
        scale_dtype=t.float32,
        scale_granularity="token_head",
    ):
        for value in (num_blocks, block_size, num_kv_heads, head_dim):
            if not isinstance(value, int) or isinstance(value, bool) or value <= 0:
                raise ValueError("Cache dimensions must be positive integers")

        self.num_blocks = num_blocks
        self.block_size = block_size
        self.cache_dtype = cache_dtype
        self.scale_dtype = scale_dtype
        self.scale_granularity = scale_granularity

        shape = (num_blocks, block_size, num_kv_heads, head_dim)
        self.k = t.empty(shape, device=device, dtype=cache_dtype)
        self.v = t.empty_like(self.k)

        self.quantized = cache_dtype == t.float8_e4m3fn
        if self.quantized:
            self.k_scales = t.empty(shape[:3], device=device, dtype=scale_dtype)
            self.v_scales = t.empty_like(self.k_scales)
        else:
            self.k_scales = None
            self.v_scales = None

    @t.no_grad()
    def append_kv(self, blocks, offsets, ks, vs):
        """Write ks/vs [T, H_kv, D] at (blocks[t], offsets[t]); metadata checks never sync."""
        expected = (blocks.numel(), *self.k.shape[2:])
        if blocks.ndim != 1 or offsets.shape != blocks.shape or ks.shape != expected or vs.shape != expected:
            raise ValueError("K/V and cache locations must describe the same packed tokens")
        if blocks.dtype not in (t.int32, t.int64) or offsets.dtype not in (t.int32, t.int64):
            raise ValueError("Cache locations must be integer tensors")
        # Device indices first (get_device: no device objects); a CPU or meta cache, or
        # any mismatch, takes the full comparison.
        dev = self.k.get_device()
        if dev < 0 or any(x.get_device() != dev for x in (blocks, offsets, ks, vs)):
            if any(x.device != self.k.device for x in (blocks, offsets, ks, vs)):
                raise ValueError("K/V and cache locations must be on the cache device")

        if self.quantized:
            quantize_append_wrapper(self, ks, vs, blocks, offsets)
        elif self.k.device.type == "cuda":
            store_append(self, ks, vs, blocks, offsets)
        else:
            # Host-memory plain cache: the reference's indexed store.
            self.k[blocks, offsets] = ks.to(self.cache_dtype)
            self.v[blocks, offsets] = vs.to(self.cache_dtype)


def native_available() -> bool:
    """True when libkvfp8.so loads (it is required for every device cache operation)."""
    try:
        _native.lib()
        return True
    except _native.NativeLibraryError:
        return False

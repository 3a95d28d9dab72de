"""Dense per-slot K/V cache, reference `src/torch_llm/inference/kv_cache.py:4-125`.

Layout (API, indexed directly by callers and tests):
    k_cache, v_cache  [batch_size, cache_max_seq_len, num_kv_heads, head_dim]  f16/bf16/f32
    seq_lens          [batch_size] int32, tokens held per slot

The reference keeps this dense cache beside the paged one as its simple
reference; the continuous runtime uses `PagedKVCache`. The validation and its
errors follow the reference line by line; like the reference, the capacity and
slot checks read device values. The writes on a GPU are one launch of the HIP
cast-and-scatter kernel (`kvfp8_store_append`), addressing the dense cache as
`batch_size` pages of `cache_max_seq_len` slots: the row of a token is its
cache slot and its column the slot's current length plus its offset in the
prompt. Caches in host memory keep the reference's indexed store.
"""

from __future__ import annotations

import torch as t

from aiproj_amd.kernals.kv_cache.quantized_append import store_rows


class KVCache:
    """Dense reference cache. The continuous runtime uses PagedKVCache instead."""

    def __init__(self, batch_size, cache_max_seq_len, num_kv_heads, head_dim, dtype, device):
        # Reference kv_cache.py:8-32.
        for value in (batch_size, cache_max_seq_len, num_kv_heads, head_dim):
            if not isinstance(value, int) or isinstance(value, bool) or value <= 0:
                raise ValueError("Cache dimensions must be positive integers")
        if dtype not in (t.float16, t.bfloat16, t.float32):
            raise ValueError("Unsupported KV cache dtype")

        self.batch_size = batch_size
        self.cache_max_seq_len = cache_max_seq_len
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.k_cache = t.empty((batch_size, cache_max_seq_len, num_kv_heads, head_dim), dtype=dtype, device=device)
        self.v_cache = t.empty_like(self.k_cache)
        self.seq_lens = t.zeros(batch_size, dtype=t.int32, device=device)

    def slots(self, cache_slots):
        """The slot indices a call addresses (all slots when None), reference kv_cache.py:35-56."""
        if cache_slots is None:
            return t.arange(self.batch_size, device=self.k_cache.device)
        slots = t.as_tensor(cache_slots, device=self.k_cache.device)
        if slots.ndim != 1:
            raise ValueError("cache_slots must be a vector of integer indices")
        if slots.numel() == 0:
            return slots.to(t.long)
        if slots.dtype not in (t.int32, t.int64):
            raise ValueError("cache_slots must be a vector of integer indices")
        if not bool(((slots >= 0) & (slots < self.batch_size)).all()) or slots.unique().numel() != slots.numel():
            raise ValueError("cache_slots must be unique, valid cache indices")
        return slots

    def check_kv(self, new_k, new_v, num_tokens):
        shape = (num_tokens, self.num_kv_heads, self.head_dim)
        if new_k.shape != shape or new_v.shape != shape:
            raise ValueError(f"Expected K/V shape {shape}")
        if new_k.device != self.k_cache.device or new_v.device != self.k_cache.device:
            raise ValueError("K/V must be on the cache device")

    def _store(self, rows, cols, new_k, new_v):
        if self.k_cache.device.type == "cuda":
            store_rows(self.k_cache, self.v_cache, new_k, new_v, rows, cols, what="KVCache")
        else:
            self.k_cache[rows, cols] = new_k.to(self.k_cache.dtype)
            self.v_cache[rows, cols] = new_v.to(self.v_cache.dtype)

    @t.no_grad()
    def append_decode(self, new_k, new_v, cache_slots=None):
        """One token per addressed slot at its current length, reference kv_cache.py:67-79."""
        slots = self.slots(cache_slots)
        self.check_kv(new_k, new_v, slots.numel())
        positions = self.seq_lens[slots]
        if not bool((positions < self.cache_max_seq_len).all()):
            raise ValueError("Decode would exceed cache capacity")
        self._store(slots, positions, new_k, new_v)
        self.seq_lens[slots] += 1

    @t.no_grad()
    def append_prefill(self, new_k, new_v, cu_seqlens, cache_slots=None):
        """Packed prompts (cu_seqlens offsets) after each slot's current length,
        reference kv_cache.py:82-118."""
        slots = self.slots(cache_slots)
        self.check_kv(new_k, new_v, new_k.shape[0])
        if cu_seqlens.device != self.k_cache.device or cu_seqlens.dtype not in (t.int32, t.int64):
            raise ValueError("cu_seqlens must be integer metadata on the cache device")
        if cu_seqlens.shape != (slots.numel() + 1,):
            raise ValueError("cu_seqlens must contain one boundary per request plus the end")
        lengths = cu_seqlens[1:] - cu_seqlens[:-1]
        if int(cu_seqlens[0]) != 0 or int(cu_seqlens[-1]) != new_k.shape[0] or not bool((lengths >= 0).all()):
            raise ValueError("Invalid cumulative sequence lengths")
        if not bool((self.seq_lens[slots] + lengths <= self.cache_max_seq_len).all()):
            raise ValueError("Prefill would exceed cache capacity")

        total = new_k.shape[0]
        token_slots = t.repeat_interleave(slots, lengths, output_size=total)
        starts = t.repeat_interleave(cu_seqlens[:-1], lengths, output_size=total)
        positions = self.seq_lens[token_slots] + t.arange(total, device=self.k_cache.device) - starts
        self._store(token_slots, positions, new_k, new_v)
        self.seq_lens[slots] += lengths

    def clear(self, cache_slots=None):
        # Stale storage is unreachable once the lengths are reset: no fill of the cache.
        self.seq_lens[self.slots(cache_slots)] = 0

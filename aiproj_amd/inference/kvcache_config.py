"""KV-cache configuration, reference `src/torch_llm/inference/kvcache_config.py:7-47`.

Same fields, defaults and validation as the reference: every size is a positive int
(bool rejected), the block size is a power of two, the cache dtype is one of
f16/bf16/f32/float8_e4m3fn (FP8 is opt-in, bf16 is the default), scales are float32
and the only scale granularity is "token_head" (one scale per token per KV head).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch as t

SUPPORTED_CACHE_DTYPES = (t.float16, t.bfloat16, t.float32, t.float8_e4m3fn)


def _is_positive_int(value) -> bool:
    return isinstance(value, int) and not isinstance(value, bool) and value > 0


@dataclass
class KVCacheConfig:
    num_blocks: int = 4096
    block_size: int = 16
    max_cache_slots: int = 64
    cache_max_seq_len: int = 2048

    kv_cache_dtype: t.dtype = t.bfloat16
    kv_scale_dtype: t.dtype = t.float32
    scale_granularity: str = "token_head"

    def __post_init__(self):
        sizes = (self.num_blocks, self.block_size, self.max_cache_slots, self.cache_max_seq_len)
        if not all(_is_positive_int(value) for value in sizes):
            raise ValueError("All cache dimensions must be positive integers.")
        if self.block_size & (self.block_size - 1):
            raise ValueError("Block size must be a power of 2.")
        if self.kv_cache_dtype not in SUPPORTED_CACHE_DTYPES:
            raise ValueError(
                "KVCache dtype must be in: [t.float16, t.bfloat16, t.float32, t.float8_e4m3fn]"
            )
        if self.kv_scale_dtype != t.float32:
            raise ValueError("KVScale dtype must be t.float32")
        if self.scale_granularity != "token_head":
            raise ValueError("scale granularity is only supported for token_head")

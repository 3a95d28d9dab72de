"""MI355X-native FP8 paged KV-cache path (gfx950 HIP kernels behind the torch_llm API).

Module layout mirrors the reference package `torch_llm` so callers swap the import
prefix only:
  aiproj_amd.inference.kvcache_config   <- torch_llm.inference.kvcache_config
  aiproj_amd.inference.paged_kv_cache   <- torch_llm.inference.paged_kv_cache
  aiproj_amd.inference.page_allocator   <- torch_llm.inference.page_allocator
  aiproj_amd.kernals.kv_cache.quantized_append <- torch_llm.kernals.kv_cache.quantized_append
  aiproj_amd.kernals.decode_attention   <- torch_llm.kernals.decode_attention
"""

__version__ = "0.1.0"

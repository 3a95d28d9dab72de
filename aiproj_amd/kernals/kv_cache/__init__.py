"""KV-cache write kernels (reference `torch_llm/kernals/kv_cache`)."""

"""Paged KV-cache storage, configuration and page metadata (reference `torch_llm/inference`)."""

"""Model pieces on the FP8 paged KV-cache path (mirrors reference `torch_llm.model`)."""

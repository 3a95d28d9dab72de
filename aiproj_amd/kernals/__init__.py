"""Kernel wrappers (reference `torch_llm/kernals`; the reference's spelling is kept)."""

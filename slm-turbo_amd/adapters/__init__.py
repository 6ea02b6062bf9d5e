"""Serving-framework adapters of the packed 4-bit KV path (vLLM backend)."""

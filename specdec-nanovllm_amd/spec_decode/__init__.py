"""Speculative-decoding verification on the gfx950 kernels (mirrors nanovllm.spec_decode)."""

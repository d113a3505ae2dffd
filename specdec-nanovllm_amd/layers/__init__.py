"""Mirror of ``nanovllm.layers`` (attention call site, W8A16 linear)."""

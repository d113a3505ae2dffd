"""Mirror of ``nanovllm.kernels`` (paged decode attention entry points)."""

"""Mirror of ``nanovllm.utils`` (forward context)."""

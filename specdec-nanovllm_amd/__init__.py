"""specdec_nanovllm_amd — MI355X (gfx950) decode hot path of specdec-nanovllm.

Hand-written HIP kernels behind a C ABI (``include/specdec_amd.h``,
``libspecdec_amd.so``): paged decode/verify attention (with the
``store_kvcache`` slot write fused in, or standalone), the W8A16 int8
weight-only linear, the draft step's neighbour ops (RMSNorm, q/k norm + RoPE,
SiLU*up, sampling) and rejection-sampling verification. ``ops`` holds the
torch-facing wrappers; ``kernels``, ``layers``, ``spec_decode``, ``utils`` and
``flash_attn_compat`` mirror the reference modules of the same names so the
reference can switch with an import swap.

The directory name carries a hyphen, so it is imported under the name
``specdec_nanovllm_amd`` (``__graft_entry__.load_package()`` registers it).
"""
from . import ops
from .ops import paged_attention, store_kvcache, w8a16_linear

__all__ = ["ops", "paged_attention", "store_kvcache", "w8a16_linear"]

"""specdec_nanovllm_amd — MI355X (gfx950) decode hot path of specdec-nanovllm.

Three hand-written HIP kernels behind a C ABI (``include/specdec_amd.h``,
``libspecdec_amd.so``): paged decode/verify attention, the ``store_kvcache``
slot write and the W8A16 int8 weight-only linear. ``ops`` holds the
torch-facing wrappers; ``kernels``, ``layers``, ``utils`` and
``flash_attn_compat`` mirror the reference modules of the same names so the
reference can switch with an import swap.

The directory name carries a hyphen, so it is imported under the name
``specdec_nanovllm_amd`` (``__graft_entry__.load_package()`` registers it).
"""
from . import ops
from .ops import paged_attention, store_kvcache, w8a16_linear

__all__ = ["ops", "paged_attention", "store_kvcache", "w8a16_linear"]

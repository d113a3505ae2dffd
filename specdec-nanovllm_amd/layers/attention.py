"""Attention call site — drop-in for ``nanovllm/layers/attention.py``.

``store_kvcache`` keeps the reference signature and asserts
(attention.py:33-40) and runs the gfx950 slot-write kernel. ``Attention`` keeps
the constructor and ``forward(q, k, v)`` contract (attention.py:43-82): write
the new K/V rows through the slot mapping, then

* decode (``not context.is_prefill``): paged attention of one query row per
  sequence over ``context_lens`` keys; the output has flash-attn's
  (B, 1, Hq, D) shape, as at attention.py:77-81;
* verify / prefix-cache prefill (``block_tables`` set): paged varlen attention
  with bottom-right causal masking, (total_q, Hq, D).

Plain prefill over contiguous k/v is not on the decode path and raises
``NotImplementedError``.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import ops
from ..flash_attn_compat import flash_attn_varlen_func, flash_attn_with_kvcache
from ..utils.context import get_context


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor):
    ops.store_kvcache(key, value, k_cache, v_cache, slot_mapping)


class Attention(nn.Module):

    def __init__(self, num_heads, head_dim, scale, num_kv_heads):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
        context = get_context()
        k_cache, v_cache = self.k_cache, self.v_cache
        if k_cache.numel() and v_cache.numel():
            store_kvcache(k, v, k_cache, v_cache, context.slot_mapping)
        if context.is_prefill:
            if context.block_tables is None:
                raise NotImplementedError("prefill over contiguous k/v is outside the decode "
                                          "hot path served by this library")
            return flash_attn_varlen_func(q, k_cache, v_cache,
                                          max_seqlen_q=context.max_seqlen_q,
                                          cu_seqlens_q=context.cu_seqlens_q,
                                          max_seqlen_k=context.max_seqlen_k,
                                          cu_seqlens_k=context.cu_seqlens_k,
                                          softmax_scale=self.scale, causal=True,
                                          block_table=context.block_tables)
        # q is (B, Hq, D), or (Hq, D) when the batch holds one sequence.
        q_in = q.unsqueeze(0).unsqueeze(0) if q.dim() == 2 else q.unsqueeze(1)
        return flash_attn_with_kvcache(q_in, k_cache, v_cache,
                                       cache_seqlens=context.context_lens,
                                       block_table=context.block_tables,
                                       softmax_scale=self.scale, causal=True)

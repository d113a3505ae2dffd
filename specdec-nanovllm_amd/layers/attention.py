"""Attention call site — drop-in for ``nanovllm/layers/attention.py``.

``store_kvcache`` keeps the reference signature and asserts
(attention.py:33-40) and runs the gfx950 slot-write kernel. ``Attention`` keeps
the constructor and ``forward(q, k, v)`` contract (attention.py:43-82): write
the new K/V rows through the slot mapping, then (both in one fused launch)

* decode (``not context.is_prefill``): paged attention of one query row per
  sequence over ``context_lens`` keys; the output has flash-attn's
  (B, 1, Hq, D) shape, as at attention.py:77-81;
* verify / prefix-cache prefill (``block_tables`` set): paged varlen attention
  with bottom-right causal masking, (total_q, Hq, D);
* plain prefill (contiguous k / v, no block table): the store, then the
  varlen causal prefill kernel over the contiguous rows.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import ops
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
        has_cache = bool(k_cache.numel() and v_cache.numel())
        if context.is_prefill:  # attention.py:62-70
            G = self.num_heads // self.num_kv_heads
            if (has_cache and context.block_tables is not None
                    and G * int(context.max_seqlen_q) <= 32):
                # speculative verify / short prefix-cache rows: store_kvcache of k / v
                # and the paged attention in one call
                return ops.paged_attention(q, k_cache, v_cache, context.block_tables,
                                           self.scale, cu_seqlens_k=context.cu_seqlens_k,
                                           cu_seqlens_q=context.cu_seqlens_q,
                                           max_seqlen_q=int(context.max_seqlen_q),
                                           key=k, value=v, slot_mapping=context.slot_mapping)
            if has_cache:
                store_kvcache(k, v, k_cache, v_cache, context.slot_mapping)
            if context.block_tables is not None:  # prefix cache: keys come from the pages
                if not has_cache:
                    raise RuntimeError("prefix-cached prefill needs the paged k_cache / v_cache")
                k, v = k_cache, v_cache
            return ops.prefill_attention(q, k, v, context.cu_seqlens_q, context.cu_seqlens_k,
                                         int(context.max_seqlen_q), self.scale,
                                         block_table=context.block_tables)
        if not has_cache:
            raise RuntimeError("Attention needs its paged k_cache / v_cache")
        # decode (attention.py:71-81): q is (B, Hq, D), or (Hq, D) for one sequence;
        # the result has flash_attn_with_kvcache's (B, 1, Hq, D) shape
        if q.dim() == 2:
            q, k, v = q.unsqueeze(0), k.reshape(1, *k.shape[-2:]), v.reshape(1, *v.shape[-2:])
        if not (q.stride(-1) == 1 and q.stride(0) % 8 == 0 and q.stride(1) % 8 == 0):
            q = q.contiguous()
        o = ops.paged_attention(q, k_cache, v_cache, context.block_tables, self.scale,
                                context_lens=context.context_lens,
                                key=k, value=v, slot_mapping=context.slot_mapping)
        return o.unsqueeze(1)

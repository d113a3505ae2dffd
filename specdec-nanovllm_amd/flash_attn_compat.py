"""The two flash-attn entry points the reference engine calls, restricted to
the paged cases on the decode hot path and served by the gfx950 kernel.

* ``flash_attn_with_kvcache`` — the decode call at
  nanovllm/layers/attention.py:78-81 (``q`` of shape (B, S, Hq, D) against the
  paged cache, ``cache_seqlens`` keys per sequence, bottom-right causal).
* ``flash_attn_varlen_func`` with ``block_table`` — the speculative-verify
  call at attention.py:67-70 (``cu_seqlens_q`` steps of k+1 rows,
  ``cu_seqlens_k[b+1] - cu_seqlens_k[b]`` keys, bottom-right causal), as set
  up by ``prepare_verify`` (nanovllm/engine/model_runner.py:492-584).

* ``flash_attn_varlen_func`` without ``block_table`` (or with one and many
  rows per sequence) — the prefill call at attention.py:64-70, contiguous K/V
  (or the prefix-cached pages), served by the prefill kernel.

Supported: head_dim 128; causal (bottom-right) whenever a sequence has several
query rows. The decode kernel takes (Hq / Hkv) * q rows per sequence <= 32 (decode
and verify); longer query blocks go to the prefill kernel.
"""
from __future__ import annotations

import torch

from . import ops


def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, rotary_cos=None,
                            rotary_sin=None, cache_seqlens=None, cache_batch_idx=None,
                            block_table=None, softmax_scale=None, causal=False, **unused):
    """Paged attention of ``q`` (B, S, Hq, D) over the cache; returns (B, S, Hq, D)."""
    if k is not None or v is not None or rotary_cos is not None or cache_batch_idx is not None:
        raise NotImplementedError("only the read-only paged form is supported "
                                  "(write new K/V with store_kvcache first)")
    if block_table is None or cache_seqlens is None:
        raise NotImplementedError("paged KV (block_table, cache_seqlens) is required")
    B, S, Hq, D = q.shape
    if S > 1 and not causal:
        raise NotImplementedError("non-causal attention with several query rows")
    scale = softmax_scale if softmax_scale is not None else D ** -0.5
    if isinstance(cache_seqlens, int):
        cache_seqlens = torch.full((B,), cache_seqlens, dtype=torch.int32, device=q.device)
    q2 = q.reshape(B * S, Hq, D)
    if not (q2.stride(-1) == 1 and q2.stride(0) % 8 == 0 and q2.stride(1) % 8 == 0):
        q2 = q2.contiguous()
    cu_q = None
    if S > 1:
        cu_q = torch.arange(0, (B + 1) * S, S, dtype=torch.int32, device=q.device)
    o = ops.paged_attention(q2, k_cache, v_cache, block_table, scale,
                            context_lens=cache_seqlens, cu_seqlens_q=cu_q, max_seqlen_q=S)
    return o.view(B, S, Hq, D)


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                           dropout_p=0.0, softmax_scale=None, causal=False, block_table=None,
                           **unused):
    """Variable-length attention of ``q`` (total_q, Hq, D); ``k``/``v`` are the
    paged caches when ``block_table`` is given, contiguous (total_k, Hkv, D)
    rows otherwise. Returns (total_q, Hq, D)."""
    if dropout_p:
        raise NotImplementedError("dropout")
    if int(max_seqlen_q) > 1 and not causal:
        raise NotImplementedError("non-causal attention with several query rows")
    scale = softmax_scale if softmax_scale is not None else q.shape[-1] ** -0.5
    if block_table is not None and (q.shape[1] // k.shape[2]) * int(max_seqlen_q) <= 32:
        return ops.paged_attention(q, k, v, block_table, scale, cu_seqlens_k=cu_seqlens_k,
                                   cu_seqlens_q=cu_seqlens_q, max_seqlen_q=int(max_seqlen_q))
    return ops.prefill_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q), scale,
                                 block_table=block_table)

"""Paged decode attention — drop-in for ``nanovllm/kernels/paged_decode_attn.py``.

The reference module offers three Triton kernels (v1 per query head, v2
GQA-shared, v3 split-KV + combine) behind ``paged_decode_attention``
(paged_decode_attn.py:352-469). All three compute the same math; here every
version runs the one gfx950 kernel (GQA-shared K/V, split-KV across
workgroups, MFMA for Q.K^T and P.V), whose split plan is chosen by the
library. The Triton tuning knobs (``block_n``, ``splits``, ``num_warps``,
``num_stages``) are accepted for signature compatibility and ignored.

Shapes (as the reference):
    q           : (num_seqs, num_q_heads, head_dim)            bf16 / fp16
    k_cache     : (num_blocks, block_size, num_kv_heads, head_dim)  "interleaved"
                  (num_blocks, num_kv_heads, block_size, head_dim)  "head_major"
    block_table : (num_seqs, max_blocks) int32, unused columns -1
    context_lens: (num_seqs,) int32
    returns     : (num_seqs, num_q_heads, head_dim)
"""
from __future__ import annotations

from .. import ops


def paged_decode_attention(q, k_cache, v_cache, block_table, context_lens, scale,
                           version=2, block_n=128, splits=8,
                           num_warps=None, num_stages=None, layout="interleaved"):
    """Paged decode attention (one query token per sequence).

    Raises ``ValueError`` for an unknown ``version`` and ``AssertionError``
    when num_q_heads is not a multiple of num_kv_heads, as the reference does
    (paged_decode_attn.py:384-385, 467-468).
    """
    if version not in (1, 2, 3):
        raise ValueError(f"unknown version: {version}")
    del block_n, splits, num_warps, num_stages
    return ops.paged_attention(q.contiguous(), k_cache, v_cache, block_table, scale,
                               context_lens=context_lens, layout=layout)

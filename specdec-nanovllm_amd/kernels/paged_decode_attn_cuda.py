"""Drop-in for ``nanovllm/kernels/paged_decode_attn_cuda.py``.

The reference JIT-compiles a CUDA sm_86 kernel and exposes
``paged_decode_attention_cuda`` (full call) and
``paged_decode_attention_cuda_partial`` (main kernel only, for timing)
(paged_decode_attn_cuda.py:52-91). Here both call the prebuilt gfx950 library;
nothing is compiled at import time. The reference kernel only accepts GQA
ratio 4 and head_dim 128 (paged_decode_attn_cuda.cu:1406-1407); this one takes
any ratio with ratio * q_len <= 32 at head_dim 128. ``splits``, ``block_n``,
``warps``, ``stages`` and ``fused`` are accepted and ignored.
"""
from __future__ import annotations

from .. import ops


def paged_decode_attention_cuda(q, k_cache, v_cache, block_table, context_lens,
                                scale, splits=8, block_n=64, warps=4, stages=3,
                                fused=True):
    """Paged decode attention; returns (num_seqs, num_q_heads, head_dim)."""
    del splits, block_n, warps, stages, fused
    return ops.paged_attention(q.contiguous(), k_cache, v_cache, block_table, scale,
                               context_lens=context_lens)


def paged_decode_attention_cuda_partial(q, k_cache, v_cache, block_table,
                                        context_lens, scale, splits=8,
                                        block_n=64, warps=4, stages=3, fused=None):
    """Run only the split-KV main kernel (no combine) so its time can be
    measured alone. Returns the output tensor, in which only sequences that
    fit in a single split are final (the reference returns its raw partial
    max buffer instead; both are timing aids, not results)."""
    del splits, block_n, warps, stages, fused
    return ops.paged_attention(q.contiguous(), k_cache, v_cache, block_table, scale,
                               context_lens=context_lens, main_only=True)

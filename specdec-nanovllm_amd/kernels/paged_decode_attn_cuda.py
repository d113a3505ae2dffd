"""Drop-in for ``nanovllm/kernels/paged_decode_attn_cuda.py``.

The reference JIT-compiles a CUDA sm_86 kernel and exposes
``paged_decode_attention_cuda`` (full call) and
``paged_decode_attention_cuda_partial`` (main kernel only, for timing)
(paged_decode_attn_cuda.py:52-91); its extension also exports the combine-only
and read-only measurement twins (paged_decode_attn_cuda.cu:1544-1555,1244-1281),
served here by ``paged_decode_attention_cuda_combine`` and
``paged_decode_attention_cuda_read_only``. All call the prebuilt gfx950 library;
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


def paged_decode_attention_cuda_combine(q, k_cache, v_cache, block_table, context_lens,
                                        scale, workspace, out):
    """Run only the merge kernel over ``workspace`` as a
    ``paged_decode_attention_cuda_partial``-style call (``ops.paged_attention``
    with ``twin="main"`` and the same workspace) left it, finishing ``out``."""
    return ops.paged_attention(q.contiguous(), k_cache, v_cache, block_table, scale,
                               context_lens=context_lens, twin="combine",
                               workspace=workspace, out=out)


def paged_decode_attention_cuda_read_only(q, k_cache, v_cache, block_table, context_lens,
                                          splits=8, block_n=64, warps=4, stages=3):
    """The main kernel's loads alone (same grid, order and prefetch), no math and
    no output: the access pattern's floor. ``q`` fixes the GQA ratio of the
    plan; it is read as the main kernel reads it. Returns nothing useful."""
    del splits, block_n, warps, stages
    ops.paged_attention(q.contiguous(), k_cache, v_cache, block_table, q.shape[-1] ** -0.5,
                        context_lens=context_lens, twin="floor")

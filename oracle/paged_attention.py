"""Paged decode / verify attention restated in numpy (float64 by default).

Test infrastructure only (see oracle/__init__.py).

Per sequence b (nanovllm/kernels/paged_decode_attn.py:472-495):
  1. gather the pages block_table[b, :ceil(L/bs)] of the cache and keep the
     first L rows -> K, V of shape (L, Hkv, D)                (:486-489)
  2. query head h uses kv head h // G, G = Hq / Hkv — the reference
     repeat_interleaves K/V over heads (:490-491); here the same pairing is
     done by grouping the query heads per kv head, which multiplies the same
     numbers without materialising the copies
  3. logits = q . K^T * scale, softmax over keys, times V       (:492-494)
  4. L == 0 -> zeros                                            (:483-485)
Verify (q_len n > 1, nanovllm/layers/attention.py:64-70 with causal=True and
nanovllm/engine/model_runner.py:522-533): query row i of a sequence with L
keys sees keys [0, L - n + i] (flash-attn's bottom-right causal alignment;
the rows sit at positions L-n .. L-1). A row that sees no key outputs zeros.
"""
import numpy as np


def gather_pages(cache: np.ndarray, bt_row, L: int, block_size: int) -> np.ndarray:
    """(L, Hkv, D) rows of one sequence from a (num_blocks, bs, Hkv, D) cache."""
    nblk = -(-L // block_size)
    phys = np.asarray(bt_row[:nblk], dtype=np.int64)
    return cache[phys].reshape(nblk * block_size, cache.shape[2], cache.shape[3])[:L]


def attend(qs: np.ndarray, K: np.ndarray, V: np.ndarray, scale: float,
           dtype=np.float64) -> np.ndarray:
    """Bottom-right causal attention of nq query rows (nq, Hq, D) over L keys
    K, V (L, Hkv, D) -> (nq, Hq, D)."""
    nq, Hq, D = qs.shape
    L, Hkv, _ = K.shape
    G = Hq // Hkv
    out = np.zeros((nq, Hq, D), dtype=dtype)
    if L == 0 or nq == 0:
        return out
    qg = qs.astype(dtype).reshape(nq, Hkv, G, D).transpose(1, 0, 2, 3).reshape(Hkv, nq * G, D)
    kt = K.astype(dtype).transpose(1, 2, 0)            # (Hkv, D, L)
    vv = V.astype(dtype).transpose(1, 0, 2)            # (Hkv, L, D)
    logits = np.matmul(qg, kt) * dtype(scale)          # (Hkv, nq*G, L), row = i*G + g
    last = L - nq + np.repeat(np.arange(nq), G)        # last visible key per row
    masked = np.arange(L)[None, :] > last[:, None]     # (nq*G, L)
    logits = np.where(masked[None], -np.inf, logits)
    seen = ~masked.all(axis=1)                         # rows with at least one key
    m = np.where(seen[None, :, None], logits.max(axis=2, keepdims=True), 0.0)
    p = np.exp(logits - m)
    p /= np.where(seen[None, :, None], p.sum(axis=2, keepdims=True), 1.0)
    o = np.matmul(p, vv)                               # (Hkv, nq*G, D)
    o = o.reshape(Hkv, nq, G, D).transpose(1, 0, 2, 3).reshape(nq, Hq, D)
    return o.astype(dtype)


def paged_attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                    block_table: np.ndarray, context_lens, scale: float,
                    cu_seqlens_q=None, dtype=np.float64) -> np.ndarray:
    """q (total_q, Hq, D); caches (num_blocks, bs, Hkv, D); block_table (B, W);
    context_lens (B,) keys per sequence; cu_seqlens_q (B+1,) or None (one row
    per sequence). Returns (total_q, Hq, D) in ``dtype``."""
    q = np.asarray(q)
    bs = k_cache.shape[1]
    out = np.zeros(q.shape, dtype=dtype)
    for b in range(len(context_lens)):
        L = int(context_lens[b])
        if cu_seqlens_q is None:
            q0, nq = b, 1
        else:
            q0, nq = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1]) - int(cu_seqlens_q[b])
        if L <= 0 or nq <= 0:
            continue
        K = gather_pages(k_cache, block_table[b], L, bs)
        V = gather_pages(v_cache, block_table[b], L, bs)
        out[q0:q0 + nq] = attend(q[q0:q0 + nq], K, V, scale, dtype)
    return out


def algorithmic_bytes(context_lens, num_q_heads, num_kv_heads, head_dim, elem_bytes,
                      q_rows_per_seq=1):
    """Bytes a decode/verify step must move at minimum: every visible K and V
    row once, q read and o written once (block tables and lengths excluded)."""
    kv = sum(int(L) for L in context_lens) * num_kv_heads * head_dim * elem_bytes * 2
    qo = 2 * len(context_lens) * q_rows_per_seq * num_q_heads * head_dim * elem_bytes
    return kv + qo

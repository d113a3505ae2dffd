"""Paged KV-cache addressing and the store_kvcache scatter (numpy, bit-exact).

Test infrastructure only (see oracle/__init__.py).
"""
import numpy as np

PAD_SLOT = -1  # nanovllm/spec_decode/graph_pad.py:33 — slot -1 writes nothing


def slot_of(block_table_row: np.ndarray, pos, block_size: int):
    """Flat cache slot of key position(s) ``pos`` of one sequence:
    ``block_table[pos // bs] * bs + pos % bs``
    (nanovllm/engine/model_runner.py:475 for decode, :535-548 for verify,
    nanovllm/spec_decode/draft_proposer.py:527-550 for draft steps)."""
    pos = np.asarray(pos, dtype=np.int64)
    return np.asarray(block_table_row, dtype=np.int64)[pos // block_size] * block_size + \
        pos % block_size


def decode_slots(block_tables, context_lens, block_size):
    """Slot of the newest token (position len-1) of each sequence
    (nanovllm/engine/model_runner.py:466-482)."""
    return np.array([slot_of(bt, int(L) - 1, block_size) for bt, L in
                     zip(block_tables, context_lens)], dtype=np.int32)


def verify_slots(block_tables, lens, k, block_size):
    """Slots of positions len-1 .. len+k-1 for each sequence, concatenated
    (nanovllm/engine/model_runner.py:522-548: n = k+1 rows starting at len-1)."""
    out = []
    for bt, L in zip(block_tables, lens):
        out.extend(slot_of(bt, np.arange(int(L) - 1, int(L) + k), block_size).tolist())
    return np.array(out, dtype=np.int32)


def store_kvcache(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray,
                  v_cache: np.ndarray, slot_mapping: np.ndarray) -> None:
    """In-place scatter: for every i with slot s = slot_mapping[i] != -1, the
    (num_kv_heads, head_dim) rows key[i] / value[i] become cache rows
    (s // block_size, s % block_size) — nanovllm/layers/attention.py:21-30
    (``cache.flat[s*D:(s+1)*D] = key[i]`` with D = num_kv_heads * head_dim).
    Works on any element type (use uint16 views for bf16: pure bit copy)."""
    assert k_cache.flags.c_contiguous and v_cache.flags.c_contiguous, \
        "caches must be C-contiguous so the flat slot view aliases them"
    n = key.shape[0]
    D = key.shape[1] * key.shape[2]
    kflat = k_cache.reshape(-1, D)
    vflat = v_cache.reshape(-1, D)
    for i in range(n):
        s = int(slot_mapping[i])
        if s == PAD_SLOT:
            continue
        kflat[s] = key[i].reshape(D)
        vflat[s] = value[i].reshape(D)

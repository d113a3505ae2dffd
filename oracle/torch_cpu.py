"""The reference's CPU paths restated in torch (fp32 on the host) — TEST
INFRASTRUCTURE ONLY (see oracle/__init__.py): the timed CPU baseline of
bench.py, pinned against this package's numpy restatement in
tests/test_oracle_torch_cpu.py.

  paged_attention  per sequence: gather the pages, softmax(q K^T scale) V in
                   fp32, zeros for a sequence without keys
                   (nanovllm/kernels/paged_decode_attn.py:472-495), with the
                   bottom-right causal rows of verify when cu_seqlens_q is
                   given (nanovllm/layers/attention.py:64-70)
  dequant_linear   fp32 q * scale (per channel), then x @ W^T
                   (nanovllm/layers/quant.py:151-159)
  store_kvcache    row i of key / value to slot slot_mapping[i], -1 skipped
                   (nanovllm/layers/attention.py:10-40)
"""
import torch


def paged_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    block_table: torch.Tensor, context_lens, scale: float,
                    cu_seqlens_q=None) -> torch.Tensor:
    """q (total_q, Hq, D) fp32; caches (num_blocks, bs, Hkv, D); block_table
    (B, W); context_lens (B,) keys per sequence. Returns (total_q, Hq, D) fp32."""
    bs, Hkv, D = k_cache.shape[1], k_cache.shape[2], k_cache.shape[3]
    Hq = q.shape[1]
    G = Hq // Hkv
    out = torch.zeros(q.shape, dtype=torch.float32)
    for b in range(len(context_lens)):
        L = int(context_lens[b])
        if cu_seqlens_q is None:
            q0, nq = b, 1
        else:
            q0, nq = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1]) - int(cu_seqlens_q[b])
        if L <= 0 or nq <= 0:
            continue
        pages = block_table[b, :(L + bs - 1) // bs].long()
        K = k_cache[pages].reshape(-1, Hkv, D)[:L].float().permute(1, 2, 0)  # (Hkv, D, L)
        V = v_cache[pages].reshape(-1, Hkv, D)[:L].float().transpose(0, 1)   # (Hkv, L, D)
        qs = q[q0:q0 + nq].float().reshape(nq, Hkv, G, D).permute(1, 0, 2, 3)
        s = torch.matmul(qs.reshape(Hkv, nq * G, D), K) * scale               # (Hkv, nq*G, L)
        if nq > 1:
            last = L - nq + torch.arange(nq).repeat_interleave(G)            # row i*G+g
            s = s.masked_fill(torch.arange(L)[None, :] > last[:, None], float("-inf"))
        o = torch.matmul(torch.softmax(s, dim=-1), V)                         # (Hkv, nq*G, D)
        out[q0:q0 + nq] = o.reshape(Hkv, nq, G, D).permute(1, 0, 2, 3).reshape(nq, Hq, D)
    return out


def dequant_linear(x: torch.Tensor, qweight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """fp32 dequantize-then-matmul with a per-channel scale: x (M, K), qweight
    (N, K) int8, scale (N,) -> (M, N) fp32."""
    w = qweight.to(torch.float32) * scale.to(torch.float32)[:, None]
    return x.float() @ w.T


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """In place: cache row slot_mapping[i] (flattened over blocks and positions)
    gets key[i] / value[i]; slot -1 leaves the cache as it is."""
    keep = slot_mapping >= 0
    rows = slot_mapping[keep].long()
    width = key.shape[1] * key.shape[2]
    k_cache.view(-1, width)[rows] = key.reshape(-1, width)[keep]
    v_cache.view(-1, width)[rows] = value.reshape(-1, width)[keep]

"""Seeded synthetic inputs for the configurations the hot path is measured on.

C1  paged decode, Qwen3-0.6B attention geometry (16q / 8kv / 128), B=1, L=1000,
    64-block pool, block table = 4 blocks of a seeded permutation.
C2  paged decode, Qwen3-4B attention geometry (32q / 8kv / 128), B in {1,8,32},
    L ~ U[512, 4096], 2048-block pool, one new K/V row per sequence written
    through slot_mapping before attention.
C3  speculative verify at Qwen3-4B geometry: B=8, q_len = k+1 = 7, len ~
    U[1500, 2600], slots for positions len-1 .. len+5, keys [0, len+6).
C4  W8A16 linear: w = clip(round(N(0,1) * 40), +-127) int8, per-channel fp16
    scales ~ U[1e-3, 4e-3], x ~ N(0,1) fp16, M in {1,7,16,56}, Qwen3-0.6B shapes.

Index data (lengths, tables, slots) comes from a CPU ``torch.Generator`` so it
is identical on every machine; the large K/V pools are drawn on the device.
"""
from __future__ import annotations

import math

import torch

QWEN3_4B_ATTN = dict(num_q_heads=32, num_kv_heads=8, head_dim=128)
QWEN3_06B_ATTN = dict(num_q_heads=16, num_kv_heads=8, head_dim=128)
# (name, N, K) of the Qwen3-0.6B linears (C4)
W8A16_SHAPES = [("qkv", 4096, 1024), ("gate_up", 6144, 1024), ("down", 1024, 3072),
                ("o_proj", 1024, 2048), ("lm_head", 151936, 1024)]
W8A16_MS = (1, 7, 16, 56)


def _randn(shape, gen, device, dtype):
    return torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(dtype)


def device_generator(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def block_tables_for(lens, block_size: int, num_blocks: int, gen: torch.Generator,
                     width: int | None = None, sets: int = 1):
    """``sets`` block tables for the same lengths, each a run of consecutive
    entries of one seeded permutation of the pool (so sets never share a page),
    padded with -1 to ``width`` columns."""
    need = [math.ceil(int(L) / block_size) for L in lens]
    width = width or max(max(need), 1)
    total = sum(need)
    if total * sets > num_blocks:
        raise ValueError(f"{sets} sets x {total} pages exceed the {num_blocks}-page pool")
    perm = torch.randperm(num_blocks, generator=gen).to(torch.int32)
    tables = []
    used = 0
    for _ in range(sets):
        bt = torch.full((len(lens), width), -1, dtype=torch.int32)
        for b, n in enumerate(need):
            bt[b, :n] = perm[used:used + n]
            used += n
        tables.append(bt)
    return tables


def slots_for(bt: torch.Tensor, positions_per_seq, block_size: int) -> torch.Tensor:
    """Flat slots ``bt[p // bs] * bs + p % bs`` of the given positions, concatenated."""
    out = []
    for b, positions in enumerate(positions_per_seq):
        for p in positions:
            out.append(int(bt[b, p // block_size]) * block_size + p % block_size)
    return torch.tensor(out, dtype=torch.int32)


def decode_case(batch: int, *, num_q_heads=32, num_kv_heads=8, head_dim=128, block_size=256,
                num_blocks=2048, ctx_range=(512, 4096), width=None, seed=0, sets=1,
                dtype=torch.bfloat16, device="cuda"):
    """C2-style decode step inputs. Lengths count the new token (position L-1)."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(ctx_range[0], ctx_range[1] + 1, (batch,), generator=g, dtype=torch.int32)
    if width is None:
        width = math.ceil(ctx_range[1] / block_size)
    tables = block_tables_for(lens.tolist(), block_size, num_blocks, g, width, sets)
    dg = device_generator(device, seed + 1)
    cache_shape = (num_blocks, block_size, num_kv_heads, head_dim)
    case = dict(
        lens=lens, tables=tables, block_size=block_size,
        num_q_heads=num_q_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
        k_cache=_randn(cache_shape, dg, device, dtype),
        v_cache=_randn(cache_shape, dg, device, dtype),
        q=_randn((batch, num_q_heads, head_dim), dg, device, dtype),
        k_new=_randn((batch, num_kv_heads, head_dim), dg, device, dtype),
        v_new=_randn((batch, num_kv_heads, head_dim), dg, device, dtype),
        slots=[slots_for(bt, [[int(L) - 1] for L in lens], block_size) for bt in tables],
        scale=head_dim ** -0.5,
    )
    return case


def verify_case(batch: int = 8, k: int = 6, *, num_q_heads=32, num_kv_heads=8, head_dim=128,
                block_size=256, num_blocks=2048, len_range=(1500, 2600), seed=0,
                dtype=torch.bfloat16, device="cuda", sets: int = 1):
    """C3 speculative-verify inputs: ``k+1`` query rows per sequence at positions
    len-1 .. len+k-1, keys [0, len+k). ``keys`` = len + k per sequence.

    The lengths come from the first seed >= ``seed`` for which at least one
    sequence's k+1 rows straddle a page boundary (C3 requires such a row);
    ``seed_used`` records it. ``sets`` > 1 adds ``tables`` / ``slot_sets``:
    that many block tables over disjoint pages of the pool (the first is
    ``table``) with their slots, for timing on pages not yet read."""
    for s in range(seed, seed + 1000):
        g = torch.Generator().manual_seed(s)
        lens = torch.randint(len_range[0], len_range[1] + 1, (batch,), generator=g,
                             dtype=torch.int32)
        if k == 0 or any((int(L) - 1) // block_size != (int(L) + k - 1) // block_size
                         for L in lens):
            break
    seed = s
    keys = lens + k
    width = math.ceil((len_range[1] + k) / block_size)
    tables = block_tables_for(keys.tolist(), block_size, num_blocks, g, width, sets)
    bt = tables[0]
    n = k + 1
    cu_q = torch.arange(0, (batch + 1) * n, n, dtype=torch.int32)
    cu_k = torch.zeros(batch + 1, dtype=torch.int32)
    cu_k[1:] = torch.cumsum(keys, 0)
    positions = [list(range(int(L) - 1, int(L) + k)) for L in lens]
    dg = device_generator(device, seed + 1)
    cache_shape = (num_blocks, block_size, num_kv_heads, head_dim)
    return dict(
        seed_used=seed,
        lens=lens, keys=keys, table=bt, cu_q=cu_q, cu_k=cu_k, k=k, block_size=block_size,
        num_q_heads=num_q_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
        crosses_page=any((int(L) - 1) // block_size != (int(L) + k - 1) // block_size
                         for L in lens),
        k_cache=_randn(cache_shape, dg, device, dtype),
        v_cache=_randn(cache_shape, dg, device, dtype),
        q=_randn((batch * n, num_q_heads, head_dim), dg, device, dtype),
        k_new=_randn((batch * n, num_kv_heads, head_dim), dg, device, dtype),
        v_new=_randn((batch * n, num_kv_heads, head_dim), dg, device, dtype),
        slots=slots_for(bt, positions, block_size),
        tables=tables,
        slot_sets=[slots_for(t, positions, block_size) for t in tables],
        scale=head_dim ** -0.5,
    )


def w8a16_case(M: int, N: int, K: int, *, seed=0, act_dtype=torch.float16,
               scale_dtype=torch.float16, device="cuda"):
    """C4 inputs: int8 weight, per-channel scale, activation."""
    g = device_generator(device, seed)
    w = torch.clamp(torch.round(torch.randn((N, K), generator=g, device=device) * 40),
                    -127, 127).to(torch.int8)
    s = (torch.rand((N,), generator=g, device=device) * 3e-3 + 1e-3).to(scale_dtype)
    x = torch.randn((M, K), generator=g, device=device).to(act_dtype)
    return dict(w=w, s=s, x=x)

"""Write the committed fixtures in tests/golden/ (run: python tests/golden/make_golden.py).

The reference repository ships no golden vectors for the decode hot path, so
these fixtures are produced here from seeded numpy inputs and torch LIBRARY
routines only — never from the oracle under test:
  * attention: torch.nn.functional.scaled_dot_product_attention (float64),
    with ``enable_gqa=True`` for the head grouping and
    ``torch.nn.attention.bias.causal_lower_right`` for flash-attn's
    bottom-right causal alignment of verify rows;
  * W8A16: torch.nn.functional.linear on float64 dequantized weights;
  * store_kvcache: torch ``index_copy_`` on the flat (slot, Hkv*D) cache view.
Large inputs are not stored: they are regenerated from the recorded seed with
numpy's PCG64 (bit-stable across platforms) and checked against stored sums.
"""
import os

import numpy as np
import torch
import torch.nn.functional as F
from torch.nn.attention.bias import causal_lower_right

HERE = os.path.dirname(os.path.abspath(__file__))


def c1_inputs(seed=0):
    """C1: Qwen3-0.6B attention geometry, B=1, L=1000, 64-block pool of 256
    tokens, table = 4 pages of a seeded permutation; q, K, V ~ N(0, 1) fp32."""
    rng = np.random.Generator(np.random.PCG64(seed))
    q = rng.standard_normal((1, 16, 128), dtype=np.float32)
    k = rng.standard_normal((64, 256, 8, 128), dtype=np.float32)
    v = rng.standard_normal((64, 256, 8, 128), dtype=np.float32)
    bt = rng.permutation(64)[:4].astype(np.int32).reshape(1, 4)
    return q, k, v, bt, np.array([1000], dtype=np.int32)


def sdpa_paged(q, k, v, bt_row, L, nq, scale):
    """Library attention of nq rows over the first L rows of the listed pages."""
    kt = torch.from_numpy(k).double()[torch.from_numpy(bt_row).long()]
    vt = torch.from_numpy(v).double()[torch.from_numpy(bt_row).long()]
    kt = kt.reshape(-1, k.shape[2], k.shape[3])[:L]          # (L, Hkv, D)
    vt = vt.reshape(-1, v.shape[2], v.shape[3])[:L]
    qt = torch.from_numpy(q).double().permute(1, 0, 2)[None]  # (1, Hq, nq, D)
    kt = kt.permute(1, 0, 2)[None]
    vt = vt.permute(1, 0, 2)[None]
    mask = causal_lower_right(nq, L) if nq > 1 else None
    o = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale,
                                       enable_gqa=True)
    return o[0].permute(1, 0, 2).numpy()                      # (nq, Hq, D)


def make_c1():
    q, k, v, bt, lens = c1_inputs(0)
    out = sdpa_paged(q, k, v, bt[0], int(lens[0]), 1, 128 ** -0.5)
    np.savez_compressed(os.path.join(HERE, "c1_decode.npz"), seed=0, block_table=bt,
                        context_lens=lens, scale=128 ** -0.5, out=out,
                        q_sum=np.float64(q.sum(dtype=np.float64)),
                        k_sum=np.float64(k.sum(dtype=np.float64)),
                        v_sum=np.float64(v.sum(dtype=np.float64)))


def make_verify():
    """Small verify case: 2 sequences, 3 query rows each, GQA 4/2, D=16,
    page 4, keys 7 and 10 spread over permuted pages (rows cross pages)."""
    rng = np.random.Generator(np.random.PCG64(1))
    nblk, bs, hkv, hq, d, nq = 8, 4, 2, 4, 16, 3
    k = rng.standard_normal((nblk, bs, hkv, d), dtype=np.float32)
    v = rng.standard_normal((nblk, bs, hkv, d), dtype=np.float32)
    lens = np.array([7, 10], dtype=np.int32)
    perm = rng.permutation(nblk).astype(np.int32)
    bt = np.full((2, 3), -1, dtype=np.int32)
    bt[0, :2] = perm[:2]
    bt[1, :3] = perm[2:5]
    q = rng.standard_normal((2 * nq, hq, d), dtype=np.float32)
    cu_q = np.array([0, 3, 6], dtype=np.int32)
    out = np.concatenate([sdpa_paged(q[cu_q[b]:cu_q[b + 1]], k, v, bt[b][bt[b] >= 0],
                                     int(lens[b]), nq, 0.3) for b in range(2)])
    np.savez_compressed(os.path.join(HERE, "verify_small.npz"), q=q, k_cache=k, v_cache=v,
                        block_table=bt, context_lens=lens, cu_seqlens_q=cu_q, scale=0.3,
                        out=out)


def make_w8a16():
    rng = np.random.Generator(np.random.PCG64(2))
    M, N, K, G = 3, 48, 128, 64
    x = rng.standard_normal((M, K)).astype(np.float16)
    w = np.clip(np.rint(rng.standard_normal((N, K)) * 40), -127, 127).astype(np.int8)
    s = rng.uniform(1e-3, 4e-3, N).astype(np.float16)
    sg = rng.uniform(1e-3, 4e-3, (N, K // G)).astype(np.float16)
    bias = rng.standard_normal(N).astype(np.float16)
    xt = torch.from_numpy(x).double()
    wt = torch.from_numpy(w).double()
    y = F.linear(xt, wt * torch.from_numpy(s).double()[:, None], torch.from_numpy(bias).double())
    wg = (wt.view(N, K // G, G) * torch.from_numpy(sg).double()[:, :, None]).view(N, K)
    yg = F.linear(xt, wg)
    np.savez_compressed(os.path.join(HERE, "w8a16_small.npz"), x=x, w=w, scale=s,
                        scale_group=sg, group_size=G, bias=bias, y=y.numpy(),
                        y_group=yg.numpy())


def make_store():
    rng = np.random.Generator(np.random.PCG64(3))
    nblk, bs, hkv, d, n = 3, 4, 2, 4, 5
    kc = rng.integers(0, 2 ** 16, (nblk, bs, hkv, d), dtype=np.uint16)
    vc = rng.integers(0, 2 ** 16, (nblk, bs, hkv, d), dtype=np.uint16)
    key = rng.integers(0, 2 ** 16, (n, hkv, d), dtype=np.uint16)
    val = rng.integers(0, 2 ** 16, (n, hkv, d), dtype=np.uint16)
    slots = np.array([0, 5, -1, 11, 6], dtype=np.int32)
    keep = slots != -1
    idx = torch.from_numpy(slots[keep].astype(np.int64))
    ek = torch.from_numpy(kc.astype(np.int32)).view(-1, hkv * d)
    ev = torch.from_numpy(vc.astype(np.int32)).view(-1, hkv * d)
    ek.index_copy_(0, idx, torch.from_numpy(key[keep].astype(np.int32)).view(-1, hkv * d))
    ev.index_copy_(0, idx, torch.from_numpy(val[keep].astype(np.int32)).view(-1, hkv * d))
    np.savez_compressed(os.path.join(HERE, "store_small.npz"), k_cache=kc, v_cache=vc,
                        key=key, value=val, slot_mapping=slots,
                        k_expected=ek.numpy().astype(np.uint16).reshape(kc.shape),
                        v_expected=ev.numpy().astype(np.uint16).reshape(vc.shape))


if __name__ == "__main__":
    make_c1()
    make_verify()
    make_w8a16()
    make_store()
    print("fixtures written to", HERE)

"""GPU parity of the variable-length causal (prefill) attention kernel
(csrc/prefill_attention.hip, through the C ABI) against float64 attention on
the CPU of the same 16-bit inputs (the oracle's ``attend``): per sequence,
softmax(q K^T * scale) V with row t seeing keys [0, nk - nq + t] (bottom-right
causal, flash-attn varlen semantics, nanovllm/layers/attention.py:64-70). Tolerance as for decode:
|o - ref| <= 2e-3 + 1e-2 |ref|. Covers contiguous K/V batches with ragged
lengths (1 .. 513 rows, tile edges), GQA ratios 1 / 4 / 8, fp16, the
prefix-cached paged form (nk > nq), the flash_attn_varlen_func dispatch and
the attention layer's prefill branch with its store_kvcache.
"""
import math

import numpy as np
import pytest
import torch

from conftest import assert_close_attn, to_np
from oracle import paged_attention as opa
from specdec_nanovllm_amd import ops, workloads
from specdec_nanovllm_amd.flash_attn_compat import flash_attn_varlen_func
from specdec_nanovllm_amd.layers.attention import Attention
from specdec_nanovllm_amd.utils.context import reset_context, set_context

pytestmark = pytest.mark.gpu
DEV = "cuda"


def ref_varlen(q, k, v, cu_q, cu_k, scale):
    """float64 per-sequence bottom-right causal attention, k/v (total_k, Hkv, D):
    the pinned oracle's ``attend`` (checked against torch SDPA with
    causal_lower_right in tests/test_oracle_attention.py) on each sequence."""
    q, k, v = to_np(q.float()), to_np(k.float()), to_np(v.float())
    out = np.zeros(q.shape, dtype=np.float64)
    for b in range(len(cu_q) - 1):
        qs, qe, ks, ke = int(cu_q[b]), int(cu_q[b + 1]), int(cu_k[b]), int(cu_k[b + 1])
        out[qs:qe] = opa.attend(q[qs:qe], k[ks:ke], v[ks:ke], scale)
    return out


def make(lens_q, lens_k, hq, hkv, dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    tq, tk = sum(lens_q), sum(lens_k)
    q = torch.randn((tq, hq, 128), generator=g).to(dtype)
    k = torch.randn((tk, hkv, 128), generator=g).to(dtype)
    v = torch.randn((tk, hkv, 128), generator=g).to(dtype)
    cu_q = torch.tensor([0] + list(np.cumsum(lens_q)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(lens_k)), dtype=torch.int32)
    return q, k, v, cu_q, cu_k


@pytest.mark.parametrize("hq,hkv,dtype", [(32, 8, torch.bfloat16), (8, 8, torch.bfloat16),
                                          (32, 4, torch.float16), (16, 8, torch.float16)])
def test_contiguous_varlen_causal(hq, hkv, dtype):
    lens = [1, 17, 64, 200, 513, 16, 15]
    q, k, v, cu_q, cu_k = make(lens, lens, hq, hkv, dtype, seed=hq + hkv)
    scale = 128 ** -0.5
    o = ops.prefill_attention(q.to(DEV), k.to(DEV), v.to(DEV), cu_q.to(DEV), cu_k.to(DEV),
                              max(lens), scale)
    assert_close_attn(to_np(o.float()), ref_varlen(q, k, v, cu_q, cu_k, scale),
                      what=f"prefill {hq}/{hkv} {dtype}")


def test_more_keys_than_queries_and_empty_sequences():
    # chunked-prefill shape (nk > nq: earlier keys fully visible) plus empty rows/keys
    lq, lk = [40, 0, 7, 100], [300, 5, 7, 100]
    q, k, v, cu_q, cu_k = make(lq, lk, 32, 8, seed=3)
    o = ops.prefill_attention(q.to(DEV), k.to(DEV), v.to(DEV), cu_q.to(DEV), cu_k.to(DEV),
                              max(lq), 0.1)
    assert_close_attn(to_np(o.float()), ref_varlen(q, k, v, cu_q, cu_k, 0.1), what="nk > nq")


def test_fewer_keys_than_queries():
    # nk < nq: under the bottom-right rule the first nq - nk rows see no key (zeros) and
    # the rest see a growing prefix; tiles past the few-key tiles still run
    lq, lk = [600, 40], [500, 1]
    q, k, v, cu_q, cu_k = make(lq, lk, 32, 8, seed=13)
    o = to_np(ops.prefill_attention(q.to(DEV), k.to(DEV), v.to(DEV), cu_q.to(DEV),
                                    cu_k.to(DEV), max(lq), 0.1).float())
    ref = ref_varlen(q, k, v, cu_q, cu_k, 0.1)
    seen = np.zeros(sum(lq), dtype=bool)  # rows that see at least one key
    for b in range(len(lq)):
        t = np.arange(lq[b])
        seen[int(cu_q[b]) + t] = lk[b] - lq[b] + t >= 0
    assert np.all(o[~seen] == 0)
    assert_close_attn(o[seen], ref[seen], what="nk < nq")


def _paged(k, v, cu_k, bs, seed):
    """Scatter contiguous k/v rows into a shuffled page pool; returns caches + table."""
    lens = (cu_k[1:] - cu_k[:-1]).tolist()
    g = torch.Generator().manual_seed(seed)
    need = sum(math.ceil(L / bs) for L in lens)
    nblk = need + 3
    perm = torch.randperm(nblk, generator=g)
    width = max(math.ceil(L / bs) for L in lens)
    bt = torch.full((len(lens), width), -1, dtype=torch.int32)
    kc = torch.randn((nblk, bs) + tuple(k.shape[1:]), generator=g).to(k.dtype)
    vc = torch.randn((nblk, bs) + tuple(v.shape[1:]), generator=g).to(v.dtype)
    n = 0
    for b, L in enumerate(lens):
        for pgi in range(math.ceil(L / bs)):
            blk = int(perm[n])
            n += 1
            bt[b, pgi] = blk
            a, e = pgi * bs, min(L, (pgi + 1) * bs)
            kc[blk, : e - a] = k[int(cu_k[b]) + a: int(cu_k[b]) + e]
            vc[blk, : e - a] = v[int(cu_k[b]) + a: int(cu_k[b]) + e]
    return kc, vc, bt


@pytest.mark.parametrize("bs", [256, 16])
def test_paged_prefix_cache(bs):
    lq, lk = [300, 33, 1], [1000, 33, 129]
    q, k, v, cu_q, cu_k = make(lq, lk, 32, 8, seed=bs)
    kc, vc, bt = _paged(k, v, cu_k, bs, seed=bs)
    scale = 128 ** -0.5
    o = ops.prefill_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), cu_q.to(DEV), cu_k.to(DEV),
                              max(lq), scale, block_table=bt.to(DEV))
    assert_close_attn(to_np(o.float()), ref_varlen(q, k, v, cu_q, cu_k, scale),
                      what=f"paged prefill bs={bs}")


def test_flash_attn_varlen_dispatch():
    lens = [50, 120]
    q, k, v, cu_q, cu_k = make(lens, lens, 32, 8, seed=9)
    ref = ref_varlen(q, k, v, cu_q, cu_k, 0.09)
    o = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), cu_q.to(DEV), cu_k.to(DEV),
                               max(lens), max(lens), softmax_scale=0.09, causal=True)
    assert_close_attn(to_np(o.float()), ref, what="compat contiguous")
    kc, vc, bt = _paged(k, v, cu_k, 256, seed=9)
    o = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), cu_q.to(DEV), cu_k.to(DEV),
                               max(lens), max(lens), softmax_scale=0.09, causal=True,
                               block_table=bt.to(DEV))
    assert_close_attn(to_np(o.float()), ref, what="compat paged long q")


def test_attention_layer_prefill_stores_and_attends():
    lens = [70, 9]
    q, k, v, cu_q, cu_k = make(lens, lens, 32, 8, seed=11)
    layer = Attention(32, 128, 128 ** -0.5, 8)
    nblk, bs = 8, 256
    layer.k_cache = torch.zeros((nblk, bs, 8, 128), dtype=torch.bfloat16, device=DEV)
    layer.v_cache = torch.zeros_like(layer.k_cache)
    bt = torch.tensor([[3, -1], [5, -1]], dtype=torch.int32)
    slots = workloads.slots_for(bt, [list(range(L)) for L in lens], bs)
    set_context(True, cu_seqlens_q=cu_q.to(DEV), cu_seqlens_k=cu_k.to(DEV),
                max_seqlen_q=max(lens), max_seqlen_k=max(lens), slot_mapping=slots.to(DEV))
    try:
        o = layer(q.to(DEV), k.to(DEV), v.to(DEV))
    finally:
        reset_context()
    assert_close_attn(to_np(o.float()), ref_varlen(q, k, v, cu_q, cu_k, 128 ** -0.5),
                      what="layer prefill")
    assert torch.equal(layer.k_cache[3, :70].cpu(), k[:70]) and torch.equal(layer.v_cache[5, :9].cpu(), v[70:])

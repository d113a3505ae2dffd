"""Pins of the attention oracle (CPU only).

Each check is chosen so a plausible slip in oracle/paged_attention.py fails
it: a wrong page/offset index (placement invariance, brute force, golden), a
wrong GQA head pairing (library SDPA with enable_gqa, repeated heads), a wrong
causal alignment (library causal_lower_right, verify golden), a dropped scale
or softmax normaliser (closed forms, brute force).
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention.bias import causal_lower_right

from oracle import paged_attention as opa

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _pool(rng, nblk, bs, hkv, d):
    return (rng.standard_normal((nblk, bs, hkv, d)), rng.standard_normal((nblk, bs, hkv, d)))


def _table(rng, lens, bs, nblk, width=None):
    need = [math.ceil(L / bs) for L in lens]
    width = width or max(max(need), 1)
    perm = rng.permutation(nblk)
    bt = np.full((len(lens), width), -1, dtype=np.int64)
    used = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[used:used + n]
        used += n
    return bt


def test_c1_golden_from_library_sdpa():
    g = np.load(os.path.join(GOLDEN, "c1_decode.npz"))
    rng = np.random.Generator(np.random.PCG64(int(g["seed"])))
    q = rng.standard_normal((1, 16, 128), dtype=np.float32)
    k = rng.standard_normal((64, 256, 8, 128), dtype=np.float32)
    v = rng.standard_normal((64, 256, 8, 128), dtype=np.float32)
    bt = rng.permutation(64)[:4].astype(np.int32).reshape(1, 4)
    assert np.array_equal(bt, g["block_table"])
    assert k.sum(dtype=np.float64) == g["k_sum"] and v.sum(dtype=np.float64) == g["v_sum"]
    assert q.sum(dtype=np.float64) == g["q_sum"]
    out = opa.paged_attention(q, k, v, bt, g["context_lens"], float(g["scale"]))
    np.testing.assert_allclose(out, g["out"], rtol=1e-12, atol=1e-13)
    # the fp32 restatement (the CPU baseline leg) agrees to fp32 precision
    out32 = opa.paged_attention(q, k, v, bt, g["context_lens"], float(g["scale"]),
                                dtype=np.float32)
    np.testing.assert_allclose(out32, g["out"], rtol=1e-4, atol=1e-5)


def test_verify_golden_bottom_right_causal():
    g = np.load(os.path.join(GOLDEN, "verify_small.npz"))
    out = opa.paged_attention(g["q"], g["k_cache"], g["v_cache"], g["block_table"],
                              g["context_lens"], float(g["scale"]), g["cu_seqlens_q"])
    np.testing.assert_allclose(out, g["out"], rtol=1e-12, atol=1e-13)


@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 8), (8, 8), (6, 2)])
def test_decode_matches_library_sdpa(hq, hkv):
    rng = np.random.default_rng(hq + hkv)
    bs, d = 16, 32
    lens = [1, 15, 16, 17, 50]
    bt = _table(rng, lens, bs, 20)
    k, v = _pool(rng, 20, bs, hkv, d)
    q = rng.standard_normal((len(lens), hq, d))
    out = opa.paged_attention(q, k, v, bt, lens, 0.2)
    for b, L in enumerate(lens):
        K = torch.from_numpy(k[bt[b, :math.ceil(L / bs)]].reshape(-1, hkv, d)[:L])
        V = torch.from_numpy(v[bt[b, :math.ceil(L / bs)]].reshape(-1, hkv, d)[:L])
        ref = F.scaled_dot_product_attention(
            torch.from_numpy(q[b]).view(1, hq, 1, d), K.permute(1, 0, 2)[None],
            V.permute(1, 0, 2)[None], scale=0.2, enable_gqa=True)[0, :, 0]
        np.testing.assert_allclose(out[b], ref.numpy(), rtol=1e-12, atol=1e-13)


@pytest.mark.parametrize("nq,L", [(7, 7), (7, 20), (3, 100), (2, 1), (5, 3)])
def test_verify_mask_matches_causal_lower_right(nq, L):
    rng = np.random.default_rng(nq * 1000 + L)
    hq, hkv, d, bs = 4, 2, 8, 8
    bt = _table(rng, [L], bs, 16)
    k, v = _pool(rng, 16, bs, hkv, d)
    q = rng.standard_normal((nq, hq, d))
    out = opa.paged_attention(q, k, v, bt, [L], 0.5, np.array([0, nq]))
    K = torch.from_numpy(k[bt[0, :math.ceil(L / bs)]].reshape(-1, hkv, d)[:L])
    V = torch.from_numpy(v[bt[0, :math.ceil(L / bs)]].reshape(-1, hkv, d)[:L])
    mask = causal_lower_right(nq, L)._materialize(device="cpu")
    qt = torch.from_numpy(q).permute(1, 0, 2)[None]
    ref = F.scaled_dot_product_attention(qt, K.permute(1, 0, 2)[None].repeat_interleave(2, 1),
                                         V.permute(1, 0, 2)[None].repeat_interleave(2, 1),
                                         attn_mask=mask, scale=0.5)[0].permute(1, 0, 2).numpy()
    seen = mask.any(dim=1).numpy()  # rows with no visible key are zero in the oracle
    np.testing.assert_allclose(out[seen], ref[seen], rtol=1e-12, atol=1e-13)
    assert np.all(out[~seen] == 0)


def test_uniform_keys_average_values():
    # all keys equal -> every logit equal -> softmax uniform -> mean of V rows
    rng = np.random.default_rng(5)
    bs, L = 8, 21
    k = np.ones((4, bs, 2, 4))
    v = rng.standard_normal((4, bs, 2, 4))
    bt = np.array([[2, 0, 3]])
    q = rng.standard_normal((1, 4, 4))
    out = opa.paged_attention(q, k, v, bt, [L], 1.0)
    rows = v[[2, 0, 3]].reshape(-1, 2, 4)[:L]
    np.testing.assert_allclose(out[0, :2], np.repeat(rows.mean(0)[:1], 2, 0), rtol=1e-12)
    np.testing.assert_allclose(out[0, 2:], np.repeat(rows.mean(0)[1:], 2, 0), rtol=1e-12)


def test_one_dominant_key_selects_its_value():
    bs, d = 4, 8
    k = np.zeros((3, bs, 1, d))
    v = np.arange(3 * bs * d, dtype=np.float64).reshape(3, bs, 1, d)
    k[1, 2, 0, 0] = 1.0          # position 4 + 2 = 6 in table order [0, 1, 2]
    q = np.zeros((1, 1, d))
    q[0, 0, 0] = 1e4
    out = opa.paged_attention(q, k, v, np.array([[0, 1, 2]]), [10], 1.0)
    np.testing.assert_allclose(out[0, 0], v[1, 2, 0], rtol=1e-12)


def test_zero_length_rows_are_zero():
    rng = np.random.default_rng(6)
    k, v = _pool(rng, 4, 8, 2, 4)
    q = rng.standard_normal((2, 4, 4))
    out = opa.paged_attention(q, k, v, np.array([[0], [-1]]), [0, 0], 1.0)
    assert np.all(out == 0)


def test_placement_and_padding_invariance():
    rng = np.random.default_rng(7)
    bs, hkv, d = 8, 2, 8
    lens = [30, 9]
    bt = _table(rng, lens, bs, 12)
    k, v = _pool(rng, 12, bs, hkv, d)
    q = rng.standard_normal((2, 4, d))
    out = opa.paged_attention(q, k, v, bt, lens, 0.3)
    perm = rng.permutation(12)          # move page p to perm[p]
    k2, v2 = np.empty_like(k), np.empty_like(v)
    k2[perm], v2[perm] = k, v
    bt2 = np.full((2, bt.shape[1] + 3), -1)
    bt2[:, :bt.shape[1]] = np.where(bt >= 0, perm[np.maximum(bt, 0)], -1)
    np.testing.assert_array_equal(opa.paged_attention(q, k2, v2, bt2, lens, 0.3), out)


def test_gqa_equals_repeated_kv_heads():
    rng = np.random.default_rng(8)
    bs, d = 8, 8
    k, v = _pool(rng, 6, bs, 2, d)
    bt = np.array([[4, 1, 5]])
    q = rng.standard_normal((1, 6, d))
    out = opa.paged_attention(q, k, v, bt, [19], 0.4)
    rep = opa.paged_attention(q, np.repeat(k, 3, axis=2), np.repeat(v, 3, axis=2), bt, [19], 0.4)
    np.testing.assert_allclose(out, rep, rtol=1e-13, atol=1e-14)


def test_verify_single_row_equals_decode():
    rng = np.random.default_rng(9)
    k, v = _pool(rng, 6, 8, 2, 8)
    bt = np.array([[3, 0, 4], [5, 1, -1]])
    q = rng.standard_normal((2, 4, 8))
    dec = opa.paged_attention(q, k, v, bt, [20, 16], 0.4)
    ver = opa.paged_attention(q, k, v, bt, [20, 16], 0.4, np.array([0, 1, 2]))
    np.testing.assert_array_equal(dec, ver)


def test_brute_force_loops_tiny():
    rng = np.random.default_rng(10)
    bs, hq, hkv, d = 3, 4, 2, 3
    k, v = _pool(rng, 5, bs, hkv, d)
    bt = np.array([[4, 2, 0], [1, 3, -1]])
    lens = [8, 4]
    cu = np.array([0, 2, 5])
    q = rng.standard_normal((5, hq, d))
    out = opa.paged_attention(q, k, v, bt, lens, 0.7, cu)
    for b in range(2):
        L, nq = lens[b], cu[b + 1] - cu[b]
        for i in range(nq):
            for h in range(hq):
                kvh = h // (hq // hkv)
                w = []
                for j in range(L - nq + i + 1):
                    page, off = bt[b][j // bs], j % bs
                    w.append(math.exp(0.7 * sum(q[cu[b] + i, h, t] * k[page, off, kvh, t]
                                                for t in range(d))))
                for t in range(d):
                    num = sum(w[j] * v[bt[b][j // bs], j % bs, kvh, t] for j in range(len(w)))
                    assert abs(out[cu[b] + i, h, t] - num / sum(w)) < 1e-12


def test_algorithmic_bytes_formula():
    # C2-style: per token K + V rows of 8 heads x 128 dims x 2 bytes = 4096 B
    b = opa.algorithmic_bytes([1000, 3], 32, 8, 128, 2)
    assert b == 1003 * 4096 + 2 * 2 * 32 * 128 * 2

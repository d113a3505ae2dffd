"""The torch-CPU restatement (the timed CPU baseline of bench.py) against the
numpy oracle, which the other oracle tests pin to library routines and closed
forms: decode and verify attention (GQA, ragged lengths, zero-length rows,
pages crossed by the verify rows), W8A16 dequantize-then-matmul, and the
slot scatter (bit-exact, -1 skipped)."""
import numpy as np
import torch

from oracle import kvcache as okv
from oracle import paged_attention as opa
from oracle import torch_cpu as otc
from oracle import w8a16 as ow8


def _case(lens, hq, hkv, bs=16, d=128, seed=0):
    rng = np.random.default_rng(seed)
    pages = sum(-(-L // bs) for L in lens) + 2
    kc = rng.standard_normal((pages, bs, hkv, d)).astype(np.float32)
    vc = rng.standard_normal((pages, bs, hkv, d)).astype(np.float32)
    perm = rng.permutation(pages)
    width = max(max(-(-L // bs) for L in lens), 1)
    bt = np.full((len(lens), width), -1, dtype=np.int64)
    used = 0
    for b, L in enumerate(lens):
        n = -(-L // bs)
        bt[b, :n] = perm[used:used + n]
        used += n
    return rng, kc, vc, bt


def test_decode_matches_numpy_oracle():
    lens = [1, 0, 37, 100, 64]
    rng, kc, vc, bt = _case(lens, 16, 4)
    q = rng.standard_normal((len(lens), 16, 128)).astype(np.float32)
    want = opa.paged_attention(q, kc, vc, bt, lens, 0.088)
    got = otc.paged_attention(torch.from_numpy(q), torch.from_numpy(kc), torch.from_numpy(vc),
                              torch.from_numpy(bt), lens, 0.088).numpy()
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)
    assert not got[1].any()  # no keys: zeros


def test_verify_rows_match_numpy_oracle():
    lens = [40, 17, 3]  # keys per sequence; 7 / 2 / 3 query rows, bottom-right causal
    cu = np.array([0, 7, 9, 12])
    rng, kc, vc, bt = _case(lens, 8, 8)
    q = rng.standard_normal((12, 8, 128)).astype(np.float32)
    want = opa.paged_attention(q, kc, vc, bt, lens, 0.1, cu)
    got = otc.paged_attention(torch.from_numpy(q), torch.from_numpy(kc), torch.from_numpy(vc),
                              torch.from_numpy(bt), lens, 0.1, torch.from_numpy(cu)).numpy()
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)


def test_dequant_linear_matches_numpy_oracle():
    rng = np.random.default_rng(3)
    w = np.clip(np.rint(rng.standard_normal((96, 128)) * 40), -127, 127).astype(np.int8)
    s = rng.uniform(1e-3, 4e-3, 96).astype(np.float32)
    x = rng.standard_normal((5, 128)).astype(np.float32)
    want = ow8.int8_linear(x, w, s)
    got = otc.dequant_linear(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(s))
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-5, atol=1e-6)


def test_store_matches_numpy_oracle_bitwise():
    rng = np.random.default_rng(4)
    kc = rng.standard_normal((6, 16, 2, 128)).astype(np.float32)
    vc = rng.standard_normal((6, 16, 2, 128)).astype(np.float32)
    key = rng.standard_normal((5, 2, 128)).astype(np.float32)
    val = rng.standard_normal((5, 2, 128)).astype(np.float32)
    slots = np.array([3, -1, 95, 17, 40], dtype=np.int32)
    kt, vt = torch.from_numpy(kc.copy()), torch.from_numpy(vc.copy())
    otc.store_kvcache(torch.from_numpy(key), torch.from_numpy(val), kt, vt, torch.from_numpy(slots))
    okv.store_kvcache(key, val, kc, vc, slots)
    assert np.array_equal(kt.numpy(), kc) and np.array_equal(vt.numpy(), vc)

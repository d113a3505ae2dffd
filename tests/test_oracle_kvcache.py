"""Pins of the KV-cache addressing / scatter oracle (CPU only)."""
import os

import numpy as np

from oracle import kvcache as okv

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_store_golden_from_index_copy():
    g = np.load(os.path.join(GOLDEN, "store_small.npz"))
    kc, vc = g["k_cache"].copy(), g["v_cache"].copy()
    okv.store_kvcache(g["key"], g["value"], kc, vc, g["slot_mapping"])
    assert np.array_equal(kc, g["k_expected"]) and np.array_equal(vc, g["v_expected"])


def test_store_brute_force_and_pad_slot():
    rng = np.random.default_rng(0)
    nblk, bs, hkv, d = 4, 8, 2, 3
    kc = rng.integers(0, 65536, (nblk, bs, hkv, d), dtype=np.uint16)
    vc = rng.integers(0, 65536, (nblk, bs, hkv, d), dtype=np.uint16)
    key = rng.integers(0, 65536, (6, hkv, d), dtype=np.uint16)
    val = rng.integers(0, 65536, (6, hkv, d), dtype=np.uint16)
    slots = np.array([3, -1, 8, 31, 16, -1], dtype=np.int32)
    k0, v0 = kc.copy(), vc.copy()
    okv.store_kvcache(key, val, kc, vc, slots)
    for blk in range(nblk):
        for off in range(bs):
            s = blk * bs + off
            hit = [i for i in range(6) if slots[i] == s]
            ek = key[hit[0]] if hit else k0[blk, off]
            ev = val[hit[0]] if hit else v0[blk, off]
            assert np.array_equal(kc[blk, off], ek) and np.array_equal(vc[blk, off], ev)


def test_slot_formula_closed_form():
    bt = np.array([7, 2, 9])
    bs = 256
    assert okv.slot_of(bt, 0, bs) == 7 * 256
    assert okv.slot_of(bt, 255, bs) == 7 * 256 + 255
    assert okv.slot_of(bt, 256, bs) == 2 * 256
    assert okv.slot_of(bt, 600, bs) == 9 * 256 + 88
    np.testing.assert_array_equal(okv.slot_of(bt, np.arange(254, 259), bs),
                                  [7 * 256 + 254, 7 * 256 + 255, 512, 513, 514])


def test_decode_and_verify_slot_positions():
    # decode writes position len-1; verify writes len-1 .. len+k-1 (k+1 rows)
    bt = np.array([[5, 1, 3], [0, 4, -1]])
    lens = np.array([256, 300])
    np.testing.assert_array_equal(okv.decode_slots(bt, lens, 256), [5 * 256 + 255, 4 * 256 + 43])
    v = okv.verify_slots(bt, lens, 2, 256)
    np.testing.assert_array_equal(v, [5 * 256 + 255, 256, 257, 4 * 256 + 43, 4 * 256 + 44,
                                      4 * 256 + 45])

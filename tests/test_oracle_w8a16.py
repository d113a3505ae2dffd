"""Pins of the W8A16 oracle (CPU only): dequantize-then-matmul against torch's
F.linear (golden), closed forms for the quantizer (round half to even, amax
row -> +-127, the 1e-8 floor), and per-group == per-channel when the group
scales of a row are equal."""
import os

import numpy as np
import torch

from oracle import bf16 as obf16
from oracle import w8a16 as ow8

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_linear_golden_from_library():
    g = np.load(os.path.join(GOLDEN, "w8a16_small.npz"))
    y = ow8.int8_linear(g["x"], g["w"], g["scale"], g["bias"])
    np.testing.assert_allclose(y, g["y"], rtol=1e-13, atol=1e-13)
    yg = ow8.int8_linear(g["x"], g["w"], g["scale_group"], None, "per_group", int(g["group_size"]))
    np.testing.assert_allclose(yg, g["y_group"], rtol=1e-13, atol=1e-13)


def test_per_group_equals_per_channel_with_equal_group_scales():
    rng = np.random.default_rng(1)
    w = rng.integers(-127, 128, (8, 256)).astype(np.int8)
    s = rng.uniform(1e-3, 4e-3, 8)
    x = rng.standard_normal((3, 256))
    a = ow8.int8_linear(x, w, s)
    b = ow8.int8_linear(x, w, np.repeat(s[:, None], 4, 1), None, "per_group", 64)
    np.testing.assert_allclose(a, b, rtol=1e-14)


def test_identity_weight():
    x = np.random.default_rng(2).standard_normal((2, 16))
    w = (np.eye(16) * 50).astype(np.int8)
    np.testing.assert_allclose(ow8.int8_linear(x, w, np.full(16, 0.02)), x, rtol=1e-14)


def test_brute_force_tiny():
    rng = np.random.default_rng(3)
    w = rng.integers(-127, 128, (3, 4)).astype(np.int8)
    s = rng.uniform(0.5, 2.0, 3)
    x = rng.standard_normal((2, 4))
    bias = rng.standard_normal(3)
    y = ow8.int8_linear(x, w, s, bias)
    for m in range(2):
        for n in range(3):
            assert abs(y[m, n] - (sum(x[m, k] * int(w[n, k]) * s[n] for k in range(4)) +
                                  bias[n])) < 1e-12


def test_quantize_round_half_even_closed_form():
    # amax 127 -> scale exactly 1: q = round_half_even(w)
    w = np.array([[127.0, 63.5, -63.5, 0.5, 1.5, 2.5, -2.5, -127.0]], dtype=np.float32)
    q, s = ow8.quantize_weight(w)
    np.testing.assert_array_equal(q[0], [127, 64, -64, 0, 2, 2, -2, -127])
    assert s[0] == 1.0
    # torch.round is the reference's rounding and agrees
    assert torch.equal(torch.round(torch.from_numpy(w)).to(torch.int8), torch.from_numpy(q))


def test_quantize_extremes_and_floor():
    w = np.zeros((2, 8), dtype=np.float32)
    w[1, 3] = -3.0
    q, s = ow8.quantize_weight(w)
    assert np.all(q[0] == 0) and s[0] == obf16.round_f32(np.float32(1e-8))
    assert q[1, 3] == -127 and np.all(np.delete(q[1], 3) == 0)
    assert s[1] == obf16.round_f32(np.float32(3.0) / np.float32(127))


def test_quantize_per_group_closed_form():
    w = np.zeros((1, 8), dtype=np.float32)
    w[0, :4] = [1.0, -2.0, 0.5, 2.0]      # group 0 amax 2
    w[0, 4:] = [10.0, 0, 0, -5.0]         # group 1 amax 10
    q, s = ow8.quantize_weight(w, "per_group", 4)
    s0, s1 = np.float32(2.0) / np.float32(127), np.float32(10.0) / np.float32(127)
    np.testing.assert_array_equal(q[0], np.clip(np.rint(w[0] / np.repeat([s0, s1], 4)), -127, 127))
    np.testing.assert_array_equal(s[0], obf16.round_f32(np.array([s0, s1], dtype=np.float32)))


def test_bf16_rounding_matches_torch():
    x = np.random.default_rng(4).standard_normal(10000).astype(np.float32) * 100
    x[:4] = [1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 65504.0]  # ties
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(obf16.f32_to_bits(x), ref)


def test_algorithmic_bytes_formula():
    assert ow8.algorithmic_bytes(1, 151936, 1024) == 151936 * 1024 + 2 * 151936 + 2048 + 2 * 151936

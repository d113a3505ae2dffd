"""Pins of oracle/decoder_ops.py (CPU): the draft step's neighbour ops.

Each function is checked against something other than its own formula:
library routines in float64 (torch rms_norm / silu, complex rotation), closed
forms and exact invariants (constant rows, power-of-two scaling, position 0),
the published Philox4x32-10 known-answer vectors (Random123 kat_vectors), and
a chi-square test of the sampling law.
"""
import numpy as np
import pytest
import torch

from oracle import bf16
from oracle import decoder_ops as od


def bf16_vals(shape, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return bf16.round_f32((rng.standard_normal(shape) * scale).astype(np.float32))


def ulps(got, ref):
    """Distance in bf16 units of the larger magnitude (2^-7 relative per unit)."""
    mag = np.maximum(np.abs(ref), np.abs(got))
    unit = np.where(mag > 0, 2.0 ** (np.floor(np.log2(np.maximum(mag, 1e-30))) - 7), 1e-30)
    return np.abs(got - ref) / unit


# ------------------------------------------------------------------- RMSNorm
def test_rmsnorm_matches_float64_library_within_rounding():
    x = bf16_vals((7, 1024), 1)
    w = bf16_vals((1024,), 2, 0.1) + 1.0
    w = bf16.round_f32(w)
    got = od.rmsnorm(x, w, 1e-6)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (1024,),
                                       torch.from_numpy(w).double(), 1e-6).numpy()
    assert ulps(got, ref).max() <= 1.5  # two bf16 roundings


def test_rmsnorm_closed_forms():
    w = bf16.round_f32(np.linspace(0.5, 2.0, 64).astype(np.float32))
    # a constant row normalises to +-1, so the output is the weight (sign of c)
    for c in (3.0, -0.25):
        x = np.full((1, 64), c, np.float32)
        out = od.rmsnorm(x, w, 0.0)
        assert np.array_equal(out[0], bf16.round_f32(np.sign(c) * w))
    # power-of-two scaling of the row is exact end to end
    x = bf16_vals((3, 256), 3)
    w2 = bf16_vals((256,), 4)
    assert np.array_equal(od.rmsnorm(x, w2, 0.0), od.rmsnorm(x * 8.0, w2, 0.0))


def test_add_rmsnorm_residual_and_consistency():
    x = bf16_vals((5, 512), 5)
    r = bf16_vals((5, 512), 6)
    w = bf16_vals((512,), 7)
    out, res = od.add_rmsnorm(x, r, w, 1e-6)
    assert np.array_equal(res, bf16.round_f32(x + r))
    # a zero residual reduces to the plain norm, bit for bit
    out0, res0 = od.add_rmsnorm(x, np.zeros_like(x), w, 1e-6)
    assert np.array_equal(out0, od.rmsnorm(x, w, 1e-6)) and np.array_equal(res0, x)
    # the norm is of the fp32 sum, not of the rounded residual: they can differ
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x + r).double(), (512,),
                                       torch.from_numpy(w).double(), 1e-6).numpy()
    assert ulps(out, ref).max() <= 1.5


# ---------------------------------------------------------------------- RoPE
def test_rope_is_a_complex_rotation():
    T, H, D = 6, 4, 128
    x = bf16_vals((T, H, D), 8)
    cs = od.rope_cache(4096, D, 1e6)
    pos = np.array([0, 1, 17, 255, 1000, 4095])
    got = od.rope(x, pos, cs)
    z = (x[..., :64].astype(np.float64) + 1j * x[..., 64:].astype(np.float64))
    ang = np.exp(1j * np.arctan2(cs[pos, 64:], cs[pos, :64]).astype(np.float64))[:, None, :]
    rot = z * ang
    ref = np.concatenate([rot.real, rot.imag], axis=-1)
    assert np.abs(got - ref).max() <= 2.0 ** -7 * np.abs(ref).max() * 2
    # position 0: cos 1, sin 0, the identity
    assert np.array_equal(od.rope(x[:1], np.array([0]), cs), x[:1])


def test_rope_cache_closed_form():
    cs = od.rope_cache(2048, 128, 1e6)
    p = np.arange(2048, dtype=np.float64)[:, None]
    ang = p * (1e6 ** (-np.arange(0, 128, 2, dtype=np.float64) / 128))[None, :]
    # fp32 angles: absolute error about p * 2^-24 radians
    assert np.abs(cs[:, :64] - np.cos(ang)).max() < 5e-4
    assert np.abs(cs[:, 64:] - np.sin(ang)).max() < 5e-4
    assert np.array_equal(cs[0], np.r_[np.ones(64), np.zeros(64)].astype(np.float32))


def test_qk_norm_rope_composes():
    q = bf16_vals((3, 16, 128), 9)
    k = bf16_vals((3, 8, 128), 10)
    qw = bf16_vals((128,), 11)
    kw = bf16_vals((128,), 12)
    cs = od.rope_cache(64, 128, 1e6)
    pos = np.array([5, 0, 63])
    qo, ko = od.qk_norm_rope(q, k, pos, cs, qw, kw, 1e-6)
    assert np.array_equal(qo, od.rope(od.rmsnorm(q, qw, 1e-6), pos, cs))
    assert np.array_equal(ko, od.rope(od.rmsnorm(k, kw, 1e-6), pos, cs))
    qn, kn = od.qk_norm_rope(q, k, pos, cs)  # no weights: RoPE only
    assert np.array_equal(qn, od.rope(q, pos, cs))


# ------------------------------------------------------------------ SiLU*up
def test_silu_mul_matches_library():
    x = bf16_vals((4, 2 * 3072), 13, 3.0)
    got = od.silu_mul(x)
    g, u = torch.from_numpy(x[:, :3072]).double(), torch.from_numpy(x[:, 3072:]).double()
    ref = (torch.nn.functional.silu(g) * u).numpy()
    assert ulps(got, ref).max() <= 1.5
    z = np.zeros((1, 16), np.float32)
    z[0, 8:] = 5.0
    assert np.array_equal(od.silu_mul(z), np.zeros((1, 8), np.float32))  # silu(0) = 0


# ------------------------------------------------------------------ sampling
def test_philox_known_answers():
    # Random123 kat_vectors for philox4x32_10
    cases = [
        ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
        ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
        ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
         (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
    ]
    for c, k, want in cases:
        got = od.philox4x32_10(*c, *k)
        assert tuple(int(v) for v in got) == want


def test_argmax_first_brute_force():
    rng = np.random.default_rng(14)
    x = rng.integers(-3, 3, size=(50, 9)).astype(np.float32)  # many ties
    want = [min(i for i in range(9) if row[i] == row.max()) for row in x]
    assert od.argmax_first(x).tolist() == want


def test_sample_law_chi_square():
    rows, V, T = 40000, 5, 0.7
    logits = np.tile(np.array([1.0, 0.2, -0.5, 0.9, 0.0], np.float32), (rows, 1))
    toks = od.sample(logits, np.full(rows, T, np.float32), seed=1234, offset=7)
    p = np.exp(logits[0] / T) / np.exp(logits[0] / T).sum()
    counts = np.bincount(toks, minlength=V)
    chi2 = (((counts - rows * p) ** 2) / (rows * p)).sum()
    assert chi2 < 20.5  # 4 degrees of freedom, p ~ 4e-4


def test_sample_greedy_limits_and_determinism():
    rng = np.random.default_rng(15)
    logits = rng.standard_normal((64, 1000)).astype(np.float32)
    greedy = od.argmax_first(logits)
    assert np.array_equal(od.sample(logits, np.zeros(64, np.float32), 1, 0), greedy)
    # a tiny temperature makes the noise negligible next to the logit gaps
    assert np.array_equal(od.sample(logits, np.full(64, 1e-6, np.float32), 1, 0), greedy)
    a = od.sample(logits, np.ones(64, np.float32), 99, 5)
    assert np.array_equal(a, od.sample(logits, np.ones(64, np.float32), 99, 5))
    assert not np.array_equal(a, od.sample(logits, np.ones(64, np.float32), 99, 6))

"""GPU parity of the draft step's neighbour kernels (csrc/decoder_ops.hip,
through the C ABI) against oracle/decoder_ops.py on the same inputs.

Tolerances: the residual written by the fused add is bit-exact. The only
free choice elsewhere is the fp32 rsqrt / exp (an ulp apart between
implementations); an ulp there can flip the first of the two 16-bit roundings
of RMSNorm (x * r, then * w) or SiLU*up (silu, then * up), so these agree to
two units of the 16-bit output at each element's magnitude; q/k norm + RoPE
mixes two such values per output and agrees to four units of the head's
largest output. Greedy
argmax is exact (first index among ties, as torch.argmax); sampled tokens
equal the oracle's except where the oracle's two best race keys are within
1e-4 (fp32 log rounding), and follow softmax(l / T) by a chi-square test.
"""
import numpy as np
import pytest
import torch

from conftest import bits16, to_np
from oracle import decoder_ops as od
from specdec_nanovllm_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
DT = {"bf16": torch.bfloat16, "f16": torch.float16}


def rand(shape, seed, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def assert_units(got, ref, what, dt="bf16", units=2, per_row=False):
    """|got - ref| <= units x one unit of the 16-bit format (bf16 2^-7, fp16
    2^-10 relative) at each element's magnitude, or at the row's largest
    magnitude with per_row."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    mag = np.maximum(np.abs(got), np.abs(ref))
    if per_row:
        mag = np.broadcast_to(mag.max(axis=-1, keepdims=True), mag.shape)
    mant = {"bf16": 7, "f16": 10}[dt]
    unit = np.where(mag > 0, 2.0 ** (np.floor(np.log2(np.maximum(mag, 1e-30))) - mant), 0)
    bad = np.abs(got - ref) > units * unit + 1e-30
    assert not bad.any(), (f"{what}: {bad.sum()} elements beyond {units} units, worst "
                           f"{np.abs(got - ref).max():.3g}")


# ------------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("rows,H", [(1, 1024), (7, 1024), (56, 2560), (3, 128), (2, 8192)])
def test_rmsnorm(dt, rows, H):
    x = rand((rows, H), rows * 31 + H, DT[dt])
    w = (1 + rand((H,), H, DT[dt], 0.1)).to(DT[dt])
    got = ops.rmsnorm(x.to(DEV), w.to(DEV), 1e-6)
    ref = od.rmsnorm(to_np(x.float()), to_np(w.float()), 1e-6, dt)
    assert_units(to_np(got.float()), ref, f"rmsnorm {dt} {rows}x{H}", dt)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_add_rmsnorm_residual_exact(dt):
    x = rand((9, 1024), 1, DT[dt])
    r = rand((9, 1024), 2, DT[dt])
    w = rand((1024,), 3, DT[dt])
    out, res = ops.rmsnorm(x.to(DEV), w.to(DEV), 1e-6, residual=r.to(DEV))
    ref_out, ref_res = od.add_rmsnorm(to_np(x.float()), to_np(r.float()), to_np(w.float()),
                                      1e-6, dt)
    assert np.array_equal(to_np(res.float()), ref_res)
    assert_units(to_np(out.float()), ref_out, f"add_rmsnorm {dt}", dt)


def test_rmsnorm_in_place_aliases():
    x = rand((4, 1024), 4, torch.bfloat16).to(DEV)
    r = rand((4, 1024), 5, torch.bfloat16).to(DEV)
    w = rand((1024,), 6, torch.bfloat16).to(DEV)
    want_out, want_res = ops.rmsnorm(x, w, 1e-6, residual=r)
    # out over x, residual_out over the residual (the engine's in-place use)
    lib = __import__("specdec_nanovllm_amd._lib", fromlist=["x"])
    L = lib.load()
    rc = L.sd_rmsnorm(x.data_ptr(), 1024, r.data_ptr(), 1024, w.data_ptr(), x.data_ptr(), 1024,
                      r.data_ptr(), 1024, 4, 1024, 1e-6, lib.SD_BF16,
                      lib.stream_ptr(x.device))
    lib.check(rc)
    torch.cuda.synchronize()
    assert torch.equal(x, want_out) and torch.equal(r, want_res)


# ------------------------------------------------------------ q/k norm + RoPE
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("T,hq,hkv,norm", [(1, 16, 8, True), (16, 16, 8, True), (56, 32, 8, True),
                                            (5, 4, 2, False)])
def test_qk_norm_rope_in_place_on_qkv(dt, T, hq, hkv, norm):
    D = 128
    qkv = rand((T, (hq + 2 * hkv) * D), T * 7 + hq, DT[dt]).to(DEV)
    before = qkv.clone()
    q = qkv[:, :hq * D].view(T, hq, D)
    k = qkv[:, hq * D:(hq + hkv) * D].view(T, hkv, D)
    qw = rand((D,), 1, DT[dt]).to(DEV) if norm else None
    kw = rand((D,), 2, DT[dt]).to(DEV) if norm else None
    cs = torch.from_numpy(od.rope_cache(4096, D, 1e6)).to(DEV)
    g = torch.Generator().manual_seed(T)
    pos = torch.randint(0, 4096, (T,), generator=g)
    ops.qk_norm_rope(q, k, pos.to(DEV), cs, qw, kw, 1e-6)
    rq, rk = od.qk_norm_rope(to_np(before[:, :hq * D].view(T, hq, D).float()),
                             to_np(before[:, hq * D:(hq + hkv) * D].view(T, hkv, D).float()),
                             pos.numpy(), cs.cpu().numpy(),
                             None if qw is None else to_np(qw.float()),
                             None if kw is None else to_np(kw.float()), 1e-6, dt)
    assert_units(to_np(q.float()), rq, "q", dt, units=4, per_row=True)
    assert_units(to_np(k.float()), rk, "k", dt, units=4, per_row=True)
    # v is not touched
    assert np.array_equal(bits16(qkv[:, (hq + hkv) * D:]), bits16(before[:, (hq + hkv) * D:]))


def test_rope_position_zero_and_out_of_range():
    D = 128
    q = rand((3, 4, D), 11, torch.bfloat16).to(DEV)
    k = rand((3, 2, D), 12, torch.bfloat16).to(DEV)
    q0, k0 = q.clone(), k.clone()
    cs = torch.from_numpy(od.rope_cache(64, D, 1e6)).to(DEV)
    # position 0 without norm is the identity; 64 and -1 have no cache row: left alone
    ops.qk_norm_rope(q, k, torch.tensor([0, 64, -1], device=DEV), cs)
    assert torch.equal(q, q0) and torch.equal(k, k0)


@pytest.mark.parametrize("dt,bs", [("bf16", 256), ("f16", 16)])
def test_qk_norm_rope_store_is_rope_then_store(dt, bs):
    # one launch = qk_norm_rope then store_kvcache: q, k and both caches bit for bit;
    # slot -1 rows are not written, a position without a cos/sin row stores k as is
    D, T, hq, hkv, nblk = 128, 6, 16, 8, 5
    qkv = rand((T, (hq + 2 * hkv) * D), 40 + bs, DT[dt]).to(DEV)
    q = qkv[:, :hq * D].view(T, hq, D)
    k = qkv[:, hq * D:(hq + hkv) * D].view(T, hkv, D)
    v = qkv[:, (hq + hkv) * D:].view(T, hkv, D)
    qw, kw = rand((D,), 3, DT[dt]).to(DEV), rand((D,), 4, DT[dt]).to(DEV)
    cs = torch.from_numpy(od.rope_cache(512, D, 1e6)).to(DEV)
    pos = torch.tensor([5, 0, 511, 512, 100, 7], device=DEV)
    slots = torch.tensor([3, -1, nblk * bs - 1, 9, 2 * bs, nblk * bs], dtype=torch.int32, device=DEV)
    kc = rand((nblk, bs, hkv, D), 5, DT[dt]).to(DEV)
    vc = rand((nblk, bs, hkv, D), 6, DT[dt]).to(DEV)
    qkv2, kc2, vc2 = qkv.clone(), kc.clone(), vc.clone()
    q2 = qkv2[:, :hq * D].view(T, hq, D)
    k2 = qkv2[:, hq * D:(hq + hkv) * D].view(T, hkv, D)
    v2 = qkv2[:, (hq + hkv) * D:].view(T, hkv, D)
    ops.qk_norm_rope(q, k, pos, cs, qw, kw, 1e-6, v=v, k_cache=kc, v_cache=vc, slot_mapping=slots)
    ops.qk_norm_rope(q2, k2, pos, cs, qw, kw, 1e-6)
    ops.store_kvcache(k2, v2, kc2, vc2, slots)
    torch.cuda.synchronize()
    assert torch.equal(qkv, qkv2)
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)


# ------------------------------------------------------------------ SiLU*up
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("rows,I", [(1, 3072), (16, 3072), (56, 9728), (3, 8)])
def test_silu_mul(dt, rows, I):
    x = rand((rows, 2 * I), rows + I, DT[dt], 3.0)
    got = ops.silu_mul(x.to(DEV))
    ref = od.silu_mul(to_np(x.float()), dt)
    assert_units(to_np(got.float()), ref, f"silu_mul {dt} {rows}x{I}", dt)


# ------------------------------------------------------------------ sampling
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("rows,V", [(1, 151936), (16, 151936), (3, 1000), (2, 1)])
def test_greedy_equals_torch_argmax(dtype, rows, V):
    logits = rand((rows, V), V + rows, torch.float32, 4.0).to(dtype).to(DEV)
    got = ops.sample(logits)
    assert torch.equal(got, torch.argmax(logits, dim=-1))


def test_greedy_ties_take_first_index():
    logits = torch.zeros((4, 5000), device=DEV)
    logits[0, [7, 4000]] = 3.0
    logits[1, [4999, 12]] = 1.0
    logits[3, :] = -2.0
    got = ops.sample(logits).tolist()
    assert got == [7, 12, 0, 0]


def test_sampled_tokens_match_oracle():
    rows, V = 24, 5000
    logits = rand((rows, V), 77, torch.float32, 2.0)
    temps = torch.linspace(0.3, 1.5, rows)
    temps[5] = 0.0  # greedy row
    state = torch.tensor([0x1234_5678_9ABC, 42], dtype=torch.int64)
    got = ops.sample(logits.to(DEV), temps.to(DEV), state.to(DEV)).cpu().numpy()
    want = od.sample(logits.numpy(), temps.numpy(), int(state[0]), int(state[1]))
    keys = od.sample_keys(logits.numpy(), np.where(temps.numpy() > 0, temps.numpy(), 1),
                          int(state[0]), int(state[1]))
    # exact on every row whose two best race keys are further apart than the
    # key's rounding (the kernel forms keys in the log2 domain with the native
    # log: a few float32 ulps of |key| <= ~20, far below 1e-3); a measured
    # near-tie may take either of its tied columns
    top2 = np.sort(keys, axis=-1)[:, -2:]
    tie = (top2[:, 1] - top2[:, 0] < 1e-3) & (temps.numpy() > 0)
    assert np.array_equal(got[~tie], want[~tie]), np.nonzero((got != want) & ~tie)[0]
    for r in np.nonzero(tie)[0]:
        assert keys[r, want[r]] - keys[r, got[r]] < 1e-3, f"row {r}: {got[r]} vs {want[r]}"
    assert tie.sum() <= 2, f"{tie.sum()} near-ties in {rows} rows"


def test_sampling_law_on_gpu():
    rows, V, T = 40000, 5, 0.7
    base = torch.tensor([1.0, 0.2, -0.5, 0.9, 0.0])
    logits = base.repeat(rows, 1).to(DEV)
    state = torch.tensor([987654321, 3], dtype=torch.int64, device=DEV)
    toks = ops.sample(logits, torch.full((rows,), T, device=DEV), state).cpu().numpy()
    p = torch.softmax(base / T, 0).numpy()
    counts = np.bincount(toks, minlength=V)
    chi2 = (((counts - rows * p) ** 2) / (rows * p)).sum()
    assert chi2 < 20.5


# ------------------------------------------------------- reference-named modules
def test_reference_named_modules():
    from specdec_nanovllm_amd.layers.activation import SiluAndMul
    from specdec_nanovllm_amd.layers.layernorm import RMSNorm
    from specdec_nanovllm_amd.layers.rotary_embedding import get_rope
    x = rand((5, 1024), 31, torch.bfloat16).to(DEV)
    r = rand((5, 1024), 32, torch.bfloat16).to(DEV)
    norm = RMSNorm(1024).to(DEV).to(torch.bfloat16)
    assert torch.equal(norm(x), ops.rmsnorm(x, norm.weight, 1e-6))
    o, res = norm(x, r)
    o2, res2 = ops.rmsnorm(x, norm.weight, 1e-6, residual=r)
    assert torch.equal(o, o2) and torch.equal(res, res2)
    gu = rand((3, 2 * 512), 33, torch.bfloat16).to(DEV)
    assert torch.equal(SiluAndMul()(gu), ops.silu_mul(gu))
    rope = get_rope(128, 128, 4096, 1e6).to(DEV)
    q = rand((4, 16 * 128), 34, torch.bfloat16).to(DEV)
    k = rand((4, 8 * 128), 35, torch.bfloat16).to(DEV)
    pos = torch.tensor([0, 5, 100, 4095], device=DEV)
    q2, k2 = rope(pos, q, k)
    assert q2.shape == q.shape and torch.equal(q2.view(4, 16, 128)[0], q.view(4, 16, 128)[0])
    rq, rk = od.qk_norm_rope(to_np(q.float()).reshape(4, 16, 128), to_np(k.float()).reshape(4, 8, 128),
                             pos.cpu().numpy(), rope.cos_sin_cache.view(4096, 128).cpu().numpy())
    assert_units(to_np(q2.float()).reshape(4, 16, 128), rq, "rope q", units=4, per_row=True)
    assert_units(to_np(k2.float()).reshape(4, 8, 128), rk, "rope k", units=4, per_row=True)

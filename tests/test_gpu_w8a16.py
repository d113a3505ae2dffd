"""GPU parity of the W8A16 fused-dequantization linear against float64
dequantize-then-matmul (nanovllm/layers/quant.py:151-159,209-223).

Tolerance: the fused kernel rounds only at the 16-bit output, so
    |y - ref| <= r |ref| + 2^-17 * (|x| @ |w|^T * s)             (elementwise)
with r = 2^-9 for fp16 output and 2^-8 for bf16 output (twice the half-ulp
output rounding, plus fp32 accumulation slack), and
max|y - ref| / max|ref| <= 2e-3 (fp16) or 4e-3 (bf16; the reference reports
0.3-0.4 % for its bf16 output, docs/W8A16量化-开发记录.md:272-274).
"""
import numpy as np
import pytest
import torch

from conftest import to_np
from oracle import w8a16 as ow8
from specdec_nanovllm_amd import _lib, ops, workloads
from specdec_nanovllm_amd.layers.linear import ReplicatedLinear
from specdec_nanovllm_amd.layers.quant import apply_int8_quant, int8_linear, quantize_weight

pytestmark = pytest.mark.gpu
DEV = "cuda"


def check(y, x, w, s, bias=None, gran="per_channel", gs=128, out_rel=2.0 ** -9, what=""):
    xn, wn, sn = to_np(x).astype(np.float64), to_np(w), to_np(s).astype(np.float64)
    bn = None if bias is None else to_np(bias).astype(np.float64)
    ref = ow8.int8_linear(xn, wn, sn, bn, gran, gs)
    mag = np.abs(xn) @ np.abs(ow8.dequantize_weight(wn, sn, gran, gs)).T
    got = to_np(y).astype(np.float64)
    bound = out_rel * np.abs(ref) + 2.0 ** -17 * mag + 1e-30
    excess = np.abs(got - ref) - bound
    assert excess.max() <= 0, f"{what}: max excess {excess.max():.3g}"
    rel = np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)
    rel_max = 2e-3 if y.dtype == torch.float16 else 4e-3
    assert rel <= rel_max, f"{what}: max|y-ref|/max|ref| = {rel:.3g}"


@pytest.mark.parametrize("name,N,K", workloads.W8A16_SHAPES)
@pytest.mark.parametrize("M", workloads.W8A16_MS)
def test_c4_shapes_fp16(name, N, K, M):
    c = workloads.w8a16_case(M, N, K, seed=N + K + M)
    y = ops.w8a16_linear(c["x"], c["w"], c["s"])
    assert y.shape == (M, N) and y.dtype == torch.float16
    check(y, c["x"], c["w"], c["s"], what=f"{name} M={M}")


@pytest.mark.parametrize("M", [1, 7, 16, 56])
def test_bf16_activations_and_scales(M):
    c = workloads.w8a16_case(M, 6144, 1024, seed=M, act_dtype=torch.bfloat16,
                             scale_dtype=torch.bfloat16)
    y = ops.w8a16_linear(c["x"], c["w"], c["s"])
    assert y.dtype == torch.bfloat16
    check(y, c["x"], c["w"], c["s"], out_rel=2.0 ** -8, what=f"bf16 M={M}")


@pytest.mark.parametrize("gs", [64, 128, 256])
@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_per_group(gs, act):
    M, N, K = 5, 1024, 2048
    c = workloads.w8a16_case(M, N, K, seed=gs, act_dtype=act)
    g = workloads.device_generator(DEV, 5)
    s = (torch.rand((N, K // gs), generator=g, device=DEV) * 3e-3 + 1e-3).to(act)
    y = ops.w8a16_linear(c["x"], c["w"], s, group_size=gs)
    check(y, c["x"], c["w"], s, gran="per_group", gs=gs,
          out_rel=2.0 ** -9 if act == torch.float16 else 2.0 ** -8, what=f"group {gs}")


@pytest.mark.parametrize("M,N,K", [(3, 1000, 1024), (100, 512, 256), (33, 4096, 64),
                                   (1, 16, 64), (2, 17, 128), (64, 3072, 1024)])
def test_ragged_shapes_and_bias(M, N, K):
    c = workloads.w8a16_case(M, N, K, seed=M * N)
    bias = torch.randn((N,), device=DEV).to(torch.float16)
    y = ops.w8a16_linear(c["x"], c["w"], c["s"], bias)
    check(y, c["x"], c["w"], c["s"], bias, what=f"{M}x{N}x{K}")


@pytest.mark.parametrize("M", [1, 3, 12, 33, 40, 64, 65])
@pytest.mark.parametrize("gs", [0, 64, 128])
def test_wide_path_scales_and_bias(M, gs):
    # N = 33000 rows of K = 1024: the wide path (whole rows per wave, activation rows and
    # the row groups' scales and bias staged in LDS), ragged last row group, fp32 scales;
    # 33..64 rows are one 64-row block, 65 two
    N, K = 33000, 1024
    c = workloads.w8a16_case(M, N, K, seed=M + gs)
    g = workloads.device_generator(DEV, 11)
    shape = (N,) if gs == 0 else (N, K // gs)
    s = (torch.rand(shape, generator=g, device=DEV) * 3e-3 + 1e-3).to(torch.float32)
    bias = torch.randn((N,), generator=g, device=DEV).to(torch.float16)
    y = ops.w8a16_linear(c["x"], c["w"], s, bias, group_size=gs)
    check(y, c["x"], c["w"], s, bias, gran="per_group" if gs else "per_channel", gs=gs or 128,
          what=f"wide M={M} group={gs}")


def test_full_int8_range_including_minus_128():
    M, N, K = 4, 256, 512
    w = torch.arange(N * K, device=DEV).remainder(256).sub(128).to(torch.int8).view(N, K)
    s = torch.full((N,), 1e-3, device=DEV).to(torch.float16)
    x = torch.randn((M, K), device=DEV).to(torch.float16)
    check(ops.w8a16_linear(x, w, s), x, w, s, what="full int8 range")
    xb = x.to(torch.bfloat16)
    check(ops.w8a16_linear(xb, w, s.to(torch.bfloat16)), xb, w, s.to(torch.bfloat16),
          out_rel=2.0 ** -8, what="full int8 range bf16")


def test_identity_weight_returns_scaled_input():
    K = 256
    w = (torch.eye(K, device=DEV) * 100).to(torch.int8)
    s = torch.full((K,), 0.01, device=DEV).to(torch.float32)
    x = torch.randn((3, K), device=DEV).to(torch.float16)
    y = ops.w8a16_linear(x, w, s)
    # y = x * (100 * 0.01) up to the scale's fp32 rounding and the fp16 output rounding
    np.testing.assert_allclose(to_np(y), to_np(x), rtol=2.0 ** -10, atol=0)


def test_leading_dims_and_mirror_int8_linear():
    c = workloads.w8a16_case(6, 4096, 1024, seed=9, act_dtype=torch.bfloat16,
                             scale_dtype=torch.bfloat16)
    x3 = c["x"].view(2, 3, 1024)
    y = int8_linear(x3, c["w"], c["s"])
    assert y.shape == (2, 3, 4096)
    assert torch.equal(y.view(6, 4096), ops.w8a16_linear(c["x"], c["w"], c["s"]))
    y2 = int8_linear(x3, c["w"], c["s"], out_features=1000)
    assert torch.equal(y2.view(6, 1000), y.view(6, 4096)[:, :1000])


def test_linear_dispatch_after_apply_int8_quant():
    torch.manual_seed(0)
    lin = ReplicatedLinear(1024, 3072).to(DEV)
    lin.weight.data = (torch.randn((3072, 1024), device=DEV) * 0.02).to(torch.bfloat16)
    model = torch.nn.Sequential()
    model.add_module("down", lin)
    x = torch.randn((7, 1024), device=DEV).to(torch.bfloat16)
    w_bf16 = lin.weight.data.clone()
    report = apply_int8_quant(model, ["down"])
    assert report[0]["shape"] == [3072, 1024] and lin.weight.dtype == torch.int8
    q, s = quantize_weight(w_bf16)
    assert torch.equal(lin.weight, q) and torch.equal(lin.weight_scale, s)
    y = lin(x)
    check(y, x, lin.weight, lin.weight_scale, out_rel=2.0 ** -8, what="LinearBase int8")
    lin.to(DEV)  # nn.Module._apply still works on the module


def test_split_plans_are_deterministic():
    c = workloads.w8a16_case(1, 1024, 3072, seed=2)
    a = ops.w8a16_linear(c["x"], c["w"], c["s"])
    for _ in range(3):
        assert torch.equal(a, ops.w8a16_linear(c["x"], c["w"], c["s"]))


def test_errors():
    c = workloads.w8a16_case(1, 64, 96, seed=1)
    with pytest.raises(RuntimeError):  # K % 64 != 0 is not supported
        ops.w8a16_linear(c["x"], c["w"], c["s"])
    with pytest.raises(AssertionError):
        ops.w8a16_linear(c["x"], c["w"].float(), c["s"])
    with pytest.raises(RuntimeError):  # CPU tensors: no fallback
        ops.w8a16_linear(c["x"].cpu(), c["w"].cpu(), c["s"].cpu())


@pytest.mark.parametrize("M,N,K,gs,act", [(1, 1024, 3072, 0, torch.bfloat16),
                                          (2, 1024, 1024, 0, torch.bfloat16),
                                          (7, 1024, 3072, 0, torch.float16),
                                          (56, 1024, 3072, 0, torch.bfloat16),
                                          (3, 33000, 1024, 0, torch.bfloat16),
                                          (20, 33000, 1024, 128, torch.float16),
                                          (40, 33000, 1024, 0, torch.bfloat16),
                                          (1, 16411, 2048, 0, torch.bfloat16)])
def test_silu_linear_is_silu_mul_then_linear(M, N, K, gs, act):
    # the down projection fed straight from gate_up (narrow K-split path and the
    # wide path with staged activations): bit-identical to the two-launch form
    c = workloads.w8a16_case(M, N, K, seed=M + N, act_dtype=act)
    g = workloads.device_generator(DEV, 17)
    gu = (torch.randn((M, 2 * K), generator=g, device=DEV) * 2).to(act)
    s = c["s"] if not gs else (torch.rand((N, K // gs), generator=g, device=DEV) * 3e-3 + 1e-3).to(act)
    bias = torch.randn((N,), generator=g, device=DEV).to(act)
    # the C entry point itself (the Python op would take two launches for the
    # larger activations), then the op
    lib = _lib.load()
    fused = torch.empty((M, N), dtype=act, device=DEV)
    rc = lib.sd_w8a16_silu_linear(gu.data_ptr(), gu.stride(0), c["w"].data_ptr(), c["w"].stride(0),
                                  s.data_ptr(), _lib.dtype_code(s.dtype), gs, bias.data_ptr(),
                                  fused.data_ptr(), fused.stride(0), M, N, K, _lib.dtype_code(act),
                                  _lib.stream_ptr(torch.device(DEV)))
    _lib.check(rc)
    two = ops.w8a16_linear(ops.silu_mul(gu), c["w"], s, bias, group_size=gs)
    assert torch.equal(fused, two)
    assert torch.equal(ops.w8a16_silu_linear(gu, c["w"], s, bias, group_size=gs), two)


@pytest.mark.parametrize("M,N,K,gs,act,res", [(1, 4096, 1024, 0, torch.bfloat16, True),
                                              (1, 2048, 2560, 0, torch.bfloat16, True),
                                              (2, 2048, 1024, 0, torch.float16, True),
                                              (1, 512, 4096, 0, torch.float16, False),
                                              (16, 6144, 1024, 0, torch.bfloat16, True),
                                              (40, 1024, 1024, 0, torch.bfloat16, True),
                                              (3, 512, 1152, 0, torch.float16, True),
                                              (2, 1024, 8192, 0, torch.bfloat16, False),
                                              (9, 33000, 1024, 128, torch.float16, True),
                                              (24, 33000, 1024, 0, torch.bfloat16, True),
                                              (48, 33000, 1024, 0, torch.bfloat16, True),
                                              (1, 151936, 1024, 0, torch.bfloat16, True),
                                              (1, 16411, 2048, 0, torch.float16, False),
                                              # staged 4 rows per wave: a short last wave,
                                              # lanes past K, no residual
                                              (13, 2048, 576, 0, torch.bfloat16, True),
                                              (5, 4096, 1024, 0, torch.float16, False),
                                              (16, 512, 64, 0, torch.bfloat16, True),
                                              (11, 6144, 1024, 0, torch.bfloat16, True)])
def test_rmsnorm_linear_is_rmsnorm_then_linear(M, N, K, gs, act, res):
    # add + RMSNorm formed while staging: bit-identical to rmsnorm then the
    # linear, residual_out identical to rmsnorm's (one row block per 16 or 32
    # rows; K = 1152 leaves the last chunk column partly empty)
    c = workloads.w8a16_case(M, N, K, seed=M + N + K, act_dtype=act)
    g = workloads.device_generator(DEV, 19)
    x = (torch.randn((M, K), generator=g, device=DEV) * 2).to(act)
    r = (torch.randn((M, K), generator=g, device=DEV)).to(act) if res else None
    nw = (1 + 0.1 * torch.randn((K,), generator=g, device=DEV)).to(act)
    s = c["s"] if not gs else (torch.rand((N, K // gs), generator=g, device=DEV) * 3e-3 + 1e-3).to(act)
    bias = torch.randn((N,), generator=g, device=DEV).to(act)
    if res:
        h, want_res = ops.rmsnorm(x, nw, 1e-6, residual=r)
    else:
        h, want_res = ops.rmsnorm(x, nw, 1e-6), None
    two = ops.w8a16_linear(h, c["w"], s, bias, group_size=gs)
    lib = _lib.load()
    fused = torch.empty((M, N), dtype=act, device=DEV)
    ro = torch.full((M, K), float("nan"), dtype=act, device=DEV) if res else None
    rc = lib.sd_w8a16_rmsnorm_linear(
        x.data_ptr(), x.stride(0), None if r is None else r.data_ptr(), K,
        None if ro is None else ro.data_ptr(), K, nw.data_ptr(), 1e-6, c["w"].data_ptr(),
        c["w"].stride(0), s.data_ptr(), _lib.dtype_code(s.dtype), gs, bias.data_ptr(),
        fused.data_ptr(), fused.stride(0), M, N, K, _lib.dtype_code(act),
        _lib.stream_ptr(torch.device(DEV)))
    _lib.check(rc)
    assert torch.equal(fused, two)
    if res:
        assert torch.equal(ro, want_res)
        ro2 = torch.empty_like(ro)
        assert torch.equal(ops.w8a16_rmsnorm_linear(x, nw, 1e-6, c["w"], s, bias, gs, residual=r,
                                                    residual_out=ro2), two)
        assert torch.equal(ro2, want_res)
        # residual_out not wanted
        assert torch.equal(ops.w8a16_rmsnorm_linear(x, nw, 1e-6, c["w"], s, bias, gs,
                                                    residual=r), two)
    else:
        assert torch.equal(ops.w8a16_rmsnorm_linear(x, nw, 1e-6, c["w"], s, bias, gs), two)


def test_rmsnorm_linear_falls_back_past_the_staging_lds():
    # 16 rows of K = 4096 do not fit the staging LDS: the op runs rmsnorm and
    # the linear (same results); the C entry reports the shape as unsupported
    M, N, K = 16, 2048, 4096
    c = workloads.w8a16_case(M, N, K, seed=5)
    g = workloads.device_generator(DEV, 23)
    x = torch.randn((M, K), generator=g, device=DEV).to(torch.bfloat16)
    r = torch.randn((M, K), generator=g, device=DEV).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn((K,), generator=g, device=DEV)).to(torch.bfloat16)
    h, want_res = ops.rmsnorm(x, nw, 1e-6, residual=r)
    two = ops.w8a16_linear(h, c["w"], c["s"])
    ro = torch.empty_like(x)
    assert torch.equal(ops.w8a16_rmsnorm_linear(x, nw, 1e-6, c["w"], c["s"], residual=r,
                                                residual_out=ro), two)
    assert torch.equal(ro, want_res)


def test_rmsnorm_linear_rejects_aliased_residual():
    M, N, K = 2, 512, 1024
    c = workloads.w8a16_case(M, N, K, seed=6)
    x = torch.randn((M, K), device=DEV).to(torch.bfloat16)
    r = torch.randn((M, K), device=DEV).to(torch.bfloat16)
    nw = torch.ones((K,), device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="overlap"):
        ops.w8a16_rmsnorm_linear(x, nw, 1e-6, c["w"], c["s"], residual=r, residual_out=r)
    # a partial overlap (residual_out starting at the second row of x) is refused too
    buf = torch.empty((3, K), device=DEV, dtype=torch.bfloat16)
    buf[:2] = x
    with pytest.raises(ValueError, match="overlap"):
        ops.w8a16_rmsnorm_linear(buf[:2], nw, 1e-6, c["w"], c["s"], residual=r,
                                 residual_out=buf[1:3])


@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("K,gs", [(1024, 0), (2560, 0), (2048, 128), (4096, 0), (3072, 64)])
@pytest.mark.parametrize("act", [torch.bfloat16, torch.float16])
def test_row_streaming_path(M, K, gs, act):
    # one or two activation rows at small K with a per-channel scale take the
    # row-streaming kernel (whole 1 KB weight rows per load, activations in
    # registers): bias, a partial last 1024-column chunk (K = 2560), N not a
    # multiple of the rows per wave. The per-group cases, and two rows past
    # M * ceil(K / 1024) = 4 (K = 3072, 4096), check the tiled kernel on the
    # other side of the dispatch rule at the same shapes.
    N = 3001
    c = workloads.w8a16_case(M, N, K, seed=K + M, act_dtype=act)
    g = workloads.device_generator(DEV, K + 7)
    if gs:
        s = (torch.rand((N, K // gs), generator=g, device=DEV) * 3e-3 + 1e-3).to(act)
    else:
        s = c["s"]
    bias = torch.randn((N,), generator=g, device=DEV).to(act)
    y = ops.w8a16_linear(c["x"], c["w"], s, bias, group_size=gs)
    check(y, c["x"], c["w"], s, bias, "per_group" if gs else "per_channel", gs,
          out_rel=2.0 ** -9 if act == torch.float16 else 2.0 ** -8, what=f"rows M={M} K={K} gs={gs}")


@pytest.mark.parametrize("M,N,K,act,norm,res", [(1, 6144, 1024, torch.bfloat16, True, True),
                                                (1, 6144, 1024, torch.bfloat16, False, False),
                                                (2, 6144, 1024, torch.float16, True, True),
                                                (1, 2048, 2048, torch.float16, True, False),
                                                (2, 512, 2048, torch.bfloat16, False, False),
                                                (1, 8192, 4096, torch.bfloat16, True, True),
                                                (1, 272, 1024, torch.bfloat16, True, True),
                                                (3, 6144, 1024, torch.bfloat16, True, True),
                                                (4, 6144, 1024, torch.bfloat16, True, False),
                                                (7, 6144, 1024, torch.bfloat16, False, False),
                                                (16, 6144, 1024, torch.float16, True, True),
                                                (16, 2048, 2048, torch.bfloat16, True, True),
                                                (56, 6144, 1024, torch.float16, False, False),
                                                (56, 6144, 1024, torch.bfloat16, True, True),
                                                (5, 2064, 1024, torch.bfloat16, False, False),
                                                (11, 6144, 1024, torch.bfloat16, True, False)])
def test_gate_up_silu_is_linear_then_silu_mul(M, N, K, act, norm, res):
    """The gate_up projection with the SiLU epilogue (paired gate / up rows on
    the row-streaming path, paired gate / up tiles on the K-split path with the
    plain projection's K split; the separate launches past them) equals the
    projection (with its RMSNorm) followed by the SiLU kernel, bit for bit."""
    c = workloads.w8a16_case(M, N, K, seed=M * 7 + N, act_dtype=act)
    g = workloads.device_generator(DEV, 31)
    x = (torch.randn((M, K), generator=g, device=DEV) * 2).to(act)
    r = torch.randn((M, K), generator=g, device=DEV).to(act) if res else None
    nw = (1 + 0.1 * torch.randn((K,), generator=g, device=DEV)).to(act) if norm else None
    bias = torch.randn((N,), generator=g, device=DEV).to(act) if M in (2, 7, 56) else None
    if norm:
        ro_two = torch.empty_like(x) if res else None
        gu = ops.w8a16_rmsnorm_linear(x, nw, 1e-6, c["w"], c["s"], bias, residual=r,
                                      residual_out=ro_two)
    else:
        gu = ops.w8a16_linear(x, c["w"], c["s"], bias)
    two = ops.silu_mul(gu)
    ro = torch.empty_like(x) if res else None
    got = ops.w8a16_gate_up_silu(x, c["w"], c["s"], nw, 1e-6, residual=r, residual_out=ro,
                                 bias=bias)
    assert got.shape == (M, N // 2)
    assert torch.equal(got.view(torch.int16), two.view(torch.int16))
    if res:
        assert torch.equal(ro, ro_two)


def test_gate_up_silu_entry_refuses_shapes_off_its_paths():
    # 3 rows (not the row path) of 2064 weight rows (pairs not in whole 16-row tiles)
    c = workloads.w8a16_case(3, 2064, 1024, seed=5)
    y = torch.empty((3, 1032), dtype=torch.float16, device=DEV)
    lib = _lib.load()
    rc = lib.sd_w8a16_gate_up_silu(c["x"].data_ptr(), c["x"].stride(0), None, 0, None, 0, None,
                                   1e-6, c["w"].data_ptr(), c["w"].stride(0), c["s"].data_ptr(),
                                   _lib.dtype_code(c["s"].dtype), None, y.data_ptr(), y.stride(0),
                                   3, 2064, 1024, _lib.SD_F16, _lib.stream_ptr(torch.device(DEV)))
    assert rc == _lib.SD_ERR_UNSUPPORTED and b"row-streaming" in lib.sd_last_error()


# ------------------------------------------------- wide matrices at one row
@pytest.mark.parametrize("N,K", [(151936, 1024), (16411, 2048), (32771, 1024), (8209, 4096)])
@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("scale_f32", [False, True])
def test_row_cyclic_rows_on_wide_matrices(N, K, act, scale_f32):
    # one activation row on more than 32 MiB of weights takes the row-cyclic
    # kernel (row n on wave n % W, four rows per lane reduction, scales gathered
    # 64 rows at a time): N not a multiple of 4, of the waves, or of 64; 1 - 4
    # column chunks; bias; 16-bit and fp32 scales
    assert N * K > 32 << 20
    c = workloads.w8a16_case(1, N, K, seed=N + K, act_dtype=act)
    s = c["s"].float() if scale_f32 else c["s"]
    g = workloads.device_generator(DEV, N)
    bias = torch.randn((N,), generator=g, device=DEV).to(act)
    y = ops.w8a16_linear(c["x"], c["w"], s, bias)
    check(y, c["x"], c["w"], s, bias,
          out_rel=2.0 ** -9 if act == torch.float16 else 2.0 ** -8, what=f"cyclic N={N} K={K}")
    # every output written exactly once: a second call into a NaN-filled
    # buffer gives the same bits
    out = torch.full_like(y, float("nan"))
    ops.w8a16_linear(c["x"], c["w"], s, bias, out=out)
    assert torch.equal(out, y)
    # without bias: the same sums less the bias, within the output rounding
    y0 = ops.w8a16_linear(c["x"], c["w"], s)
    check(y0, c["x"], c["w"], s, out_rel=2.0 ** -9 if act == torch.float16 else 2.0 ** -8,
          what=f"cyclic N={N} K={K} no bias")


def test_two_rows_on_wide_matrices_stay_on_the_tiled_kernel():
    # M = 2 past 32 MiB is not a row-kernel shape: same tolerance via the tiled path
    c = workloads.w8a16_case(2, 151936, 1024, seed=2)
    check(ops.w8a16_linear(c["x"], c["w"], c["s"]), c["x"], c["w"], c["s"], what="M=2 lm_head")


# ----------------------------------------------------- measurement twins
@pytest.mark.parametrize("M,N,K", [(1, 151936, 1024), (7, 151936, 1024), (56, 151936, 1024),
                                   (1, 4096, 1024), (16, 1024, 3072), (56, 6144, 1024)])
@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_floor_twin_runs_the_plan_and_writes_nothing(M, N, K, act):
    # sd_w8a16_floor: the same plan with no math leaves the output untouched
    # (its store is guarded by a condition on the loaded data that these
    # inputs never meet) and leaves the real call's result unchanged after it
    c = workloads.w8a16_case(M, N, K, seed=M + N, act_dtype=act)
    sentinel = torch.full((M, N), 7.0, dtype=act, device=DEV)
    out = sentinel.clone()
    ops.w8a16_linear(c["x"], c["w"], c["s"], out=out, twin="floor")
    torch.cuda.synchronize()
    assert torch.equal(out, sentinel)
    y = ops.w8a16_linear(c["x"], c["w"], c["s"])
    check(y, c["x"], c["w"], c["s"], out_rel=2.0 ** -9 if act == torch.float16 else 2.0 ** -8,
          what=f"after floor M={M} N={N}")
    with pytest.raises(RuntimeError, match="per-channel"):
        ops.w8a16_linear(c["x"], c["w"], torch.ones((N, K // 128), device=DEV, dtype=act),
                         group_size=128, twin="floor")


def test_stream_read_ceiling_reads_and_writes_nothing():
    buf = torch.randint(0, 255, (64 << 20,), dtype=torch.uint8, device=DEV)
    sink = torch.full((4,), 5, dtype=torch.int32, device=DEV)
    for wg in (0, 256, 1536):
        ops.stream_read(buf, sink, wg)
    torch.cuda.synchronize()
    assert sink.tolist() == [5, 5, 5, 5]
    lib = _lib.load()
    assert lib.sd_stream_read(buf.data_ptr(), 15, sink.data_ptr(), 0, None) == _lib.SD_ERR_VALUE
    assert lib.sd_stream_read(buf.data_ptr() + 8, 1024, sink.data_ptr(), 0,
                              None) == _lib.SD_ERR_VALUE

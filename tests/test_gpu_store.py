"""GPU parity of the store_kvcache slot write: bit-exact against the oracle
scatter (nanovllm/layers/attention.py:10-40), -1 and out-of-range slots write
nothing, strided key/value views, 2- and 4-byte elements."""
import numpy as np
import pytest
import torch

from conftest import bits16
from oracle import kvcache as okv
from specdec_nanovllm_amd import ops, workloads
from specdec_nanovllm_amd.layers.attention import store_kvcache as mirror_store

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _caches(nblk, bs, hkv, d, dtype, seed):
    g = workloads.device_generator(DEV, seed)
    kc = torch.randn((nblk, bs, hkv, d), generator=g, device=DEV).to(dtype)
    vc = torch.randn((nblk, bs, hkv, d), generator=g, device=DEV).to(dtype)
    return kc, vc


def _host(t):
    if t.element_size() == 2:
        return bits16(t)
    return t.detach().cpu().numpy().copy()


@pytest.mark.parametrize("batch", [1, 8, 32])
def test_c2_decode_row_write_bit_exact(batch):
    case = workloads.decode_case(batch, seed=batch, num_blocks=512, ctx_range=(512, 4096))
    kc, vc = case["k_cache"], case["v_cache"]
    kc_h, vc_h = _host(kc), _host(vc)
    slots = case["slots"][0]
    ops.store_kvcache(case["k_new"], case["v_new"], kc, vc, slots.to(DEV))
    torch.cuda.synchronize()
    okv.store_kvcache(_host(case["k_new"]), _host(case["v_new"]), kc_h, vc_h, slots.numpy())
    assert np.array_equal(_host(kc), kc_h)
    assert np.array_equal(_host(vc), vc_h)


def test_c3_verify_rows_cross_page_boundaries():
    case = workloads.verify_case(seed=3, num_blocks=256)
    assert case["crosses_page"]
    kc, vc = case["k_cache"], case["v_cache"]
    kc_h, vc_h = _host(kc), _host(vc)
    ops.store_kvcache(case["k_new"], case["v_new"], kc, vc, case["slots"].to(DEV))
    torch.cuda.synchronize()
    okv.store_kvcache(_host(case["k_new"]), _host(case["v_new"]), kc_h, vc_h,
                      case["slots"].numpy())
    assert np.array_equal(_host(kc), kc_h)
    assert np.array_equal(_host(vc), vc_h)
    # the slots are the closed-form ones of the verify positions
    bt = case["table"].numpy()
    exp = okv.verify_slots(bt, case["lens"].numpy(), case["k"], case["block_size"])
    assert np.array_equal(exp, case["slots"].numpy())


def test_pad_and_out_of_range_slots_write_nothing():
    kc, vc = _caches(8, 16, 2, 128, torch.bfloat16, 7)
    before_k, before_v = _host(kc), _host(vc)
    n = 6
    key = torch.randn((n, 2, 128), device=DEV).to(torch.bfloat16)
    val = torch.randn((n, 2, 128), device=DEV).to(torch.bfloat16)
    slots = torch.tensor([-1, 5, 8 * 16, -7, 127, 2 ** 30], dtype=torch.int32)
    ops.store_kvcache(key, val, kc, vc, slots.to(DEV))
    torch.cuda.synchronize()
    ok = torch.tensor([-1, 5, -1, -1, 127, -1], dtype=torch.int32)  # in-range subset
    okv.store_kvcache(_host(key), _host(val), before_k, before_v, ok.numpy())
    assert np.array_equal(_host(kc), before_k)
    assert np.array_equal(_host(vc), before_v)


def test_strided_views_from_fused_qkv():
    # k and v as column slices of one (N, (Hq + 2 Hkv) * D) projection output
    hq, hkv, d, n = 16, 8, 128, 9
    qkv = torch.randn((n, (hq + 2 * hkv) * d), device=DEV).to(torch.bfloat16)
    k = qkv[:, hq * d:(hq + hkv) * d].view(n, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(n, hkv, d)
    assert k.stride(0) == (hq + 2 * hkv) * d
    kc, vc = _caches(4, 256, hkv, d, torch.bfloat16, 11)
    kc_h, vc_h = _host(kc), _host(vc)
    slots = torch.tensor([0, 255, 256, 257, 511, 700, 1023, -1, 300], dtype=torch.int32)
    mirror_store(k, v, kc, vc, slots.to(DEV))
    torch.cuda.synchronize()
    okv.store_kvcache(bits16(k), bits16(v), kc_h, vc_h, slots.numpy())
    assert np.array_equal(_host(kc), kc_h)
    assert np.array_equal(_host(vc), vc_h)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_other_element_sizes(dtype):
    kc, vc = _caches(4, 32, 4, 64, dtype, 13)
    kc_h, vc_h = _host(kc), _host(vc)
    key = torch.randn((5, 4, 64), device=DEV).to(dtype)
    val = torch.randn((5, 4, 64), device=DEV).to(dtype)
    slots = torch.tensor([3, 31, 32, -1, 127], dtype=torch.int32)
    ops.store_kvcache(key, val, kc, vc, slots.to(DEV))
    torch.cuda.synchronize()
    okv.store_kvcache(_host(key), _host(val), kc_h, vc_h, slots.numpy())
    assert np.array_equal(_host(kc), kc_h)
    assert np.array_equal(_host(vc), vc_h)


def test_reference_asserts():
    kc, vc = _caches(2, 16, 2, 128, torch.bfloat16, 1)
    key = torch.randn((3, 2, 128), device=DEV).to(torch.bfloat16)
    with pytest.raises(AssertionError):  # slot count mismatch (attention.py:39)
        ops.store_kvcache(key, key, kc, vc, torch.zeros(2, dtype=torch.int32, device=DEV))
    with pytest.raises(AssertionError):  # head rows not contiguous (attention.py:37)
        kt = torch.randn((3, 128, 2), device=DEV).to(torch.bfloat16).transpose(1, 2)
        ops.store_kvcache(kt, kt, kc, vc, torch.zeros(3, dtype=torch.int32, device=DEV))

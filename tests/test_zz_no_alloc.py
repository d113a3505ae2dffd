"""sd_paged_attention_noalloc: the static-scratch form of sd_paged_attention.

Through the C ABI (ctypes), the no-allocation entry point must give bit for
bit the output of sd_paged_attention with a torch-allocated workspace (same
kernels, same plan), and both must sit within the attention tolerance
|o - ref| <= 2e-3 + 1e-2 |ref| of the float64 oracle. Two calls in a row on
the shared scratch, the second with a smaller input, then a verify-shaped call
(the largest scratch of the three), then sizes beyond the scratch, which must
be refused before any launch.
"""

import numpy as np
import pytest
import torch

from conftest import assert_close_attn, bits16, to_np
from oracle import paged_attention as opa
from specdec_nanovllm_amd import _lib, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCRATCH_BYTES = 32 << 20  # SD_NOALLOC_SCRATCH_BYTES


def _compact(k_cache, v_cache, bt):
    bt = bt.cpu()
    used = sorted(set(int(x) for x in bt.flatten().tolist() if x >= 0))
    remap = {p: i for i, p in enumerate(used)}
    idx = torch.tensor(used, dtype=torch.long, device=k_cache.device)
    kc = to_np(k_cache[idx]).astype(np.float32)
    vc = to_np(v_cache[idx]).astype(np.float32)
    bt2 = np.array([[remap.get(int(x), -1) for x in row] for row in bt.tolist()],
                   dtype=np.int64).reshape(bt.shape)
    return kc, vc, bt2


def _call(noalloc, q, kc, vc, bt, ctx, cuk, cuq, max_qlen, hq, hkv, out):
    """One call of sd_paged_attention(_noalloc) through ctypes; returns the status."""
    lib = _lib.load()
    nblk, bs = kc.shape[0], kc.shape[1]
    B, width = bt.shape
    stream = torch.cuda.current_stream().cuda_stream
    common = (q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(),
              kc.stride(0), kc.stride(1), kc.stride(2), nblk, bs, bt.data_ptr(), bt.stride(0),
              width, None if ctx is None else ctx.data_ptr(),
              None if cuk is None else cuk.data_ptr(), None if cuq is None else cuq.data_ptr(),
              max_qlen, q.shape[0], B, hq, hkv, 128, 128 ** -0.5, _lib.SD_BF16,
              out.data_ptr(), out.stride(0), out.stride(1))
    if noalloc:
        return lib.sd_paged_attention_noalloc(*common, 0, stream)
    nbytes = lib.sd_paged_attention_workspace_size(B, max_qlen, hq, hkv, 128, width * bs, 0)
    assert 0 < nbytes <= SCRATCH_BYTES, nbytes
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    return lib.sd_paged_attention(*common, ws.data_ptr(), nbytes, 0, stream)


def _both(q, kc, vc, bt, ctx=None, cuk=None, cuq=None, max_qlen=1, hq=32, hkv=8):
    o_ws = torch.full_like(q, float("nan"))
    o_na = torch.full_like(q, float("nan"))
    assert _call(False, q, kc, vc, bt, ctx, cuk, cuq, max_qlen, hq, hkv, o_ws) == _lib.SD_OK
    rc = _call(True, q, kc, vc, bt, ctx, cuk, cuq, max_qlen, hq, hkv, o_na)
    assert rc == _lib.SD_OK, _lib.load().sd_last_error()
    torch.cuda.synchronize()
    return o_ws, o_na


def _check_decode(case, b_take):
    bt = case["tables"][0][:b_take].contiguous()
    lens = case["lens"][:b_take].contiguous()
    q = case["q"][:b_take].contiguous()
    o_ws, o_na = _both(q, case["k_cache"], case["v_cache"], bt.to(DEV), ctx=lens.to(DEV))
    assert np.array_equal(bits16(o_na), bits16(o_ws)), f"B={b_take}: not bit-identical"
    kc, vc, bt2 = _compact(case["k_cache"], case["v_cache"], bt)
    ref = opa.paged_attention(to_np(q), kc, vc, bt2, lens.numpy(), case["scale"])
    assert_close_attn(to_np(o_na), ref, what=f"noalloc decode B={b_take}")


def test_noalloc_matches_workspace_entry_two_calls():
    case = workloads.decode_case(32, seed=11)
    print("noalloc: C2 decode B=32 then B=8 (smaller), seed 11", flush=True)
    _check_decode(case, 32)
    _check_decode(case, 8)  # second call on the same scratch, smaller input


def test_noalloc_verify_rows():
    c = workloads.verify_case(8, 6, seed=3)
    print(f"noalloc: C3 verify B=8 q_len 7, seed {c['seed_used']}", flush=True)
    bt = c["table"].to(DEV)
    cuq, cuk = c["cu_q"].to(DEV), c["cu_k"].to(DEV)
    o_ws, o_na = _both(c["q"], c["k_cache"], c["v_cache"], bt, cuk=cuk, cuq=cuq, max_qlen=7)
    assert np.array_equal(bits16(o_na), bits16(o_ws)), "verify: not bit-identical"
    kc, vc, bt2 = _compact(c["k_cache"], c["v_cache"], c["table"])
    ref = opa.paged_attention(to_np(c["q"]), kc, vc, bt2, c["keys"].numpy(), c["scale"],
                              c["cu_q"].numpy())
    assert_close_attn(to_np(o_na), ref, what="noalloc verify")


def test_noalloc_refuses_sizes_beyond_scratch():
    lib = _lib.load()
    B, hq, hkv = 3000, 32, 1  # 32 rows per pair: 50 MB of partials for the sequences alone
    need = lib.sd_paged_attention_workspace_size(B, 1, hq, hkv, 128, 256, 0)
    assert need > SCRATCH_BYTES, need
    q = torch.zeros((B, hq, 128), dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros((2, 256, hkv, 128), dtype=torch.bfloat16, device=DEV)
    bt = torch.zeros((B, 1), dtype=torch.int32, device=DEV)
    ctx = torch.ones(B, dtype=torch.int32, device=DEV)
    out = torch.zeros_like(q)
    rc = _call(True, q, kc, kc, bt, ctx, None, None, 1, hq, hkv, out)
    assert rc == _lib.SD_ERR_UNSUPPORTED
    assert b"static scratch" in lib.sd_last_error()
    torch.cuda.synchronize()
    assert int(out.abs().max()) == 0, "a refused call wrote its output"
    # the scratch still serves a call that fits, afterwards
    test_noalloc_matches_workspace_entry_two_calls()

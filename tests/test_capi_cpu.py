"""The C-ABI library without a GPU: it opens, exports exactly what
include/specdec_amd.h declares, the ctypes table matches the header's
parameter counts, and argument validation (which returns before any HIP call)
reports the reference's error kinds. No kernel is launched here."""
import ctypes
import os
import re
import subprocess

import pytest
import torch

from specdec_nanovllm_amd import _lib, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "specdec_amd.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(sd_[a-z_0-9]+)\s*\(([^;]*?)\)\s*;",
                         text, flags=re.M | re.S):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_header_parses():
    fns = header_functions()
    assert {"sd_abi_version", "sd_last_error", "sd_store_kvcache", "sd_paged_attention",
            "sd_paged_attention_partial", "sd_paged_attention_workspace_size",
            "sd_w8a16_linear", "sd_w8a16_workspace_size"} <= set(fns)


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.library_path()],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    fns = header_functions()
    assert set(fns) <= exported, f"missing: {set(fns) - exported}"
    assert {s for s in exported if s.startswith("sd_")} == set(fns), "undeclared sd_ exports"
    for name in fns:
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)


def test_ctypes_table_matches_header_arity():
    fns = header_functions()
    assert set(_lib.SIGNATURES) == set(fns)
    for name, n in fns.items():
        assert len(_lib.SIGNATURES[name][1]) == n, name


def test_abi_version_and_empty_error():
    lib = _lib.load()
    assert lib.sd_abi_version() == _lib.ABI_VERSION == 2
    assert isinstance(lib.sd_last_error(), bytes)


def test_validation_errors_without_gpu():
    lib = _lib.load()
    # GQA divisibility -> SD_ERR_VALUE (reference: AssertionError / ValueError kind)
    rc = lib.sd_paged_attention(1, 0, 0, 1, 1, 0, 0, 0, 1, 256, 1, 1, 1, 1, None, None, 1, 1, 1,
                                30, 8, 128, 0.1, 0, 1, 0, 0, None, 0, 0, None)
    assert rc == _lib.SD_ERR_VALUE and b"GQA" in lib.sd_last_error()
    with pytest.raises(ValueError):
        _lib.check(rc)
    # head_dim 64 -> SD_ERR_UNSUPPORTED (reference: TORCH_CHECK -> RuntimeError)
    rc = lib.sd_paged_attention(16, 0, 0, 16, 16, 0, 0, 0, 1, 256, 16, 1, 1, 16, None, None, 1,
                                1, 1, 32, 8, 64, 0.1, 0, 16, 0, 0, None, 0, 0, None)
    assert rc == _lib.SD_ERR_UNSUPPORTED
    with pytest.raises(RuntimeError):
        _lib.check(rc)
    # G * q_len > 32 unsupported
    rc = lib.sd_paged_attention(16, 0, 0, 16, 16, 0, 0, 0, 1, 256, 16, 1, 1, 16, None, 16, 9,
                                9, 1, 32, 8, 128, 0.1, 0, 16, 0, 0, None, 0, 0, None)
    assert rc == _lib.SD_ERR_UNSUPPORTED
    # split workspace missing -> SD_ERR_WORKSPACE
    rc = lib.sd_paged_attention(16, 4096, 128, 16, 16, 256 * 1024, 1024, 128, 64, 256, 16, 16,
                                16, 16, None, None, 1, 32, 32, 32, 8, 128, 0.1, 0, 16, 4096,
                                128, None, 0, 0, None)
    assert rc == _lib.SD_ERR_WORKSPACE
    # W8A16: K % 64 != 0 unsupported, M < 0 invalid
    assert lib.sd_w8a16_linear(16, 96, 16, 96, 16, 1, 0, None, 16, 64, 1, 64, 96, 1, None, 0,
                               None) == _lib.SD_ERR_UNSUPPORTED
    assert lib.sd_w8a16_linear(16, 96, 16, 96, 16, 1, 0, None, 16, 64, -1, 64, 96, 1, None, 0,
                               None) == _lib.SD_ERR_VALUE
    # store: bad element size
    assert lib.sd_store_kvcache(16, 0, 0, 16, 0, 0, 16, 16, 0, 0, 0, 16, 1, 1, 8, 16, 1, 3,
                                None) == _lib.SD_ERR_UNSUPPORTED


def test_workspace_queries():
    lib = _lib.load()
    # num_splits = 4 at C2 B=32: 4 * 32 * 8 workgroups, one partial slot per
    # workgroup plus one per (sequence, kv head); 4 rows of (m, l) + 128 fp32 each
    n = lib.sd_paged_attention_workspace_size(32, 1, 32, 8, 128, 4096, 4)
    entries = (4 * 32 * 8 + 32 * 8) * 4
    assert n == (entries * 8 + 255) // 256 * 256 + entries * 128 * 4
    # verify rows (7 x 4) widen every slot; the default plan follows the device
    nv = lib.sd_paged_attention_workspace_size(8, 7, 32, 8, 128, 2816, 4)
    ev = (4 * 8 * 8 + 8 * 8) * 28
    assert nv == (ev * 8 + 255) // 256 * 256 + ev * 128 * 4
    assert lib.sd_paged_attention_workspace_size(32, 1, 32, 8, 128, 4096, 0) > 0
    assert lib.sd_paged_attention_workspace_size(0, 1, 32, 8, 128, 4096, 0) == 0
    # W8A16 is one launch for every shape (K splits are added inside a workgroup)
    for M, N, K in [(1, 151936, 1024), (1, 1024, 3072), (56, 4096, 1024)]:
        assert lib.sd_w8a16_workspace_size(M, N, K, 0) == 0


def test_ops_refuse_cpu_tensors():
    # the product path never falls back to CPU math
    k = torch.zeros((2, 16, 2, 128), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.store_kvcache(torch.zeros((1, 2, 128), dtype=torch.bfloat16),
                          torch.zeros((1, 2, 128), dtype=torch.bfloat16), k, k.clone(),
                          torch.zeros(1, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.paged_attention(torch.zeros((1, 4, 128), dtype=torch.bfloat16), k, k,
                            torch.zeros((1, 1), dtype=torch.int32), 0.1,
                            context_lens=torch.ones(1, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.w8a16_linear(torch.zeros((1, 64), dtype=torch.float16),
                         torch.zeros((8, 64), dtype=torch.int8), torch.ones(8))


@pytest.mark.skipif(torch.cuda.device_count() > 0,
                    reason="fake device addresses: only where no GPU can be reached")
def test_w8a16_rejects_overlapping_outputs():
    """Other workgroups still read x / residual while one writes y or
    residual_out, so any shared byte is refused before a launch."""
    lib = _lib.load()
    M, N, K = 2, 4096, 1024
    x, res, w, s, nw = 0x100000, 0x200000, 0x300000, 0x400000, 0x500000
    row = K * 2

    def norm_call(res_out, y):
        return lib.sd_w8a16_rmsnorm_linear(x, K, res, K, res_out, K, nw, 1e-6, w, K, s,
                                           _lib.SD_BF16, 0, None, y, N, M, N, K,
                                           _lib.SD_BF16, None)

    free = 0x600000
    # residual_out: partly over the second row of x, or over the residual's tail
    assert norm_call(x + row, free) == _lib.SD_ERR_VALUE
    assert b"overlap" in lib.sd_last_error()
    assert norm_call(res + row + 512, free) == _lib.SD_ERR_VALUE
    # y over x, over the residual, or over residual_out
    assert norm_call(free, x + 16) == _lib.SD_ERR_VALUE
    assert norm_call(free, res - 16) == _lib.SD_ERR_VALUE
    assert norm_call(free, free + 2 * row - 16) == _lib.SD_ERR_VALUE
    # plain and SiLU forms: y over the activation rows
    assert lib.sd_w8a16_linear(x, K, w, K, s, _lib.SD_BF16, 0, None, x + row, N, M, N, K,
                               _lib.SD_BF16, None, 0, None) == _lib.SD_ERR_VALUE
    assert lib.sd_w8a16_silu_linear(x, 2 * K, w, K, s, _lib.SD_BF16, 0, None, x + 3 * row, N,
                                    M, N, K, _lib.SD_BF16, None) == _lib.SD_ERR_VALUE


@pytest.mark.skipif(torch.cuda.device_count() > 0,
                    reason="fake device addresses: only where no GPU can be reached")
def test_w8a16_refuses_rows_past_24_bits():
    """The tiled kernel forms a weight row's byte offset with one 24 x 24-bit
    multiply-add, so 2^24 rows or more (even of a short row, under the 4 GiB
    span) are refused before a launch; 2^24 - 16 rows pass the check."""
    lib = _lib.load()
    x, w, s, y = 0x100000, 0x200000, 0x300000, 0x40000000
    K = 64
    for N in ((1 << 24), (1 << 24) + 16):
        rc = lib.sd_w8a16_linear(x, K, w, K, s, _lib.SD_F16, 0, None, y, N, 1, N, K,
                                 _lib.SD_F16, None, 0, None)
        assert rc == _lib.SD_ERR_UNSUPPORTED, N
        assert b"2^24 rows" in lib.sd_last_error()
    # the stride limit holds on its own too
    assert lib.sd_w8a16_linear(x, 1 << 24, w, 1 << 24, s, _lib.SD_F16, 0, None, y, 16, 1, 16,
                               K, _lib.SD_F16, None, 0, None) == _lib.SD_ERR_UNSUPPORTED


# ------------------------------------------------------------------ argument sweep
HOSTILE = {
    ctypes.c_void_p: [None, 0x1001, 0xFFFFFFFFFFFFF000],
    ctypes.c_int64: [0, -1, 2**31, 2**62, -(2**63)],
    ctypes.c_int32: [0, -1, 2**31 - 1, -(2**31)],
    ctypes.c_float: [float("nan"), float("inf"), -1.0, 0.0],
    ctypes.c_size_t: [0, 2**63],
}


# Plausible values per entry (argument index -> value), so that the sweep's
# single-argument mutations reach the checks behind the first ones: decode
# attention at Qwen3-4B geometry (16 sequences, 32 / 8 heads of 128, 256-token
# pages), a 128-dim store, head_dim 128 for the RoPE and prefill entries.
_ATTN = {1: 4096, 2: 128, 5: 256 * 1024, 6: 1024, 7: 128, 8: 64, 9: 256, 11: 16, 12: 16,
         14: None, 15: None, 16: 1, 17: 16, 18: 16, 19: 32, 20: 8, 21: 128, 23: 0,
         25: 4096, 26: 128, 28: 1 << 30, 29: 0}
PLAUSIBLE = {
    "sd_paged_attention": _ATTN,
    "sd_paged_attention_partial": _ATTN,
    "sd_paged_attention_combine": _ATTN,
    "sd_paged_attention_floor": _ATTN,
    "sd_paged_attention_noalloc": {i: v for i, v in _ATTN.items() if i < 27} | {27: 0},
    "sd_paged_attention_store": {1: 1024, 2: 128, 4: 1024, 5: 128}
                                | {i + 7: v for i, v in _ATTN.items()},
    "sd_store_kvcache": {1: 1024, 2: 128, 4: 1024, 5: 128, 8: 256 * 1024, 9: 1024, 10: 128,
                         12: 16, 13: 8, 14: 128, 15: 256, 16: 64, 17: 2},
    "sd_qk_norm_rope": {1: 4096, 2: 128, 4: 1024, 5: 128, 7: 32, 8: 8, 9: 128, 14: 128,
                        15: 4096, 16: 0},
    "sd_prefill_attention": {1: 4096, 2: 128, 5: 1024, 6: 128, 7: 256 * 1024, 8: 64, 9: 256,
                             11: 16, 12: 16, 15: 64, 16: 1024, 17: 16, 18: 32, 19: 8,
                             20: 128, 22: 0, 24: 4096, 25: 128},
    # no dtype to leave invalid: two bad arguments (a ragged byte count, a misaligned
    # sink), so that no single mutation reaches a launch on a host without a GPU
    "sd_stream_read": {1: 15, 2: 0x10000001},
}


def _baseline(name, argtypes):
    out = []
    for i, t in enumerate(argtypes):
        if t is ctypes.c_void_p:
            out.append(0x10000000 + i * 0x1000000)  # 16-byte aligned, never dereferenced
        elif t is ctypes.c_int64:
            out.append(64)
        elif t is ctypes.c_int32:
            out.append(16)
        elif t is ctypes.c_float:
            out.append(0.125)
        else:
            out.append(0)
    for i, v in PLAUSIBLE.get(name, {}).items():
        out[i] = v
    if argtypes[-1] is ctypes.c_void_p:
        out[-1] = None  # the stream: a host handle, always the default stream here
    return out


@pytest.mark.skipif(torch.cuda.device_count() > 0,
                    reason="fake device addresses: only where no GPU can be reached")
def test_argument_sweep_returns_status_codes():
    """Every entry point, every argument set in turn to a hostile value (NULL,
    misaligned or top-of-space pointers, 0 / -1 / extreme sizes, NaN and inf):
    each call returns a status code and leaves a message, never crashes. Run
    under AddressSanitizer + UndefinedBehaviorSanitizer by
    test_capi_sanitized_cpu.py, where an overflow or out-of-bounds access in
    the host-side checks aborts the run."""
    lib = _lib.load()
    calls = 0
    for name, (res, argtypes) in _lib.SIGNATURES.items():
        if not argtypes:
            continue
        fn = getattr(lib, name)
        base = _baseline(name, argtypes)
        mutable = argtypes[:-1] if argtypes[-1] is ctypes.c_void_p else argtypes
        for i, t in enumerate(mutable):
            for v in HOSTILE[t]:
                args = list(base)
                args[i] = v
                rc = fn(*args)
                calls += 1
                if res is ctypes.c_int:
                    assert 0 <= rc <= _lib.SD_ERR_HIP, (name, i, v, rc)
                    assert isinstance(lib.sd_last_error(), bytes)
    assert calls > 500

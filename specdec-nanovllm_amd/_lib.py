"""ctypes binding of ``libspecdec_amd.so`` — the C ABI declared in
``include/specdec_amd.h``.

torch is imported before the library is opened: the library needs
``libamdhip64.so.7`` by soname, and loading it after torch makes it bind to
the HIP runtime torch already mapped (one runtime per process, so streams and
device pointers are shared). There is no fallback: if the library is missing
or was built for another ABI, every op raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

_HERE = os.path.dirname(os.path.abspath(__file__))
# SPECDEC_AMD_LIBRARY: another build of the same library (a sanitizer build
# for the host-side checks, for instance)
LIB_PATH = os.environ.get("SPECDEC_AMD_LIBRARY") or os.path.join(_HERE, "libspecdec_amd.so")
ABI_VERSION = 2

SD_OK, SD_ERR_VALUE, SD_ERR_UNSUPPORTED, SD_ERR_WORKSPACE, SD_ERR_HIP = range(5)
SD_BF16, SD_F16, SD_F32 = 0, 1, 2

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/specdec_amd.h one to one.
SIGNATURES = {
    "sd_abi_version": (ctypes.c_int, []),
    "sd_last_error": (ctypes.c_char_p, []),
    "sd_store_kvcache": (ctypes.c_int, [
        _p, _i64, _i64,            # key, strides (tok, head)
        _p, _i64, _i64,            # value, strides
        _p, _p, _i64, _i64, _i64,  # k_cache, v_cache, strides (block, pos, head)
        _p, _i64,                  # slot_mapping, num_tokens
        _i32, _i32, _i32, _i64,    # num_kv_heads, head_dim, block_size, num_blocks
        _i32, _p]),                # elem_bytes, stream
    "sd_paged_attention_workspace_size": (_sz, [_i32, _i32, _i32, _i32, _i32, _i64, _i32]),
    "sd_paged_attention": (ctypes.c_int, [
        _p, _i64, _i64,                 # q, strides (tok, head)
        _p, _p, _i64, _i64, _i64, _i64,  # k_cache, v_cache, strides, num_blocks
        _i32, _p, _i64, _i32,           # block_size, block_table, bt_stride, max_blocks
        _p, _p, _p,                     # context_lens, cu_seqlens_k, cu_seqlens_q
        _i32, _i64, _i32, _i32, _i32, _i32,  # max_qlen, total_q, seqs, hq, hkv, head_dim
        _f32, _i32,                     # scale, dtype
        _p, _i64, _i64,                 # out, strides
        _p, _sz, _i32, _p]),            # workspace, bytes, num_splits, stream
    "sd_w8a16_workspace_size": (_sz, [_i64, _i64, _i64, _i32]),
    "sd_w8a16_silu_linear": (ctypes.c_int, [
        _p, _i64, _p, _i64,             # gate_up, stride, w, w_stride
        _p, _i32, _i32, _p,             # scale, scale_dtype, group_size, bias
        _p, _i64,                       # y, y_stride
        _i64, _i64, _i64, _i32, _p]),   # M, N, K, dtype, stream
    "sd_w8a16_rmsnorm_linear": (ctypes.c_int, [
        _p, _i64, _p, _i64, _p, _i64,   # x, stride, residual, stride, residual_out, stride
        _p, _f32, _p, _i64,             # norm_weight, eps, w, w_stride
        _p, _i32, _i32, _p,             # scale, scale_dtype, group_size, bias
        _p, _i64,                       # y, y_stride
        _i64, _i64, _i64, _i32, _p]),   # M, N, K, dtype, stream
    "sd_w8a16_gate_up_silu": (ctypes.c_int, [
        _p, _i64, _p, _i64, _p, _i64,   # x, stride, residual, stride, residual_out, stride
        _p, _f32, _p, _i64,             # norm_weight (or NULL), eps, w, w_stride
        _p, _i32, _p,                   # scale, scale_dtype, bias
        _p, _i64,                       # y, y_stride
        _i64, _i64, _i64, _i32, _p]),   # M, N, K, dtype, stream
    "sd_stream_read": (ctypes.c_int, [_p, _i64, _p, _i32, _p]),  # src, bytes, sink, wgs, stream
    "sd_w8a16_floor": (ctypes.c_int, [
        _p, _i64, _p, _i64,             # x, x_stride, w, w_stride
        _p, _i32, _p,                   # scale, scale_dtype, bias
        _p, _i64,                       # y, y_stride
        _i64, _i64, _i64, _i32, _p]),   # M, N, K, dtype, stream
    "sd_w8a16_linear": (ctypes.c_int, [
        _p, _i64, _p, _i64,             # x, x_stride, w, w_stride
        _p, _i32, _i32, _p,             # scale, scale_dtype, group_size, bias
        _p, _i64,                       # y, y_stride
        _i64, _i64, _i64, _i32,         # M, N, K, dtype
        _p, _sz, _p]),                  # workspace, bytes, stream
}
SIGNATURES.update({
    "sd_rmsnorm": (ctypes.c_int, [
        _p, _i64, _p, _i64,             # x, stride, residual, stride
        _p, _p, _i64, _p, _i64,         # weight, out, stride, residual_out, stride
        _i64, _i32, _f32, _i32, _p]),   # rows, hidden, eps, dtype, stream
    "sd_qk_norm_rope": (ctypes.c_int, [
        _p, _i64, _i64, _p, _i64, _i64,  # q, strides (tok, head), k, strides
        _i64, _i32, _i32, _i32,         # tokens, hq, hkv, head_dim
        _p, _p, _f32,                   # q_weight, k_weight, eps
        _p, _p, _i64, _i64,             # positions, cos_sin, stride, max_position
        _i32, _p]),                     # dtype, stream
    "sd_qk_norm_rope_store": (ctypes.c_int, [
        _p, _i64, _i64, _p, _i64, _i64,  # q, strides, k, strides
        _p, _i64, _i64, _i64,            # v, strides, tokens
        _i32, _i32, _i32, _p, _p, ctypes.c_float,  # Hq, Hkv, head_dim, q_w, k_w, eps
        _p, _p, _i64, _i64,              # positions, cos_sin, stride, max_position
        _p, _p, _i64, _i64, _i64,        # k_cache, v_cache, block/pos/head strides
        _i64, _i32, _p, _i32, _p]),      # num_blocks, block_size, slots, dtype, stream
    "sd_silu_mul": (ctypes.c_int, [_p, _i64, _p, _i64, _i64, _i32, _i32, _p]),
    "sd_sample_workspace_size": (ctypes.c_size_t, [_i64, _i32]),
    "sd_sample": (ctypes.c_int, [
        _p, _i64, _i32, _i64, _i32,     # logits, stride, dtype, rows, vocab
        _p, _p, _p,                     # temperatures, rng_state, out_tokens
        _p, ctypes.c_size_t, _p]),      # workspace, bytes, stream
    "sd_quantize_int8": (ctypes.c_int, [
        _p, _i64, _i32, _p, _i64,       # w, stride, dtype, q, stride
        _p, _i64, _i32, _i32, _p]),     # scale, N, K, group_size, stream
    "sd_prefill_attention": (ctypes.c_int, [
        _p, _i64, _i64, _p, _p,         # q, strides (tok, head), k, v
        _i64, _i64, _i64, _i64, _i32,   # kv strides (tok, head, block), num_blocks, block_size
        _p, _i64, _i32,                 # block_table, bt_stride, max_blocks
        _p, _p, _i32, _i64, _i32,       # cu_q, cu_k, max_seqlen_q, total_q, num_seqs
        _i32, _i32, _i32, _f32, _i32,   # hq, hkv, head_dim, scale, dtype
        _p, _i64, _i64, _p]),           # out, strides, stream
    "sd_verify_batch_workspace_size": (_sz, [_i64, _i32, _i32]),
    "sd_verify_batch": (ctypes.c_int, [
        _p, _i64, _i64, _i32,           # draft, strides (b, k), dtype
        _p, _i64, _i64, _i32,           # target, strides, dtype
        _p, _i64, _p, _i32, _p,         # tokens, stride, temperatures, point_mass, rng_state
        _i64, _i32, _i32,               # batch, k, vocab
        _p, _p, _p,                     # accepted, bonus, accept_mask
        _p, _sz, _p]),                  # workspace, bytes, stream
})
SIGNATURES["sd_paged_attention_partial"] = SIGNATURES["sd_paged_attention"]
SIGNATURES["sd_paged_attention_combine"] = SIGNATURES["sd_paged_attention"]
SIGNATURES["sd_paged_attention_floor"] = SIGNATURES["sd_paged_attention"]
# sd_paged_attention without (workspace, workspace_bytes): the static-scratch form
_attn_args = SIGNATURES["sd_paged_attention"][1]
SIGNATURES["sd_paged_attention_noalloc"] = (ctypes.c_int, _attn_args[:-4] + _attn_args[-2:])
SIGNATURES["sd_paged_attention_store"] = (ctypes.c_int, [
    _p, _i64, _i64,                 # key (new rows), strides (tok, head)
    _p, _i64, _i64,                 # value, strides
    _p,                             # slot_mapping
    *SIGNATURES["sd_paged_attention"][1]])

_lib = None


def library_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Open the library (once) and declare every exported signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
            "g.build()'` (hipcc, gfx950). There is no CPU fallback.")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.sd_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"libspecdec_amd ABI {ver} != expected {ABI_VERSION}; rebuild")
    _lib = lib
    return lib


def check(rc: int) -> None:
    """Map a nonzero sd_status to the exception the reference raises."""
    if rc == SD_OK:
        return
    msg = load().sd_last_error().decode(errors="replace")
    if rc == SD_ERR_VALUE:
        raise ValueError(msg)
    raise RuntimeError(msg)


_DTYPES = {torch.bfloat16: SD_BF16, torch.float16: SD_F16, torch.float32: SD_F32}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPES[dt]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {dt}") from None


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one ROCm device; returns it. CPU tensors are an error (no fallback)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"specdec_nanovllm_amd ops run only on a ROCm GPU; got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def stream_ptr(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream

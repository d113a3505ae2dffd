"""Torch-facing wrappers of the three hot-path kernels.

Each function validates shapes the way the reference does (``assert`` where the
reference asserts), allocates the output and the split workspace with torch's
caching allocator on the current stream (so the call is graph-capturable and
reentrant across streams), and enqueues the HIP kernels through the C ABI on
``torch.cuda.current_stream()``. Nothing here computes on the CPU.
"""
from __future__ import annotations

import torch

from . import _lib


def _workspace(nbytes: int, dev: torch.device) -> torch.Tensor | None:
    if nbytes <= 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=dev)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _i32(t: torch.Tensor | None) -> torch.Tensor | None:
    if t is None:
        return None
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


# --------------------------------------------------------------------------- store
def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Write token rows of key/value into the paged cache at ``slot_mapping``.

    Contract of ``store_kvcache`` (nanovllm/layers/attention.py:33-40): key and
    value are (N, num_kv_heads, head_dim) with contiguous heads, the caches are
    (num_blocks, block_size, num_kv_heads, head_dim) with stride(1) equal to
    num_kv_heads * head_dim, and slot -1 skips the row.
    """
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    assert k_cache.stride() == v_cache.stride() and k_cache.shape == v_cache.shape
    assert key.dtype == value.dtype == k_cache.dtype == v_cache.dtype
    assert k_cache.dim() == 4 and k_cache.shape[2] == num_heads and k_cache.shape[3] == head_dim
    dev = _lib.require_device(key, value, k_cache, v_cache, slot_mapping)
    if N == 0:
        return
    slots = _i32(slot_mapping.reshape(-1))
    lib = _lib.load()
    with torch.cuda.device(dev):
        rc = lib.sd_store_kvcache(
            key.data_ptr(), key.stride(0), key.stride(1),
            value.data_ptr(), value.stride(0), value.stride(1),
            k_cache.data_ptr(), v_cache.data_ptr(),
            k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
            slots.data_ptr(), N, num_heads, head_dim, k_cache.shape[1], k_cache.shape[0],
            key.element_size(), _lib.stream_ptr(dev))
    _lib.check(rc)


# ----------------------------------------------------------------------- attention
def _cache_geometry(k_cache: torch.Tensor, layout: str):
    if layout == "head_major":
        # (num_blocks, num_kv_heads, block_size, head_dim)
        num_blocks, num_kv_heads, block_size, head_dim = k_cache.shape
        sb, sh, sp = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    elif layout == "interleaved":
        # (num_blocks, block_size, num_kv_heads, head_dim): nano-vllm / flash-attn layout
        num_blocks, block_size, num_kv_heads, head_dim = k_cache.shape
        sb, sp, sh = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    else:
        raise ValueError(f"unknown layout: {layout}")
    return num_blocks, block_size, num_kv_heads, head_dim, sb, sp, sh


def paged_attention_workspace_bytes(num_seqs: int, max_seqlen_q: int, num_q_heads: int,
                                    num_kv_heads: int, max_ctx: int, num_splits: int = 0,
                                    device: torch.device | str | None = None) -> int:
    """Bytes of the split-KV workspace ``paged_attention`` uses for these sizes on
    ``device`` (the plan follows the device's compute units)."""
    lib = _lib.load()
    with torch.cuda.device(torch.device(device) if device is not None else
                           torch.cuda.current_device()):
        return int(lib.sd_paged_attention_workspace_size(
            int(num_seqs), int(max_seqlen_q), int(num_q_heads), int(num_kv_heads), 128,
            int(max_ctx), int(num_splits)))


def paged_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    block_table: torch.Tensor, scale: float, *,
                    context_lens: torch.Tensor | None = None,
                    cu_seqlens_k: torch.Tensor | None = None,
                    cu_seqlens_q: torch.Tensor | None = None, max_seqlen_q: int = 1,
                    layout: str = "interleaved", num_splits: int = 0,
                    out: torch.Tensor | None = None, main_only: bool = False,
                    key: torch.Tensor | None = None, value: torch.Tensor | None = None,
                    slot_mapping: torch.Tensor | None = None,
                    no_alloc: bool = False, twin: str | None = None,
                    workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Paged decode (``cu_seqlens_q is None``: one query row per sequence) or
    speculative-verify attention (rows ``cu_seqlens_q[b]:cu_seqlens_q[b+1]``,
    bottom-right causal), GQA, split-KV.

    q: (total_q, num_q_heads, head_dim); keys per sequence from ``context_lens``
    (B,) or ``cu_seqlens_k`` (B+1,). Returns ``out`` (same shape/dtype as q).
    ``main_only`` runs only the split-KV main kernel (measurement twin; the
    same as ``twin="main"``). The other measurement twins: ``twin="combine"``
    runs only the merge over ``workspace`` as a ``twin="main"`` call with the
    same arguments left it; ``twin="floor"`` issues only the main kernel's loads
    (no math, ``out`` untouched). ``workspace`` (uint8, at least the size the
    library asks for) replaces the workspace otherwise allocated per call.

    ``key``/``value`` (total_q, num_kv_heads, head_dim) with ``slot_mapping``
    (total_q,): store_kvcache of these rows fused into the same launch — the
    ``Attention.forward`` sequence (nanovllm/layers/attention.py:59-82). The
    same cache as ``store_kvcache`` and the output of attention afterwards up to
    rounding (the new keys are scored in fp32 in the merge launch), for the
    engine's slot layout: sequence b's rows are its last n_b keys (slot -1: not
    written).

    ``no_alloc`` runs the same kernels on the library's static device scratch
    (``sd_paged_attention_noalloc``) instead of a workspace from torch's
    allocator; pass ``out`` as well to allocate nothing at all. Calls that
    overlap in time on one device share that scratch and race.
    """
    if q.dim() != 3:
        raise ValueError(f"q must be (tokens, heads, head_dim), got {tuple(q.shape)}")
    total_q, num_q_heads, head_dim = q.shape
    num_blocks, block_size, num_kv_heads, hd_c, sb, sp, sh = _cache_geometry(k_cache, layout)
    assert num_q_heads % num_kv_heads == 0, \
        f"GQA needs num_q_heads divisible by num_kv_heads: {num_q_heads} vs {num_kv_heads}"
    assert hd_c == head_dim, f"head_dim mismatch: q {head_dim} vs cache {hd_c}"
    assert k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride()
    assert k_cache.dtype == v_cache.dtype == q.dtype, "q and caches must share one dtype"
    assert k_cache.stride(-1) == 1 and q.stride(-1) == 1
    assert block_table.dim() == 2, "block_table must be (num_seqs, max_blocks)"
    if (context_lens is None) == (cu_seqlens_k is None):
        raise ValueError("give exactly one of context_lens / cu_seqlens_k")
    dev = _lib.require_device(q, k_cache, v_cache, block_table, context_lens, cu_seqlens_k,
                              cu_seqlens_q, out)
    num_seqs = block_table.shape[0]
    bt = _i32(block_table)
    ctx = _i32(context_lens)
    cuk = _i32(cu_seqlens_k)
    cuq = _i32(cu_seqlens_q)
    if cuq is None:
        max_seqlen_q = 1
        if total_q != num_seqs:
            raise ValueError(f"decode expects one query row per sequence: q has {total_q} rows, "
                             f"block_table {num_seqs}")
    if out is None:
        out = torch.empty_like(q)
    else:
        assert out.shape == q.shape and out.dtype == q.dtype and out.stride(-1) == 1
    if main_only:
        twin = "main"
    if twin not in (None, "main", "combine", "floor"):
        raise ValueError(f"unknown twin: {twin}")
    fused = key is not None
    assert not (no_alloc and (fused or twin)), "no_alloc is the plain attention call"
    assert not (fused and twin), "the measurement twins are plain attention calls"
    if fused:
        assert value is not None and slot_mapping is not None
        assert key.shape == (total_q, num_kv_heads, head_dim) and value.shape == key.shape
        assert key.dtype == value.dtype == q.dtype
        assert key.stride(-1) == 1 and value.stride(-1) == 1
        assert slot_mapping.numel() == total_q
        _lib.require_device(key, value, slot_mapping)
    if total_q == 0 or (num_seqs == 0 and not fused):
        return out  # (num_seqs == 0 with new rows: the library only stores them)
    lib = _lib.load()
    max_blocks = bt.shape[1]
    fn = {None: lib.sd_paged_attention, "main": lib.sd_paged_attention_partial,
          "combine": lib.sd_paged_attention_combine,
          "floor": lib.sd_paged_attention_floor}[twin]
    new_rows = ()
    if fused:
        slots = _i32(slot_mapping.reshape(-1))
        fn = lib.sd_paged_attention_store
        new_rows = (key.data_ptr(), key.stride(0), key.stride(1),
                    value.data_ptr(), value.stride(0), value.stride(1), slots.data_ptr())
    if no_alloc:
        with torch.cuda.device(dev):
            rc = lib.sd_paged_attention_noalloc(
                q.data_ptr(), q.stride(0), q.stride(1),
                k_cache.data_ptr(), v_cache.data_ptr(), sb, sp, sh, num_blocks,
                block_size, bt.data_ptr(), bt.stride(0), max_blocks,
                _ptr(ctx), _ptr(cuk), _ptr(cuq),
                int(max_seqlen_q), total_q, num_seqs, num_q_heads, num_kv_heads, head_dim,
                float(scale), _lib.dtype_code(q.dtype),
                out.data_ptr(), out.stride(0), out.stride(1), int(num_splits),
                _lib.stream_ptr(dev))
        _lib.check(rc)
        return out
    with torch.cuda.device(dev):
        # the plan (and so the workspace) depends on the device's compute units
        ws_bytes = lib.sd_paged_attention_workspace_size(
            num_seqs, int(max_seqlen_q), num_q_heads, num_kv_heads, head_dim,
            max_blocks * block_size, int(num_splits))
        if workspace is not None:
            assert workspace.dtype == torch.uint8 and workspace.is_contiguous()
            if workspace.numel() < ws_bytes:
                raise RuntimeError(f"workspace of {workspace.numel()} bytes, {ws_bytes} needed")
            _lib.require_device(workspace)
            ws, ws_bytes = workspace, workspace.numel()
        else:
            ws = _workspace(ws_bytes, dev)
        rc = fn(*new_rows, q.data_ptr(), q.stride(0), q.stride(1),
                k_cache.data_ptr(), v_cache.data_ptr(), sb, sp, sh, num_blocks,
                block_size, bt.data_ptr(), bt.stride(0), max_blocks,
                _ptr(ctx), _ptr(cuk), _ptr(cuq),
                int(max_seqlen_q), total_q, num_seqs, num_q_heads, num_kv_heads, head_dim,
                float(scale), _lib.dtype_code(q.dtype),
                out.data_ptr(), out.stride(0), out.stride(1),
                _ptr(ws), ws_bytes, int(num_splits), _lib.stream_ptr(dev))
    _lib.check(rc)
    return out


def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
                      max_seqlen_q: int, scale: float, block_table: torch.Tensor | None = None,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """Variable-length causal attention (the prefill call of the attention layer,
    nanovllm/layers/attention.py:64-70): q (total_q, Hq, 128); ``k``/``v`` are
    contiguous (total_k, Hkv, 128) rows when ``block_table`` is None, else the
    paged caches (num_blocks, block_size, Hkv, 128). Row t of sequence b sees
    keys [0, nk_b - nq_b + t]. Returns (total_q, Hq, 128)."""
    total_q, num_q_heads, head_dim = q.shape
    assert k.shape == v.shape and k.stride() == v.stride()
    assert q.stride(-1) == 1 and k.stride(-1) == 1
    num_seqs = cu_seqlens_q.numel() - 1
    cuq, cuk = _i32(cu_seqlens_q), _i32(cu_seqlens_k)
    assert cuk.numel() == num_seqs + 1
    if block_table is None:
        assert k.dim() == 3, "contiguous k/v must be (total_k, Hkv, D)"
        num_kv_heads = k.shape[1]
        s_tok, s_head, s_blk, num_blocks, block_size = k.stride(0), k.stride(1), 0, 0, 0
        bt, bt_stride, max_blocks = None, 0, 0
    else:
        assert k.dim() == 4, "paged k/v cache must be (num_blocks, block_size, Hkv, D)"
        num_blocks, block_size, num_kv_heads, _ = k.shape
        s_blk, s_tok, s_head = k.stride(0), k.stride(1), k.stride(2)
        bt = _i32(block_table)
        bt_stride, max_blocks = bt.stride(0), bt.shape[1]
    assert num_q_heads % num_kv_heads == 0, "GQA needs num_q_heads % num_kv_heads == 0"
    dev = _lib.require_device(q, k, v, cuq, cuk, bt, out)
    if out is None:
        out = torch.empty_like(q)
    if num_seqs <= 0 or total_q == 0:
        return out
    lib = _lib.load()
    with torch.cuda.device(dev):
        rc = lib.sd_prefill_attention(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
                                      v.data_ptr(), s_tok, s_head, s_blk, num_blocks, block_size,
                                      _ptr(bt), bt_stride, max_blocks, cuq.data_ptr(),
                                      cuk.data_ptr(), int(max_seqlen_q), total_q, num_seqs,
                                      num_q_heads, num_kv_heads, head_dim, float(scale),
                                      _lib.dtype_code(q.dtype), out.data_ptr(), out.stride(0),
                                      out.stride(1), _lib.stream_ptr(dev))
    _lib.check(rc)
    return out


# -------------------------------------------------------------------------- w8a16
def w8a16_linear(x: torch.Tensor, qweight: torch.Tensor, scale: torch.Tensor,
                 bias: torch.Tensor | None = None, group_size: int = 0,
                 out: torch.Tensor | None = None, twin: str | None = None) -> torch.Tensor:
    """y = x @ (qweight * scale)^T + bias with the dequantization fused.

    x: (..., K) fp16/bf16; qweight: (N, K) int8; scale: (N,) when
    ``group_size == 0`` else (N, K // group_size); returns (..., N) in x.dtype.
    ``twin="floor"``: the measurement twin instead (sd_w8a16_floor: the same
    plan, grid and loads with no math; per-channel scales only); the output
    is left unwritten.
    """
    if twin not in (None, "floor"):
        raise ValueError(f"unknown twin {twin!r}")
    assert qweight.dtype == torch.int8, f"qweight must be int8, got {qweight.dtype}"
    assert qweight.dim() == 2
    N, K = qweight.shape
    x2 = x.reshape(-1, x.shape[-1])
    M = x2.shape[0]
    assert x2.shape[1] == K, f"K mismatch: x {tuple(x2.shape)} vs w {tuple(qweight.shape)}"
    if x2.stride(-1) != 1 or (M > 1 and x2.stride(0) % 8 != 0):
        x2 = x2.contiguous()
    qw = qweight if qweight.is_contiguous() else qweight.contiguous()
    sc = scale.contiguous()
    if group_size:
        assert sc.numel() == N * (K // group_size), "per-group scale must be (N, K // group_size)"
    else:
        assert sc.numel() == N, "per-channel scale must have N entries"
    b = None if bias is None else bias.to(x.dtype).contiguous()
    dev = _lib.require_device(x2, qw, sc, b, out)
    if out is None:
        y = torch.empty((M, N), device=dev, dtype=x.dtype)
    else:
        y = out.reshape(M, N)
        assert y.dtype == x.dtype and y.stride(-1) == 1
    if M == 0:
        return y.view(*x.shape[:-1], N)
    lib = _lib.load()
    if twin == "floor":
        if group_size:
            raise RuntimeError("w8a16 floor twin: per-channel scales only")
        with torch.cuda.device(dev):
            rc = lib.sd_w8a16_floor(
                x2.data_ptr(), x2.stride(0), qw.data_ptr(), qw.stride(0),
                sc.data_ptr(), _lib.dtype_code(sc.dtype), _ptr(b),
                y.data_ptr(), y.stride(0), M, N, K, _lib.dtype_code(x.dtype),
                _lib.stream_ptr(dev))
        _lib.check(rc)
        return y.view(*x.shape[:-1], N)
    ws_bytes = lib.sd_w8a16_workspace_size(M, N, K, int(group_size))
    ws = _workspace(ws_bytes, dev)
    with torch.cuda.device(dev):
        rc = lib.sd_w8a16_linear(
            x2.data_ptr(), x2.stride(0), qw.data_ptr(), qw.stride(0),
            sc.data_ptr(), _lib.dtype_code(sc.dtype), int(group_size), _ptr(b),
            y.data_ptr(), y.stride(0), M, N, K, _lib.dtype_code(x.dtype),
            _ptr(ws), ws_bytes, _lib.stream_ptr(dev))
    _lib.check(rc)
    return y.view(*x.shape[:-1], N)



def w8a16_silu_linear(gate_up: torch.Tensor, qweight: torch.Tensor, scale: torch.Tensor,
                      bias: torch.Tensor | None = None, group_size: int = 0,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """w8a16_linear(silu_mul(gate_up), ...): the MLP's act_fn and down_proj
    (layers/activation.py:6-11 then the W8A16 linear). gate_up: (..., 2K); the
    activation is SiluAndMul's, bit for bit. One launch while the fused form
    stages its activation rows in LDS (min(M, 16) (2K + 16) <= 33,024 bytes),
    the two separate launches otherwise (the faster of the two there)."""
    assert qweight.dtype == torch.int8 and qweight.dim() == 2
    N, K = qweight.shape
    g2 = gate_up.reshape(-1, gate_up.shape[-1])
    M = g2.shape[0]
    assert g2.shape[1] == 2 * K, f"gate_up {tuple(g2.shape)} needs 2K = {2 * K} columns"
    if g2.stride(-1) != 1 or (M > 1 and g2.stride(0) % 8 != 0) or g2.data_ptr() % 16:
        g2 = g2.contiguous()
    qw = qweight if qweight.is_contiguous() else qweight.contiguous()
    sc = scale.contiguous()
    if group_size:
        assert sc.numel() == N * (K // group_size), "per-group scale must be (N, K // group_size)"
    else:
        assert sc.numel() == N, "per-channel scale must have N entries"
    if min(M, 16) * (2 * K + 16) > 33024:
        y = w8a16_linear(silu_mul(g2), qw, sc, bias, group_size, out)
        return y.view(*gate_up.shape[:-1], N)
    b = None if bias is None else bias.to(gate_up.dtype).contiguous()
    dev = _lib.require_device(g2, qw, sc, b, out)
    if out is None:
        y = torch.empty((M, N), device=dev, dtype=gate_up.dtype)
    else:
        y = out.reshape(M, N)
        assert y.dtype == gate_up.dtype and y.stride(-1) == 1
    if M == 0:
        return y.view(*gate_up.shape[:-1], N)
    lib = _lib.load()
    with torch.cuda.device(dev):
        rc = lib.sd_w8a16_silu_linear(
            g2.data_ptr(), g2.stride(0), qw.data_ptr(), qw.stride(0),
            sc.data_ptr(), _lib.dtype_code(sc.dtype), int(group_size), _ptr(b),
            y.data_ptr(), y.stride(0), M, N, K, _lib.dtype_code(gate_up.dtype),
            _lib.stream_ptr(dev))
    _lib.check(rc)
    return y.view(*gate_up.shape[:-1], N)


# Rows up to which the add + RMSNorm runs inside the projection's launch (the
# fused entry points accept more; past this the two launches measured faster):
# up to 16 rows of at most 1024 columns, where each wave of a workgroup
# normalises up to 4 rows in one round trip, and up to 4 rows of wider ones,
# where the waves take their rows one at a time.
NORM_FUSED_MAX_ROWS = 16
NORM_FUSED_MAX_ROWS_WIDE = 4


def _norm_fused(M: int, K: int) -> bool:
    limit = NORM_FUSED_MAX_ROWS if K <= 1024 else NORM_FUSED_MAX_ROWS_WIDE
    return M <= limit and K % 8 == 0 and K <= 8192


def w8a16_rmsnorm_linear(x: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                         qweight: torch.Tensor, scale: torch.Tensor,
                         bias: torch.Tensor | None = None, group_size: int = 0,
                         residual: torch.Tensor | None = None,
                         residual_out: torch.Tensor | None = None,
                         out: torch.Tensor | None = None) -> torch.Tensor:
    """w8a16_linear(rmsnorm(x, norm_weight, eps, residual)[0], ...): a decoder
    layer's RMSNorm (layers/layernorm.py:16-47) feeding the next projection.
    The normalised rows equal ``rmsnorm``'s bit for bit. With ``residual``,
    ``residual_out`` (sharing no byte with x, residual or the output; None:
    not written)
    receives bf16(x + residual), ``rmsnorm``'s second output. One launch for
    up to 16 rows at K <= 1024 and up to 4 rows above: at one or two rows
    every wave of the row-streaming GEMV forms the norm of its columns; from
    three rows the tiled kernel's workgroups normalise their rows while
    staging them. More rows, or rows that do not fit the staging LDS, take the
    two separate launches (same results)."""
    assert qweight.dtype == torch.int8 and qweight.dim() == 2
    N, K = qweight.shape
    assert x.shape[-1] == K and norm_weight.shape == (K,)
    assert residual_out is None or residual is not None, "residual_out needs a residual"
    x2 = _rows16(x, "x")
    M = x2.shape[0]
    nw = norm_weight.to(x.dtype).contiguous()
    qw = qweight if qweight.is_contiguous() else qweight.contiguous()
    sc = scale.contiguous()
    if group_size:
        assert sc.numel() == N * (K // group_size), "per-group scale must be (N, K // group_size)"
    else:
        assert sc.numel() == N, "per-channel scale must have N entries"
    r2 = ro = None
    if residual is not None:
        assert residual.shape == x.shape and residual.dtype == x.dtype
        r2 = _rows16(residual, "residual")
    if residual_out is not None:
        assert residual_out.shape == x.shape and residual_out.dtype == x.dtype
        ro = residual_out.reshape(M, K)
        assert ro.stride(-1) == 1 and ro.data_ptr() % 16 == 0 and (M <= 1 or ro.stride(0) % 8 == 0)
    b = None if bias is None else bias.to(x.dtype).contiguous()
    dev = _lib.require_device(x2, nw, qw, sc, b, r2, ro, out)
    if out is None:
        y = torch.empty((M, N), device=dev, dtype=x.dtype)
    else:
        y = out.reshape(M, N)
        assert y.dtype == x.dtype and y.stride(-1) == 1
    shape = (*x.shape[:-1], N)
    if M == 0:
        return y.view(shape)
    rc = _lib.SD_ERR_UNSUPPORTED
    if _norm_fused(M, K):
        lib = _lib.load()
        with torch.cuda.device(dev):
            rc = lib.sd_w8a16_rmsnorm_linear(
                x2.data_ptr(), x2.stride(0), _ptr(r2), 0 if r2 is None else r2.stride(0),
                _ptr(ro), 0 if ro is None else ro.stride(0), nw.data_ptr(), float(eps),
                qw.data_ptr(), qw.stride(0), sc.data_ptr(), _lib.dtype_code(sc.dtype),
                int(group_size), _ptr(b), y.data_ptr(), y.stride(0), M, N, K,
                _lib.dtype_code(x.dtype), _lib.stream_ptr(dev))
    if rc == _lib.SD_ERR_UNSUPPORTED:
        # more rows, or rows that do not fit the staging LDS: the RMSNorm launch
        # (writing residual_out itself), then the plain linear
        h = torch.empty_like(x2)
        rsum = ro if ro is not None or r2 is None else torch.empty_like(r2)
        lib = _lib.load()
        with torch.cuda.device(dev):
            rc = lib.sd_rmsnorm(x2.data_ptr(), x2.stride(0), _ptr(r2),
                                0 if r2 is None else r2.stride(0), nw.data_ptr(), h.data_ptr(),
                                h.stride(0), _ptr(rsum), 0 if rsum is None else rsum.stride(0), M,
                                K, float(eps), _lib.dtype_code(x.dtype), _lib.stream_ptr(dev))
        _lib.check(rc)
        w8a16_linear(h, qw, sc, b, group_size, y)
        return y.view(shape)
    _lib.check(rc)
    return y.view(shape)


def w8a16_gate_up_silu(x: torch.Tensor, qweight: torch.Tensor, scale: torch.Tensor,
                       norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                       residual: torch.Tensor | None = None,
                       residual_out: torch.Tensor | None = None,
                       bias: torch.Tensor | None = None,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    """silu_mul(w8a16_linear(a, qweight, scale)) of the MLP (models/qwen3.py
    Qwen3MLP.forward: gate_up_proj then act_fn), with a = x, or a =
    rmsnorm(x, norm_weight, eps, residual) when ``norm_weight`` is given
    (``residual_out`` as in ``w8a16_rmsnorm_linear``). qweight (2I, K) =
    [gate; up], per-channel scale (2I,); returns (..., I), bit for bit the
    separate calls. One launch on the row-streaming path (one or two rows,
    weights up to 32 MiB: a wave streams gate row i with up row I + i and
    forms the pair's SiLU once) and on the K-split path of narrow layers (a
    workgroup takes gate tile g and up tile g with the plain projection's K
    split; with the norm, above 16 rows at K <= 1024 or 4 rows above, the
    RMSNorm launch comes first);
    other shapes take the separate launches."""
    assert qweight.dtype == torch.int8 and qweight.dim() == 2
    N, K = qweight.shape
    assert N % 2 == 0 and x.shape[-1] == K
    assert residual_out is None or residual is not None, "residual_out needs a residual"
    assert residual is None or norm_weight is not None, "a residual needs the norm weight"
    x2 = _rows16(x, "x")
    M = x2.shape[0]
    nw = None if norm_weight is None else norm_weight.to(x.dtype).contiguous()
    qw = qweight if qweight.is_contiguous() else qweight.contiguous()
    sc = scale.contiguous()
    assert sc.numel() == N, "per-channel scale must have N entries"
    r2 = ro = None
    if residual is not None:
        assert residual.shape == x.shape and residual.dtype == x.dtype
        r2 = _rows16(residual, "residual")
    if residual_out is not None:
        assert residual_out.shape == x.shape and residual_out.dtype == x.dtype
        ro = residual_out.reshape(M, K)
        assert ro.stride(-1) == 1 and ro.data_ptr() % 16 == 0 and (M <= 1 or ro.stride(0) % 8 == 0)
    b = None if bias is None else bias.to(x.dtype).contiguous()
    dev = _lib.require_device(x2, nw, qw, sc, b, r2, ro, out)
    shape = (*x.shape[:-1], N // 2)
    if out is None:
        y = torch.empty((M, N // 2), device=dev, dtype=x.dtype)
    else:
        y = out.reshape(M, N // 2)
        assert y.dtype == x.dtype and y.stride(-1) == 1
    if M == 0:
        return y.view(shape)
    lib = _lib.load()
    xa, ra, roa, nwa = x2, r2, ro, nw
    if nw is not None and not _norm_fused(M, K) and K % 8 == 0 and K <= 8192:
        # past the rows where the staged norm pays (every workgroup normalises
        # all of them): the RMSNorm launch (writing residual_out itself), then
        # the paired projection on the normalised rows
        xa = torch.empty_like(x2)
        rsum = ro if ro is not None or r2 is None else torch.empty_like(r2)
        with torch.cuda.device(dev):
            rc = lib.sd_rmsnorm(x2.data_ptr(), x2.stride(0), _ptr(r2),
                                0 if r2 is None else r2.stride(0), nw.data_ptr(), xa.data_ptr(),
                                xa.stride(0), _ptr(rsum), 0 if rsum is None else rsum.stride(0), M,
                                K, float(eps), _lib.dtype_code(x.dtype), _lib.stream_ptr(dev))
        _lib.check(rc)
        ra = roa = nwa = None
    with torch.cuda.device(dev):
        rc = lib.sd_w8a16_gate_up_silu(
            xa.data_ptr(), xa.stride(0), _ptr(ra), 0 if ra is None else ra.stride(0),
            _ptr(roa), 0 if roa is None else roa.stride(0), _ptr(nwa), float(eps),
            qw.data_ptr(), qw.stride(0), sc.data_ptr(), _lib.dtype_code(sc.dtype), _ptr(b),
            y.data_ptr(), y.stride(0), M, N, K, _lib.dtype_code(x.dtype), _lib.stream_ptr(dev))
    if rc == _lib.SD_ERR_UNSUPPORTED and (nwa is None or (K % 8 == 0 and K <= 8192)):
        # neither the row-streaming nor the K-split path: the projection, then
        # the SiLU launch
        if nwa is None:
            gu = w8a16_linear(xa, qw, sc, b)
        else:
            gu = w8a16_rmsnorm_linear(x2, nw, eps, qw, sc, b, residual=r2, residual_out=ro)
        silu_mul(gu, out=y)
        return y.view(shape)
    _lib.check(rc)
    return y.view(shape)


def quantize_int8(w: torch.Tensor, group_size: int = 0):
    """Symmetric int8 quantization of a 2-D weight on the GPU (the W8A16
    format's producer, nanovllm/layers/quant.py:123-148): per row (group_size
    0) or per group of columns, scale = max(max|w| / 127, 1e-8) in fp32,
    q = clamp(round_half_even(w / scale), -127, 127). Returns (q int8 (N, K),
    scale bf16 (N, K // group) — the fp32 scale rounded after q)."""
    assert w.dim() == 2, f"expects a 2-D weight, got {tuple(w.shape)}"
    N, K = w.shape
    G = group_size if group_size > 0 else K
    assert K % G == 0, "group_size must divide K"
    if w.stride(-1) != 1 or w.data_ptr() % 16 or (N > 1 and w.stride(0) % 8):
        w = w.contiguous()
    dev = _lib.require_device(w)
    q = torch.empty((N, K), dtype=torch.int8, device=dev)
    scale = torch.empty((N, K // G), dtype=torch.bfloat16, device=dev)
    if N:
        lib = _lib.load()
        with torch.cuda.device(dev):
            rc = lib.sd_quantize_int8(w.data_ptr(), w.stride(0), _lib.dtype_code(w.dtype),
                                      q.data_ptr(), q.stride(0), scale.data_ptr(), N, K,
                                      int(group_size), _lib.stream_ptr(dev))
        _lib.check(rc)
    return q, scale


# --------------------------------------------------------------- draft-step neighbours
def _rows16(t: torch.Tensor, what: str) -> torch.Tensor:
    """2-D (rows, width) view with a unit last stride and 16-byte aligned rows."""
    t2 = t.reshape(-1, t.shape[-1])
    if t2.stride(-1) != 1 or t2.data_ptr() % 16 or (t2.shape[0] > 1 and t2.stride(0) % 8):
        t2 = t2.contiguous()
    return t2


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
            residual: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """RMSNorm.forward (nanovllm/layers/layernorm.py:16-47) over the last dim.

    ``residual is None``: returns ``bf16(bf16(x * rsqrt(mean(x^2) + eps)) * weight)``.
    Otherwise returns ``(out, residual_out)`` with ``s = x + residual`` in fp32,
    ``residual_out = s`` rounded to the dtype and ``out`` the norm of ``s``.
    """
    H = x.shape[-1]
    x2 = _rows16(x, "x")
    assert weight.shape == (H,), "weight must be (hidden,)"
    w = weight.to(x.dtype).contiguous()
    r2 = None if residual is None else _rows16(residual, "residual")
    if r2 is not None:
        assert residual.shape == x.shape and residual.dtype == x.dtype
    dev = _lib.require_device(x2, w, r2, out)
    o = torch.empty_like(x2) if out is None else out.reshape(-1, H)
    ro = None if r2 is None else torch.empty_like(r2)
    rows = x2.shape[0]
    if rows:
        lib = _lib.load()
        with torch.cuda.device(dev):
            rc = lib.sd_rmsnorm(x2.data_ptr(), x2.stride(0), _ptr(r2), 0 if r2 is None else r2.stride(0),
                                w.data_ptr(), o.data_ptr(), o.stride(0), _ptr(ro),
                                0 if ro is None else ro.stride(0), rows, H, float(eps),
                                _lib.dtype_code(x.dtype), _lib.stream_ptr(dev))
        _lib.check(rc)
    o = o.view(x.shape)
    if residual is None:
        return o
    return o, ro.view(x.shape)


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor,
                 cos_sin_cache: torch.Tensor, q_weight: torch.Tensor | None = None,
                 k_weight: torch.Tensor | None = None, eps: float = 1e-6,
                 v: torch.Tensor | None = None, k_cache: torch.Tensor | None = None,
                 v_cache: torch.Tensor | None = None,
                 slot_mapping: torch.Tensor | None = None) -> None:
    """In place on q (T, Hq, 128) and k (T, Hkv, 128) (strided views allowed):
    per-head RMSNorm with q_weight / k_weight (skipped when None), then
    rotate-half RoPE at ``positions`` from ``cos_sin_cache`` (max_pos, [1,] 128)
    fp32 = [cos | sin] (nanovllm/models/qwen3.py:80-88,
    layers/rotary_embedding.py:6-48).

    With ``v``, ``k_cache``, ``v_cache`` and ``slot_mapping``: also
    store_kvcache of the finished k rows and of v (layers/attention.py:33-40)
    in the same launch; caches (num_blocks, block_size, Hkv, 128)."""
    assert q.dim() == 3 and k.dim() == 3 and q.shape[0] == k.shape[0]
    assert q.shape[-1] == 128 and k.shape[-1] == 128 and q.stride(-1) == 1 and k.stride(-1) == 1
    assert q.dtype == k.dtype
    assert (q_weight is None) == (k_weight is None)
    T = q.shape[0]
    cs = cos_sin_cache.reshape(cos_sin_cache.shape[0], -1)
    assert cs.dtype == torch.float32 and cs.shape[1] >= 128 and cs.stride(-1) == 1
    pos = positions.reshape(-1)
    if pos.dtype != torch.int64:
        pos = pos.to(torch.int64)
    pos = pos.contiguous()
    assert pos.numel() == T
    qw = None if q_weight is None else q_weight.to(q.dtype).contiguous()
    kw = None if k_weight is None else k_weight.to(q.dtype).contiguous()
    dev = _lib.require_device(q, k, pos, cs, qw, kw)
    if T == 0:
        return
    lib = _lib.load()
    if k_cache is not None:
        assert v is not None and v_cache is not None and slot_mapping is not None
        assert v.shape == k.shape and v.stride(-1) == 1 and v.dtype == k.dtype
        assert k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride()
        assert k_cache.dtype == k.dtype and k_cache.shape[2:] == k.shape[1:]
        slots = _i32(slot_mapping.reshape(-1)).contiguous()
        assert slots.numel() == T
        _lib.require_device(v, k_cache, v_cache, slots)
        with torch.cuda.device(dev):
            rc = lib.sd_qk_norm_rope_store(
                q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
                v.data_ptr(), v.stride(0), v.stride(1), T, q.shape[1], k.shape[1], 128,
                _ptr(qw), _ptr(kw), float(eps), pos.data_ptr(), cs.data_ptr(), cs.stride(0),
                cs.shape[0], k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0),
                k_cache.stride(1), k_cache.stride(2), k_cache.shape[0], k_cache.shape[1],
                slots.data_ptr(), _lib.dtype_code(q.dtype), _lib.stream_ptr(dev))
        _lib.check(rc)
        return
    with torch.cuda.device(dev):
        rc = lib.sd_qk_norm_rope(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0),
                                 k.stride(1), T, q.shape[1], k.shape[1], 128, _ptr(qw), _ptr(kw),
                                 float(eps), pos.data_ptr(), cs.data_ptr(), cs.stride(0),
                                 cs.shape[0], _lib.dtype_code(q.dtype), _lib.stream_ptr(dev))
    _lib.check(rc)


def silu_mul(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """SiluAndMul (nanovllm/layers/activation.py:6-11): x (..., 2I) -> (..., I)."""
    W = x.shape[-1]
    assert W % 2 == 0
    x2 = _rows16(x, "x")
    dev = _lib.require_device(x2, out)
    o = torch.empty((x2.shape[0], W // 2), dtype=x.dtype, device=dev) if out is None \
        else out.reshape(-1, W // 2)
    if x2.shape[0]:
        lib = _lib.load()
        with torch.cuda.device(dev):
            rc = lib.sd_silu_mul(x2.data_ptr(), x2.stride(0), o.data_ptr(), o.stride(0),
                                 x2.shape[0], W // 2, _lib.dtype_code(x.dtype),
                                 _lib.stream_ptr(dev))
        _lib.check(rc)
    return o.view(*x.shape[:-1], W // 2)


# Philox (seed, offset) per device for calls that bring no rng_state: seeded
# from torch's initial seed, its offset advanced on the stream after each draw
# (so graph replays draw fresh noise too).
_RNG_STATES: dict = {}


def default_rng_state(dev: torch.device) -> torch.Tensor:
    st = _RNG_STATES.get(dev.index)
    if st is None:
        st = torch.tensor([torch.initial_seed() & 0x7FFFFFFFFFFFFFFF, 0], dtype=torch.int64,
                          device=dev)
        _RNG_STATES[dev.index] = st
    return st


def sample(logits: torch.Tensor, temperatures: torch.Tensor | None = None,
           rng_state: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """One token per row of logits (rows, vocab): greedy argmax when
    ``temperatures`` is None (or a row's temperature is <= 0), otherwise the
    exponential-race draw of ``Sampler.forward`` (nanovllm/layers/sampler.py:6-12)
    with Philox noise keyed by ``rng_state`` = (seed, offset) int64 on the device.
    A given ``rng_state`` is the caller's to advance; without one the device's
    default state is used and advanced."""
    assert logits.dim() == 2 and logits.stride(-1) == 1
    rows, V = logits.shape
    t = None
    advance = False
    if temperatures is not None:
        t = temperatures.reshape(-1).to(torch.float32).contiguous()
        assert t.numel() == rows
        if rng_state is None:
            rng_state, advance = default_rng_state(logits.device), True
        assert rng_state.numel() == 2 and rng_state.dtype == torch.int64
    dev = _lib.require_device(logits, t, rng_state, out)
    o = torch.empty(rows, dtype=torch.int64, device=dev) if out is None else out
    assert o.dtype == torch.int64 and o.numel() == rows and o.is_contiguous()
    if rows:
        lib = _lib.load()
        with torch.cuda.device(dev):
            ws_bytes = lib.sd_sample_workspace_size(rows, V)
            ws = _workspace(ws_bytes, dev)
            rc = lib.sd_sample(logits.data_ptr(), logits.stride(0), _lib.dtype_code(logits.dtype),
                               rows, V, _ptr(t), _ptr(rng_state), o.data_ptr(), _ptr(ws),
                               ws_bytes, _lib.stream_ptr(dev))
        _lib.check(rc)
        if advance:
            rng_state[1:].add_(1)
    return o


def verify_batch(draft: torch.Tensor, target_logits: torch.Tensor, draft_tokens: torch.Tensor,
                 temperatures: torch.Tensor | None = None, draft_is_point_mass: bool = False,
                 rng_state: torch.Tensor | None = None):
    """Rejection-sampling verification (nanovllm/spec_decode/verify.py:39-183):
    returns (accepted (B,) int64, bonus (B,) int64, accept_mask (B, k) bool).

    ``draft`` (B, k, V): the draft's raw logits, or its probabilities with
    ``draft_is_point_mass``; ``target_logits`` (B, k + 1, V); the row dims may
    be strided, the vocabulary contiguous. Noise is Philox keyed by
    ``rng_state`` (seed, offset) on the device; without one the device's
    default state is used and advanced."""
    assert draft.dim() == 3 and target_logits.dim() == 3 and draft_tokens.dim() == 2
    B, k, V = draft.shape
    assert target_logits.shape[0] == B and target_logits.shape[2] == V
    assert target_logits.shape[1] == k + 1, "target_logits must hold k + 1 rows"
    assert draft_tokens.shape == (B, k)
    assert draft.stride(-1) == 1 and target_logits.stride(-1) == 1
    tok = draft_tokens if draft_tokens.dtype == torch.int64 else draft_tokens.to(torch.int64)
    if tok.stride(-1) != 1:
        tok = tok.contiguous()
    t = None if temperatures is None else temperatures.reshape(-1).to(torch.float32).contiguous()
    if t is not None and t.numel() == 1 and B > 1:
        t = t.expand(B).contiguous()
    advance = rng_state is None
    if advance:
        rng_state = default_rng_state(draft.device)
    dev = _lib.require_device(draft, target_logits, tok, t, rng_state)
    accepted = torch.empty(B, dtype=torch.int64, device=dev)
    bonus = torch.empty(B, dtype=torch.int64, device=dev)
    mask = torch.empty((B, k), dtype=torch.bool, device=dev)
    if B:
        lib = _lib.load()
        with torch.cuda.device(dev):
            ws_bytes = lib.sd_verify_batch_workspace_size(B, k, V)
            ws = _workspace(ws_bytes, dev)
            rc = lib.sd_verify_batch(draft.data_ptr(), draft.stride(0), draft.stride(1),
                                     _lib.dtype_code(draft.dtype), target_logits.data_ptr(),
                                     target_logits.stride(0), target_logits.stride(1),
                                     _lib.dtype_code(target_logits.dtype), tok.data_ptr(),
                                     tok.stride(0), _ptr(t), int(bool(draft_is_point_mass)),
                                     rng_state.data_ptr(), B, k, V, accepted.data_ptr(),
                                     bonus.data_ptr(), mask.data_ptr(), _ptr(ws), ws_bytes,
                                     _lib.stream_ptr(dev))
        _lib.check(rc)
        if advance:
            rng_state[1:].add_(1)
    return accepted, bonus, mask


# ---------------------------------------------------------------------- measurement
def stream_read(buf: torch.Tensor, sink: torch.Tensor, workgroups: int = 0) -> None:
    """One streaming read of ``buf`` (sd_stream_read): the box's read ceiling,
    the bench's second denominator beside the 8 TB/s data-sheet peak.
    ``sink``: at least one int32 of device memory, practically never written.
    ``workgroups`` <= 0 takes the library's default (six per CU)."""
    assert buf.is_contiguous() and sink.dtype == torch.int32 and sink.numel() >= 1
    dev = _lib.require_device(buf, sink)
    nbytes = buf.numel() * buf.element_size() // 16 * 16
    with torch.cuda.device(dev):
        rc = _lib.load().sd_stream_read(buf.data_ptr(), nbytes, sink.data_ptr(),
                                         int(workgroups), _lib.stream_ptr(dev))
    _lib.check(rc)

"""W8A16 quantization and dequantize-then-matmul restated in numpy.

Test infrastructure only (see oracle/__init__.py).
"""
import numpy as np

from . import bf16

QMAX = 127


def _grouped(w: np.ndarray, granularity: str, group_size: int) -> np.ndarray:
    N, K = w.shape
    if granularity == "per_channel":
        return w.reshape(N, 1, K)
    if granularity == "per_group":
        assert group_size > 0 and K % group_size == 0
        return w.reshape(N, K // group_size, group_size)
    raise ValueError(granularity)


def quantize_weight(w: np.ndarray, granularity: str = "per_channel", group_size: int = 128):
    """nanovllm/layers/quant.py:123-148. In fp32: scale = max(amax / 127, 1e-8)
    over the channel (or group); q = clip(round_half_even(w / scale), -127, 127).
    Returns (q int8 (N, K), scale as bf16 values held in float32 — (N,) or
    (N, K // group_size)); q uses the unrounded fp32 scale, as in the reference."""
    wf = np.asarray(w, dtype=np.float32)
    N, K = wf.shape
    g = _grouped(wf, granularity, group_size)
    scale = np.maximum(np.abs(g).max(axis=2, keepdims=True) / np.float32(QMAX),
                       np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.rint(g / scale), -QMAX, QMAX).astype(np.int8).reshape(N, K)
    scale = scale.reshape(N) if granularity == "per_channel" else scale.reshape(N, K // group_size)
    return q, bf16.round_f32(scale)


def dequantize_weight(q: np.ndarray, scale: np.ndarray, granularity: str = "per_channel",
                      group_size: int = 128, dtype=np.float64) -> np.ndarray:
    """nanovllm/layers/quant.py:151-159: q * scale per channel or per group."""
    N, K = q.shape
    qf = q.astype(dtype)
    s = np.asarray(scale, dtype=dtype)
    if granularity == "per_channel":
        return qf * s.reshape(N, 1)
    return (qf.reshape(N, K // group_size, group_size) *
            s.reshape(N, K // group_size, 1)).reshape(N, K)


def int8_linear(x: np.ndarray, q: np.ndarray, scale: np.ndarray, bias=None,
                granularity: str = "per_channel", group_size: int = 128,
                dtype=np.float64) -> np.ndarray:
    """y = x @ dequantize(q, scale).T (+ bias), all in ``dtype`` — the
    dequantize-then-matmul that the fused kernel must match
    (the math of nanovllm/layers/quant.py:209-223)."""
    x2 = np.asarray(x, dtype=dtype).reshape(-1, q.shape[1])
    y = x2 @ dequantize_weight(q, scale, granularity, group_size, dtype).T
    if bias is not None:
        y = y + np.asarray(bias, dtype=dtype)
    return y.reshape(*np.shape(x)[:-1], q.shape[0])


def algorithmic_bytes(M: int, N: int, K: int, act_bytes: int = 2, scale_bytes: int = 2,
                      group_size: int = 0) -> int:
    """Minimum HBM bytes of one call: int8 weight once, scales, x read, y written."""
    nscale = N if group_size == 0 else N * (K // group_size)
    return N * K + nscale * scale_bytes + act_bytes * M * K + act_bytes * M * N

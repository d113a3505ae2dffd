"""W8A16 (int8 weight, 16-bit activation) — drop-in for ``nanovllm/layers/quant.py``.

* ``int8_linear`` — the fused-dequantization linear (quant.py:262-310), served
  by the gfx950 kernel: int8 weights stream from HBM once and become 16-bit
  floats only in registers; fp32 accumulation; the per-channel scale
  multiplies the fp32 accumulator. The output dtype is the activation dtype
  (the reference always writes bf16, and only ever receives bf16).
* ``quantize_weight`` — the symmetric quantizer (quant.py:123-148) on the gfx950
  quantize kernel (bit-identical to the reference's fp32 formula; a weight on
  the CPU is an error, as for every op here); ``dequantize_weight`` — the
  reference dequantization (quant.py:151-159) in plain torch, for checking.
* ``hf_names_to_modules`` — checkpoint tensor names to engine module names
  (quant.py:31-63).
* ``apply_int8_quant`` — in-place swap of named linear layers to int8
  (quant.py:66-117).
"""
from __future__ import annotations

import re

import torch
import torch.nn as nn

from .. import ops

QMAX = 127


def quantize_weight(w: torch.Tensor, granularity: str = "per_channel", group_size: int = 128):
    """Symmetric int8 quantization (zero point 0) of a 2-D weight ``[N, K]``.

    scale = max(|w| over the channel or group) / 127, floored at 1e-8, computed
    in fp32; q = clamp(round_half_even(w / scale), -127, 127). Returns
    ``(q int8 [N, K], scale bf16 [N] or [N, K // group_size])`` — the scale is
    rounded to bf16 only after q has been computed with the fp32 value.
    """
    assert w.dim() == 2, f"expects a 2-D weight, got {tuple(w.shape)}"
    N, K = w.shape
    if granularity == "per_channel":
        q, scale = ops.quantize_int8(w, 0)
        return q, scale.view(N)
    if granularity == "per_group":
        assert group_size > 0 and K % group_size == 0
        return ops.quantize_int8(w, group_size)
    raise ValueError(granularity)


# Checkpoint (HF) tensor names -> engine module names: q/k/v are one qkv_proj
# and gate/up one gate_up_proj in the engine (quant.py:31-38).
_HF_TO_ENGINE = [
    (re.compile(r"^(.*)\.self_attn\.(?:q|k|v)_proj\.weight$"), r"\1.self_attn.qkv_proj"),
    (re.compile(r"^(.*)\.self_attn\.o_proj\.weight$"), r"\1.self_attn.o_proj"),
    (re.compile(r"^(.*)\.mlp\.(?:gate|up)_proj\.weight$"), r"\1.mlp.gate_up_proj"),
    (re.compile(r"^(.*)\.mlp\.down_proj\.weight$"), r"\1.mlp.down_proj"),
]


def hf_names_to_modules(hf_names):
    """quant.py:41-63: the engine modules a quant_config's ``quantized_layers``
    name. A packed module must be complete (q, k and v; gate and up), else
    ValueError — never a half-quantized module."""
    groups = {}
    for n in hf_names:
        for rx, rep in _HF_TO_ENGINE:
            if rx.match(n):
                groups.setdefault(rx.sub(rep, n), set()).add(n)
                break
        else:
            raise ValueError(f"unrecognised quantized layer name: {n}")
    for mod, src in groups.items():
        if mod.endswith("qkv_proj") and len(src) != 3:
            raise ValueError(f"{mod} needs q, k and v together, got {sorted(src)}")
        if mod.endswith("gate_up_proj") and len(src) != 2:
            raise ValueError(f"{mod} needs gate and up together, got {sorted(src)}")
    return sorted(groups)


def dequantize_weight(q: torch.Tensor, scale: torch.Tensor,
                      granularity: str = "per_channel", group_size: int = 128):
    """fp32 ``q * scale`` (per channel or per group); for checking only."""
    N, K = q.shape
    qf = q.to(torch.float32)
    sf = scale.to(torch.float32)
    if granularity == "per_channel":
        return qf * sf.view(N, 1)
    return (qf.view(N, K // group_size, group_size) * sf.view(N, K // group_size, 1)).view(N, K)


def int8_linear(x: torch.Tensor, qweight: torch.Tensor, scale: torch.Tensor,
                bias: torch.Tensor | None = None,
                granularity: str = "per_channel", group_size: int = 128,
                out_features: int | None = None, cfg_: dict | None = None):
    """y = x @ dequant(qweight).T + bias with the dequantization fused.

    x: [..., K] bf16/fp16; qweight: [N, K] int8; scale: [N] (per_channel) or
    [N, K // group_size] (per_group). ``cfg_`` (Triton tile overrides in the
    reference) is accepted and ignored.
    """
    del cfg_
    assert qweight.dtype == torch.int8
    if granularity not in ("per_channel", "per_group"):
        raise ValueError(granularity)
    N = qweight.shape[0]
    if out_features and out_features != N:
        qweight = qweight[:out_features]
        scale = scale[:out_features]
    gs = group_size if granularity == "per_group" else 0
    return ops.w8a16_linear(x, qweight, scale, bias, gs)


def apply_int8_quant(model: nn.Module, module_names, granularity: str = "per_channel",
                     group_size: int = 128, verbose: bool = False):
    """Quantize the named ``LinearBase`` submodules of ``model`` in place.

    Each module's bf16 ``weight`` becomes an int8 parameter plus a
    ``weight_scale`` parameter, and ``quant_granularity``/``quant_group_size``
    are set, so ``LinearBase._apply`` dispatches to ``int8_linear``. Returns one
    report dict per module (shape, relative error on up to 256 rows,
    saturation fraction, scale range, bytes before/after).
    """
    from .linear import LinearBase

    wanted = set(module_names)
    report = []
    for name, mod in model.named_modules():
        if name not in wanted:
            continue
        if not isinstance(mod, LinearBase):
            raise TypeError(f"{name} is a {type(mod).__name__}, not a LinearBase")
        w = mod.weight.data
        assert w.dtype == torch.bfloat16, f"{name}: weight dtype {w.dtype} is not bf16"
        q, s = quantize_weight(w, granularity, group_size)
        mod.weight = nn.Parameter(q.to(w.device).contiguous(), requires_grad=False)
        mod.weight_scale = nn.Parameter(s.to(w.device).contiguous(), requires_grad=False)
        mod.quant_granularity = granularity
        mod.quant_group_size = group_size
        rows = min(w.shape[0], 256)
        ref = w[:rows].to(torch.float32)
        err = ref - dequantize_weight(q[:rows], s[:rows], granularity, group_size)
        report.append({
            "name": name, "shape": list(w.shape),
            "rel_err": (err.norm() / ref.norm()).item(),
            "saturate_frac": (q.abs() == QMAX).float().mean().item(),
            "scale_min": float(s.float().min()), "scale_max": float(s.float().max()),
            "bytes_before": w.numel() * 2, "bytes_after": q.numel() + s.numel() * 2,
        })
        if verbose:
            print(f"  [int8] {name:<46} {tuple(w.shape)} rel_err={report[-1]['rel_err']:.5f}")
    missing = wanted - {r["name"] for r in report}
    if missing:
        raise KeyError(f"modules not found in the model: {sorted(missing)}")
    return report

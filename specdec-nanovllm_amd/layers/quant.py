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


def _error_sample(w: torch.Tensor, q: torch.Tensor, s: torch.Tensor, granularity: str,
                  group_size: int) -> float:
    """Relative Frobenius error of the dequantized weight on its first 256
    rows (a sample, so the check never expands a whole layer to fp32)."""
    n = min(w.shape[0], 256)
    ref = w[:n].float()
    return ((ref - dequantize_weight(q[:n], s[:n], granularity, group_size)).norm()
            / ref.norm()).item()


def _swap_to_int8(name: str, mod: nn.Module, granularity: str, group_size: int) -> dict:
    """Replace ``mod.weight`` (bf16) by its int8 form and a ``weight_scale``
    parameter, set the two attributes ``LinearBase._apply`` dispatches on, and
    describe what changed."""
    w = mod.weight.data
    q, s = quantize_weight(w, granularity, group_size)
    frozen = dict(requires_grad=False)
    mod.weight = nn.Parameter(q.to(w.device).contiguous(), **frozen)
    mod.weight_scale = nn.Parameter(s.to(w.device).contiguous(), **frozen)
    mod.quant_granularity, mod.quant_group_size = granularity, group_size
    sf = s.float()
    return dict(name=name, shape=list(w.shape),
                rel_err=_error_sample(w, q, s, granularity, group_size),
                saturate_frac=(q.abs() == QMAX).float().mean().item(),
                scale_min=float(sf.min()), scale_max=float(sf.max()),
                bytes_before=2 * w.numel(), bytes_after=q.numel() + 2 * s.numel())


def apply_int8_quant(model: nn.Module, module_names, granularity: str = "per_channel",
                     group_size: int = 128, verbose: bool = False):
    """Quantize the named ``LinearBase`` submodules of ``model`` in place
    (the contract of nanovllm/layers/quant.py:66-117).

    Each module's bf16 ``weight`` becomes an int8 parameter plus a
    ``weight_scale`` parameter, and ``quant_granularity``/``quant_group_size``
    are set, so ``LinearBase._apply`` dispatches to ``int8_linear``. Returns one
    report dict per module, in the model's module order (name, shape, relative
    error on up to 256 rows, saturation fraction, scale range, bytes
    before/after). Errors, as the reference raises them: ``KeyError`` for names
    the model lacks, ``TypeError`` for a module that is not a ``LinearBase``,
    ``AssertionError`` for a weight that is not bf16. Every module is checked
    before any is changed, so a refused call leaves the model as it was.
    """
    from .linear import LinearBase

    wanted = set(module_names)
    chosen = [(n, m) for n, m in model.named_modules() if n in wanted]
    absent = wanted.difference(n for n, _ in chosen)
    if absent:
        raise KeyError(f"modules not found in the model: {sorted(absent)}")
    for name, mod in chosen:
        if not isinstance(mod, LinearBase):
            raise TypeError(f"{name} is a {type(mod).__name__}, not a LinearBase")
        assert mod.weight.dtype == torch.bfloat16, \
            f"{name}: weight dtype {mod.weight.dtype} is not bf16"
    report = [_swap_to_int8(name, mod, granularity, group_size) for name, mod in chosen]
    if verbose:
        for r in report:
            print(f"int8 {r['name']}: {r['shape'][0]}x{r['shape'][1]}, "
                  f"rel err {r['rel_err']:.2e}, {r['bytes_before'] >> 10} -> "
                  f"{r['bytes_after'] >> 10} KiB")
    return report

"""Linear dispatch — the single-GPU part of ``nanovllm/layers/linear.py``.

``LinearBase._apply(x, bias)`` is the one call site of the W8A16 path in the
reference (linear.py:40-45): an int8 ``weight`` goes to ``int8_linear`` with
the module's ``weight_scale``/``quant_granularity``/``quant_group_size``,
anything else to ``F.linear``. Tensor-parallel sharding and its all-reduce are
not part of this single-GPU library (tp_size is 1).

``nn.Module`` already uses the name ``_apply(fn)`` for ``.to()``/``.cuda()``;
the reference overrides it with the linear dispatch, which breaks those calls.
Here a callable first argument is forwarded to ``nn.Module._apply``, so both
uses work.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .quant import int8_linear


class LinearBase(nn.Module):

    def __init__(self, input_size: int, output_size: int, bias: bool = False,
                 tp_dim: int | None = None):
        super().__init__()
        self.tp_dim = tp_dim
        self.tp_rank = 0
        self.tp_size = 1
        self.quant_granularity = "per_channel"
        self.quant_group_size = 128
        self.weight = nn.Parameter(torch.empty(output_size, input_size))
        if bias:
            self.bias = nn.Parameter(torch.empty(output_size))
        else:
            self.register_parameter("bias", None)

    def _apply(self, x, bias=None, *args, **kwargs):
        if callable(x) and not isinstance(x, torch.Tensor):
            return super()._apply(x, *(() if bias is None else (bias,)), *args, **kwargs)
        if self.weight.dtype == torch.int8:
            return int8_linear(x, self.weight, self.weight_scale, bias,
                               self.quant_granularity, self.quant_group_size)
        return F.linear(x, self.weight, bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError


class ReplicatedLinear(LinearBase):

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._apply(x, self.bias)

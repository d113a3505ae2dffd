"""``RMSNorm`` with the reference's interface (nanovllm/layers/layernorm.py:6-47)
on the HIP kernel ``sd_rmsnorm``: ``forward(x)`` is the plain norm,
``forward(x, residual)`` the fused residual add + norm returning
``(normed, new_residual)``; fp32 arithmetic with the module's bf16 roundings."""
from __future__ import annotations

import torch
from torch import nn

from .. import ops


class RMSNorm(nn.Module):

    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        if residual is None:
            return ops.rmsnorm(x, self.weight, self.eps)
        return ops.rmsnorm(x, self.weight, self.eps, residual=residual)

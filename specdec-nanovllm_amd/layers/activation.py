"""``SiluAndMul`` with the reference's interface (nanovllm/layers/activation.py:6-11)
on the HIP kernel ``sd_silu_mul``: x (..., 2I) = [gate | up] -> silu(gate) * up."""
from __future__ import annotations

import torch
from torch import nn

from .. import ops


class SiluAndMul(nn.Module):

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return ops.silu_mul(x)

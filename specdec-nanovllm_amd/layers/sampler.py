"""``Sampler`` with the reference's interface (nanovllm/layers/sampler.py:6-12) on
the HIP sampling kernel: logits / T, softmax, then argmax(probs / E) with
E ~ Exp(1) — computed in one pass as argmax(l / T - log E) — and greedy argmax
for rows whose temperature is <= 0. The noise is this library's Philox stream
(``ops.default_rng_state``), so draws match the reference in law, not sample
for sample."""
from __future__ import annotations

import torch
from torch import nn

from .. import ops


class Sampler(nn.Module):

    def forward(self, logits: torch.Tensor, temperatures: torch.Tensor) -> torch.Tensor:
        if logits.stride(-1) != 1:
            logits = logits.contiguous()
        return ops.sample(logits, temperatures)

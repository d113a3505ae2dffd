"""``verify_batch`` with the reference's signature and result type
(nanovllm/spec_decode/verify.py:29-183), on the fused HIP kernels of
``csrc/verify.hip``.

The algorithm is the reference's: q = softmax(draft / T) (or the given
probabilities for a point-mass draft), p = softmax(target / T); candidate j is
accepted with probability min(1, p_j[x_j] / q_j[x_j]); the accepted length is
the first rejection; the bonus token is drawn from normalize(max(0, p_a - q_a))
with q padded by a zero row (so "all accepted" draws from p_k). The random
numbers are this library's counter-based Philox noise rather than torch's
generator, so a draw matches the reference in law, not sample for sample.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from .. import ops


@dataclass
class VerifyResult:
    """Same fields as the reference's (verify.py:29-36)."""
    accepted: torch.Tensor      # (batch,) accepted prefix length
    bonus: torch.Tensor         # (batch,) the extra token of this round (always valid)
    n_proposed: torch.Tensor    # (batch,) candidates proposed
    accept_mask: torch.Tensor   # (batch, k) per-candidate acceptance


@torch.no_grad()
def verify_batch(draft_probs: torch.Tensor, target_logits: torch.Tensor,
                 draft_tokens: torch.Tensor, temperatures: Optional[torch.Tensor] = None,
                 draft_is_point_mass: bool = False,
                 rng_state: Optional[torch.Tensor] = None) -> VerifyResult:
    """verify.py:39-183. ``draft_probs`` are the draft's raw logits (the
    reference's historical name) or, with ``draft_is_point_mass``, its
    probabilities; ``target_logits`` holds k + 1 rows per sequence."""
    batch, k, _ = draft_probs.shape
    if temperatures is not None and temperatures.dim() == 0:
        temperatures = temperatures.reshape(1).expand(batch)
    accepted, bonus, mask = ops.verify_batch(draft_probs, target_logits, draft_tokens,
                                             temperatures, draft_is_point_mass, rng_state)
    n_proposed = torch.full((batch,), k, dtype=torch.long, device=draft_probs.device)
    return VerifyResult(accepted=accepted, bonus=bonus, n_proposed=n_proposed, accept_mask=mask)

"""Switch load-balancing loss on the gfx950 aux-loss kernels.

``load_balancing_loss_func`` keeps the signature and result of transformers'
(TF models/qwen3_moe/modeling_qwen3_moe.py:514-593, including the
attention-mask branch), and ``sequence_parallel_load_balancing_loss`` that of
parallel/parallel/engine/model_parallel/sequence_parallel.py:239-280.  The
forward and the closed-form backward are one kernel each; the top-k
selection is the router's, so counts match the routing exactly.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import ops
from .groups import require_single_rank


def _aux(logits: Tensor, num_experts: int, top_k: int, token_weight: Tensor | None) -> Tensor:
    aux, _ = ops.aux_loss_fwd(logits, token_weight, num_experts, top_k)
    return aux


def load_balancing_loss_func(
    gate_logits: Tensor | tuple[Tensor, ...] | None,
    num_experts: int | None = None,
    top_k: int = 2,
    attention_mask: Tensor | None = None,
) -> Tensor | int:
    """Switch aux loss over the concatenated router logits of every layer."""
    if gate_logits is None or not isinstance(gate_logits, tuple):
        return 0
    device = gate_logits[0].device
    if len(gate_logits) == 1:
        logits = gate_logits[0]
    else:
        logits = torch.cat([g.to(device) for g in gate_logits], dim=0)
    if num_experts is None:
        num_experts = logits.shape[-1]
    token_weight = None
    if attention_mask is not None:
        batch, seq = attention_mask.shape
        layers = logits.shape[0] // (batch * seq)
        token_weight = attention_mask.to(device=device, dtype=torch.float32).reshape(1, -1).expand(layers, -1)
        token_weight = token_weight.reshape(-1).contiguous()
    return _aux(logits, num_experts, top_k, token_weight)


def sequence_parallel_load_balancing_loss(
    router_logits: tuple[Tensor, ...] | None,
    *,
    num_experts: int,
    top_k: int,
    group,
) -> Tensor | None:
    """Aux loss over the global SP token population; one rank holds all of it here."""
    if not router_logits:
        return None
    require_single_rank(group, "sequence-parallel load-balancing loss")
    logits = router_logits[0] if len(router_logits) == 1 else torch.cat(tuple(router_logits), dim=0)
    return _aux(logits, num_experts, top_k, None)

"""The step before the MoE block: post_attention_layernorm -> router -> top-k -> aux.

In the reference a decoder layer normalises its residual stream with
``post_attention_layernorm`` (TF/models/qwen3_moe/modeling_qwen3_moe.py:345),
the MoE block's router takes the normalised rows
(``Qwen3MoeTopKRouter.forward``, :258-267), and the model later recomputes
the softmax and top-k of the same logits inside ``load_balancing_loss_func``
(:550-552).  ``norm_router_aux`` runs the norm kernel once (its output is
what the experts read) and one router pass whose top-k kernel also produces
the aux-loss partial sums, so the aux loss needs no second softmax or top-k.
Gradients flow to the residual stream, the norm weight and the router
weight through the ops' autograd.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import ops

__all__ = ["norm_router_aux"]


def norm_router_aux(
    hidden: Tensor,
    norm_weight: Tensor,
    router_weight: Tensor,
    top_k: int,
    *,
    eps: float = 1e-6,
    norm_topk_prob: bool = True,
    attention_mask: Tensor | None = None,
    logit_bias: Tensor | None = None,
) -> tuple[Tensor, tuple[Tensor, Tensor, Tensor], Tensor]:
    """(x, (router_logits, scores, indices), aux) for hidden [..., H] (bf16).

    ``x`` has hidden's shape and is the MoE block's input; the router 3-tuple
    is the reference router's output for ``x`` (fp32 logits); ``aux`` equals
    ``load_balancing_loss_func((router_logits,), E, top_k, attention_mask)``
    for this layer.  ``attention_mask`` [B, S] weights tokens as in the
    reference's masked branch.
    """
    x, _ = ops.rmsnorm_fwd(hidden, norm_weight, float(eps))
    H = hidden.shape[-1]
    tw = None
    if attention_mask is not None:
        tw = attention_mask.to(device=hidden.device, dtype=torch.float32).reshape(-1)
        if tw.numel() != x.numel() // H:
            raise ValueError(f"attention_mask has {tw.numel()} entries for {x.numel() // H} tokens")
    logits, scores, idx, aux, _stats = ops.router_aux_fwd(x.reshape(-1, H), router_weight, top_k, norm_topk_prob, tw,
                                                          logit_bias)
    return x, (logits, scores, idx), aux

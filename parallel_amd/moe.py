"""Qwen3-MoE block modules and the transformers experts plugin, on gfx950 kernels.

Module tree, parameter layout and call signatures are those of transformers'
Qwen3-MoE (TF = transformers, pinned 5.14.1 by the reference, 5.15.0 here):

  SparseMoeBlock.forward(h [B,S,H]) -> [B,S,H]      TF modeling_qwen3_moe.py:270-281
    .gate    TopKRouter -> (logits [T,E] f32, scores [T,k], indices [T,k])   :249-267
    .experts Experts(hidden [T,H], top_k_index, top_k_weights) -> [T,H]     :209-246
             gate_up_proj [E,2I,H], down_proj [E,H,I]                        :218-219

so the EP hooks of parallel/parallel/engine/model_parallel/expert_parallel.py
(which match ``*.mlp.gate`` / ``*.mlp.experts``) attach unchanged.  The same
experts function is also registered in transformers' ``ExpertsInterface``
(TF integrations/moe.py:481-506) under the name ``"mi355x"``, so a stock
``Qwen3MoeSparseMoeBlock`` runs on these kernels with
``config._experts_implementation = "mi355x"``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor, nn

from . import ops

EXPERTS_IMPLEMENTATION = "mi355x"


@dataclass
class MoeConfig:
    """The Qwen3MoeConfig fields the expert path reads (TF configuration_qwen3_moe.py:86-108)."""

    hidden_size: int
    num_experts: int
    num_experts_per_tok: int
    moe_intermediate_size: int
    norm_topk_prob: bool = False  # transformers' default
    router_aux_loss_coef: float = 0.001
    hidden_act: str = "silu"


class TopKRouter(nn.Module):
    """Qwen3MoeTopKRouter: softmax top-k over the router logits, optional
    renormalisation.  The logits are fp32, or, under CUDA bf16 autocast (the
    reference's default AMP, parallel/parallel/engine/engine.py:141), those
    of a bf16 linear with bf16 scores, as the reference module gives there."""

    def __init__(self, config):
        super().__init__()
        self.top_k = config.num_experts_per_tok
        self.num_experts = config.num_experts
        self.norm_topk_prob = config.norm_topk_prob
        self.hidden_dim = config.hidden_size
        self.weight = nn.Parameter(torch.zeros(self.num_experts, self.hidden_dim))

    def forward(self, hidden_states: Tensor) -> tuple[Tensor, Tensor, Tensor]:
        hidden_states = hidden_states.reshape(-1, self.hidden_dim)
        if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
            with torch.autocast("cuda", enabled=False):
                return ops.router_fwd_bf16(hidden_states.to(torch.bfloat16), self.weight.to(torch.bfloat16),
                                           self.top_k, self.norm_topk_prob)[:3]
        return ops.router_fwd(hidden_states, self.weight, self.top_k, self.norm_topk_prob)


def _check_gated_silu(module) -> None:
    act = getattr(getattr(module, "config", None), "hidden_act", "silu")
    if act != "silu":
        raise NotImplementedError(f"the fused expert epilogue implements SwiGLU (silu), not {act!r}")
    if getattr(module, "has_bias", False):
        raise NotImplementedError("expert biases are not supported by the mi355x experts implementation")
    if getattr(module, "is_transposed", False):
        raise NotImplementedError("transposed expert weights are not supported by the mi355x experts implementation")
    if not getattr(module, "has_gate", True) or not getattr(module, "is_concatenated", True):
        raise NotImplementedError("the mi355x experts implementation expects concatenated [gate; up] weights")


def mi355x_experts_forward(self, hidden_states: Tensor, top_k_index: Tensor, top_k_weights: Tensor) -> Tensor:
    """ExpertsInterface function with the signature of grouped_mm_experts_forward
    (TF integrations/moe.py:377-382).  Expert ids equal to ``self.num_experts``
    are the EP sentinel and contribute nothing (TF integrations/moe.py:405-437)."""
    _check_gated_silu(self)
    if self.gate_up_proj.shape[0] != self.num_experts:
        raise ValueError(f"gate_up_proj holds {self.gate_up_proj.shape[0]} experts, module says {self.num_experts}")
    out = ops.experts(hidden_states, top_k_index, top_k_weights, self.gate_up_proj, self.down_proj,
                      accumulate_grad=bool(getattr(self, "fuse_grad_accumulation", False)))
    return out.to(hidden_states.dtype)


class Experts(nn.Module):
    """Qwen3MoeExperts parameters, forward on the gfx950 grouped-GEMM path.

    ``fuse_grad_accumulation`` (off by default) adds each backward's weight
    gradients into existing ``.grad`` tensors inside the weight-gradient GEMM
    (see ``ops.experts``); it skips the parameters' post-accumulate-grad hooks."""

    fuse_grad_accumulation = False

    def __init__(self, config):
        super().__init__()
        self.config = config
        self.num_experts = config.num_experts
        self.hidden_dim = config.hidden_size
        self.intermediate_dim = config.moe_intermediate_size
        self.gate_up_proj = nn.Parameter(torch.empty(self.num_experts, 2 * self.intermediate_dim, self.hidden_dim))
        self.down_proj = nn.Parameter(torch.empty(self.num_experts, self.hidden_dim, self.intermediate_dim))
        self.has_gate, self.has_bias, self.is_transposed, self.is_concatenated = True, False, False, True

    def forward(self, hidden_states: Tensor, top_k_index: Tensor, top_k_weights: Tensor) -> Tensor:
        return mi355x_experts_forward(self, hidden_states, top_k_index, top_k_weights)


class SparseMoeBlock(nn.Module):
    """Qwen3MoeSparseMoeBlock: router then experts, [B,S,H] in and out."""

    def __init__(self, config):
        super().__init__()
        self.experts = Experts(config)
        self.gate = TopKRouter(config)

    def forward(self, hidden_states: Tensor) -> Tensor:
        batch_size, sequence_length, hidden_dim = hidden_states.shape
        flat = hidden_states.view(-1, hidden_dim)
        _, routing_weights, selected_experts = self.gate(flat)
        out = self.experts(flat, selected_experts, routing_weights)
        return out.reshape(batch_size, sequence_length, hidden_dim)


def register_experts_implementation(name: str = EXPERTS_IMPLEMENTATION) -> bool:
    """Registers the gfx950 experts function in transformers' ExpertsInterface.

    Returns False when transformers is not importable (the standalone modules
    above do not need it)."""
    try:
        from transformers.integrations.moe import ALL_EXPERTS_FUNCTIONS
    except ImportError:
        return False
    ALL_EXPERTS_FUNCTIONS.register(name, mi355x_experts_forward)
    return True

"""Expert ownership and the EP hook runtimes, with the reference's contracts.

Mirrors parallel/parallel/engine/model_parallel/expert_parallel.py:12-231:
``ExpertPartition`` (contiguous ownership, ``owner``, ``localize_routes``),
``verify_expert_modules``, ``ReplicatedTokenExpertParallel`` (router output
hook + expert input/output hooks) and ``SequenceParallelExpertParallel``
(dispatch before the experts, combine after).  The expert modules they wrap
run on the gfx950 kernels; the rank boundary is the one-rank loopback of this
single-GPU build.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .groups import require_single_rank
from .token_dispatch import TokenDispatcher


@dataclass(frozen=True)
class ExpertPartition:
    """Contiguous expert ownership and replicated-token route localization."""

    num_experts: int
    ep_size: int
    ep_rank: int

    def __post_init__(self):
        if self.ep_size < 1:
            raise ValueError("ep_size must be positive")
        if not 0 <= self.ep_rank < self.ep_size:
            raise ValueError("ep_rank is outside the expert-parallel group")
        if self.num_experts % self.ep_size:
            raise ValueError(
                f"num_experts ({self.num_experts}) must be divisible by ep_size ({self.ep_size})"
            )

    @property
    def local_count(self) -> int:
        return self.num_experts // self.ep_size

    @property
    def start(self) -> int:
        return self.ep_rank * self.local_count

    @property
    def stop(self) -> int:
        return self.start + self.local_count

    @property
    def global_experts(self) -> range:
        return range(self.start, self.stop)

    def owner(self, global_expert: torch.Tensor) -> torch.Tensor:
        return torch.div(global_expert, self.local_count, rounding_mode="floor")

    def localize_routes(self, global_indices: torch.Tensor, scores: torch.Tensor):
        """Local indices (non-local -> sentinel ``local_count``), zeroed non-local scores, locality mask."""
        if global_indices.shape != scores.shape:
            raise ValueError("Expert indices and scores must have the same shape")
        local_mask = self.owner(global_indices) == self.ep_rank
        local_indices = (global_indices - self.start).masked_fill(~local_mask, self.local_count)
        local_scores = scores.masked_fill(~local_mask, 0)
        return local_indices, local_scores, local_mask


def local_expert_range(num_experts: int, ep_size: int, ep_rank: int) -> range:
    return ExpertPartition(num_experts, ep_size, ep_rank).global_experts


def verify_expert_modules(model, partition: ExpertPartition) -> None:
    expert_modules = [
        (name, module)
        for name, module in model.named_modules()
        if name.endswith(".mlp.experts") and hasattr(module, "num_experts")
    ]
    if not expert_modules:
        raise RuntimeError("Expert-parallel plan found no expert modules")
    mismatched = [f"{name}={m.num_experts}" for name, m in expert_modules if m.num_experts != partition.local_count]
    if mismatched:
        raise RuntimeError(
            f"Expected {partition.local_count} local experts per rank, got " + ", ".join(mismatched)
        )


class _RankBoundary:
    """Shared hook bookkeeping (install once, remove on close)."""

    def __init__(self):
        self._handles = []

    def close(self) -> None:
        for handle in self._handles:
            handle.remove()
        self._handles.clear()


class ReplicatedTokenExpertParallel(_RankBoundary):
    """Replicated-token EP: every rank routes all tokens, keeps its own experts.

    With one rank the gradient and output all-reduces are the identity; routes
    to experts another rank would own become the sentinel and are skipped by
    the expert kernels."""

    def __init__(self, partition: ExpertPartition, group):
        super().__init__()
        require_single_rank(group, "replicated-token expert parallelism")
        self.partition = partition
        self.group = group

    def _router_output_hook(self, module, inputs, outputs):
        router_logits, scores, global_indices, *extra = outputs
        local_indices, local_scores, _ = self.partition.localize_routes(global_indices, scores)
        return router_logits, local_scores, local_indices, *extra

    def _experts_input_hook(self, module, inputs):
        return inputs

    def _experts_output_hook(self, module, inputs, output):
        return output

    def apply(self, model) -> None:
        if self._handles:
            raise RuntimeError("Expert parallel hooks are already installed")
        routers, experts = [], []
        for name, module in model.named_modules():
            if name.endswith(".mlp.gate"):
                routers.append(module)
            elif name.endswith(".mlp.experts"):
                experts.append(module)
        if not routers or len(routers) != len(experts):
            raise RuntimeError(
                f"Expected paired MoE routers and experts, got {len(routers)} routers and "
                f"{len(experts)} expert modules"
            )
        for router in routers:
            self._handles.append(router.register_forward_hook(self._router_output_hook))
        for expert_module in experts:
            self._handles.append(expert_module.register_forward_pre_hook(self._experts_input_hook))
            self._handles.append(expert_module.register_forward_hook(self._experts_output_hook))


class SequenceParallelExpertParallel(_RankBoundary):
    """Route local tokens to expert owners and back around every expert module."""

    def __init__(self, partition: ExpertPartition, group):
        super().__init__()
        self.partition = partition
        self.group = group
        self.dispatcher = TokenDispatcher(partition, group)
        self._states = {}

    def _experts_input_hook(self, module, inputs):
        hidden_states, global_indices, routing_weights = inputs
        hidden, indices, weights, state = self.dispatcher.dispatch(hidden_states, global_indices, routing_weights)
        self._states.setdefault(id(module), []).append(state)
        return hidden, indices, weights

    def _experts_output_hook(self, module, inputs, output):
        states = self._states.get(id(module))
        if not states:
            raise RuntimeError("Expert output has no matching token dispatch")
        return self.dispatcher.combine(output, states.pop())

    def apply(self, model) -> None:
        if self._handles:
            raise RuntimeError("Expert parallel hooks are already installed")
        experts = [m for name, m in model.named_modules() if name.endswith(".mlp.experts")]
        if not experts:
            raise RuntimeError("Sequence-parallel EP found no expert modules")
        for module in experts:
            self._handles.append(module.register_forward_pre_hook(self._experts_input_hook))
            self._handles.append(module.register_forward_hook(self._experts_output_hook))

    def close(self) -> None:
        super().close()
        self._states.clear()

"""Expert ownership and the expert-parallel hooks of one rank's share.

Public API of parallel/parallel/engine/model_parallel/expert_parallel.py:12-231,
kept so that callers and plans written for the reference attach unchanged:
``ExpertPartition(num_experts, ep_size, ep_rank)`` with ``local_count``,
``start``, ``stop``, ``global_experts``, ``owner`` and ``localize_routes``;
``local_expert_range``; ``verify_expert_modules``; and the two runtimes
``ReplicatedTokenExpertParallel`` and ``SequenceParallelExpertParallel`` with
``apply(model)`` / ``close()``.  Exception types are the reference's
(``ValueError`` for partitions and shapes, ``RuntimeError`` for hook misuse).

This build runs one process per GPU and no collectives.  A process group of
one process (``None`` included) may still carry a partition with
``ep_size > 1``: the process then computes rank ``ep_rank``'s share of the
layer, as if the other ranks held no source tokens.  Every quantity the
reference sums over ranks (the expert outputs, the router's and the hidden
states' gradients) is then this rank's term of that sum, so adding the shares
of ranks 0..ep_size-1 gives the whole layer.  Larger groups are refused
(``groups.require_single_rank``).

How the runtimes map onto the kernels:

* replicated tokens: every rank routes all tokens.  The router's forward hook
  rewrites its (logits, scores, indices) output to this rank's local expert
  ids, with non-local routes sent to the sentinel id ``local_count`` and their
  scores zeroed.  The expert kernels' counting sort places sentinel slots past
  the last expert and skips them, so non-local routes cost no GEMM work.  The
  reference's all-reduces at the expert boundary are identities within one
  process and are not installed.
* sequence-parallel tokens: a pre-hook on each experts module dispatches the
  routes to their owner ranks (``TokenDispatcher``: one counting-sort launch
  sequence gives the owner-major send buffer, splits and local ids), and a
  forward hook combines the returned rows into source-token order.  The
  dispatch state travels from the pre-hook to the hook on a per-module stack,
  so nested calls of one module (activation recomputation) pair correctly.
"""

from __future__ import annotations

from collections import defaultdict
from dataclasses import dataclass

import torch

from .groups import require_single_rank
from .token_dispatch import TokenDispatcher

ROUTER_SUFFIX = ".mlp.gate"
EXPERTS_SUFFIX = ".mlp.experts"


@dataclass(frozen=True)
class ExpertPartition:
    """Contiguous ownership: rank r owns global experts [r * E_l, (r + 1) * E_l)."""

    num_experts: int
    ep_size: int
    ep_rank: int

    def __post_init__(self):
        if self.ep_size < 1:
            raise ValueError(f"ep_size must be positive, got {self.ep_size}")
        if self.ep_rank < 0 or self.ep_rank >= self.ep_size:
            raise ValueError(f"ep_rank {self.ep_rank} is outside the expert-parallel group of {self.ep_size}")
        if self.num_experts % self.ep_size != 0:
            raise ValueError(f"{self.num_experts} experts cannot be split evenly over ep_size {self.ep_size} "
                             "(num_experts must be divisible by ep_size)")

    @property
    def local_count(self) -> int:
        return self.num_experts // self.ep_size

    @property
    def start(self) -> int:
        return self.local_count * self.ep_rank

    @property
    def stop(self) -> int:
        return self.local_count * (self.ep_rank + 1)

    @property
    def global_experts(self) -> range:
        return range(self.start, self.stop)

    def owner(self, global_expert: torch.Tensor) -> torch.Tensor:
        """Owner rank of each global expert id (floor division, as ids may be any integer)."""
        return global_expert.div(self.local_count, rounding_mode="floor")

    def localize_routes(self, global_indices: torch.Tensor, scores: torch.Tensor):
        """(local ids, scores, locality mask) of routes given by global expert ids.

        A route is local when its id lies in [start, stop); local ids are
        id - start, every other route gets the sentinel ``local_count`` and a
        zero score (whose gradient is then zero too)."""
        if global_indices.shape != scores.shape:
            raise ValueError(f"expert indices {tuple(global_indices.shape)} and scores {tuple(scores.shape)} "
                             "must have the same shape")
        offset = global_indices - self.start
        local_mask = (offset >= 0) & (offset < self.local_count)
        local_indices = torch.where(local_mask, offset, torch.full_like(offset, self.local_count))
        local_scores = torch.where(local_mask, scores, torch.zeros_like(scores))
        return local_indices, local_scores, local_mask


def local_expert_range(num_experts: int, ep_size: int, ep_rank: int) -> range:
    """Global ids of the experts rank ``ep_rank`` owns."""
    return ExpertPartition(num_experts, ep_size, ep_rank).global_experts


def _moe_children(model) -> tuple[list, list]:
    """(routers, expert modules) of a model, by the module names MoE decoder layers use."""
    routers, experts = [], []
    for name, module in model.named_modules():
        if name.endswith(ROUTER_SUFFIX):
            routers.append(module)
        elif name.endswith(EXPERTS_SUFFIX):
            experts.append(module)
    return routers, experts


def verify_expert_modules(model, partition: ExpertPartition) -> None:
    """Checks that every experts module of the model holds exactly this rank's experts."""
    counts = {name: module.num_experts for name, module in model.named_modules()
              if name.endswith(EXPERTS_SUFFIX) and hasattr(module, "num_experts")}
    if not counts:
        raise RuntimeError(f"no '*{EXPERTS_SUFFIX}' modules with num_experts found for the expert-parallel plan")
    wrong = sorted(f"{name}={n}" for name, n in counts.items() if n != partition.local_count)
    if wrong:
        raise RuntimeError(f"each rank should hold {partition.local_count} local experts, but "
                           + ", ".join(wrong))


class _HookRuntime:
    """Owns the hook handles of one runtime; ``apply`` installs once, ``close`` removes."""

    def __init__(self, partition: ExpertPartition, group):
        require_single_rank(group, type(self).__name__)
        self.partition = partition
        self.group = group
        self._handles: list = []

    def _hook(self, module, kind: str, fn) -> None:
        register = module.register_forward_pre_hook if kind == "pre" else module.register_forward_hook
        self._handles.append(register(fn))

    def _begin_apply(self) -> None:
        if self._handles:
            raise RuntimeError(f"{type(self).__name__} hooks are already installed; close() them first")

    def close(self) -> None:
        while self._handles:
            self._handles.pop().remove()


class ReplicatedTokenExpertParallel(_HookRuntime):
    """Every rank routes all tokens and runs its own experts on them."""

    def _localize_router_output(self, module, inputs, outputs):
        router_logits, scores, global_indices, *rest = outputs
        local_indices, local_scores, _ = self.partition.localize_routes(global_indices, scores)
        return (router_logits, local_scores, local_indices, *rest)

    def apply(self, model) -> None:
        self._begin_apply()
        routers, experts = _moe_children(model)
        if not routers or len(routers) != len(experts):
            raise RuntimeError(f"replicated-token EP needs one '*{ROUTER_SUFFIX}' per '*{EXPERTS_SUFFIX}' module, "
                               f"found {len(routers)} routers and {len(experts)} expert modules")
        for router in routers:
            self._hook(router, "post", self._localize_router_output)


class SequenceParallelExpertParallel(_HookRuntime):
    """Each rank routes its own tokens; they are dispatched to the expert owners and back."""

    def __init__(self, partition: ExpertPartition, group):
        super().__init__(partition, group)
        self.dispatcher = TokenDispatcher(partition, group)
        self._in_flight: defaultdict[int, list] = defaultdict(list)

    def _dispatch(self, module, inputs):
        hidden_states, global_indices, routing_weights = inputs
        hidden, local_experts, weights, state = self.dispatcher.dispatch(hidden_states, global_indices,
                                                                         routing_weights)
        self._in_flight[id(module)].append(state)
        return hidden, local_experts, weights

    def _combine(self, module, inputs, output):
        pending = self._in_flight.get(id(module))
        if not pending:
            raise RuntimeError("an experts module returned without a dispatch from its pre-hook "
                               "(no dispatch state to combine with)")
        return self.dispatcher.combine(output, pending.pop())

    def apply(self, model) -> None:
        self._begin_apply()
        _, experts = _moe_children(model)
        if not experts:
            raise RuntimeError(f"sequence-parallel EP found no '*{EXPERTS_SUFFIX}' modules to wrap")
        for module in experts:
            self._hook(module, "pre", self._dispatch)
            self._hook(module, "post", self._combine)

    def close(self) -> None:
        super().close()
        self._in_flight.clear()

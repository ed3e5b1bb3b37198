"""TokenDispatcher on the gfx950 permute/combine kernels.

API of parallel/parallel/engine/model_parallel/token_dispatch.py:11-174:
``TokenDispatcher(partition, group)``, ``.dispatch(hidden [T,H],
global_indices [T,k], scores [T,k]) -> (hidden [R,H], local_experts [R,1],
scores [R,1], DispatchState)``, ``.combine(expert_output [R,H], state) ->
[T,H]``, ``DispatchState`` and ``variable_all_to_all``.

The owner-rank sort, the send splits, the row gather and the local expert ids
come from one stable counting-sort launch sequence (``moe_permute_fwd`` with
divisor = local expert count), and the combine is a gather over the inverse
permutation instead of an atomic ``index_add``.  On one GPU the exchange is the
loopback of a one-rank group: the send buffer is the receive buffer, in the
reference's receive layout (source-rank-major, flat (token, k) order inside a
source block).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops
from .groups import group_size, require_single_rank


def variable_all_to_all(value, send_splits, receive_splits, group, *, mode="", detail=""):
    """Variable-split exchange (token_dispatch.py:62-68); the one-rank loopback here."""
    require_single_rank(group, f"variable_all_to_all({mode or 'exchange'})")
    if sum(send_splits) != value.shape[0] or tuple(send_splits) != tuple(receive_splits):
        raise ValueError(
            f"one-rank exchange needs send == receive splits covering {value.shape[0]} rows, "
            f"got {tuple(send_splits)} / {tuple(receive_splits)}"
        )
    return value


@dataclass
class DispatchState:
    send_splits: tuple[int, ...]
    receive_splits: tuple[int, ...]
    source_tokens: torch.Tensor
    num_source_tokens: int
    # Inverse of the dispatch order (slot t*k+j -> send row), used by the
    # gather-form combine, and the routes per token.
    pos_of_slot: torch.Tensor | None = None
    top_k: int = 1


class TokenDispatcher:
    """Dispatch top-k routes to expert owners and restore source-token order."""

    def __init__(self, partition, group):
        self.partition = partition
        self.group = group
        self.world_size = group_size(group)
        if self.world_size != partition.ep_size:
            raise ValueError(
                f"partition has ep_size={partition.ep_size} but the group has {self.world_size} ranks"
            )

    def _exchange_splits(self, send_counts: torch.Tensor):
        """(send, receive) splits as tuples; one small device-to-host copy (token_dispatch.py:86-99)."""
        send = tuple(int(c) for c in send_counts.tolist())
        require_single_rank(self.group, "split exchange")
        return send, send

    def dispatch(self, hidden_states, global_indices, scores):
        if global_indices.shape != scores.shape:
            raise ValueError("Expert indices and scores must have the same shape")
        tokens, top_k = global_indices.shape
        send_hidden, send_experts, send_scores, source_tokens, pos_of_slot, counts = ops.dispatch_fwd(
            hidden_states, global_indices, scores, self.partition.local_count, self.partition.ep_size
        )
        send_splits, receive_splits = self._exchange_splits(counts)
        received_hidden = variable_all_to_all(
            send_hidden, send_splits, receive_splits, self.group, mode="dispatch_hidden", detail="routes"
        )
        received_experts = variable_all_to_all(
            send_experts, send_splits, receive_splits, self.group, mode="dispatch_experts", detail="routes"
        )
        received_scores = variable_all_to_all(
            send_scores, send_splits, receive_splits, self.group, mode="dispatch_scores", detail="routes"
        )
        state = DispatchState(send_splits, receive_splits, source_tokens, tokens, pos_of_slot, top_k)
        return received_hidden, received_experts.unsqueeze(-1), received_scores.unsqueeze(-1), state

    def combine(self, expert_output: torch.Tensor, state: DispatchState):
        returned = variable_all_to_all(
            expert_output, state.receive_splits, state.send_splits, self.group, mode="combine_hidden",
            detail="routes"
        )
        if state.pos_of_slot is None:
            raise ValueError("DispatchState has no inverse permutation; it was not produced by this dispatcher")
        return ops.combine_rows_fwd(returned, state.pos_of_slot, state.num_source_tokens, state.top_k)

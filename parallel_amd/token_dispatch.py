"""TokenDispatcher on the gfx950 permute/combine kernels.

API of parallel/parallel/engine/model_parallel/token_dispatch.py:11-174:
``TokenDispatcher(partition, group)``, ``.dispatch(hidden [T,H],
global_indices [T,k], scores [T,k]) -> (hidden [R,H], local_experts [R,1],
scores [R,1], DispatchState)``, ``.combine(expert_output [R,H], state) ->
[T,H]``, ``DispatchState`` and ``variable_all_to_all``.

The owner-rank sort, the send splits, the row gather and the local expert ids
come from one stable counting-sort launch sequence (``moe_permute_fwd`` with
divisor = local expert count), and the combine is a gather over the inverse
permutation instead of an atomic ``index_add``.

This build exchanges nothing between processes.  Within one process the
group holds rank ``partition.ep_rank`` of an ``ep_size``-rank expert-parallel
group whose other ranks are absent: they send this rank no rows and return no
rows.  The exchange therefore keeps the block this rank sends to itself and
drops the others; in the reference's receive layout (source-rank-major,
flat (token, k) order within a source) that block is the whole receive
buffer.  With ``ep_size == 1`` the exchange is the identity.  The combine of a
share returns zeros for the routes owned by absent ranks, so the shares of
all ranks sum to the full layer.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import ops
from .groups import require_single_rank


def _block_start(splits, rank: int) -> int:
    return sum(int(s) for s in splits[:rank])


def variable_all_to_all(value, send_splits, receive_splits, group, *, mode="", detail="", rank=None):
    """Variable-split exchange (token_dispatch.py:62-68) within one process.

    The process is rank ``rank`` (0 when the splits have one entry): its send
    block ``rank`` becomes its receive block ``rank`` and must have the same
    size; every other receive block is empty (zeros: the sender is absent) and
    every other send block is dropped.  Differentiable: the gradient runs the
    reverse exchange."""
    require_single_rank(group, f"variable_all_to_all({mode or 'exchange'})")
    send_splits, receive_splits = tuple(int(s) for s in send_splits), tuple(int(s) for s in receive_splits)
    if len(send_splits) != len(receive_splits):
        raise ValueError(f"send splits {send_splits} and receive splits {receive_splits} differ in length")
    if sum(send_splits) != value.shape[0]:
        raise ValueError(f"send splits {send_splits} do not cover the {value.shape[0]} rows to send")
    if rank is None:
        if len(send_splits) != 1:
            raise ValueError("a one-process exchange over several ranks needs the process's rank")
        rank = 0
    if send_splits[rank] != receive_splits[rank]:
        raise ValueError(f"rank {rank} sends itself {send_splits[rank]} rows but expects {receive_splits[rank]}")
    if len(send_splits) == 1:
        return value
    block = value.narrow(0, _block_start(send_splits, rank), send_splits[rank])
    before = _block_start(receive_splits, rank)
    after = sum(receive_splits) - before - receive_splits[rank]
    if before == 0 and after == 0:
        return block
    # rows from absent senders are zeros (F.pad pads the leading dimension last in its spec)
    return F.pad(block, (0, 0) * (value.dim() - 1) + (before, after))


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
        require_single_rank(group, "TokenDispatcher")
        self.partition = partition
        self.group = group
        self.world_size = partition.ep_size
        self.rank = partition.ep_rank

    def _exchange_splits(self, send_counts: torch.Tensor):
        """(send, receive) splits as tuples; one small device-to-host copy (token_dispatch.py:86-99).

        Only this rank sends rows to this rank; the absent ranks send none."""
        send = tuple(int(c) for c in send_counts.tolist())
        receive = tuple(send[self.rank] if src == self.rank else 0 for src in range(self.world_size))
        return send, receive

    def _exchange(self, value, send_splits, receive_splits, mode):
        return variable_all_to_all(value, send_splits, receive_splits, self.group, mode=mode, detail="routes",
                                   rank=self.rank)

    def dispatch(self, hidden_states, global_indices, scores):
        if global_indices.shape != scores.shape:
            raise ValueError("Expert indices and scores must have the same shape")
        tokens, top_k = global_indices.shape
        send_hidden, send_experts, send_scores, source_tokens, pos_of_slot, counts = ops.dispatch_fwd(
            hidden_states, global_indices, scores, self.partition.local_count, self.partition.ep_size
        )
        send_splits, receive_splits = self._exchange_splits(counts)
        received_hidden = self._exchange(send_hidden, send_splits, receive_splits, "dispatch_hidden")
        received_experts = self._exchange(send_experts, send_splits, receive_splits, "dispatch_experts")
        received_scores = self._exchange(send_scores, send_splits, receive_splits, "dispatch_scores")
        state = DispatchState(send_splits, receive_splits, source_tokens, tokens, pos_of_slot, top_k)
        return received_hidden, received_experts.unsqueeze(-1), received_scores.unsqueeze(-1), state

    def combine(self, expert_output: torch.Tensor, state: DispatchState):
        returned = self._exchange(expert_output, state.receive_splits, state.send_splits, "combine_hidden")
        if state.pos_of_slot is None:
            raise ValueError("DispatchState has no inverse permutation; it was not produced by this dispatcher")
        return ops.combine_rows_fwd(returned, state.pos_of_slot, state.num_source_tokens, state.top_k)

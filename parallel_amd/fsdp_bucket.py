"""Expert weight gradients written straight into an FSDP unit's gradient bucket.

The reference's FSDP unit reduces a whole unit's gradients with one
reduce-scatter (``DPParamUnit.start_gradient_reduction``,
parallel/parallel/engine/_dp_param_unit.py:373-498). Its input is a
rank-major bucket ``[world, bucket_numel]``. Every parameter takes a flat
slot of ``padded_numel`` elements at ``bucket_offset`` in each rank's chunk
(:268-277). Rank r's slot holds rows ``[r * padded_rows, ...)`` of the
parameter's gradient, with ``padded_rows = ceil(rows / world)`` (:200-202),
and is zero past the parameter's last row. The reference first materialises
each full gradient and then copies it into the bucket (:395-417); for the
expert projections (EXPERT placement on dim 0,
parallel/parallel/engine/model_parallel/models/qwen3_moe.py:81-84) that is a
1.2 GB read and write per layer at Qwen3-30B-A3B sizes.

``experts_backward_into_bucket`` runs the expert backward on the same kernels
as ``ops.experts_bwd``. The weight-gradient GEMM writes expert g's block
directly at its slot in rank ``g // padded_rows``'s chunk, so the full
gradients never exist. The bucket is then the reduce-scatter input as is.
Other parameters of the unit are packed with ``pack_gradient``, the
reference's copy.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch
from torch import Tensor

from . import ops
from ._lib import call, ptr

__all__ = ["BucketSlot", "GradBucketLayout", "experts_backward_into_bucket", "pack_gradient"]


@dataclass(frozen=True)
class BucketSlot:
    """One parameter's place in every rank's chunk of the unit bucket."""

    name: str
    shape: tuple[int, ...]
    padded_rows: int
    bucket_offset: int
    padded_numel: int


@dataclass(frozen=True)
class GradBucketLayout:
    """The flat layout of one FSDP unit (_dp_param_unit.py:200-202, :268-277)."""

    world_size: int
    slots: tuple[BucketSlot, ...]
    bucket_numel: int

    @classmethod
    def from_named_shapes(cls, named_shapes: Sequence[tuple[str, Sequence[int]]], world_size: int) -> "GradBucketLayout":
        if world_size < 1:
            raise ValueError(f"world_size must be >= 1, got {world_size}")
        slots, offset = [], 0
        for name, shape in named_shapes:
            shape = tuple(int(d) for d in shape)
            if not shape:
                raise ValueError(f"FSDP parameter {name} must have at least one dimension")
            padded_rows = (shape[0] + world_size - 1) // world_size
            padded_numel = padded_rows
            for size in shape[1:]:
                padded_numel *= size
            slots.append(BucketSlot(name, shape, padded_rows, offset, padded_numel))
            offset += padded_numel
        return cls(world_size, tuple(slots), offset)

    @classmethod
    def from_module(cls, module: torch.nn.Module, world_size: int) -> "GradBucketLayout":
        return cls.from_named_shapes([(n, p.shape) for n, p in module.named_parameters()], world_size)

    def slot(self, name: str) -> BucketSlot:
        for s in self.slots:
            if s.name == name:
                return s
        raise KeyError(f"no parameter {name!r} in the bucket layout")

    def new_bucket(self, dtype: torch.dtype, device) -> Tensor:
        """The zero-filled reduce-scatter input [world_size, bucket_numel]."""
        return torch.zeros(self.world_size, self.bucket_numel, dtype=dtype, device=device)

    def shard_view(self, bucket: Tensor, name: str, rank: int) -> Tensor:
        """Rank ``rank``'s padded slot of ``name`` as [padded_rows, *shape[1:]]."""
        s = self.slot(name)
        return bucket[rank].narrow(0, s.bucket_offset, s.padded_numel).view(s.padded_rows, *s.shape[1:])


def _check_bucket(bucket: Tensor, layout: GradBucketLayout) -> None:
    if bucket.shape != (layout.world_size, layout.bucket_numel) or not bucket.is_contiguous():
        raise ValueError(f"bucket must be a contiguous [{layout.world_size}, {layout.bucket_numel}] tensor, "
                         f"got {tuple(bucket.shape)}")


def pack_gradient(bucket: Tensor, layout: GradBucketLayout, name: str, grad: Tensor) -> None:
    """Copies a full gradient into its slots (the reference's per-parameter copy)."""
    _check_bucket(bucket, layout)
    s = layout.slot(name)
    if tuple(grad.shape) != s.shape:
        raise ValueError(f"gradient of {name} has shape {tuple(grad.shape)}, the layout {s.shape}")
    for rank in range(layout.world_size):
        start = rank * s.padded_rows
        rows = min(s.padded_rows, max(s.shape[0] - start, 0))
        if rows:
            layout.shard_view(bucket, name, rank)[:rows].copy_(grad.narrow(0, start, rows))


def experts_backward_into_bucket(d_out: Tensor, top_k_weights: Tensor, gate_up_proj: Tensor, down_proj: Tensor,
                                 saved: Sequence[Tensor], bucket: Tensor, layout: GradBucketLayout, *,
                                 names: tuple[str, str] = ("gate_up_proj", "down_proj"),
                                 accumulate: bool = False) -> tuple[Tensor, Tensor]:
    """The expert backward with dW written into ``bucket``; returns (d_hidden, d_weights).

    ``saved`` is (xp, pre, act, y, pos_of_slot, offsets) from ``ops.experts_fwd``;
    ``names`` are the two projections' names in ``layout``. With ``accumulate``
    the gradients are added to the bucket's contents (torch's bf16 add);
    otherwise they overwrite them. Slots past the last expert are never
    written (zero in a bucket from ``new_bucket``).
    """
    ops._require_gpu(d_out, bucket, gate_up_proj, down_proj)
    _check_bucket(bucket, layout)
    if bucket.dtype not in (torch.bfloat16, torch.float32) or bucket.device != d_out.device:
        raise ValueError("bucket must be a bf16 or fp32 tensor on the gradients' device")
    xp, pre, act, y, pos_of_slot, offsets = saved
    params = dict(zip(names, (gate_up_proj, down_proj)))
    E = gate_up_proj.shape[0]
    S = xp.shape[0]
    elt = bucket.element_size()
    s = torch.cuda.current_stream(d_out.device).cuda_stream

    def wgrad(proj, dc, a, n, k):
        name = names[0] if proj == "gate_up_proj" else names[1]
        slot = layout.slot(name)
        if slot.shape != tuple(params[name].shape):
            raise ValueError(f"{name}: layout shape {slot.shape} != parameter shape {tuple(params[name].shape)}")
        base = bucket.data_ptr() + slot.bucket_offset * elt
        call("moe_grouped_gemm_wgrad_bucket", ptr(dc), ptr(a), ptr(offsets), E, S, n, k, base, slot.padded_rows,
             layout.bucket_numel, 1 if bucket.dtype == torch.float32 else 0, 1 if accumulate else 0, s,
             tag="up_wgrad" if proj == "gate_up_proj" else "down_wgrad")
        return None

    d_hidden, d_w, _, _ = ops.experts_bwd_kernels(d_out, top_k_weights, gate_up_proj, down_proj, xp, pre, act, y,
                                                  pos_of_slot, offsets, wgrad)
    return d_hidden, d_w

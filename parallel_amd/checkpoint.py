"""Qwen3-MoE safetensors checkpoints -> one rank's expert and router weights.

Hub checkpoints store every expert as separate projections,
``model.layers.{L}.mlp.experts.{e}.{gate,up,down}_proj.weight`` ([I,H],
[I,H], [H,I]), and the router as ``model.layers.{L}.mlp.gate.weight``
([E,H]). The expert kernels take the packed parameters of the reference
module, ``gate_up_proj [E,2I,H]`` with the gate rows first and
``down_proj [E,H,I]`` (``TF/models/qwen3_moe/modeling_qwen3_moe.py:218-219``).
transformers builds them on load by stacking the experts and concatenating
gate and up (``TF/conversion_mapping.py`` qwen2_moe rules:
``MergeModulelist(dim=0)`` then ``Concatenate(dim=1)``). Under expert
parallelism each rank keeps the contiguous slice
``[rank * E / ep, (rank + 1) * E / ep)`` of dim 0
(``TF/integrations/tensor_parallel.py:1066-1085``, the same ownership as
``ExpertPartition``).

``load_moe_layer`` does that for one decoder layer, reading only the local
experts' tensors from memory-mapped shards and copying each straight into its
slot of the packed device tensors, so the host never holds more than one
expert projection. Checkpoints that already store the packed form
(``mlp.experts.gate_up_proj`` / ``mlp.experts.down_proj``) are sliced on dim 0.
Only local paths are read; nothing is fetched.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass
from pathlib import Path

import torch

from .expert_parallel import ExpertPartition

__all__ = ["MoeLayerWeights", "load_moe_layer", "checkpoint_files"]

_INDEX = "model.safetensors.index.json"


@dataclass
class MoeLayerWeights:
    """One rank's weights of a Qwen3-MoE sparse block, in the kernels' layout."""

    gate_up_proj: torch.Tensor  # [E_local, 2I, H], gate rows [0, I), up rows [I, 2I)
    down_proj: torch.Tensor  # [E_local, H, I]
    router_weight: torch.Tensor  # [E, H] (replicated: every rank routes over all experts)
    norm_weight: torch.Tensor | None  # [H] post_attention_layernorm weight, when present
    partition: ExpertPartition


def checkpoint_files(path: str | os.PathLike) -> dict[str, Path]:
    """Tensor name -> shard file for a checkpoint directory or a single file."""
    path = Path(path)
    if path.is_file():
        return {name: path for name in _names(path)}
    index = path / _INDEX
    if index.exists():
        weight_map = json.loads(index.read_text())["weight_map"]
        return {name: path / shard for name, shard in weight_map.items()}
    files = sorted(path.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no safetensors files under {path}")
    out: dict[str, Path] = {}
    for f in files:
        for name in _names(f):
            out[name] = f
    return out


def _names(file: Path) -> list[str]:
    from safetensors import safe_open

    with safe_open(str(file), framework="pt") as fh:
        return list(fh.keys())


class _Reader:
    """Lazily opened shards; tensors are read one at a time (memory-mapped)."""

    def __init__(self, files: dict[str, Path]):
        self.files = files
        self.handles: dict[Path, object] = {}

    def has(self, name: str) -> bool:
        return name in self.files

    def get(self, name: str) -> torch.Tensor:
        from safetensors import safe_open

        f = self.files[name]
        if f not in self.handles:
            self.handles[f] = safe_open(str(f), framework="pt")
        return self.handles[f].get_tensor(name)

    def get_slice(self, name: str, start: int, stop: int) -> torch.Tensor:
        from safetensors import safe_open

        f = self.files[name]
        if f not in self.handles:
            self.handles[f] = safe_open(str(f), framework="pt")
        return self.handles[f].get_slice(name)[start:stop]


def _prefix(files: dict[str, Path], layer: int) -> str:
    for cand in (f"model.layers.{layer}.", f"model.language_model.layers.{layer}.", f"layers.{layer}."):
        if any(n.startswith(cand + "mlp.") for n in files):
            return cand
    raise KeyError(f"no MoE block of layer {layer} in the checkpoint")


def load_moe_layer(
    path: str | os.PathLike,
    layer: int,
    *,
    ep_size: int = 1,
    ep_rank: int = 0,
    device: torch.device | str | None = None,
    dtype: torch.dtype | None = None,
) -> MoeLayerWeights:
    """Reads layer ``layer``'s router, norm and local expert weights.

    ``dtype`` defaults to the checkpoint's; ``device`` to the CPU. Raises
    ``ValueError`` when the experts do not split evenly over ``ep_size`` or
    the per-expert shapes disagree, and ``KeyError`` for a missing tensor.
    """
    files = checkpoint_files(path)
    rd = _Reader(files)
    pre = _prefix(files, layer)
    router = rd.get(pre + "mlp.gate.weight")
    num_experts, hidden = router.shape
    part = ExpertPartition(num_experts=num_experts, ep_size=ep_size, ep_rank=ep_rank)
    dev = torch.device(device) if device is not None else torch.device("cpu")
    norm_name = pre + "post_attention_layernorm.weight"
    norm = rd.get(norm_name) if rd.has(norm_name) else None
    out_dtype = dtype or router.dtype

    fused_gu, fused_dn = pre + "mlp.experts.gate_up_proj", pre + "mlp.experts.down_proj"
    if rd.has(fused_gu):
        gu = rd.get_slice(fused_gu, part.start, part.stop)
        dn = rd.get_slice(fused_dn, part.start, part.stop)
        if gu.shape[0] != part.local_count or gu.shape[2] != hidden or dn.shape[1] != hidden:
            raise ValueError(f"packed expert shapes {tuple(gu.shape)} / {tuple(dn.shape)} do not match H={hidden}")
        gate_up = gu.to(device=dev, dtype=out_dtype).contiguous()
        down = dn.to(device=dev, dtype=out_dtype).contiguous()
    else:
        first = rd.get(pre + f"mlp.experts.{part.start}.gate_proj.weight")
        inter = first.shape[0]
        gate_up = torch.empty(part.local_count, 2 * inter, hidden, device=dev, dtype=out_dtype)
        down = torch.empty(part.local_count, hidden, inter, device=dev, dtype=out_dtype)
        for i, e in enumerate(part.global_experts):
            g = rd.get(pre + f"mlp.experts.{e}.gate_proj.weight")
            u = rd.get(pre + f"mlp.experts.{e}.up_proj.weight")
            d = rd.get(pre + f"mlp.experts.{e}.down_proj.weight")
            if g.shape != (inter, hidden) or u.shape != (inter, hidden) or d.shape != (hidden, inter):
                raise ValueError(
                    f"expert {e}: gate {tuple(g.shape)}, up {tuple(u.shape)}, down {tuple(d.shape)} "
                    f"do not match I={inter}, H={hidden}"
                )
            gate_up[i, :inter].copy_(g)
            gate_up[i, inter:].copy_(u)
            down[i].copy_(d)
    return MoeLayerWeights(
        gate_up_proj=gate_up,
        down_proj=down,
        router_weight=router.to(device=dev, dtype=out_dtype),
        norm_weight=None if norm is None else norm.to(device=dev, dtype=out_dtype),
        partition=part,
    )

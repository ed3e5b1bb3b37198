"""Writes the golden vectors in this directory from transformers' Qwen3-MoE block.

The arithmetic of the reference's expert path lives in transformers (the
reference pins 5.14.1; 5.15.0 is installed in the build container and 5.14.1
is unavailable offline).  This script runs transformers' own
Qwen3MoeSparseMoeBlock (experts_implementation "grouped_mm", the reference's
default, TF modeling_utils.py:1965-1966) and load_balancing_loss_func on the
CPU in fp32, on inputs regenerated from the seeded recipe in
parallel_amd/workloads.py (rounded to bfloat16 values, held in fp32), and
stores outputs and gradients as .npz fixtures.

Run from the repository root:  python tests/golden/make_golden.py
Nothing here runs on the GPU box; the fixtures are data.
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from parallel_amd.workloads import WORKLOADS, Workload, make_block_inputs  # noqa: E402

OUT_DIR = Path(__file__).resolve().parent

CASES = {
    # C1 of the benchmark configs: H 256, E 8, top-2, I 128, renormalised, 512 tokens.
    "c1": (WORKLOADS["c1"], 1234),
    # The reference tests' tiny shape (tests/test_model_parallel.py:27-46), transformers' default
    # norm_topk_prob=False, with a wider hidden so the GPU kernels' 8-element rows apply.
    "tiny": (Workload("tiny", 1, 48, 64, 4, 2, 16, norm_topk_prob=False, aux_coef=0.01, dtype="fp32"), 7),
}


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().contiguous().numpy().tobytes()).hexdigest()[:16]


def run_case(name: str, w: Workload, seed: int) -> dict[str, np.ndarray]:
    import transformers
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock, load_balancing_loss_func

    cfg = Qwen3MoeConfig(
        hidden_size=w.hidden, num_experts=w.experts, num_experts_per_tok=w.top_k,
        moe_intermediate_size=w.intermediate, norm_topk_prob=w.norm_topk_prob,
        router_aux_loss_coef=w.aux_coef, hidden_act="silu",
    )
    cfg._experts_implementation = "grouped_mm"
    block = Qwen3MoeSparseMoeBlock(cfg).float()
    # bf16-representable values held in fp32: the GPU's bf16 path and this fp32
    # run then start from identical inputs.
    inp = {k: v.float() for k, v in make_block_inputs(w, seed=seed, dtype=torch.bfloat16).items()}
    with torch.no_grad():
        block.gate.weight.copy_(inp["router_weight"])
        block.experts.gate_up_proj.copy_(inp["gate_up_proj"])
        block.experts.down_proj.copy_(inp["down_proj"])
    captured = {}
    block.gate.register_forward_hook(lambda m, i, o: captured.update(router=o))
    x = inp["x"].clone().requires_grad_(True)
    out = block(x.view(w.batch, w.seq, w.hidden)).view(w.tokens, w.hidden)
    logits, scores, indices = captured["router"]
    aux = load_balancing_loss_func((logits,), w.experts, w.top_k, None)
    loss = (out * inp["d_out"]).sum() + w.aux_coef * aux
    loss.backward()
    # Eager experts on the same routing, as an independent check of the grouped path.
    cfg_e = Qwen3MoeConfig(**{k: getattr(cfg, k) for k in (
        "hidden_size", "num_experts", "num_experts_per_tok", "moe_intermediate_size", "norm_topk_prob",
        "router_aux_loss_coef", "hidden_act")})
    cfg_e._experts_implementation = "eager"
    eager = Qwen3MoeSparseMoeBlock(cfg_e).float()
    eager.load_state_dict(block.state_dict())
    with torch.no_grad():
        out_eager = eager(inp["x"].view(w.batch, w.seq, w.hidden)).view(w.tokens, w.hidden)
    # EP sentinel case: the experts called with localized routes of rank 0 of ep=2
    # (ids of the other half -> sentinel num_experts/2 after slicing the weights).
    half = w.experts // 2
    cfg_s = Qwen3MoeConfig(**{**{k: getattr(cfg, k) for k in (
        "hidden_size", "num_experts_per_tok", "moe_intermediate_size", "norm_topk_prob",
        "router_aux_loss_coef", "hidden_act")}, "num_experts": half})
    cfg_s._experts_implementation = "grouped_mm"
    local = Qwen3MoeSparseMoeBlock(cfg_s).float()
    with torch.no_grad():
        local.experts.gate_up_proj.copy_(inp["gate_up_proj"][:half])
        local.experts.down_proj.copy_(inp["down_proj"][:half])
        mask = indices < half
        local_idx = indices.masked_fill(~mask, half)
        local_scores = scores.detach().masked_fill(~mask, 0)
        out_local = local.experts(inp["x"], local_idx, local_scores)

    meta = {
        "transformers": transformers.__version__,
        "torch": torch.__version__,
        "seed": seed,
        "x_sha": digest(inp["x"]),
        "gate_up_sha": digest(inp["gate_up_proj"]),
        # transformers' eager experts on the same routing, as a check of its grouped path
        "eager_vs_grouped_maxabs": float((out_eager - out.detach()).abs().max()),
    }
    print(name, meta)
    return {
        "meta": np.array(repr(meta)),
        "logits": logits.detach().numpy(),
        "scores": scores.detach().numpy(),
        "indices": indices.numpy(),
        "out": out.detach().numpy(),
        "aux": aux.detach().numpy(),
        "dx": x.grad.numpy(),
        "d_router": block.gate.weight.grad.numpy(),
        "d_gate_up": block.experts.gate_up_proj.grad.numpy(),
        "d_down": block.experts.down_proj.grad.numpy(),
        "sentinel_local_idx": local_idx.numpy(),
        "sentinel_out": out_local.numpy(),
    }


def main() -> None:
    torch.set_num_threads(1)  # reproducible CPU reduction order
    for name, (w, seed) in CASES.items():
        arrays = run_case(name, w, seed)
        path = OUT_DIR / f"{name}_qwen3_moe_block.npz"
        np.savez_compressed(path, **arrays)
        print(f"wrote {path} ({path.stat().st_size // 1024} KiB)")


if __name__ == "__main__":
    main()

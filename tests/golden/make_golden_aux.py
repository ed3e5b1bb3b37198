"""Writes tests/golden/aux_masked.npz from transformers' load_balancing_loss_func.

The aux loss's attention-mask branch (TF models/qwen3_moe/modeling_qwen3_moe.py:556-589)
expands a [batch, seq] 0/1 mask over every layer's router logits (layer-major
concatenation) and over the top-k slots, and normalises the per-expert counts
and probability sums by the unmasked token count.  This script runs that
function itself (transformers 5.15.0 here; the reference pins 5.14.1) on
seeded logits of several layers with real padding and holes in the mask, and
stores inputs, the loss and its gradient with respect to every layer's logits
(autograd through the same function).

Run from the repository root:  python tests/golden/make_golden_aux.py
Nothing here runs on the GPU box; the fixture is data.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "aux_masked.npz"

# (name, layers, batch, seq, experts, top_k, seed)
CASES = [
    ("small", 3, 2, 48, 16, 4, 21),
    ("c2", 2, 2, 256, 128, 8, 22),
]


def make_case(layers, batch, seq, experts, top_k, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    logits = (rng.standard_normal((layers, batch * seq, experts)) * 1.5).astype(np.float32)
    mask = np.ones((batch, seq), dtype=np.float32)
    mask[0, seq - seq // 4:] = 0  # right padding in the first sequence
    mask[1, : seq // 8] = 0  # left padding in the second
    holes = rng.random((batch, seq)) < 0.1
    mask[holes] = 0
    return logits, mask


def main() -> None:
    from transformers.models.qwen3_moe.modeling_qwen3_moe import load_balancing_loss_func

    torch.set_num_threads(1)
    arrays = {}
    for name, layers, batch, seq, experts, top_k, seed in CASES:
        logits, mask = make_case(layers, batch, seq, experts, top_k, seed)
        leaves = [torch.from_numpy(l).clone().requires_grad_() for l in logits]
        aux = load_balancing_loss_func(tuple(leaves), experts, top_k, torch.from_numpy(mask))
        aux.backward()
        unmasked = load_balancing_loss_func(tuple(torch.from_numpy(l) for l in logits), experts, top_k, None)
        arrays.update({
            f"{name}_logits": logits,
            f"{name}_mask": mask,
            f"{name}_meta": np.array([layers, batch, seq, experts, top_k, seed], dtype=np.int64),
            f"{name}_aux": aux.detach().numpy(),
            f"{name}_aux_unmasked": unmasked.numpy(),
            f"{name}_d_logits": np.stack([l.grad.numpy() for l in leaves]),
        })
        print(name, f"aux {float(aux):.6f} (unmasked {float(unmasked):.6f}), masked tokens {int((mask == 0).sum())}")
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size // 1024} KiB)")


if __name__ == "__main__":
    main()

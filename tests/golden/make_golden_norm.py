"""Writes golden vectors of transformers' Qwen3MoeRMSNorm (the block-input norm).

Runs transformers' own module (TF modeling_qwen3_moe.py:285-299, installed
5.15.0; the reference pins 5.14.1, unavailable offline) in bfloat16 on the
CPU, forward and backward, on seeded inputs, and stores inputs, outputs and
gradients as fp32 .npz (every value is a bfloat16 value).

Run from the repository root:  python tests/golden/make_golden_norm.py
Nothing here runs on the GPU box; the fixtures are data.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "qwen3_moe_rmsnorm.npz"

CASES = {"h256": (64, 256, 11), "h2048": (24, 2048, 12)}  # rows, hidden, seed
EPS = 1e-6


def main() -> None:
    import transformers
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeRMSNorm

    out = {"transformers_version": np.array(transformers.__version__)}
    for name, (T, H, seed) in CASES.items():
        g = torch.Generator().manual_seed(seed)
        h = (torch.randn(T, H, generator=g) * 2.0).to(torch.bfloat16)
        h[0] = 0.75  # a constant row: x = w * bf16(c / sqrt(c^2 + eps))
        w = (1.0 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
        dx = torch.randn(T, H, generator=g).to(torch.bfloat16)
        norm = Qwen3MoeRMSNorm(H, eps=EPS).to(torch.bfloat16)
        with torch.no_grad():
            norm.weight.copy_(w)
        hh = h.clone().requires_grad_()
        x = norm(hh)
        x.backward(dx)
        for key, val in dict(h=h, w=w, dx=dx, x=x.detach(), dh=hh.grad, dw=norm.weight.grad).items():
            out[f"{name}_{key}"] = val.float().numpy()
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()

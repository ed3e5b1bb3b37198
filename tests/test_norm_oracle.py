"""CPU pins of the block-input norm's oracle (TF modeling_qwen3_moe.py:294-299).

The fixtures are transformers' own Qwen3MoeRMSNorm in bfloat16, forward and
backward (tests/golden/make_golden_norm.py).  Independent checks: a constant
row's closed form, scale invariance, and the analytic gradient the kernels
use against fp64 autograd.
"""

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import moe_oracle as O

EPS = 1e-6


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN / "qwen3_moe_rmsnorm.npz")


@pytest.mark.parametrize("case", ["h256", "h2048"])
def test_oracle_matches_transformers_module(gold, case):
    h = torch.from_numpy(gold[f"{case}_h"]).bfloat16().requires_grad_()
    w = torch.from_numpy(gold[f"{case}_w"]).bfloat16().requires_grad_()
    dx = torch.from_numpy(gold[f"{case}_dx"]).bfloat16()
    x = O.rmsnorm(h, w, EPS)
    x.backward(dx)
    assert torch.equal(x.float(), torch.from_numpy(gold[f"{case}_x"]))
    assert torch.equal(h.grad.float(), torch.from_numpy(gold[f"{case}_dh"]))
    assert torch.equal(w.grad.float(), torch.from_numpy(gold[f"{case}_dw"]))


def test_constant_row_closed_form(gold):
    h, w, x = (gold[f"h256_{k}"] for k in ("h", "w", "x"))
    c = float(h[0, 0])
    assert (h[0] == c).all()
    hs = torch.tensor(c / np.sqrt(c * c + EPS), dtype=torch.float32).bfloat16().float()
    expect = (torch.from_numpy(w).bfloat16() * hs.bfloat16()).float().numpy()
    np.testing.assert_array_equal(x[0], expect)


def test_scale_invariance():
    g = torch.Generator().manual_seed(3)
    h = torch.randn(16, 128, generator=g).bfloat16()
    w = torch.ones(128).bfloat16()
    a, b = O.rmsnorm(h, w, 0.0), O.rmsnorm(h * 4, w, 0.0)  # x4 is exact in bf16
    assert torch.equal(a, b)


def test_analytic_gradient_matches_autograd_fp64():
    """dh = r*dhs - (r^3/H) h sum(dhs h), the formula the backward kernel evaluates."""
    g = torch.Generator().manual_seed(5)
    T, H = 6, 40
    h = torch.randn(T, H, generator=g, dtype=torch.float64).requires_grad_()
    w = torch.randn(H, generator=g, dtype=torch.float64)
    dx = torch.randn(T, H, generator=g, dtype=torch.float64)
    x = w * (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + EPS))
    x.backward(dx)
    hd = h.detach()
    r = torch.rsqrt(hd.pow(2).mean(-1, keepdim=True) + EPS)
    dhs = dx * w
    dh = r * dhs - (r ** 3 / H) * hd * (dhs * hd).sum(-1, keepdim=True)
    torch.testing.assert_close(h.grad, dh, rtol=1e-12, atol=1e-12)

"""The step before the MoE block on the GPU: block-input RMSNorm and the router
with the aux loss from its own top-k, against transformers' golden vectors
and the CPU oracle (TF modeling_qwen3_moe.py:294-299, :258-267, :514-593)."""

import numpy as np
import pytest
import torch

from conftest import GOLDEN, close_bf16, routing_check
from oracle import moe_oracle as O
from parallel_amd import norm_router_aux, ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
EPS = 1e-6


def gen(seed):
    return torch.Generator().manual_seed(seed)


def _bit_equal_frac(a, b):
    return float((a.float().cpu() == b.float().cpu()).float().mean())


@pytest.mark.parametrize("case", ["h256", "h2048"])
def test_rmsnorm_matches_transformers_golden(case):
    gold = np.load(GOLDEN / "qwen3_moe_rmsnorm.npz")
    h = torch.from_numpy(gold[f"{case}_h"]).to(DEV, BF).requires_grad_()
    w = torch.from_numpy(gold[f"{case}_w"]).to(DEV, BF).requires_grad_()
    dx = torch.from_numpy(gold[f"{case}_dx"]).to(DEV, BF)
    x, rstd = ops.rmsnorm_fwd(h, w, EPS)
    x.backward(dx)
    torch.cuda.synchronize()
    gx, gdh, gdw = (torch.from_numpy(gold[f"{case}_{k}"]) for k in ("x", "dh", "dw"))
    # x differs from torch's only where rsqrt's last bit moves a bf16 rounding
    assert _bit_equal_frac(x, gx) > 0.995
    close_bf16(x, gx, "x", max_rel=8e-3)
    close_bf16(h.grad, gdh, "dh", max_rel=1e-2)
    close_bf16(w.grad, gdw, "dweight", max_rel=1e-2)
    assert torch.isfinite(rstd).all()


@pytest.mark.parametrize("T,H", [(1, 8), (7, 72), (4096, 2048), (33, 4096)])
def test_rmsnorm_shapes_against_oracle(T, H):
    g = gen(T * 31 + H)
    h = (torch.randn(T, H, generator=g) * 3).to(BF)
    w = (1 + 0.2 * torch.randn(H, generator=g)).to(BF)
    dx = torch.randn(T, H, generator=g).to(BF)
    hc, wc = h.clone().requires_grad_(), w.clone().requires_grad_()
    xr = O.rmsnorm(hc, wc, EPS)
    xr.backward(dx)
    hd, wd = h.to(DEV).requires_grad_(), w.to(DEV).requires_grad_()
    x, _ = ops.rmsnorm_fwd(hd, wd, EPS)
    x.backward(dx.to(DEV))
    close_bf16(x, xr, f"x T{T} H{H}", max_rel=8e-3)
    close_bf16(hd.grad, hc.grad, f"dh T{T} H{H}", max_rel=1e-2)
    close_bf16(wd.grad, wc.grad, f"dweight T{T} H{H}", max_rel=1e-2)


@pytest.mark.parametrize("T,H,E,k,masked,biased", [(4096, 2048, 128, 8, False, False), (300, 64, 64, 6, True, True),
                                                   (4, 8, 8, 2, False, False), (16400, 2048, 128, 8, True, True),
                                                   (8200, 4096, 128, 8, False, True)])
def test_router_aux_equals_router_then_aux(T, H, E, k, masked, biased):
    """One pass (router top-k + aux partials) = router_fwd then aux_loss_fwd, bit for bit."""
    g = gen(T + E)
    x = torch.randn(T, H, generator=g).to(DEV, BF)
    wr = (torch.randn(E, H, generator=g) * 0.05).to(DEV, BF)
    tw = (torch.rand(T, generator=g) > 0.3).float().to(DEV) if masked else None
    bias = (torch.randn(E, generator=g) * 0.5).to(DEV) if biased else None
    logits, scores, idx, aux, stats = ops.router_aux_fwd(x, wr, k, True, tw, bias)
    l2, s2, i2 = ops.router_fwd(x, wr, k, True, bias)
    a2, st2 = ops.aux_loss_fwd(l2, tw, E, k)
    torch.cuda.synchronize()
    assert torch.equal(logits, l2) and torch.equal(scores, s2) and torch.equal(idx, i2)
    assert torch.equal(aux, a2) and torch.equal(stats, st2)


@pytest.mark.parametrize("T,H,E,k", [(512, 256, 32, 4), (4096, 2048, 128, 8)])
def test_norm_router_aux_forward_backward_against_oracle(T, H, E, k):
    g = gen(77)
    hidden = (torch.randn(2, T // 2, H, generator=g) * 2).to(BF)
    nw = (1 + 0.1 * torch.randn(H, generator=g)).to(BF)
    wr = (torch.randn(E, H, generator=g) * 0.05).to(BF)
    mask = (torch.rand(2, T // 2, generator=g) > 0.2).float()
    gx = torch.randn(2, T // 2, H, generator=g).to(BF)
    gs = torch.randn(T, k, generator=g)
    coef = 0.37

    leaves = [t.clone().requires_grad_() for t in (hidden, nw, wr)]
    x, logits, scores, idx, aux = O.norm_router_aux(*leaves, k, eps=EPS, norm_topk_prob=True, attention_mask=mask)
    ((x.float() * gx.float()).sum() + (scores * gs).sum() + coef * aux).backward()

    dl = [t.to(DEV).requires_grad_() for t in (hidden, nw, wr)]
    xd, (ld, sd, idd), auxd = norm_router_aux(*dl, k, eps=EPS, norm_topk_prob=True, attention_mask=mask.to(DEV))
    ((xd.float() * gx.to(DEV).float()).sum() + (sd * gs.to(DEV)).sum() + coef * auxd).backward()
    torch.cuda.synchronize()

    close_bf16(xd, x, "x", max_rel=8e-3)
    close_bf16(ld, logits, "logits")
    routing_check(idd, idx, logits)
    close_bf16(sd, scores, "scores")
    assert abs(float(auxd.detach()) - float(aux.detach())) <= 1e-5 * abs(float(aux.detach())) + 1e-6
    for name, a, b in zip(("dhidden", "dnorm_weight", "drouter_weight"), dl, leaves):
        close_bf16(a.grad, b.grad, name, max_rel=2e-2)

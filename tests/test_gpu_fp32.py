"""The fp32 path: fp32 modules (the C1 configuration, hidden 256, 8 experts,
top-2, moe_intermediate 128, 512 tokens) on the fp32 kernels, against the
oracle's fp32 arithmetic: the router (TF modeling_qwen3_moe.py:258-267), the
experts (TF integrations/moe.py:377-478), the aux loss (:514-593) and the
whole block's forward and backward.

Tolerance (fp32): normwise max relative error <= 1e-4 and cosine >= 1 - 1e-7
against the oracle; the two compute the same fp32 products and differ only in
summation order.  Routing is bit-exact, as for bf16."""

import pytest
import torch

from conftest import close_bf16, routing_check
from oracle import moe_oracle as O
from parallel_amd import ops, register_experts_implementation

pytestmark = pytest.mark.gpu
DEV = "cuda"
F32 = torch.float32
AUX_COEF = 1e-3


def close_f32(actual, expected, name):
    assert actual.dtype == F32, f"{name}: dtype {actual.dtype}"
    return close_bf16(actual, expected, name, max_rel=1e-4, min_cos=1 - 1e-7)


def block_inputs(T, H, E, I, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g)
    rw = torch.randn(E, H, generator=g) * 0.02
    gu = torch.randn(E, 2 * I, H, generator=g) * 0.02
    dn = torch.randn(E, H, I, generator=g) * 0.02
    d_out = torch.randn(T, H, generator=g)
    return x, rw, gu, dn, d_out


CASES = {
    "c1": dict(T=512, H=256, E=8, I=128, k=2),
    "ragged": dict(T=77, H=100, E=6, I=40, k=3),  # no dimension a multiple of the 32-row tile
    "wide": dict(T=2048, H=1024, E=32, I=512, k=4),  # ~256 rows per expert, 1024- and 512-long reductions
}


def gpu_leaves(*ts):
    return [t.to(DEV).requires_grad_() for t in ts]


@pytest.mark.parametrize("case", list(CASES))
def test_fp32_block_matches_the_oracle(case):
    c = CASES[case]
    x, rw, gu, dn, d_out = block_inputs(c["T"], c["H"], c["E"], c["I"], seed=5)
    ref = O.block_forward_backward(x, rw, gu, dn, d_out, top_k=c["k"], norm_topk_prob=True, aux_coef=AUX_COEF)

    xg, rwg, gug, dng = gpu_leaves(x, rw, gu, dn)
    out, logits, scores, idx, aux = ops.moe_block(xg, rwg, gug, dng, c["k"], True)
    ((out * d_out.to(DEV)).sum() + AUX_COEF * aux).backward()

    routing_check(idx, ref["indices"], ref["logits"])
    close_f32(logits, ref["logits"], f"{case} logits")
    close_f32(scores, ref["scores"], f"{case} scores")
    close_f32(out, ref["out"], f"{case} out")
    a, b = float(aux.detach()), float(ref["aux"])
    assert abs(a - b) <= 1e-5 * abs(b), (a, b)
    close_f32(xg.grad, ref["dx"], f"{case} dx")
    close_f32(rwg.grad, ref["d_router"], f"{case} d_router")
    close_f32(gug.grad, ref["d_gate_up"], f"{case} d_gate_up")
    close_f32(dng.grad, ref["d_down"], f"{case} d_down")

    # the separate ops (router_aux_fwd, then experts) give the same bits
    xs, rws, gus, dns = gpu_leaves(x, rw, gu, dn)
    l2, s2, i2, a2, _ = ops.router_aux_fwd(xs, rws, c["k"], True)
    o2 = ops.experts(xs, i2, s2, gus, dns)
    ((o2 * d_out.to(DEV)).sum() + AUX_COEF * a2).backward()
    for name, a, b in (("logits", logits, l2), ("scores", scores, s2), ("indices", idx, i2), ("out", out, o2),
                       ("aux", aux, a2), ("dx", xg.grad, xs.grad), ("d_router", rwg.grad, rws.grad),
                       ("d_gate_up", gug.grad, gus.grad), ("d_down", dng.grad, dns.grad)):
        assert torch.equal(a, b), f"{case}: moe_block and the separate ops differ in {name}"


def test_fp32_aux_gradient_alone():
    """With no output gradient the router's gradients are the aux loss's alone
    (a dropped aux term would leave them zero)."""
    c = CASES["c1"]
    x, rw, gu, dn, _ = block_inputs(c["T"], c["H"], c["E"], c["I"], seed=6)
    d_out = torch.zeros(c["T"], c["H"])
    ref = O.block_forward_backward(x, rw, gu, dn, d_out, top_k=c["k"], norm_topk_prob=True, aux_coef=1.0)
    xg, rwg, gug, dng = gpu_leaves(x, rw, gu, dn)
    out, _, _, _, aux = ops.moe_block(xg, rwg, gug, dng, c["k"], True)
    ((out * d_out.to(DEV)).sum() + aux).backward()
    assert float(ref["d_router"].abs().max()) > 0
    close_f32(xg.grad, ref["dx"], "aux-only dx")
    close_f32(rwg.grad, ref["d_router"], "aux-only d_router")


@pytest.mark.parametrize("T", [77, 0])
def test_fp32_experts_with_empty_experts_and_sentinels(T):
    """An EP rank's local experts: ids in {0, 2, 5} and the sentinel E (routes
    owned by another rank), so experts 1, 3 and 4 receive no rows."""
    E, H, I, k = 6, 100, 40, 3
    g = torch.Generator().manual_seed(8)
    x = torch.randn(T, H, generator=g)
    choices = torch.tensor([0, 2, 5, E])
    idx = choices[torch.randint(0, 4, (T, k), generator=g)]
    w = torch.rand(T, k, generator=g)
    gu = torch.randn(E, 2 * I, H, generator=g) * 0.05
    dn = torch.randn(E, H, I, generator=g) * 0.05
    d_out = torch.randn(T, H, generator=g)

    xg, wg, gug, dng = gpu_leaves(x, w, gu, dn)
    out = ops.experts(xg, idx.to(DEV), wg, gug, dng)
    assert out.shape == (T, H) and out.dtype == F32
    out.backward(d_out.to(DEV))
    assert xg.grad is not None and xg.grad.shape == (T, H)
    for e in (1, 3, 4):
        assert int(gug.grad[e].count_nonzero()) == 0 and int(dng.grad[e].count_nonzero()) == 0
    if T == 0:
        assert int(gug.grad.count_nonzero()) == 0 and int(dng.grad.count_nonzero()) == 0
        return
    leaves = [t.clone().requires_grad_() for t in (x, w, gu, dn)]
    want = O.experts_grouped(leaves[0], idx, leaves[1], leaves[2], leaves[3])
    want.backward(d_out)
    close_f32(out, want, "out")
    close_f32(xg.grad, leaves[0].grad, "d_hidden")
    close_f32(wg.grad, leaves[1].grad, "d_weights")
    close_f32(gug.grad, leaves[2].grad, "d_gate_up")
    close_f32(dng.grad, leaves[3].grad, "d_down")


def test_fp32_gradients_accumulate_in_the_kernels():
    """accumulate_grad adds into existing fp32 .grad tensors: the same bits as
    autograd's fresh gradient plus the old value."""
    c = CASES["ragged"]
    x, rw, gu, dn, d_out = block_inputs(c["T"], c["H"], c["E"], c["I"], seed=9)
    old = [torch.randn(t.shape, generator=torch.Generator().manual_seed(i)) for i, t in enumerate((rw, gu, dn))]
    results = []
    for accumulate in (False, True):
        xg, rwg, gug, dng = gpu_leaves(x, rw, gu, dn)
        if accumulate:
            for p, o in zip((rwg, gug, dng), old):
                p.grad = o.to(DEV).clone()
        out, _, _, _, aux = ops.moe_block(xg, rwg, gug, dng, c["k"], True, accumulate_grad=accumulate)
        ((out * d_out.to(DEV)).sum() + AUX_COEF * aux).backward()
        results.append((rwg.grad, gug.grad, dng.grad))
    for name, fresh, acc, o in zip(("router", "gate_up", "down"), results[0], results[1], old):
        assert torch.equal(acc, o.to(DEV) + fresh), f"accumulated {name} gradient differs from old + fresh"


def test_fp32_transformers_block_runs_on_the_plugin():
    """transformers' own fp32 Qwen3MoeSparseMoeBlock with the mi355x experts:
    its output and input gradient against the unmodified block on the CPU."""
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock

    assert register_experts_implementation()

    def config():
        return Qwen3MoeConfig(hidden_size=256, num_experts=8, num_experts_per_tok=2, moe_intermediate_size=128,
                              norm_topk_prob=True)

    torch.manual_seed(0)
    ref_block = Qwen3MoeSparseMoeBlock(config())  # the experts implementation is read from the config per call
    with torch.no_grad():
        for p in ref_block.parameters():
            p.normal_(0, 0.05)
    cfg = config()
    cfg._experts_implementation = "mi355x"
    block = Qwen3MoeSparseMoeBlock(cfg)
    block.load_state_dict(ref_block.state_dict())
    block = block.to(DEV)
    x = torch.randn(2, 64, 256)
    xg = x.to(DEV).requires_grad_()
    out = block(xg)
    xr = x.clone().requires_grad_()
    want = ref_block(xr)
    out, want = (out[0], want[0]) if isinstance(out, tuple) else (out, want)
    close_f32(out, want, "fp32 plugin block out")
    out.square().sum().backward()
    want.square().sum().backward()
    close_f32(xg.grad, xr.grad, "fp32 plugin block d_hidden")
    close_f32(block.experts.gate_up_proj.grad, ref_block.experts.gate_up_proj.grad, "fp32 plugin d_gate_up")

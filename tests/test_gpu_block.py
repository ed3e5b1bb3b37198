"""Block-level parity on the GPU: router -> experts -> combine + aux loss,
forward and backward, against the CPU oracle, the transformers golden
vectors, and size-independent properties at the benchmark's full size."""

import dataclasses

import numpy as np
import pytest
import torch

from conftest import GOLDEN, close_bf16, routing_check
from oracle import moe_oracle as O
from parallel_amd import (
    ExpertPartition,
    SparseMoeBlock,
    TokenDispatcher,
    load_balancing_loss_func,
    ops,
    register_experts_implementation,
)
from parallel_amd.workloads import WORKLOADS, Workload, ep_receive_buffer, make_block_inputs, scaled

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def gpu_block_step(w: Workload, inp, logit_bias=None):
    """Forward + backward of <out, d_out> + coef * aux on the gfx950 path."""
    x = inp["x"].to(DEV).requires_grad_()
    rw = inp["router_weight"].to(DEV).requires_grad_()
    gu = inp["gate_up_proj"].to(DEV).requires_grad_()
    dn = inp["down_proj"].to(DEV).requires_grad_()
    bias = None if logit_bias is None else logit_bias.to(DEV)
    logits, scores, idx = ops.router_fwd(x, rw, w.top_k, w.norm_topk_prob, bias)
    out = ops.experts(x, idx, scores, gu, dn)
    aux = load_balancing_loss_func((logits,), w.experts, w.top_k)
    torch.autograd.backward([out, aux], [inp["d_out"].to(DEV), torch.tensor(w.aux_coef, device=DEV)])
    return dict(logits=logits.detach(), scores=scores.detach(), indices=idx, out=out.detach(), aux=aux.detach(),
                dx=x.grad, d_router=rw.grad, d_gate_up=gu.grad, d_down=dn.grad)


def oracle_step(w, inp, logit_bias=None):
    return O.block_forward_backward(inp["x"], inp["router_weight"], inp["gate_up_proj"], inp["down_proj"],
                                    inp["d_out"], top_k=w.top_k, norm_topk_prob=w.norm_topk_prob,
                                    aux_coef=w.aux_coef, logit_bias=logit_bias)


def compare(gpu, ref, tag):
    routed = O.topk_softmax(gpu["logits"].cpu(), gpu["indices"].shape[1], True)[1]
    routing_check(gpu["indices"], routed, gpu["logits"])  # on the same logits
    routing_check(gpu["indices"], ref["indices"], gpu["logits"])
    close_bf16(gpu["logits"], ref["logits"], f"{tag} logits", max_rel=1e-4, min_cos=0.999999)
    close_bf16(gpu["scores"], ref["scores"], f"{tag} scores", max_rel=1e-4, min_cos=0.999999)
    torch.testing.assert_close(gpu["aux"].cpu(), ref["aux"], rtol=1e-4, atol=1e-6)
    for key in ("out", "dx", "d_router", "d_gate_up", "d_down"):
        close_bf16(gpu[key], ref[key], f"{tag} {key}")


def test_block_c1_shape_against_oracle_and_transformers_golden():
    w = WORKLOADS["c1"]
    inp = make_block_inputs(w, seed=1234, dtype=BF)
    gpu = gpu_block_step(w, inp)
    compare(gpu, oracle_step(w, inp), "c1")
    # transformers' own fp32 block on the unrounded inputs: same bar at bf16 precision
    g = np.load(GOLDEN / "c1_qwen3_moe_block.npz")
    for key in ("out", "dx", "d_router", "d_gate_up", "d_down"):
        close_bf16(gpu[key], torch.from_numpy(g[key]), f"c1 golden {key}")


@pytest.mark.parametrize("name,tokens,experts", [("c2", 384, None), ("c5", 160, 16)])
def test_block_scaled_configs_against_oracle(name, tokens, experts):
    # C5's expert shapes (H = 4096, I = 1536) with 16 of its 128 experts: the
    # same GEMM tiles and paths, with the CPU oracle's weight gradients and
    # their float64 comparison an eighth of the full 3.2 GB per tensor.
    w = scaled(WORKLOADS[name], tokens)
    if experts is not None:
        w = dataclasses.replace(w, experts=experts)
    inp = make_block_inputs(w, seed=5, dtype=BF)
    compare(gpu_block_step(w, inp), oracle_step(w, inp), name)


def test_block_c4_imbalanced_router_with_aux_gradient():
    w = scaled(WORKLOADS["c4"], 512)
    inp = make_block_inputs(w, seed=6, dtype=BF)
    gpu = gpu_block_step(w, inp, inp["logit_bias"])
    ref = oracle_step(w, inp, inp["logit_bias"])
    compare(gpu, ref, "c4")
    counts = torch.bincount(gpu["indices"].cpu().reshape(-1), minlength=w.experts)
    assert counts.max() > 1.5 * counts.float().mean(), "the bias should skew the routing"


def test_block_c4_two_steps_accumulate_into_existing_gradients():
    """C4's dW accumulation: two forward/backward steps into pre-existing
    gradients (the expert weights' sums formed inside the weight-gradient
    kernel, the router's by autograd) against the initial gradients plus the
    oracle's two steps."""
    w = scaled(WORKLOADS["c4"], 512)
    inp = make_block_inputs(w, seed=16, dtype=BF)
    g = torch.Generator().manual_seed(17)
    d_outs = [inp["d_out"], torch.randn(w.tokens, w.hidden, generator=g).to(BF)]
    names = ("x", "router_weight", "gate_up_proj", "down_proj")
    init = {n: torch.randn(inp[n].shape, generator=g).mul(1e-2).to(BF) for n in names[1:]}
    leaves = {n: inp[n].to(DEV).requires_grad_() for n in names}
    for n in names[1:]:
        leaves[n].grad = init[n].to(DEV)
    bias = inp["logit_bias"].to(DEV)
    coef = torch.tensor(w.aux_coef, device=DEV)
    for d_out in d_outs:
        logits, scores, idx = ops.router_fwd(leaves["x"], leaves["router_weight"], w.top_k, True, bias)
        out = ops.experts(leaves["x"], idx, scores, leaves["gate_up_proj"], leaves["down_proj"], accumulate_grad=True)
        aux = load_balancing_loss_func((logits,), w.experts, w.top_k)
        torch.autograd.backward([out, aux], [d_out.to(DEV), coef])
    torch.cuda.synchronize()
    refs = [O.block_forward_backward(inp["x"], inp["router_weight"], inp["gate_up_proj"], inp["down_proj"], d,
                                     top_k=w.top_k, norm_topk_prob=True, aux_coef=w.aux_coef,
                                     logit_bias=inp["logit_bias"]) for d in d_outs]
    for n, key in (("router_weight", "d_router"), ("gate_up_proj", "d_gate_up"), ("down_proj", "d_down")):
        want = init[n].float() + refs[0][key] + refs[1][key]
        close_bf16(leaves[n].grad, want, f"c4 accumulated {key}")
    close_bf16(leaves["x"].grad, refs[0]["dx"] + refs[1]["dx"], "c4 accumulated dx")


def test_ep_share_receive_layout_c3():
    w = scaled(WORKLOADS["c3"], 384)
    _, _, (src, tok, lexp, lsc) = ep_receive_buffer(w, seed=3)
    R = src.shape[0]
    inp = make_block_inputs(w, seed=3, dtype=BF)
    xs = [inp["x"], torch.randn(w.tokens, w.hidden, generator=torch.Generator().manual_seed(99)).to(BF)]
    hidden = torch.stack([xs[s][t] for s, t in zip(src.tolist(), tok.tolist())])
    idx = torch.from_numpy(lexp).view(R, 1)
    sc = torch.from_numpy(lsc).view(R, 1)
    assert (torch.bincount(idx.view(-1), minlength=64) == 0).sum() >= 4, "some local experts must be empty"
    d_out = torch.randn(R, w.hidden, generator=torch.Generator().manual_seed(7)).to(BF)
    h = hidden.to(DEV).requires_grad_()
    s = sc.to(DEV).requires_grad_()
    gu = inp["gate_up_proj"].to(DEV).requires_grad_()
    dn = inp["down_proj"].to(DEV).requires_grad_()
    out = ops.experts(h, idx.to(DEV), s, gu, dn)
    out.backward(d_out.to(DEV))
    hr = hidden.float().requires_grad_()
    sr = sc.clone().requires_grad_()
    gr = inp["gate_up_proj"].float().requires_grad_()
    dr = inp["down_proj"].float().requires_grad_()
    ref = O.experts_grouped(hr, idx, sr, gr, dr)
    ref.backward(d_out.float())
    close_bf16(out, ref, "c3 out")
    close_bf16(h.grad, hr.grad, "c3 d_hidden")
    close_bf16(s.grad, sr.grad, "c3 d_scores")
    close_bf16(gu.grad, gr.grad, "c3 d_gate_up")
    close_bf16(dn.grad, dr.grad, "c3 d_down")
    empty = torch.bincount(idx.view(-1), minlength=64) == 0
    assert not gu.grad[empty.to(DEV)].any() and not dn.grad[empty.to(DEV)].any()


def test_sentinel_routes_match_transformers_golden():
    w = WORKLOADS["c1"]
    g = np.load(GOLDEN / "c1_qwen3_moe_block.npz")
    inp = make_block_inputs(w, seed=1234, dtype=BF)
    half = w.experts // 2
    idx = torch.from_numpy(g["sentinel_local_idx"])
    scores = torch.from_numpy(g["scores"]).masked_fill(idx == half, 0)
    out = ops.experts(inp["x"].to(DEV), idx.to(DEV), scores.to(DEV), inp["gate_up_proj"][:half].to(DEV),
                      inp["down_proj"][:half].to(DEV))
    close_bf16(out, torch.from_numpy(g["sentinel_out"]), "sentinel out")


def test_token_dispatcher_round_trip_closed_form():
    # One-rank analogue of parallel tests/test_sequence_parallel.py:17-73.
    T, H, k, E = 64, 32, 2, 4
    hidden = torch.randn(T, H, generator=torch.Generator().manual_seed(1)).to(BF).to(DEV).requires_grad_()
    raw = torch.rand(T, k, generator=torch.Generator().manual_seed(2))
    scores = (raw / raw.sum(1, keepdim=True)).to(DEV).requires_grad_()
    indices = torch.stack([torch.randperm(E, generator=torch.Generator().manual_seed(t))[:k] for t in range(T)])
    dispatcher = TokenDispatcher(ExpertPartition(E, 1, 0), None)
    received, local_idx, rscores, state = dispatcher.dispatch(hidden, indices.to(DEV), scores)
    assert state.send_splits == (T * k,) and received.shape == (T * k, H)
    ref_h, ref_e, ref_s, ref_src, _ = O.dispatch_send(hidden.detach().cpu(), indices, scores.detach().cpu(), E, 1)
    assert torch.equal(received.detach().cpu(), ref_h) and torch.equal(local_idx.cpu().view(-1), ref_e)
    assert torch.equal(state.source_tokens.cpu(), ref_src)
    combined = dispatcher.combine(received * rscores.to(received.dtype), state)
    close_bf16(combined, hidden.detach(), "round trip", max_rel=1e-2)
    combined.float().square().sum().backward()
    close_bf16(hidden.grad, 2 * combined.detach(), "d_hidden", max_rel=2e-2)
    ref_ds = 2 * (hidden.detach().float() * combined.detach().float()).sum(-1, keepdim=True).expand(T, k)
    close_bf16(scores.grad, ref_ds, "d_scores", max_rel=2e-2)


def test_transformers_block_runs_on_the_plugin():
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock

    assert register_experts_implementation()
    cfg = Qwen3MoeConfig(hidden_size=256, num_experts=8, num_experts_per_tok=2, moe_intermediate_size=128,
                         norm_topk_prob=True)
    cfg._experts_implementation = "mi355x"
    torch.manual_seed(0)
    block = Qwen3MoeSparseMoeBlock(cfg)
    with torch.no_grad():
        for p in block.parameters():
            p.normal_(0, 0.05)
    ref_block = Qwen3MoeSparseMoeBlock(cfg)
    ref_block.load_state_dict(block.state_dict())
    block = block.to(DEV, BF)
    x = torch.randn(2, 64, 256)
    xg = x.to(DEV, BF).requires_grad_()
    _, sc, ix = block.gate(xg.view(-1, 256))
    out = block.experts(xg.view(-1, 256), ix, sc)
    ref = O.experts_eager(x.to(BF).float().view(-1, 256), ix.cpu(), sc.detach().cpu().float(),
                          ref_block.experts.gate_up_proj.detach().to(BF).float(),
                          ref_block.experts.down_proj.detach().to(BF).float())
    close_bf16(out, ref, "transformers plugin out")
    out.float().square().sum().backward()
    assert block.experts.gate_up_proj.grad is not None and torch.isfinite(xg.grad.float()).all()


def test_full_c2_forward_properties_and_sampled_tokens():
    w = WORKLOADS["c2"]
    inp = make_block_inputs(w, seed=11, device=DEV, dtype=BF, weights_on_device_rng=True)
    x = inp["x"]
    logits, scores, idx = ops.router_fwd(x, inp["router_weight"], w.top_k, True)
    gu, dn = inp["gate_up_proj"], inp["down_proj"]
    out1, xp, pre, act, y, pos, offsets = ops.experts_fwd(x, idx, scores, gu, dn)
    out2 = ops.experts_fwd(x, idx, scores, gu, dn)[0]
    assert torch.equal(out1, out2), "forward must be deterministic"
    # permutation invariants at full size
    off = offsets.cpu().long()
    assert int(off[-1]) == w.slots and bool((off[1:] >= off[:-1]).all())
    p = pos.cpu().long()
    assert torch.equal(torch.sort(p).values, torch.arange(w.slots))
    ids_sorted = idx.cpu().reshape(-1)[torch.argsort(p)]
    assert bool((ids_sorted[1:] >= ids_sorted[:-1]).all())
    # linearity: doubling the activations doubles the up-projection exactly
    act2 = torch.empty_like(act)
    pre2 = torch.empty_like(pre)
    from parallel_amd import _lib
    xp2 = xp * 2
    _lib.call("moe_grouped_gemm_swiglu_fwd", xp2.data_ptr(), gu.data_ptr(), offsets.data_ptr(), w.experts, w.slots,
              w.hidden, w.intermediate, act2.data_ptr(), pre2.data_ptr(), _lib.stream_of(xp2))
    assert torch.equal(pre2, pre * 2)
    # sampled tokens against the oracle (the forward is per-token independent)
    sample = torch.randperm(w.tokens, generator=torch.Generator().manual_seed(0))[:48]
    ref = O.experts_grouped(x.cpu()[sample], idx.cpu()[sample], scores.cpu()[sample], gu.cpu(), dn.cpu())
    close_bf16(out1.cpu()[sample], ref, "c2 sampled tokens")


@pytest.mark.parametrize("name", ["c2", "c4", "c5"])
def test_full_size_backward_sampled_tokens_against_the_oracle(name):
    """The full block's input gradient (the one-op block: the router's
    top-k backward inside the combine backward, the router's dX added in the
    permute backward) on 48 sampled tokens against the oracle run on those
    tokens alone, at C2, C4 (its biased router) and C5 (H 4096).  With no
    aux term every part of a token's input gradient is the token's own: its
    k experts' backward and its router row's."""
    w = WORKLOADS[name]
    inp = make_block_inputs(w, seed=15, device=DEV, dtype=BF, weights_on_device_rng=True)
    x = inp["x"].clone().requires_grad_()
    rw, gu, dn = inp["router_weight"], inp["gate_up_proj"], inp["down_proj"]
    bias = inp.get("logit_bias")
    out, logits, _, idx, _ = ops.moe_block(x, rw, gu, dn, w.top_k, w.norm_topk_prob, None, bias)
    d_out = inp["d_out"]
    torch.autograd.backward([out], [d_out])
    torch.cuda.synchronize()
    sample = torch.randperm(w.tokens, generator=torch.Generator().manual_seed(1))[:48]
    bias_c = None if bias is None else bias.cpu()
    ref = O.block_forward_backward(x.detach().cpu()[sample], rw.cpu(), gu.cpu(), dn.cpu(), d_out.cpu()[sample],
                                   top_k=w.top_k, norm_topk_prob=w.norm_topk_prob, aux_coef=0.0, logit_bias=bias_c)
    routing_check(idx.cpu()[sample], ref["indices"], logits.detach().cpu()[sample])
    close_bf16(out.detach().cpu()[sample], ref["out"], f"{name} sampled out")
    got = x.grad.cpu()[sample].float()
    rel, _ = close_bf16(got, ref["dx"], f"{name} sampled dx")
    # The router's share of dx must be there: the oracle's input gradient
    # with the routing weights held constant (experts only) is much further
    # from the kernels' than the full one is.
    xs = x.detach().cpu()[sample].float().requires_grad_()

    def lg(t):
        return O.router_logits(t, rw.cpu()) + (0.0 if bias_c is None else bias_c.float())

    _, ix = O.topk_softmax(lg(xs), w.top_k, w.norm_topk_prob)
    sc = O.topk_softmax(lg(xs.detach()), w.top_k, w.norm_topk_prob)[0]
    y = O.experts_grouped(xs, ix, sc, gu.cpu(), dn.cpu())
    (y.float() * d_out.cpu()[sample].float()).sum().backward()
    scale = ref["dx"].float().abs().max()
    rel_experts_only = float((got - xs.grad).abs().max() / scale)
    assert rel_experts_only > 4 * rel, (rel, rel_experts_only)


def test_experts_concentrated_routing():
    """Every token routes to the same k experts: k groups of T rows (several
    evenly split m-tiles each) and E - k empty experts, forward and backward,
    against the oracle's grouped experts."""
    T, H, E, k, I = 1100, 256, 16, 4, 128
    g = torch.Generator().manual_seed(21)
    x = torch.randn(T, H, generator=g).to(BF)
    idx = torch.tensor([3, 7, 8, 15]).repeat(T, 1)
    scores = torch.softmax(torch.randn(T, k, generator=g), -1)
    gu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(BF)
    dn = (torch.randn(E, H, I, generator=g) * 0.05).to(BF)
    d_out = torch.randn(T, H, generator=g).to(BF)
    leaves = [t.clone().requires_grad_() for t in (x, scores, gu, dn)]
    ref = O.experts_grouped(leaves[0], idx, leaves[1], leaves[2], leaves[3])
    ref.backward(d_out)
    dl = [t.to(DEV).requires_grad_() for t in (x, scores, gu, dn)]
    out = ops.experts(dl[0], idx.to(DEV), dl[1], dl[2], dl[3])
    out.backward(d_out.to(DEV))
    torch.cuda.synchronize()
    close_bf16(out, ref, "concentrated out")
    for name, a, b in zip(("dx", "d_scores", "d_gate_up", "d_down"), dl, leaves):
        close_bf16(a.grad, b.grad, f"concentrated {name}")
    unused = [e for e in range(E) if e not in (3, 7, 8, 15)]
    assert not dl[2].grad[unused].any() and not dl[3].grad[unused].any(), "experts without routes get zero dW"


@pytest.mark.parametrize("k", [3, 16])
def test_experts_run_time_slot_count(k):
    """The experts op at slot counts served by the run-time-k kernels (row
    copy, combine, permute backward), forward and backward, against the
    oracle's grouped experts."""
    T, H, E, I = 257, 136, 24, 64
    g = torch.Generator().manual_seed(23 + k)
    x = torch.randn(T, H, generator=g).to(BF)
    idx = torch.rand(T, E, generator=g).topk(k, dim=1).indices
    scores = torch.softmax(torch.randn(T, k, generator=g), -1)
    gu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(BF)
    dn = (torch.randn(E, H, I, generator=g) * 0.05).to(BF)
    d_out = torch.randn(T, H, generator=g).to(BF)
    leaves = [t.clone().requires_grad_() for t in (x, scores, gu, dn)]
    ref = O.experts_grouped(leaves[0], idx, leaves[1], leaves[2], leaves[3])
    ref.backward(d_out)
    dl = [t.to(DEV).requires_grad_() for t in (x, scores, gu, dn)]
    out = ops.experts(dl[0], idx.to(DEV), dl[1], dl[2], dl[3])
    out.backward(d_out.to(DEV))
    torch.cuda.synchronize()
    close_bf16(out, ref, f"k={k} out")
    for name, a, b in zip(("dx", "d_scores", "d_gate_up", "d_down"), dl, leaves):
        close_bf16(a.grad, b.grad, f"k={k} {name}")


def test_empty_batch_through_router_and_experts():
    """A batch with no tokens (an EP rank can receive no rows): the reference's
    grouped experts return [0, H] and every weight gradient is zero.  Every
    entry point on the path sees size 0 with NULL pointers for the empty
    buffers."""
    H, E, k, I = 256, 16, 4, 128
    g = torch.Generator().manual_seed(22)
    x = torch.empty(0, H, dtype=BF, device=DEV).requires_grad_()
    rw = (torch.randn(E, H, generator=g) * 0.05).to(DEV, BF).requires_grad_()
    gu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(DEV, BF).requires_grad_()
    dn = (torch.randn(E, H, I, generator=g) * 0.05).to(DEV, BF).requires_grad_()
    logits, scores, idx = ops.router_fwd(x, rw, k, True)
    assert logits.shape == (0, E) and scores.shape == (0, k) and idx.shape == (0, k)
    out = ops.experts(x, idx, scores, gu, dn)
    assert out.shape == (0, H)
    (out.float().sum() + scores.sum() + logits.sum()).backward()
    torch.cuda.synchronize()
    assert x.grad is not None and x.grad.shape == (0, H)
    for name, p in (("router", rw), ("gate_up_proj", gu), ("down_proj", dn)):
        assert p.grad is not None and p.grad.shape == p.shape and not p.grad.any(), f"{name}: dW must be zero"

"""The benchmark configurations at full size on the GPU, backward included,
through size-independent properties (the CPU oracle cannot run these sizes
in seconds):

* every expert's forward products (pre-activations, down projection) and
  weight and input gradients against plain fp32 torch.mm references of the
  same products, computed per expert on the GPU from the kernels' own inputs
  (xp, act, d_pre, dy), the SwiGLU and the weighted combine: the persistent
  schedules' multi-round tile loops, the even m-split of large experts and
  the cost split of the weight gradients at 128 experts, all at full size;
* weight-gradient accumulation into existing gradients, fused in the kernel
  against torch's separate add, bit for bit;
* the router at full size (one, two or four 16-token row tiles per block):
  its logits against an fp32 torch product on the GPU, its routing against
  the oracle's top-k on the returned logits, bit for bit.
"""

from dataclasses import replace

import pytest
import torch

from conftest import close_bf16, routing_check
from oracle import moe_oracle as O
from parallel_amd import _lib, ops
from parallel_amd.workloads import WORKLOADS, ep_receive_buffer, make_block_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def _forward(w, seed):
    inp = make_block_inputs(w, seed=seed, device=DEV, dtype=BF, weights_on_device_rng=True)
    bias = inp.get("logit_bias")
    logits, scores, idx = ops.router_fwd(inp["x"], inp["router_weight"], w.top_k, w.norm_topk_prob, bias)
    _check_router(inp, bias, logits, scores, idx, w)
    saved = ops.experts_fwd(inp["x"], idx, scores, inp["gate_up_proj"], inp["down_proj"])
    return inp, scores, idx, saved


def _check_router(inp, bias, logits, scores, idx, w):
    """Logits within fp32 accumulation-order noise of x.float() @ wr.float().T
    (+ bias); indices and scores those of the oracle's softmax and top-k on
    the returned logits (no exact ties on continuous random inputs)."""
    ref = inp["x"].float() @ inp["router_weight"].float().t()
    if bias is not None:
        ref = ref + bias.float()
    torch.testing.assert_close(logits, ref, rtol=1e-4, atol=1e-4 * float(ref.abs().max()))
    lc = logits.cpu()
    ref_s, ref_i = O.topk_softmax(lc, w.top_k, w.norm_topk_prob)
    routing_check(idx, ref_i, lc)
    torch.testing.assert_close(scores.cpu(), ref_s.float(), rtol=2e-6, atol=1e-7)


def _dgrad(dc, wt, offsets, G, M, N, K):
    """moe_grouped_gemm_dgrad: da[M,K] = dc[M,N] . w[g] (w [G,N,K])."""
    da = torch.empty(M, K, dtype=BF, device=DEV)
    _lib.call("moe_grouped_gemm_dgrad", dc.data_ptr(), wt.data_ptr(), offsets.data_ptr(), G, M, N, K, da.data_ptr(),
              _lib.stream_of(dc))
    return da


def close_on_device(actual, expected, name, max_rel=2e-2, min_cos=0.9999):
    """close_bf16's bar (normwise max relative error, cosine) evaluated on the GPU."""
    a = actual.float().reshape(-1)
    b = expected.float().reshape(-1)
    denom = float(b.abs().max())
    rel = float((a - b).abs().max()) / max(denom, 1e-30)
    cos = float(torch.dot(a.double(), b.double()) / (a.double().norm() * b.double().norm()).clamp_min(1e-300))
    assert torch.isfinite(a).all(), f"{name}: non-finite values"
    assert rel <= max_rel and (cos >= min_cos or denom == 0), f"{name}: max rel err {rel:.3e}, cosine {cos:.6f}"
    return rel


def _backward_checks(name, w, inp, scores, saved, seed):
    """Checks the saved forward state (SwiGLU, combine, every expert's up and
    down products), runs the experts' backward on it and checks every
    expert's dW and input gradients, against fp32 products of the kernels'
    own inputs; returns the per-expert row counts."""
    E, H, I, S = w.experts, w.hidden, w.intermediate, w.slots
    out, xp, pre, act, y, pos, offsets = saved
    # forward: the SwiGLU of the saved pre-activations (gate | up) and the
    # weighted combine of the down projection's rows
    g_, u_ = pre.float()[:, :I], pre.float()[:, I:]
    close_on_device(act, torch.nn.functional.silu(g_) * u_, f"{name} act")
    T, k = w.tokens, w.top_k
    posl = pos.long().view(T, k)
    close_on_device(out, (y.float()[posl] * scores.float().unsqueeze(-1)).sum(1), f"{name} out")
    d_out = torch.randn(w.tokens, H, generator=torch.Generator(device=DEV).manual_seed(seed), device=DEV).to(BF)
    captured = {}

    def wgrad(proj, dc, a, n, k):
        captured[proj] = (dc, a)
        dw = torch.empty(E, n, k, dtype=BF, device=DEV)
        _lib.call("moe_grouped_gemm_wgrad", dc.data_ptr(), a.data_ptr(), offsets.data_ptr(), E, S, n, k,
                  dw.data_ptr(), 0, 0, _lib.stream_of(dc))
        return dw

    d_hidden, d_w, d_gu, d_dn = ops.experts_bwd_kernels(d_out, scores, inp["gate_up_proj"], inp["down_proj"], xp,
                                                        pre, act, y, pos, offsets, wgrad)
    d_pre, _ = captured["gate_up_proj"]
    dy, _ = captured["down_proj"]
    gu, dn = inp["gate_up_proj"], inp["down_proj"]
    d_act = _dgrad(dy, dn, offsets, E, S, H, I)
    d_xp = _dgrad(d_pre, gu, offsets, E, S, 2 * I, H)
    torch.cuda.synchronize()
    off = offsets.cpu().long().tolist()
    assert off[-1] == S
    counts = [off[0]] + [off[e] - off[e - 1] for e in range(1, E)]
    worst = {}
    r0 = 0
    for e in range(E):
        r1 = off[e]
        rows = slice(r0, r1)
        if r1 == r0:
            assert not d_gu[e].any() and not d_dn[e].any(), f"{name} expert {e}: empty expert needs zero dW"
        else:
            f = lambda t: t[rows].float()  # noqa: E731
            checks = (("pre", pre[rows], f(xp) @ gu[e].float().t()), ("y", y[rows], f(act) @ dn[e].float().t()),
                      ("d_gate_up", d_gu[e], f(d_pre).t() @ f(xp)), ("d_down", d_dn[e], f(dy).t() @ f(act)),
                      ("d_xp", d_xp[rows], f(d_pre) @ gu[e].float()), ("d_act", d_act[rows], f(dy) @ dn[e].float()))
            for label, got, ref in checks:
                rel = close_on_device(got, ref, f"{name} expert {e} ({r1 - r0} rows) {label}")
                worst[label] = max(worst.get(label, 0.0), rel)
        r0 = r1
    print(f"{name}: worst normwise max rel err per product over {E} experts: {worst}")
    # the combine backward's score gradient <d_out[t], y[pos(t, j)]> and the
    # permute backward's sum of each token's k input-gradient rows
    close_on_device(d_w.view(T, k), (y.float()[posl] * d_out.float().unsqueeze(1)).sum(-1), f"{name} d_scores")
    close_on_device(d_hidden, d_xp.float()[posl].sum(1), f"{name} d_hidden")
    return counts


@pytest.mark.parametrize("name,seed", [("c2", 31), ("c4", 32), ("c5", 33)])
def test_full_size_backward_every_expert(name, seed):
    w = WORKLOADS[name]
    inp, scores, idx, saved = _forward(w, seed)
    counts = _backward_checks(name, w, inp, scores, saved, seed)
    assert max(counts) > 256, "some expert must span several m-tiles"


def test_full_size_concentrated_routing():
    """C4's 16384 tokens all routed to the same 8 experts: 16384 rows each
    (64 evenly split m-tiles), 120 empty experts, and the weight gradients'
    cost split with nearly all the cost in 8 groups."""
    w = WORKLOADS["c4"]
    inp = make_block_inputs(w, seed=51, device=DEV, dtype=BF, weights_on_device_rng=True)
    g = torch.Generator(device=DEV).manual_seed(52)
    chosen = torch.tensor([3, 17, 40, 41, 77, 90, 101, 127], device=DEV)
    idx = chosen.repeat(w.tokens, 1)
    scores = torch.softmax(torch.randn(w.tokens, w.top_k, generator=g, device=DEV), -1)
    saved = ops.experts_fwd(inp["x"], idx, scores, inp["gate_up_proj"], inp["down_proj"])
    counts = _backward_checks("c4 concentrated", w, inp, scores, saved, 53)
    assert sorted(c for c in counts if c) == [w.tokens] * 8 and counts.count(0) == w.experts - 8


def test_full_c4_gradient_accumulation_fused_equals_torch_add():
    """C4 ("dW accumulation"): two backward steps into existing gradients.
    The in-kernel accumulation gives the same bits as torch adding a fresh
    dense gradient into .grad."""
    w = WORKLOADS["c4"]
    inp = make_block_inputs(w, seed=41, device=DEV, dtype=BF, weights_on_device_rng=True)
    g = torch.Generator(device=DEV).manual_seed(5)
    d_outs = [torch.randn(w.tokens, w.hidden, generator=g, device=DEV).to(BF) for _ in range(2)]
    init = [torch.randn(p.shape, generator=g, device=DEV).mul_(1e-3).to(BF)
            for p in (inp["gate_up_proj"], inp["down_proj"])]
    logits, scores, idx = ops.router_fwd(inp["x"], inp["router_weight"], w.top_k, True, inp["logit_bias"])
    grads = {}
    for fused in (False, True):
        gu = inp["gate_up_proj"].clone().requires_grad_()
        dn = inp["down_proj"].clone().requires_grad_()
        gu.grad, dn.grad = init[0].clone(), init[1].clone()
        for d_out in d_outs:
            ops.experts(inp["x"], idx, scores, gu, dn, accumulate_grad=fused).backward(d_out)
        torch.cuda.synchronize()
        grads[fused] = (gu.grad, dn.grad)
    for a, b, label in zip(grads[True], grads[False], ("d_gate_up", "d_down")):
        assert torch.equal(a, b), f"fused {label} accumulation differs from torch's add"


def test_full_c3_receive_buffer_every_expert():
    """C3 at its stated size: rank 0's receive buffer of an EP = 2 group,
    2 x 4096 source tokens x 8 slots drawn Zipf(1.2) over 128 experts (about
    24k rows, source-rank-major, expert-contiguous within a source, at least
    4 of the 64 local experts empty), through the experts forward and
    backward, with every expert's products checked as above
    (token_dispatch.py:101-158)."""
    w3 = WORKLOADS["c3"]
    _, _, (src, tok, lexp, lsc) = ep_receive_buffer(w3, seed=3)
    R = int(src.shape[0])
    inp = make_block_inputs(w3, seed=3, device=DEV, dtype=BF, weights_on_device_rng=True)
    xs = torch.randn(w3.sources, w3.tokens, w3.hidden, generator=torch.Generator(device=DEV).manual_seed(8),
                     device=DEV).to(BF)
    hidden = xs[torch.from_numpy(src).to(DEV), torch.from_numpy(tok).to(DEV)].contiguous()
    idx = torch.from_numpy(lexp).to(DEV).view(R, 1)
    sc = torch.from_numpy(lsc).to(DEV).view(R, 1)
    saved = ops.experts_fwd(hidden, idx, sc, inp["gate_up_proj"], inp["down_proj"])
    recv = replace(w3, name="c3_receive", batch=1, seq=R, top_k=1, experts=w3.local_experts, local_experts=None)
    counts = _backward_checks("c3", recv, inp, sc, saved, 62)
    assert sum(c == 0 for c in counts) >= 4, "some local experts must be empty"
    assert max(counts) > 4 * R // len(counts), "Zipf routing must be skewed"

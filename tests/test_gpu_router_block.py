"""The one-pass router (GEMM, reduction, top-k softmax and aux partials in one
kernel), the router backward with the aux loss's gradient formed in the same
pass, and the whole block as one op (``ops.moe_block``), on the GPU.

References: the CPU oracle (router_logits / topk_softmax / block_forward_backward,
following TF modeling_qwen3_moe.py:249-267, :514-593 and integrations/moe.py:377-478),
and the separate ops, whose kernels the fused paths share: where the
arithmetic is the same the results must be the same bits."""

import pytest
import torch

from conftest import close_bf16, routing_check
from oracle import moe_oracle as O
from parallel_amd import ops
from parallel_amd.workloads import WORKLOADS, make_block_inputs, scaled
from test_gpu_block import compare, gpu_block_step, oracle_step

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def gen(seed):
    return torch.Generator().manual_seed(seed)


# Every experts-per-lane width of the one-pass kernel (E = 16, 32, 64, 96/128),
# H with a partial last k-step (72, 136, 264, 520), T not a multiple of the
# block's 16 tokens (1 and 17 leave most of a block's rows empty); H above
# 4096 (4200, 8200) loads x in more than one group of 32 k-steps per wave;
# E = 120 and E = 256 take the split-K path.
ROUTER_CASES = [(257, 72, 16, 4), (300, 136, 32, 3), (1000, 520, 64, 6), (200, 264, 96, 5), (4096, 2048, 128, 8),
                (70, 4200, 128, 8), (40, 8200, 48, 2), (1, 264, 128, 8), (17, 2048, 64, 4), (129, 256, 256, 8),
                (300, 72, 120, 8),
                # past 4096 and 8192 tokens (256 CUs): two and four 16-token row tiles per block,
                # ragged last block, one or several groups of x loads per block
                (5000, 264, 128, 8), (6000, 2104, 64, 8), (8200, 264, 64, 8), (8200, 2104, 64, 8),
                (16390, 1104, 128, 8), (16400, 72, 32, 4),
                (16400, 264, 16, 2), (16390, 520, 64, 6),
                # the split-K GEMM and reduce-and-select path at many tokens
                (16400, 264, 120, 8), (9000, 136, 256, 8), (5000, 72, 320, 4)]


@pytest.mark.parametrize("T,H,E,k", ROUTER_CASES)
def test_router_aux_fwd_matches_fp32_and_the_standalone_kernels(T, H, E, k):
    x = torch.randn(T, H, generator=gen(T)).to(BF)
    w = (torch.randn(E, H, generator=gen(E)) * 0.05).to(BF)
    bias = torch.randn(E, generator=gen(7)) * 0.3
    tw = (torch.rand(T, generator=gen(8)) > 0.2).float()
    logits, scores, idx, aux, stats = ops.router_aux_fwd(x.to(DEV), w.to(DEV), k, True, tw.to(DEV), bias.to(DEV))
    ref = O.router_logits(x, w) + bias
    torch.testing.assert_close(logits.cpu(), ref, rtol=1e-4, atol=1e-5)
    routing_check(idx, O.topk_softmax(ref, k, True)[1], logits)
    # the routing and the loss are those of the standalone kernels on the returned logits, bit for bit
    s2, i2 = ops.router_topk(logits, k, True)
    assert torch.equal(i2, idx) and torch.equal(s2, scores)
    aux2, stats2 = ops.aux_loss_fwd(logits, tw.to(DEV), E, k)
    assert torch.equal(aux, aux2) and torch.equal(stats, stats2)
    ref_aux = O.load_balancing_loss((ref,), E, k, attention_mask=tw.reshape(1, T))
    torch.testing.assert_close(aux.cpu(), ref_aux, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("T,H,E,k,masked", [(1000, 256, 64, 6, True), (512, 2048, 128, 8, False),
                                             (300, 72, 120, 8, True)])
def test_router_aux_backward_is_the_two_pass_gradient_bit_for_bit(T, H, E, k, masked):
    """The aux loss's logits gradient formed inside the top-k backward gives
    the bits of moe_aux_loss_bwd's output added by the separate pass."""
    x = torch.randn(T, H, generator=gen(1)).to(BF).to(DEV)
    w = (torch.randn(E, H, generator=gen(2)) * 0.05).to(BF).to(DEV)
    tw = (torch.rand(T, generator=gen(3)) > 0.3).float().to(DEV) if masked else None
    d_scores = torch.randn(T, k, generator=gen(4)).to(DEV)
    d_logits = (torch.randn(T, E, generator=gen(5)) * 0.01).to(DEV)
    d_aux = torch.tensor(0.37, device=DEV)
    xg, wg = x.clone().requires_grad_(), w.clone().requires_grad_()
    logits, scores, idx, aux, stats = ops.router_aux_fwd(xg, wg, k, True, tw)
    torch.autograd.backward([scores, logits, aux], [d_scores, d_logits, d_aux])
    dl_aux = ops.aux_loss_bwd(logits.detach(), tw, stats, d_aux)
    dx2, dw2 = ops.router_bwd(x, w, logits.detach(), idx, d_logits + dl_aux, d_scores, True)
    assert torch.equal(xg.grad, dx2)
    assert torch.equal(wg.grad, dw2)


def block_step(w, inp, accumulate=False, grads=None, logit_bias=None):
    x = inp["x"].to(DEV).requires_grad_()
    rw = inp["router_weight"].to(DEV).requires_grad_()
    gu = inp["gate_up_proj"].to(DEV).requires_grad_()
    dn = inp["down_proj"].to(DEV).requires_grad_()
    if grads is not None:
        for p, g in zip((rw, gu, dn), grads):
            p.grad = g.clone()
    bias = None if logit_bias is None else logit_bias.to(DEV)
    out, logits, scores, idx, aux = ops.moe_block(x, rw, gu, dn, w.top_k, w.norm_topk_prob, None, bias, accumulate)
    torch.autograd.backward([out, aux], [inp["d_out"].to(DEV), torch.tensor(w.aux_coef, device=DEV)])
    return dict(logits=logits.detach(), scores=scores.detach(), indices=idx, out=out.detach(), aux=aux.detach(),
                dx=x.grad, d_router=rw.grad, d_gate_up=gu.grad, d_down=dn.grad)


@pytest.mark.parametrize("base,tokens", [("c1", 512), ("c2", 512), ("c4", 1024)])
def test_moe_block_matches_the_separate_ops_and_the_oracle(base, tokens):
    w = scaled(WORKLOADS[base], tokens)
    inp = make_block_inputs(w, seed=11, dtype=BF)
    bias = inp.get("logit_bias")
    blk = block_step(w, inp, logit_bias=bias)
    sep = gpu_block_step(w, inp, logit_bias=bias)
    compare(blk, oracle_step(w, inp, logit_bias=bias), f"{base} block")
    # Same kernels: the forward and the weight gradients are the same bits.
    for key in ("logits", "scores", "indices", "out", "aux", "d_router", "d_gate_up", "d_down"):
        assert torch.equal(blk[key], sep[key]), key
    # dX: the router's share joins the experts' in fp32 inside the permute
    # backward, one rounding where autograd rounds the experts' sum first.
    close_bf16(blk["dx"], sep["dx"], f"{base} dx against the separate ops", max_rel=1e-2, min_cos=0.99999)


@pytest.mark.parametrize("base,tokens", [("c2", 512), ("c4", 1024)])
def test_moe_block_with_score_and_logit_gradients_matches_the_separate_ops(base, tokens):
    """When the scores and logits returned by moe_block also feed the loss,
    the block's backward sums the scores' two gradients before the router's
    top-k backward (the separate-launch path, not the combine's fused one)
    and adds the logits' gradient there: the router weight's gradient is the
    separate ops' bits, the expert weights' too."""
    w = scaled(WORKLOADS[base], tokens)
    inp = make_block_inputs(w, seed=12, dtype=BF)
    bias = inp.get("logit_bias")
    bias = None if bias is None else bias.to(DEV)
    T, k, E = w.tokens, w.top_k, w.experts
    d_scores = torch.randn(T, k, generator=gen(21)).to(DEV)
    d_logits = (torch.randn(T, E, generator=gen(22)) * 0.01).to(DEV)
    coef = torch.tensor(w.aux_coef, device=DEV)
    d_out = inp["d_out"].to(DEV)
    res = []
    for fused_op in (True, False):
        a = [inp[n].to(DEV).clone().requires_grad_() for n in ("x", "router_weight", "gate_up_proj", "down_proj")]
        if fused_op:
            out, logits, scores, _, aux = ops.moe_block(*a, k, w.norm_topk_prob, None, bias)
        else:
            logits, scores, idx, aux, _ = ops.router_aux_fwd(a[0], a[1], k, w.norm_topk_prob, None, bias)
            out = ops.experts(a[0], idx, scores, a[2], a[3])
        torch.autograd.backward([out, aux, scores, logits], [d_out, coef, d_scores, d_logits])
        res.append([t.grad for t in a])
    torch.cuda.synchronize()
    (dx1, dr1, dg1, dd1), (dx2, dr2, dg2, dd2) = res
    assert torch.equal(dr1, dr2) and torch.equal(dg1, dg2) and torch.equal(dd1, dd2)
    close_bf16(dx1, dx2, f"{base} dx against the separate ops", max_rel=1e-2, min_cos=0.99999)


@pytest.mark.parametrize("name", ["c2", "c4", "c5"])
def test_moe_block_matches_the_separate_ops_at_full_size(name):
    """The benchmark configurations at full size (C4 with its biased router,
    C5 with its 4096-wide layer): moe_block gives the separate ops' bits for
    the forward, the aux loss and every weight gradient."""
    w = WORKLOADS[name]
    inp = make_block_inputs(w, seed=14, device=DEV, dtype=BF, weights_on_device_rng=True)
    bias = inp.get("logit_bias")
    # each step gets its own leaves (tensors already on the device are not copied by .to)
    blk = block_step(w, {key: t.clone() for key, t in inp.items()}, logit_bias=bias)
    sep = gpu_block_step(w, {key: t.clone() for key, t in inp.items()}, logit_bias=bias)
    torch.cuda.synchronize()
    for key in ("logits", "scores", "indices", "out", "aux", "d_router", "d_gate_up", "d_down"):
        assert torch.equal(blk[key], sep[key]), f"{name} {key}"
    close_bf16(blk["dx"], sep["dx"], f"{name} dx against the separate ops", max_rel=1e-2, min_cos=0.99999)


def test_moe_block_on_a_side_stream_gives_the_default_stream_bits():
    """Every launch goes to torch's current stream: the block's forward and
    backward issued on another stream (default priority) give the same bits
    as on the default stream."""
    w = scaled(WORKLOADS["c2"], 1024)
    inp = make_block_inputs(w, seed=15, dtype=BF)
    ref = block_step(w, inp)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        got = block_step(w, inp)
    torch.cuda.synchronize()
    for key in ("logits", "scores", "indices", "out", "aux", "dx", "d_router", "d_gate_up", "d_down"):
        assert torch.equal(got[key], ref[key]), key


def test_moe_block_accumulates_every_weight_gradient_in_the_kernels():
    w = scaled(WORKLOADS["c2"], 512)
    inp = make_block_inputs(w, seed=12, dtype=BF)
    g = gen(13)
    init = [torch.randn(inp[n].shape, generator=g).mul(1e-3).to(BF).to(DEV)
            for n in ("router_weight", "gate_up_proj", "down_proj")]
    fresh = block_step(w, inp)
    acc = block_step(w, inp, accumulate=True, grads=init)
    for key, g0 in zip(("d_router", "d_gate_up", "d_down"), init):
        assert torch.equal(acc[key], g0 + fresh[key]), key  # torch's bf16 add of the fresh gradient
    assert torch.equal(acc["dx"], fresh["dx"])


# ------------------------------------------------- bf16 router logits (AMP)


@pytest.mark.parametrize("T,H,E,k,norm", [(1000, 256, 64, 6, True), (4096, 2048, 128, 8, True),
                                          (300, 72, 120, 8, False), (257, 136, 32, 3, True),
                                          # two and four 16-token row tiles per block
                                          (6000, 2104, 64, 8, True), (8200, 2104, 64, 8, True),
                                          (16390, 1104, 128, 8, False)])
def test_bf16_logit_router_routes_bit_exactly(T, H, E, k, norm):
    """Under the reference's bf16 autocast (parallel/parallel/engine/engine.py:141)
    Qwen3MoeTopKRouter's F.linear gives bf16 logits; softmax and top-k run in
    fp32 on them and the scores are cast back to bf16 (TF
    modeling_qwen3_moe.py:258-267)."""
    x = torch.randn(T, H, generator=gen(T + 1)).to(BF)
    w = (torch.randn(E, H, generator=gen(E + 1)) * 0.05).to(BF)
    logits_b, scores, idx, logits32 = ops.router_fwd_bf16(x.to(DEV), w.to(DEV), k, norm)
    assert logits_b.dtype == BF and scores.dtype == BF and logits32.dtype == torch.float32
    lb = logits_b.cpu()
    assert torch.equal(logits32.cpu(), lb.float())
    # The bf16 logits round the fp32 sum: mostly the same bits as rounding the
    # oracle's fp32 sum, and always within one bf16 step of it plus the fp32
    # accumulation-order noise (which exceeds a bf16 step only near zero).
    ref = O.router_logits(x, w)
    want = ref.to(BF)
    step = torch.ldexp(torch.ones_like(ref), torch.frexp(ref)[1] - 8)  # one bf16 ulp at each value
    assert ((lb.float() - ref).abs() <= step + 1e-5).all()
    assert (lb == want).float().mean() > 0.99
    # Routing on these logits is exact, ties included: largest logit first,
    # equal logits in increasing expert index, the reference's fp32 softmax,
    # renormalisation and bf16 cast.
    canon = torch.argsort(-lb.float(), dim=-1, stable=True)[:, :k]
    assert torch.equal(idx.cpu(), canon)
    top = torch.softmax(lb.float(), dim=-1).gather(1, canon)
    if norm:
        top = top / top.sum(dim=-1, keepdim=True)
    assert torch.equal(scores.cpu(), top.to(BF))
    # torch.topk (the oracle) agrees wherever its tie order does not matter
    ref_s, ref_i = O.topk_softmax(lb, k, norm)
    ties = O.topk_ties(lb.float(), ref_i)
    routing_check(idx, ref_i, lb.float(), expect_ties=int(ties.sum()))


def test_bf16_logit_router_backward_and_the_autocast_module():
    from parallel_amd import TopKRouter

    T, H, E, k = 512, 256, 64, 6
    x = torch.randn(T, H, generator=gen(31)).to(BF)
    w = (torch.randn(E, H, generator=gen(32)) * 0.05).to(BF)
    d_scores = torch.randn(T, k, generator=gen(33))
    xg, wg = x.to(DEV).requires_grad_(), w.to(DEV).requires_grad_()
    logits_b, scores, idx, _ = ops.router_fwd_bf16(xg, wg, k, True)
    scores.backward(d_scores.to(DEV).to(BF))
    # fp32 autograd of the reference's softmax / gather / renormalisation on
    # the selection made (bf16 logits tie often; the selection itself is pinned
    # bit for bit above), the bf16 rounding of the logits passed straight through
    xr, wr = x.float().requires_grad_(), w.float().requires_grad_()
    lr = O.router_logits(xr, wr)
    lr = lr + (lr.to(BF).float() - lr).detach()
    sr = torch.softmax(lr, dim=-1).gather(1, idx.cpu())
    sr = sr / sr.sum(dim=-1, keepdim=True)
    sr.backward(d_scores.to(BF).float())
    close_bf16(xg.grad, xr.grad, "bf16-logit router dx")
    close_bf16(wg.grad, wr.grad, "bf16-logit router dweight")
    # The transformers-facing module takes this path under bf16 autocast.
    cfg = type("Cfg", (), dict(num_experts_per_tok=k, num_experts=E, norm_topk_prob=True, hidden_size=H))()
    router = TopKRouter(cfg).to(DEV)
    with torch.no_grad():
        router.weight.copy_(w.float())
    with torch.autocast("cuda", dtype=torch.bfloat16):
        lm, sm, im = router(x.to(DEV))
    assert lm.dtype == BF and sm.dtype == BF
    assert torch.equal(lm, logits_b.detach()) and torch.equal(im, idx) and torch.equal(sm, scores.detach())


def test_bf16_logit_router_backward_sums_its_logit_gradients_in_bf16():
    """Under bf16 autocast the reference's router logits are a bf16 tensor read
    by two consumers, the router's fp32 softmax and the aux loss
    (load_balancing_loss_func, TF modeling_qwen3_moe.py:514-593); autograd
    returns each consumer's gradient in bf16 and adds them in bf16.
    moe_router_bf16_logits_bwd with the aux loss's bf16 gradient as d_logits gives
    the bits of CPU autograd on the bf16 logits (up to the rare bf16 rounding
    flip of a one-ulp fp32 difference in the softmax path); rounding the fp32
    sum once instead differs on more than 1 % of the logits here.  Without
    renormalisation, so that every logit's softmax-path gradient is well
    conditioned (renormalised top-k makes the unselected logits' gradient
    exactly zero in exact arithmetic, and what either side computes there is
    rounding noise)."""
    from parallel_amd import _lib

    T, H, E, k, coef = 512, 256, 64, 6, 1.0
    x = torch.randn(T, H, generator=gen(41)).to(BF)
    w = (torch.randn(E, H, generator=gen(42)) * 0.05).to(BF)
    d_scores = torch.randn(T, k, generator=gen(43)).to(BF)
    logits_b, _, idx, logits32 = ops.router_fwd_bf16(x.to(DEV), w.to(DEV), k, False)
    ic = idx.cpu()

    def softmax_path(lg):
        top = torch.softmax(lg.float(), dim=-1).gather(1, ic)
        return (top.to(BF).float() * d_scores.float()).sum()

    lb = logits_b.cpu().requires_grad_()
    (softmax_path(lb) + coef * O.load_balancing_loss(lb.float(), E, k)).backward()
    la = logits_b.cpu().requires_grad_()
    (coef * O.load_balancing_loss(la.float(), E, k)).backward()
    d_add = la.grad.float()
    got = torch.empty(T, E, dtype=BF, device=DEV)
    _lib.call("moe_router_bf16_logits_bwd", logits32.data_ptr(), idx.data_ptr(), (ds := d_scores.float().to(DEV)).data_ptr(),
              (da := d_add.to(DEV)).data_ptr(), None, None, None, T, E, k, 0, got.data_ptr(), _lib.stream_of(got))
    torch.cuda.synchronize()
    got, want = got.cpu(), lb.grad
    lf = logits_b.cpu().float().requires_grad_()
    softmax_path(lf).backward()
    # A rounding flip of the softmax path's term moves the sum by one bf16
    # step of the larger term (more than one step of the sum where the two
    # terms cancel).
    term = torch.maximum(lf.grad.abs(), d_add.abs())
    ulp = torch.ldexp(torch.ones(T, E), torch.frexp(term)[1] - 8)
    assert ((got.float() - want.float()).abs() <= ulp).all(), "more than one bf16 step of a term from the reference"
    assert (got == want).float().mean() >= 0.999
    once = (lf.grad + d_add).to(BF)
    assert (once != want).float().mean() > 0.01, "the test data must separate one rounding from two"


def test_moe_block_bf16_logits_c2_routes_bit_exactly_and_matches_the_separate_ops():
    """ops.moe_block(bf16_logits=True) on the C2 layer (4096 tokens, H 2048,
    128 experts, top-8), the router as the reference runs it under bf16
    autocast (parallel/parallel/engine/engine.py:141): bf16 logits and
    scores, the routing bit-exact on those logits (largest first, equal
    logits in increasing expert index; the reference's fp32 softmax,
    renormalisation and bf16 cast, TF modeling_qwen3_moe.py:258-267); the
    same logits, scores, routes and output bits as router_fwd_bf16 followed
    by the experts, the aux loss of load_balancing_loss_func on the bf16
    logits, and the same gradients (the expert weights' bit for bit)."""
    from parallel_amd import load_balancing_loss_func

    w = WORKLOADS["c2"]
    inp = make_block_inputs(w, seed=53, device=DEV, dtype=BF, weights_on_device_rng=True)
    k, E = w.top_k, w.experts
    coef = torch.tensor(w.aux_coef, device=DEV)
    a = [inp[n].detach().clone().requires_grad_() for n in ("x", "router_weight", "gate_up_proj", "down_proj")]
    out, lg, sc, idx, aux = ops.moe_block(*a, k, w.norm_topk_prob, bf16_logits=True)
    assert lg.dtype == BF and sc.dtype == BF
    lb = lg.detach().cpu()
    canon = torch.argsort(-lb.float(), dim=-1, stable=True)[:, :k]
    assert torch.equal(idx.cpu(), canon)
    top = torch.softmax(lb.float(), dim=-1).gather(1, canon)
    assert torch.equal(sc.detach().cpu(), (top / top.sum(dim=-1, keepdim=True)).to(BF))
    b = [inp[n].detach().clone().requires_grad_() for n in ("x", "router_weight", "gate_up_proj", "down_proj")]
    lg2, sc2, idx2, _ = ops.router_fwd_bf16(b[0], b[1], k, w.norm_topk_prob)
    assert torch.equal(lg2, lg) and torch.equal(sc2, sc) and torch.equal(idx2, idx)
    out2 = ops.experts(b[0], idx2, sc2, b[2], b[3])
    assert torch.equal(out2, out)
    aux2 = load_balancing_loss_func((lg2,), E, k)
    torch.testing.assert_close(aux, aux2, rtol=1e-6, atol=0)
    d_out = inp["d_out"]
    torch.autograd.backward([out, aux], [d_out, coef])
    torch.autograd.backward([out2, aux2], [d_out, coef])
    torch.cuda.synchronize()
    for name, ga, gb in zip(("dx", "d_router", "d_gate_up", "d_down"), a, b):
        close_bf16(ga.grad, gb.grad, f"c2 bf16-logit block {name}")
    assert torch.equal(a[2].grad, b[2].grad) and torch.equal(a[3].grad, b[3].grad)


# T, H, E, k, norm, aux (with a token mask), incoming logits gradient, bf16
# logits, share of sentinel slots.  E spans the experts-per-lane widths of
# the one-wave-per-token backward (1, 2, 4, 16 per lane) and k the
# specialised and run-time slot counts.
COMBINE_ROUTER_CASES = [(4096, 2048, 128, 8, True, False, False, False, 0.0),
                        (1000, 256, 64, 6, False, True, True, False, 0.05),
                        (512, 128, 200, 4, True, True, True, True, 0.0),
                        (300, 96, 32, 3, True, False, True, False, 0.1),
                        (64, 64, 1000, 16, True, True, False, True, 0.0),
                        (33, 72, 8, 1, False, False, False, False, 0.0),
                        # more tokens than the grid's waves: a wave takes several tokens
                        (40000, 64, 64, 4, True, True, True, False, 0.02)]


@pytest.mark.parametrize("T,H,E,k,norm,aux,d_logits,bf16,sentinel", COMBINE_ROUTER_CASES)
def test_combine_router_bwd_is_the_two_launches_bit_for_bit(T, H, E, k, norm, aux, d_logits, bf16, sentinel):
    """moe_combine_router_bwd (the combine backward and the router's top-k
    backward in one launch, as ops.moe_block runs them) against
    moe_combine_bwd followed by the router top-k backward entry point on its
    d_scores: d_y, d_scores and the bf16 logits gradient, bit for bit."""
    from parallel_amd import _lib

    g = gen(T + E + k)
    I = 64
    x = torch.randn(T, H, generator=g).to(BF).to(DEV)
    wr = (torch.randn(E, H, generator=g) * 0.05).to(BF).to(DEV)
    gu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(BF).to(DEV)
    dn = (torch.randn(E, H, I, generator=g) * 0.05).to(BF).to(DEV)
    tw = (torch.rand(T, generator=g) > 0.2).float().to(DEV) if aux else None
    logits, scores, idx, _, stats = ops.router_aux_fwd(x, wr, k, norm, tw)
    if bf16:
        logits = logits.to(BF).float()  # the values of bf16 logits
    ids = idx.clone()
    if sentinel:
        ids[(torch.rand(T, k, generator=g) < sentinel).to(DEV)] = E  # slots without an expert
    _, _, _, _, y, pos, offsets = ops._experts_fwd_kernels(x, ids, scores, gu, dn)
    d_out = torch.randn(T, H, generator=g).to(BF).to(DEV)
    dl_in = (torch.randn(T, E, generator=g) * 0.01).to(DEV) if d_logits else None
    d_aux = torch.tensor([0.7], device=DEV) if aux else None
    st = stats if aux else None
    S = T * k
    s = _lib.stream_of(x)
    dy1 = torch.empty(S, H, dtype=BF, device=DEV)
    dw1 = torch.empty(T, k, device=DEV)
    dl1 = torch.empty(T, E, dtype=BF, device=DEV)
    _lib.call("moe_combine_bwd", _lib.ptr(d_out), _lib.ptr(y), _lib.ptr(pos), _lib.ptr(offsets), E,
              _lib.ptr(scores), T, H, k, _lib.ptr(dy1), _lib.ptr(dw1), s)
    if bf16:
        _lib.call("moe_router_bf16_logits_bwd", _lib.ptr(logits), _lib.ptr(ids), _lib.ptr(dw1), _lib.ptr(dl_in),
                  _lib.ptr(tw), _lib.ptr(st), _lib.ptr(d_aux), T, E, k, int(norm), _lib.ptr(dl1), s)
    elif aux:
        _lib.call("moe_router_aux_bwd_bf16", _lib.ptr(logits), _lib.ptr(ids), _lib.ptr(dw1), _lib.ptr(dl_in),
                  _lib.ptr(tw), _lib.ptr(st), _lib.ptr(d_aux), T, E, k, int(norm), _lib.ptr(dl1), s)
    else:
        _lib.call("moe_router_topk_bwd_bf16", _lib.ptr(logits), _lib.ptr(ids), _lib.ptr(dw1), _lib.ptr(dl_in), T, E,
                  k, int(norm), _lib.ptr(dl1), s)
    for with_scores in (True, False):
        dy2 = torch.full((S, H), float("nan"), dtype=BF, device=DEV)
        dw2 = torch.full((T, k), float("nan"), device=DEV)
        dl2 = torch.full((T, E), float("nan"), dtype=BF, device=DEV)
        _lib.call("moe_combine_router_bwd", _lib.ptr(d_out), _lib.ptr(y), _lib.ptr(pos), _lib.ptr(offsets), E,
                  _lib.ptr(scores), T, H, k, _lib.ptr(dy2), _lib.ptr(dw2) if with_scores else None, _lib.ptr(logits),
                  _lib.ptr(ids), _lib.ptr(dl_in), _lib.ptr(tw), _lib.ptr(st), _lib.ptr(d_aux), E, int(norm),
                  int(bf16), _lib.ptr(dl2), s)
        torch.cuda.synchronize()
        assert torch.equal(dy2, dy1), "d_y"
        assert torch.equal(dl2, dl1), "d_logits"
        if with_scores:
            assert torch.equal(dw2, dw1), "d_scores"
        else:
            assert torch.isnan(dw2).all(), "d_scores written although not asked for"

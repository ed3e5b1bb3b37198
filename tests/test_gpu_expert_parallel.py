"""Expert parallelism on the GPU: both hook runtimes installed on a model of
SparseMoeBlock layers, one rank's share at a time, on the kernels; the
dispatcher's owner-major send buffer against the oracle's restatement of
TokenDispatcher.dispatch (token_dispatch.py:101-125), bit for bit."""

import numpy as np
import pytest
import torch
from torch import nn

from conftest import GOLDEN, close_bf16
from oracle import moe_oracle as O
from parallel_amd import (
    ExpertPartition,
    Experts,
    ReplicatedTokenExpertParallel,
    SequenceParallelExpertParallel,
    SparseMoeBlock,
    TokenDispatcher,
    ops,
    verify_expert_modules,
)
from parallel_amd.workloads import WORKLOADS, make_block_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


class _Layer(nn.Module):
    def __init__(self, block):
        super().__init__()
        self.mlp = block


def ep_model(w, inp, ep, rank, layers=2):
    """A model whose decoder layers hold SparseMoeBlocks with the full router
    and rank ``rank``'s slice of the experts (dim-0 EXPERT placement,
    parallel/parallel/engine/model_parallel/models/qwen3_moe.py:64-65,81-84)."""
    part = ExpertPartition(w.experts, ep, rank)
    cfg = w.config()
    local_cfg = w.config()
    local_cfg.num_experts = part.local_count
    model = nn.Module()
    model.layers = nn.ModuleList()
    for _ in range(layers):
        block = SparseMoeBlock(cfg)
        block.experts = Experts(local_cfg)
        with torch.no_grad():
            block.gate.weight.copy_(inp["router_weight"])
            block.experts.gate_up_proj.copy_(inp["gate_up_proj"][part.start:part.stop])
            block.experts.down_proj.copy_(inp["down_proj"][part.start:part.stop])
        model.layers.append(_Layer(block))
    return model.to(DEV, BF), part


def run_share(runtime_cls, w, inp, ep, rank, layers=2):
    """Forward + backward of <block(x), d_out> through the first layer of the
    model with ``runtime_cls`` installed for (ep, rank)."""
    model, part = ep_model(w, inp, ep, rank, layers)
    verify_expert_modules(model, part)
    rt = runtime_cls(part, None)
    rt.apply(model)
    x = inp["x"].to(DEV).view(1, w.tokens, w.hidden).requires_grad_()
    block = model.layers[0].mlp
    out = block(x)
    out.backward(inp["d_out"].to(DEV).view_as(out))
    torch.cuda.synchronize()
    rt.close()
    return out.detach().view(w.tokens, w.hidden), x.grad.view(w.tokens, w.hidden), block.gate.weight.grad


@pytest.mark.parametrize("runtime_cls", [ReplicatedTokenExpertParallel, SequenceParallelExpertParallel])
def test_ep2_shares_against_golden_and_oracle(runtime_cls):
    """C1 block at ep = 2: rank 0's share equals transformers' experts on the
    localized routes (golden sentinel_out); each rank's share equals the
    oracle's experts on that rank's localized routes; the shares' outputs,
    input gradients and router gradients sum to the unsharded block's."""
    w = WORKLOADS["c1"]
    inp = make_block_inputs(w, seed=1234, dtype=BF)
    ref = O.block_forward_backward(inp["x"], inp["router_weight"], inp["gate_up_proj"], inp["down_proj"],
                                   inp["d_out"], top_k=w.top_k, norm_topk_prob=w.norm_topk_prob, aux_coef=0.0)
    g = np.load(GOLDEN / "c1_qwen3_moe_block.npz")
    ep = 2
    outs, dxs, drs = [], [], []
    for rank in range(ep):
        out, dx, dr = run_share(runtime_cls, w, inp, ep, rank)
        part = ExpertPartition(w.experts, ep, rank)
        li, ls, _ = part.localize_routes(ref["indices"], ref["scores"])
        want = O.experts_grouped(inp["x"].float(), li, ls, inp["gate_up_proj"][part.start:part.stop].float(),
                                 inp["down_proj"][part.start:part.stop].float())
        close_bf16(out, want, f"rank {rank} share")
        if rank == 0:
            close_bf16(out, torch.from_numpy(g["sentinel_out"]), "rank 0 share vs transformers")
        outs.append(out.float().cpu())
        dxs.append(dx.float().cpu())
        drs.append(dr.float().cpu())
    close_bf16(sum(outs), ref["out"], "sum of shares")
    close_bf16(sum(dxs), ref["dx"], "sum of input gradients")
    close_bf16(sum(drs), ref["d_router"], "sum of router gradients")


def test_both_runtimes_give_the_same_share():
    """The replicated-token and the dispatch runtimes compute the same rank
    share by different kernel sequences (sentinel slots skipped in place,
    against owner-major dispatch and gather-form combine)."""
    w = WORKLOADS["c1"]
    inp = make_block_inputs(w, seed=77, dtype=BF)
    for ep, rank in ((4, 1), (8, 7)):
        a = run_share(ReplicatedTokenExpertParallel, w, inp, ep, rank)
        b = run_share(SequenceParallelExpertParallel, w, inp, ep, rank)
        for name, x, y in zip(("out", "dx", "d_router"), a, b):
            close_bf16(x, y, f"ep {ep} rank {rank} {name}")


@pytest.mark.parametrize("T,E,local,seed,k,H", [(512, 128, 16, 0, 4, 64), (1000, 64, 8, 1, 4, 64), (37, 16, 4, 2, 4, 64),
                                                 (256, 8, 1, 3, 4, 64),
                                                 # the C2 layer's send side at ep = 8 and ep = 2
                                                 (4096, 128, 16, 4, 8, 2048), (4096, 128, 64, 5, 8, 2048)])
def test_dispatch_send_buffer_bit_exact(T, E, local, seed, k, H):
    """ops.dispatch_fwd at ep = E / local equals TokenDispatcher.dispatch's send
    side (the oracle's restatement) bit for bit: rows, local expert ids,
    scores, source tokens and splits."""
    k = min(k, E)
    g = torch.Generator().manual_seed(seed)
    hidden = torch.randn(T, H, generator=g).to(BF)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    scores = torch.rand(T, k, generator=g)
    ep = E // local
    sh, se, ss, src, pos, counts = ops.dispatch_fwd(hidden.to(DEV), idx.to(DEV), scores.to(DEV), local, ep)
    rh, re, rs, rsrc, rsplits = O.dispatch_send(hidden, idx, scores, local, ep)
    assert torch.equal(sh.cpu(), rh)
    assert torch.equal(se.cpu(), re)
    assert torch.equal(ss.cpu(), rs)
    assert torch.equal(src.cpu(), rsrc)
    assert tuple(counts.cpu().tolist()) == rsplits
    # pos_of_slot is the inverse of the send order
    assert torch.equal(src.cpu()[pos.cpu().long()], torch.arange(T).repeat_interleave(k))


def test_sp_runtime_c2_layer_ep2_shares_sum_to_the_block():
    """The dispatch runtime on the C2 layer (H 2048, 128 experts, top-8, I 768,
    4096 tokens) at ep = 2, each rank's share in turn (64 local experts, about
    16k routed rows each): the shares' outputs, input gradients and router
    gradients sum to the unsharded block's (ep = 1, same runtime); the block
    and each share equal the oracle's experts on 48 sampled tokens, on the
    block's own routes localized to the share
    (expert_parallel.py:124-231; the reference's tests/test_model_parallel.py:309-339)."""
    w = WORKLOADS["c2"]
    inp = make_block_inputs(w, seed=41, device=DEV, dtype=BF, weights_on_device_rng=True)
    full = run_share(SequenceParallelExpertParallel, w, inp, 1, 0, layers=1)
    shares = [run_share(SequenceParallelExpertParallel, w, inp, 2, r, layers=1) for r in range(2)]
    for i, name in enumerate(("out", "dx", "d_router")):
        close_bf16(shares[0][i].float() + shares[1][i].float(), full[i], f"c2 ep2 sum of {name}")
    x = inp["x"]
    _, scores, idx = ops.router_fwd(x, inp["router_weight"], w.top_k, w.norm_topk_prob)
    sample = torch.randperm(w.tokens, generator=torch.Generator().manual_seed(5))[:48]
    xs, ids, scs = x.cpu()[sample], idx.cpu()[sample], scores.cpu()[sample]
    gu, dn = inp["gate_up_proj"].cpu(), inp["down_proj"].cpu()
    close_bf16(full[0].cpu()[sample], O.experts_grouped(xs, ids, scs, gu, dn), "c2 block, sampled tokens")
    for rank in range(2):
        part = ExpertPartition(w.experts, 2, rank)
        li, ls, _ = part.localize_routes(ids, scs)
        want = O.experts_grouped(xs, li, ls, gu[part.start:part.stop], dn[part.start:part.stop])
        close_bf16(shares[rank][0].cpu()[sample], want, f"c2 rank {rank} share, sampled tokens")


@pytest.mark.parametrize("rank", [0, 1])
def test_zero_receive_dispatch_through_the_experts(rank):
    """The reference's zero-receive case (its tests/test_sequence_parallel.py:17-73)
    on the kernels: ep = 2 and every route owned by rank 0.  Rank 1's share
    receives no rows; dispatch, the experts on the empty receive buffer and
    the combine run without a launch error and give zero output, zero input
    and score gradients and zero weight gradients.  Rank 0's share receives
    every route and equals the oracle's experts, backward included."""
    T, H, k, E, I = 96, 64, 2, 4, 32
    g = torch.Generator().manual_seed(31)
    part = ExpertPartition(E, 2, rank)
    x = torch.randn(T, H, generator=g).to(BF)
    raw = torch.rand(T, k, generator=g) + 0.1
    sc = raw / raw.sum(1, keepdim=True)
    indices = torch.stack([torch.randperm(E // 2, generator=g)[:k] for _ in range(T)])  # all on rank 0
    gu_all = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(BF)
    dn_all = (torch.randn(E, H, I, generator=g) * 0.05).to(BF)
    hidden = x.to(DEV).requires_grad_()
    scores = sc.to(DEV).requires_grad_()
    gu = gu_all[part.start:part.stop].to(DEV).requires_grad_()
    dn = dn_all[part.start:part.stop].to(DEV).requires_grad_()
    dispatcher = TokenDispatcher(part, None)
    received, local_idx, received_scores, state = dispatcher.dispatch(hidden, indices.to(DEV), scores)
    assert local_idx.shape == (T * k if rank == 0 else 0, 1)
    assert state.send_splits == (T * k, 0) and state.receive_splits == ((T * k, 0) if rank == 0 else (0, 0))
    y = ops.experts(received, local_idx, received_scores, gu, dn)
    combined = dispatcher.combine(y, state)
    combined.float().square().sum().backward()
    torch.cuda.synchronize()
    if rank == 1:
        assert received.shape == (0, H) and y.shape == (0, H)
        assert not combined.any(), "a share that receives nothing returns zeros"
        for name, t in (("hidden", hidden), ("scores", scores), ("gate_up_proj", gu), ("down_proj", dn)):
            assert t.grad is not None and not t.grad.any(), f"{name}: gradient of an empty share must be zero"
        return
    leaves = [t.clone().float().requires_grad_() for t in (x, sc, gu_all[:E // 2], dn_all[:E // 2])]
    ref = O.experts_grouped(leaves[0], indices, leaves[1], leaves[2], leaves[3])
    ref.square().sum().backward()
    close_bf16(combined, ref, "rank 0 combined")
    for name, a, b in zip(("hidden", "scores", "gate_up_proj", "down_proj"), (hidden, scores, gu, dn), leaves):
        close_bf16(a.grad, b.grad, f"rank 0 d_{name}")

"""The block step (moe_block forward and backward) captured into a HIP graph
and replayed: every replay gives the eager step's bits, with eager work and
synchronisations between the replays."""

import pytest
import torch

from parallel_amd import ops
from parallel_amd.workloads import WORKLOADS, make_block_inputs, scaled

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
KEYS = ("out", "aux", "dx", "d_router", "d_gate_up", "d_down")


def test_moe_block_step_replays_from_a_hip_graph():
    w = scaled(WORKLOADS["c2"], 1024)
    inp = {k: v.to(DEV) for k, v in make_block_inputs(w, seed=16, dtype=BF).items()}
    coef = torch.tensor(w.aux_coef, device=DEV)
    leaves = [inp[n].clone().requires_grad_() for n in ("x", "router_weight", "gate_up_proj", "down_proj")]

    def step():
        for p in leaves:
            p.grad = None
        out, _, _, _, aux = ops.moe_block(*leaves, w.top_k, w.norm_topk_prob)
        torch.autograd.backward([out, aux], [inp["d_out"], coef])
        return out, aux

    def snapshot(out, aux):
        return dict(out=out.detach().clone(), aux=aux.detach().clone(), dx=leaves[0].grad.clone(),
                    d_router=leaves[1].grad.clone(), d_gate_up=leaves[2].grad.clone(), d_down=leaves[3].grad.clone())

    eager = snapshot(*step())
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the default stream, as capture requires
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    for p in leaves:
        p.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, _, _, _, aux = ops.moe_block(*leaves, w.top_k, w.norm_topk_prob)
        torch.autograd.backward([out, aux], [inp["d_out"], coef])
    grads = [p.grad for p in leaves]
    for replay in range(3):
        # eager work between replays, then the replay, checked against the eager step
        scratch = ops.moe_block(*[t.detach() for t in leaves], w.top_k, w.norm_topk_prob)[0]
        torch.cuda.synchronize()
        del scratch
        graph.replay()
        torch.cuda.synchronize()
        got = dict(out=out, aux=aux, dx=grads[0], d_router=grads[1], d_gate_up=grads[2], d_down=grads[3])
        for key in KEYS:
            assert torch.equal(got[key], eager[key]), f"replay {replay}: {key}"

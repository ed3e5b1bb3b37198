"""CPU tests of the expert-parallel layer: ownership, route localization, the
one-process exchange of a rank's share, and the hook runtimes' plumbing and
errors (on stand-in modules; the GPU tests run them on the kernels)."""

import pytest
import torch
from torch import nn

from oracle import moe_oracle as O
from parallel_amd import (
    ExpertPartition,
    ReplicatedTokenExpertParallel,
    SequenceParallelExpertParallel,
    local_expert_range,
    variable_all_to_all,
    verify_expert_modules,
)


def test_localize_routes_known_answer_and_oracle():
    # parallel tests/test_model_parallel.py:140-147
    p = ExpertPartition(num_experts=8, ep_size=2, ep_rank=1)
    li, ls, m = p.localize_routes(torch.tensor([[0, 6], [4, 3]]), torch.tensor([[0.2, 0.8], [0.7, 0.3]]))
    assert li.tolist() == [[4, 2], [0, 4]] and m.tolist() == [[False, True], [True, False]]
    torch.testing.assert_close(ls, torch.tensor([[0.0, 0.8], [0.7, 0.0]]))
    # every rank of several partitions against the oracle's floor-division owner rule, including ids
    # outside [0, E) (never local)
    g = torch.Generator().manual_seed(0)
    for E, ep in ((8, 1), (8, 2), (12, 3), (128, 8)):
        idx = torch.randint(-3, E + 3, (50, 4), generator=g)
        sc = torch.rand(50, 4, generator=g)
        for r in range(ep):
            got = ExpertPartition(E, ep, r).localize_routes(idx, sc)
            want = O.localize_routes(idx, sc, E, ep, r)
            for a, b in zip(got, want):
                assert torch.equal(a, b)
        assert list(local_expert_range(E, ep, ep - 1)) == list(range(E - E // ep, E))


def test_localized_scores_pass_gradient_only_for_local_routes():
    p = ExpertPartition(8, 2, 0)
    sc = torch.rand(3, 2, requires_grad=True)
    _, ls, m = p.localize_routes(torch.tensor([[1, 5], [7, 0], [3, 3]]), sc)
    ls.sum().backward()
    assert torch.equal(sc.grad, m.float())


def test_owner_is_floor_division():
    p = ExpertPartition(8, 2, 0)
    assert p.owner(torch.tensor([-1, 0, 3, 4, 7, 8])).tolist() == [-1, 0, 0, 1, 1, 2]


def test_one_process_exchange_of_a_share():
    """Rank 1 of 3: keeps its self block on dispatch, pads absent ranks' rows
    with zeros on the way back; the gradient is the reverse exchange."""
    value = torch.arange(12.0).view(6, 2).requires_grad_()
    send, recv = (2, 3, 1), (0, 3, 0)
    got = variable_all_to_all(value, send, recv, None, rank=1)
    assert got.tolist() == [[4.0, 5.0], [6.0, 7.0], [8.0, 9.0]]
    back = variable_all_to_all(got * 10, recv, send, None, rank=1)
    assert back[:2].abs().sum() == 0 and back[5].abs().sum() == 0 and torch.equal(back[2:5], got * 10)
    back.sum().backward()
    assert value.grad.tolist() == [[0.0, 0.0]] * 2 + [[10.0, 10.0]] * 3 + [[0.0, 0.0]]
    assert variable_all_to_all(value, (6,), (6,), None) is value
    with pytest.raises(ValueError, match="rank"):
        variable_all_to_all(value, send, recv, None)
    with pytest.raises(ValueError, match="expects"):
        variable_all_to_all(value, send, (0, 2, 0), None, rank=1)
    with pytest.raises(ValueError, match="cover"):
        variable_all_to_all(value, (2, 2, 1), recv, None, rank=1)


class _Router(nn.Module):
    def __init__(self, idx, scores):
        super().__init__()
        self.idx, self.scores = idx, scores

    def forward(self, x):
        return torch.zeros(x.shape[0], 8), self.scores, self.idx


class _Experts(nn.Module):
    def __init__(self, num_experts):
        super().__init__()
        self.num_experts = num_experts
        self.seen = []

    def forward(self, hidden, idx, weights):
        self.seen.append((idx, weights))
        return hidden


class _Mlp(nn.Module):
    def __init__(self, idx, scores, local):
        super().__init__()
        self.gate = _Router(idx, scores)
        self.experts = _Experts(local)

    def forward(self, x):
        _, s, i = self.gate(x)
        return self.experts(x, i, s)


class _Layer(nn.Module):
    def __init__(self, *a):
        super().__init__()
        self.mlp = _Mlp(*a)


def _model(n_layers=2, local=4):
    idx = torch.tensor([[0, 6], [4, 3]])
    sc = torch.tensor([[0.2, 0.8], [0.7, 0.3]])
    m = nn.Module()
    m.layers = nn.ModuleList(_Layer(idx, sc, local) for _ in range(n_layers))
    return m


def test_replicated_token_runtime_localizes_router_outputs():
    model = _model()
    rt = ReplicatedTokenExpertParallel(ExpertPartition(8, 2, 1), None)
    rt.apply(model)
    with pytest.raises(RuntimeError, match="already installed"):
        rt.apply(model)
    model.layers[0].mlp(torch.zeros(2, 3))
    idx, w = model.layers[0].mlp.experts.seen[-1]
    assert idx.tolist() == [[4, 2], [0, 4]]
    torch.testing.assert_close(w, torch.tensor([[0.0, 0.8], [0.7, 0.0]]))
    rt.close()
    model.layers[0].mlp(torch.zeros(2, 3))
    assert model.layers[0].mlp.experts.seen[-1][0].tolist() == [[0, 6], [4, 3]], "close() removes the hooks"
    rt.apply(model)  # re-installable after close
    rt.close()


def test_runtime_errors():
    with pytest.raises(RuntimeError, match="routers"):
        bad = _model()
        del bad.layers[1].mlp.gate
        ReplicatedTokenExpertParallel(ExpertPartition(8, 2, 0), None).apply(bad)
    with pytest.raises(RuntimeError, match="no"):
        SequenceParallelExpertParallel(ExpertPartition(8, 2, 0), None).apply(nn.Linear(2, 2))
    sp = SequenceParallelExpertParallel(ExpertPartition(8, 2, 0), None)
    with pytest.raises(RuntimeError, match="dispatch"):
        sp._combine(nn.Linear(2, 2), (), torch.zeros(1))


def test_verify_expert_modules():
    verify_expert_modules(_model(local=4), ExpertPartition(8, 2, 0))
    with pytest.raises(RuntimeError, match="4 local experts.*layers.0.mlp.experts=8"):
        verify_expert_modules(_model(local=8), ExpertPartition(8, 2, 0))
    with pytest.raises(RuntimeError, match="no"):
        verify_expert_modules(nn.Linear(2, 2), ExpertPartition(8, 2, 0))


def test_partition_errors():
    for args, match in (((8, 0, 0), "positive"), ((8, 2, 2), "outside"), ((8, 2, -1), "outside"),
                        ((6, 4, 0), "divisible")):
        with pytest.raises(ValueError, match=match):
            ExpertPartition(*args)

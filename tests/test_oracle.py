"""Pins the CPU oracle: golden vectors from transformers' own Qwen3-MoE block,
the reference's known-answer tests, closed forms and brute force."""

import itertools

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import moe_oracle as O
from parallel_amd.workloads import WORKLOADS, Workload, make_block_inputs

CASES = {
    "c1": (WORKLOADS["c1"], 1234),
    "tiny": (Workload("tiny", 1, 48, 64, 4, 2, 16, norm_topk_prob=False, aux_coef=0.01, dtype="fp32"), 7),
}


@pytest.fixture(scope="module", params=sorted(CASES))
def golden_case(request):
    w, seed = CASES[request.param]
    g = dict(np.load(GOLDEN / f"{request.param}_qwen3_moe_block.npz"))
    inp = {k: v.float() for k, v in make_block_inputs(w, seed=seed, dtype=torch.bfloat16).items()}
    res = O.block_forward_backward(
        inp["x"], inp["router_weight"], inp["gate_up_proj"], inp["down_proj"], inp["d_out"], top_k=w.top_k,
        norm_topk_prob=w.norm_topk_prob, aux_coef=w.aux_coef)
    return w, inp, g, res


def test_oracle_matches_transformers_forward(golden_case):
    w, inp, g, res = golden_case
    np.testing.assert_allclose(res["logits"].numpy(), g["logits"], rtol=1e-5, atol=1e-6)
    assert np.array_equal(res["indices"].numpy(), g["indices"]), "routing indices differ from transformers"
    np.testing.assert_allclose(res["scores"].numpy(), g["scores"], rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(res["out"].numpy(), g["out"], rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(float(res["aux"]), float(g["aux"]), rtol=1e-6)


def test_oracle_matches_transformers_gradients(golden_case):
    w, inp, g, res = golden_case
    for key in ("dx", "d_router", "d_gate_up", "d_down"):
        ref = g[key]
        got = res[key].numpy()
        scale = np.abs(ref).max()
        assert np.abs(got - ref).max() <= 1e-4 * scale + 1e-7, f"{key}: {np.abs(got - ref).max()} vs scale {scale}"


def test_oracle_sentinel_routes_match_transformers(golden_case):
    w, inp, g, _ = golden_case
    half = w.experts // 2
    idx = torch.from_numpy(g["sentinel_local_idx"])
    scores = torch.from_numpy(g["scores"]).masked_fill(idx == half, 0)
    out = O.experts_grouped(inp["x"], idx, scores, inp["gate_up_proj"][:half], inp["down_proj"][:half])
    np.testing.assert_allclose(out.numpy(), g["sentinel_out"], rtol=1e-4, atol=1e-5)


def test_grouped_and_eager_experts_agree():
    gen = torch.Generator().manual_seed(3)
    T, H, E, k, I = 40, 32, 6, 3, 16
    x = torch.randn(T, H, generator=gen)
    idx = torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(T)])
    idx[5] = torch.tensor([0, 1, 2])
    w = torch.rand(T, k, generator=gen)
    gu = torch.randn(E, 2 * I, H, generator=gen) * 0.1
    dn = torch.randn(E, H, I, generator=gen) * 0.1
    a = O.experts_grouped(x, idx, w, gu, dn)
    b = O.experts_eager(x, idx, w, gu, dn)
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


def test_experts_gradients_match_finite_differences():
    gen = torch.Generator().manual_seed(5)
    T, H, E, k, I = 6, 4, 3, 2, 3
    x = torch.randn(T, H, generator=gen, dtype=torch.float64, requires_grad=True)
    idx = torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(T)])
    w = torch.rand(T, k, generator=gen, dtype=torch.float64, requires_grad=True)
    gu = (torch.randn(E, 2 * I, H, generator=gen, dtype=torch.float64) * 0.5).requires_grad_()
    dn = (torch.randn(E, H, I, generator=gen, dtype=torch.float64) * 0.5).requires_grad_()

    def f(x, w, gu, dn):
        return O.experts_grouped(x, idx, w, gu, dn, compute_dtype=torch.float64)

    assert torch.autograd.gradcheck(f, (x, w, gu, dn), eps=1e-6, atol=1e-6)


def test_stable_permutation_matches_brute_force():
    rng = np.random.default_rng(0)
    for S, E, div, nb in [(0, 4, 1, 4), (1, 4, 1, 4), (37, 5, 1, 5), (64, 8, 4, 2), (100, 3, 1, 2)]:
        ids = rng.integers(0, E, size=S)
        perm, pos, counts, offsets = O.stable_permutation(ids, div, nb)
        keys = [min(i // div, nb) for i in ids]
        brute = [s for b in range(nb + 1) for s in range(S) if keys[s] == b]
        assert perm.tolist() == brute
        assert all(pos[perm[p]] == p for p in range(S))
        assert counts.tolist() == [keys.count(b) for b in range(nb)]
        assert offsets.tolist() == list(itertools.accumulate(counts.tolist())) if nb else True


def test_stable_permutation_matches_torch_stable_sort():
    ids = torch.randint(0, 128, (32768,), generator=torch.Generator().manual_seed(1))
    perm, pos, counts, offsets = O.stable_permutation(ids.numpy(), 1, 128)
    ref_vals, ref_perm = torch.sort(ids, stable=True)
    assert np.array_equal(perm, ref_perm.numpy())
    assert np.array_equal(counts, torch.bincount(ids, minlength=128).numpy())
    hist = torch.histc(ids.float(), bins=128, min=0, max=127)
    assert np.array_equal(offsets, torch.cumsum(hist, 0, dtype=torch.int32).numpy())


def test_localize_routes_known_answer():
    # parallel tests/test_model_parallel.py:140-147
    idx = torch.tensor([[0, 6], [4, 3]])
    sc = torch.tensor([[0.2, 0.8], [0.7, 0.3]])
    li, ls, m = O.localize_routes(idx, sc, num_experts=8, ep_size=2, ep_rank=1)
    assert li.tolist() == [[4, 2], [0, 4]]
    assert ls.tolist() == [[0.0, 0.800000011920929], [0.699999988079071, 0.0]]
    assert m.tolist() == [[False, True], [True, False]]


def test_dispatch_combine_round_trip_closed_form():
    # One-rank analogue of parallel tests/test_sequence_parallel.py:17-73: with scores
    # summing to one, combine(dispatch(h) * s) == h, dh = 2h and ds = 2 * sum(h^2).
    hidden = (torch.arange(6, dtype=torch.float32).reshape(2, 3)).requires_grad_()
    scores = torch.tensor([[0.25, 0.75], [0.6, 0.4]], requires_grad=True)
    indices = torch.tensor([[0, 1], [1, 0]])
    sh, se, ss, src, splits = O.dispatch_send(hidden, indices, scores, local_count=4, ep_size=1)
    assert splits == (4,) and se.tolist() == [0, 1, 1, 0]
    combined = O.combine_index_add(sh * ss.unsqueeze(-1), src, 2)
    torch.testing.assert_close(combined, hidden)
    combined.square().sum().backward()
    torch.testing.assert_close(hidden.grad, 2 * hidden.detach())
    torch.testing.assert_close(scores.grad, 2 * hidden.detach().square().sum(-1, keepdim=True).expand_as(scores))


def test_dispatch_owner_order_is_stable():
    idx = torch.tensor([[5, 0], [2, 7], [4, 1]])
    sc = torch.rand(3, 2)
    sh, se, ss, src, splits = O.dispatch_send(torch.randn(3, 4), idx, sc, local_count=4, ep_size=2)
    # owner 0: slots 1 (e0), 2 (e2), 5 (e1); owner 1: slots 0 (e5), 3 (e7), 4 (e4)
    assert src.tolist() == [0, 1, 2, 0, 1, 2]
    assert se.tolist() == [0, 2, 1, 1, 3, 0]
    assert splits == (3, 3)


def test_aux_loss_is_top_k_for_balanced_routing():
    E, k, T = 8, 2, 64
    gen = torch.Generator().manual_seed(0)
    logits = torch.randn(T, E, generator=gen) * 0.1
    for t in range(T):  # token t prefers experts 2t, 2t+1 (mod E): counts are perfectly balanced
        logits[t, (2 * t) % E] += 5.0
        logits[t, (2 * t + 1) % E] += 4.0
    aux = O.load_balancing_loss((logits,), E, k)
    torch.testing.assert_close(aux, torch.tensor(float(k)), rtol=1e-6, atol=1e-6)


def test_aux_loss_mask_of_ones_equals_unmasked():
    logits = torch.randn(2 * 6, 5, generator=torch.Generator().manual_seed(2))
    mask = torch.ones(2, 6)
    a = O.load_balancing_loss((logits,), 5, 2)
    b = O.load_balancing_loss((logits,), 5, 2, attention_mask=mask)
    torch.testing.assert_close(a, b)


# ------------------------------------------------------------- tie detection


def _ties_brute_force(probs: torch.Tensor, k: int) -> list[bool]:
    """A token's top-k depends on how exact ties are broken iff some value is
    held by two or more experts and fewer than k experts are strictly larger
    (then at least one holder is selected and another holder's place is
    ambiguous).  Counted pairwise, without sorting."""
    out = []
    for row in probs.tolist():
        tied = False
        for v in row:
            larger = sum(1 for u in row if u > v)
            equal = sum(1 for u in row if u == v)
            tied |= equal >= 2 and larger < k
        out.append(tied)
    return out


def test_topk_ties_constructed_cases():
    E = 8
    rows = {
        "none": [3.0, 2.5, 2.0, 1.5, 1.0, 0.5, 0.0, -0.5],
        "boundary": [3.0, 2.5, 2.0, 2.0, 1.0, 0.5, 0.0, -0.5],  # 3rd == 4th with k = 3
        "inside": [3.0, 3.0, 2.0, 1.5, 1.0, 0.5, 0.0, -0.5],  # 1st == 2nd
        "below": [3.0, 2.5, 2.0, 1.0, 1.0, 0.5, 0.0, -0.5],  # 4th == 5th: outside the top 3 and its boundary
        "last_pair": [3.0, 2.5, 2.0, 1.5, 1.0, 0.5, -1.0, -1.0],
        "all_equal": [0.0] * E,
    }
    logits = torch.tensor(list(rows.values()))
    for k, expect in ((3, [False, True, True, False, False, True]), (8, [False, True, True, True, True, True]),
                      (7, [False, True, True, True, True, True]), (1, [False, False, True, False, False, True])):
        idx = torch.zeros(len(rows), k, dtype=torch.long)
        got = O.topk_ties(logits, idx).tolist()
        assert got == expect, f"k={k}: {dict(zip(rows, got))}"
        assert got == _ties_brute_force(torch.softmax(logits, -1), k), f"k={k}: brute force disagrees"


def test_topk_ties_matches_brute_force_on_random_and_planted_ties():
    g = torch.Generator().manual_seed(11)
    T, E = 400, 12
    logits = torch.randn(T, E, generator=g)
    # plant exact ties at random sorted positions in a third of the tokens
    for t in range(0, T, 3):
        order = torch.argsort(logits[t], descending=True)
        a = int(torch.randint(0, E - 1, (1,), generator=g))
        logits[t, order[a + 1]] = logits[t, order[a]]
    probs = torch.softmax(logits, -1)
    for k in (1, 2, 4, 8, 11, 12):
        got = O.topk_ties(logits, torch.zeros(T, k, dtype=torch.long))
        assert got.tolist() == _ties_brute_force(probs, k), f"k={k}"
        assert 0 < int(got.sum()) <= len(range(0, T, 3)), "only planted ties are flagged"
    # continuous random logits carry no exact ties at the benchmark's router shape
    big = torch.randn(4096, 128, generator=g)
    assert not O.topk_ties(big, torch.zeros(4096, 8, dtype=torch.long)).any()


# ------------------------------------------------------------ the CPU baseline


def test_reference_step_equals_block_forward_backward():
    """reference_step (the CPU baseline: F.grouped_mm on existing leaves) gives
    the block's outputs and gradients, in fp32 and, at bf16's tolerance, in bf16."""
    w = WORKLOADS["c1"]
    inp = {k: v.float() for k, v in make_block_inputs(w, seed=1234, dtype=torch.bfloat16).items()}
    ref = O.block_forward_backward(inp["x"], inp["router_weight"], inp["gate_up_proj"], inp["down_proj"],
                                   inp["d_out"], top_k=w.top_k, norm_topk_prob=w.norm_topk_prob, aux_coef=w.aux_coef)
    for dtype, tol in ((torch.float32, 1e-5), (torch.bfloat16, 2e-2)):
        leaves = O.make_leaves(*(inp[k].to(dtype) for k in ("x", "router_weight", "gate_up_proj", "down_proj")))
        for _ in range(2):  # a second step on the same leaves starts from cleared gradients
            out = O.reference_step(leaves, inp["d_out"], top_k=w.top_k, norm_topk_prob=w.norm_topk_prob,
                                   aux_coef=w.aux_coef, compute_dtype=dtype)
        pairs = [("out", out, ref["out"])] + [(n, l.grad, ref[n]) for n, l in
                                              zip(("dx", "d_router", "d_gate_up", "d_down"), leaves)]
        for name, got, want in pairs:
            err = float((got.float() - want).abs().max() / want.abs().max())
            assert err <= tol, f"{dtype} {name}: max rel err {err:.2e}"


@pytest.mark.parametrize("case", ["small", "c2"])
def test_aux_loss_masked_branch_matches_transformers_golden(case):
    """The attention-mask branch over several layers (layer-major logits, the
    [batch, seq] mask expanded per layer and per top-k slot) against
    transformers' own load_balancing_loss_func, forward and gradient."""
    g = np.load(GOLDEN / "aux_masked.npz")
    layers, batch, seq, E, k, _ = g[f"{case}_meta"].tolist()
    leaves = [torch.from_numpy(l).clone().requires_grad_() for l in g[f"{case}_logits"]]
    mask = torch.from_numpy(g[f"{case}_mask"])
    assert 0 < int((mask == 0).sum()) < mask.numel()
    aux = O.load_balancing_loss(tuple(leaves), E, k, attention_mask=mask)
    aux.backward()
    np.testing.assert_allclose(float(aux), float(g[f"{case}_aux"]), rtol=1e-6)
    got = np.stack([l.grad.numpy() for l in leaves])
    np.testing.assert_allclose(got, g[f"{case}_d_logits"], rtol=1e-5, atol=1e-9)
    unmasked = O.load_balancing_loss(tuple(l.detach() for l in leaves), E, k)
    np.testing.assert_allclose(float(unmasked), float(g[f"{case}_aux_unmasked"]), rtol=1e-6)
    # the mask matters: dropping it changes the loss
    assert abs(float(aux) - float(unmasked)) > 1e-4

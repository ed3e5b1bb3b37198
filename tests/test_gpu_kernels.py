"""Per-kernel parity on the GPU, through the C-ABI ops, against the CPU oracle
(integers bit-exact) and plain fp32 torch references (floating point)."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import close_bf16, routing_check
from oracle import moe_oracle as O
from parallel_amd import _lib, ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def gen(seed):
    return torch.Generator().manual_seed(seed)


# ------------------------------------------------------------------- router

# E spans every experts-per-lane instantiation (1, 2, 4, 8, 16; 200 leaves the
# last lane chunk partly empty) and k the specialised (1, 2, 4, 6, 8) and the
# generic (3, 5, 16) forms.
ROUTER_CASES = [(512, 8, 2, True), (4096, 128, 8, True), (1000, 128, 8, False), (257, 64, 4, True),
                (64, 1024, 16, True), (33, 3, 3, False), (300, 200, 6, True), (128, 384, 1, False),
                (96, 512, 5, True)]


@pytest.mark.parametrize("T,E,k,norm", ROUTER_CASES)
def test_router_topk_bit_exact_on_same_logits(T, E, k, norm):
    logits = torch.randn(T, E, generator=gen(T + E))
    scores, idx = ops.router_topk(logits.to(DEV), k, norm)
    ref_scores, ref_idx = O.topk_softmax(logits, k, norm)
    routing_check(idx, ref_idx, logits)
    torch.testing.assert_close(scores.cpu(), ref_scores, rtol=2e-6, atol=1e-7)


def test_router_topk_ties_go_to_lower_index():
    logits = torch.zeros(4, 16)
    logits[1, 5] = 1.0
    scores, idx = ops.router_topk(logits.to(DEV), 4, False)
    assert idx[0].tolist() == [0, 1, 2, 3]
    assert idx[1].tolist() == [5, 0, 1, 2]
    torch.testing.assert_close(scores[0].cpu(), torch.full((4,), 1 / 16))


@pytest.mark.parametrize("T,H,E", [(512, 256, 8), (4096, 2048, 128), (300, 72, 24)])
def test_router_logits_match_fp32(T, H, E):
    x = torch.randn(T, H, generator=gen(1)).to(BF)
    w = (torch.randn(E, H, generator=gen(2)) * 0.02).to(BF)
    logits, scores, idx = ops.router_fwd(x.to(DEV), w.to(DEV), min(8, E), True)
    ref = O.router_logits(x, w)
    torch.testing.assert_close(logits.cpu(), ref, rtol=1e-4, atol=1e-5)
    ref_s, ref_i = O.topk_softmax(logits.cpu(), min(8, E), True)
    routing_check(idx, ref_i, logits)


# Many router weight-gradient partials, the last one ragged (512-row chunks:
# 18 at 9000 tokens, 34 at 17000).  E a multiple of 32 up to 128 with H a
# multiple of 32 takes the one-pass kernel: 64-column slices (C2: 8 chunks of
# 512 tokens; 9001 tokens: 29 chunks of 320, the last ragged), 32-column
# slices (H 96, 160, 2080), experts past E read as zeros (E 32, 96), fewer
# tokens than one 64-token sub-step (37).
@pytest.mark.parametrize("T,H,norm,E,k", [(384, 256, True, 16, 4), (384, 256, False, 16, 4), (384, 256, True, 200, 6),
                                          (384, 256, False, 384, 1), (9000, 264, True, 128, 8),
                                          (17000, 136, False, 64, 6), (4096, 2048, True, 128, 8),
                                          (9001, 512, True, 128, 8), (1000, 96, False, 96, 6), (37, 64, True, 32, 4),
                                          (300, 160, False, 64, 6), (2000, 2080, True, 128, 8)])
def test_router_backward_matches_autograd(T, H, norm, E, k):
    x = torch.randn(T, H, generator=gen(3)).to(BF)
    w = (torch.randn(E, H, generator=gen(4)) * 0.05).to(BF)
    d_scores = torch.randn(T, k, generator=gen(5))
    d_logits = torch.randn(T, E, generator=gen(6)) * 0.01
    xg = x.to(DEV).requires_grad_()
    wg = w.to(DEV).requires_grad_()
    logits, scores, idx = ops.router_fwd(xg, wg, k, norm)
    torch.autograd.backward([scores, logits], [d_scores.to(DEV), d_logits.to(DEV)])
    xr = x.float().requires_grad_()
    wr = w.float().requires_grad_()
    lr = O.router_logits(xr, wr)
    sr, ir = O.topk_softmax(lr, k, norm)
    assert torch.equal(ir, idx.cpu())
    torch.autograd.backward([sr, lr], [d_scores, d_logits])
    close_bf16(xg.grad, xr.grad, "router dx")
    close_bf16(wg.grad, wr.grad, "router dweight")


@pytest.mark.parametrize("T,H,E,accumulate", [(4096, 2048, 128, False), (9001, 512, 128, True), (1000, 96, 96, False),
                                               (37, 64, 32, True), (2000, 2080, 128, False), (300, 264, 64, False)])
def test_router_gemm_backward_is_the_exact_products(T, H, E, accumulate):
    """moe_router_logits_bwd through the C ABI on given bf16 dZ, X and Wr:
    every element of dX = dZ Wr and dWr = dZ^T X within one bf16 rounding of
    the fp64 product plus an fp32-summation bound (2^-16 of the sum of the
    terms' magnitudes), which a dropped token, sub-step or column tile
    exceeds; with dwr_accumulate, dWr = bf16(old + bf16(sum)).  Covers the
    one-pass kernel's 64- and 32-column slices, ragged token chunks and E < 128
    (H 264 takes the two-kernel path)."""
    g = gen(T + H)
    dz = (torch.randn(T, E, generator=g) * 0.1).to(BF)
    x = torch.randn(T, H, generator=g).to(BF)
    w = (torch.randn(E, H, generator=g) * 0.05).to(BF)
    old = (torch.randn(E, H, generator=g) * 0.01).to(BF)
    dzd, xd, wd = dz.to(DEV), x.to(DEV), w.to(DEV)
    dx = torch.full((T, H), float("nan"), dtype=BF, device=DEV)
    dw = old.to(DEV) if accumulate else torch.full((E, H), float("nan"), dtype=BF, device=DEV)
    lib = _lib.load()
    ws = torch.empty(max(lib.moe_router_logits_bwd_workspace_bytes(T, H, E), 16), dtype=torch.uint8, device=DEV)
    _lib.call("moe_router_logits_bwd", _lib.ptr(dzd), _lib.ptr(xd), _lib.ptr(wd), _lib.ptr(dx), _lib.ptr(dw),
              int(accumulate), T, H, E, _lib.ptr(ws), ws.numel(), _lib.stream_of(dzd))
    torch.cuda.synchronize()
    a, b, c = dz.double(), x.double(), w.double()
    for name, got, ref, mag, base in (("dX", dx, a @ c, a.abs() @ c.abs(), None),
                                      ("dWr", dw, a.t() @ b, a.abs().t() @ b.abs(), old if accumulate else None)):
        got = got.cpu().double()
        fresh = ref.to(BF).double()
        want = fresh if base is None else (base.double() + fresh).to(BF).double()
        # One bf16 ulp of the product (the fp32 sum may round the other way),
        # one of the accumulated result, and the fp32 summation error.
        bound = ref.abs() * 2.0 ** -7 + mag * 2.0 ** -16 + 1e-30
        if base is not None:
            bound = bound + want.abs() * 2.0 ** -7
        err = (got - want).abs()
        assert torch.isfinite(got).all(), f"{name}: non-finite (unwritten) elements"
        bad = err > bound
        assert not bad.any(), (f"{name}: {int(bad.sum())} elements outside the bound, worst at "
                               f"{np.unravel_index(int((err / bound).argmax()), tuple(err.shape))}")


# ------------------------------------------------------------------ aux loss


@pytest.mark.parametrize("T,E,k,masked", [(512, 8, 2, False), (4096, 128, 8, False), (2 * 96, 64, 6, True),
                                           (2 * 150, 200, 6, True), (256, 384, 1, False), (128, 1024, 16, False)])
def test_aux_loss_forward_backward(T, E, k, masked):
    logits = torch.randn(T, E, generator=gen(T)) * 2
    mask = None
    if masked:
        mask = (torch.rand(2, T // 2, generator=gen(9)) > 0.3).float()
    lg = logits.to(DEV).requires_grad_()
    tw = None if mask is None else mask.reshape(-1).to(DEV)
    aux, stats = ops.aux_loss_fwd(lg, tw, E, k)
    aux.backward(torch.tensor(0.7, device=DEV))
    lr = logits.clone().requires_grad_()
    ref = O.load_balancing_loss((lr,), E, k, attention_mask=mask)
    (0.7 * ref).backward()
    torch.testing.assert_close(aux.cpu(), ref.detach(), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(lg.grad.cpu(), lr.grad, rtol=1e-4, atol=1e-8)


@pytest.mark.parametrize("case", ["small", "c2"])
def test_aux_loss_masked_layers_match_transformers_golden(case):
    """load_balancing_loss_func with an attention mask over several layers
    (the per-layer expansion of a [batch, seq] padding mask) against the
    golden loss and logits gradient that transformers' own function wrote."""
    from conftest import GOLDEN
    from parallel_amd import load_balancing_loss_func

    g = np.load(GOLDEN / "aux_masked.npz")
    layers, batch, seq, E, k, _ = g[f"{case}_meta"].tolist()
    leaves = [torch.from_numpy(l).to(DEV).requires_grad_() for l in g[f"{case}_logits"]]
    mask = torch.from_numpy(g[f"{case}_mask"]).to(DEV)
    aux = load_balancing_loss_func(tuple(leaves), E, k, mask)
    aux.backward()
    torch.testing.assert_close(aux.cpu(), torch.tensor(float(g[f"{case}_aux"])), rtol=1e-5, atol=1e-6)
    got = torch.stack([l.grad.cpu() for l in leaves])
    want = torch.from_numpy(g[f"{case}_d_logits"])
    torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-8)


def test_aux_loss_balanced_routing_is_top_k():
    E, k, T = 8, 2, 64
    logits = torch.randn(T, E, generator=gen(0)) * 0.1
    for t in range(T):
        logits[t, (2 * t) % E] += 5.0
        logits[t, (2 * t + 1) % E] += 4.0
    aux, stats = ops.aux_loss_fwd(logits.to(DEV), None, E, k)
    assert abs(float(aux) - k) < 1e-5
    assert stats.cpu().tolist() == [16.0] * E + [64.0]


# ------------------------------------------------------------------- permute


def _perm_case(T, k, E, seed, sentinel_frac=0.0, skew=None, distinct=True):
    g = gen(seed)
    if distinct and k <= E:
        keys = torch.rand(T, E, generator=g)
        if skew is not None:
            keys = keys + skew
        ids = keys.topk(k, dim=1).indices
    else:
        ids = torch.randint(0, E, (T, k), generator=g)
    if sentinel_frac:
        ids = ids.masked_fill(torch.rand(T, k, generator=g) < sentinel_frac, E)
    return ids


PERMUTE_CASES = [
    dict(T=4096, k=8, E=128, seed=1),
    dict(T=16384, k=8, E=128, seed=2, skew=torch.linspace(0, 2, 128)),
    dict(T=512, k=2, E=8, seed=3),
    dict(T=1, k=1, E=4, seed=4),
    dict(T=3000, k=4, E=64, seed=5, sentinel_frac=0.4),
    dict(T=700, k=3, E=1024, seed=6, distinct=False),
    dict(T=2049, k=1, E=2, seed=7, distinct=False),
    # 262144 and 320000 routes: 512 and 625 count blocks in every scatter block's prefix
    dict(T=32768, k=8, E=128, seed=8, skew=torch.linspace(0, 3, 128)),
    dict(T=40000, k=8, E=128, seed=9, sentinel_frac=0.1),
]


@pytest.mark.parametrize("case", PERMUTE_CASES, ids=lambda c: f"T{c['T']}k{c['k']}E{c['E']}")
def test_permute_bit_exact(case):
    case = dict(case)
    T, k, E = case["T"], case["k"], case["E"]
    ids = _perm_case(**case)
    H = 64
    hidden = torch.randn(T, H, generator=gen(11)).to(BF)
    rows, perm, pos, counts, offsets = ops.permute_fwd(hidden.to(DEV), ids.to(DEV), 1, E, True)
    r_perm, r_pos, r_counts, r_off = O.stable_permutation(ids.numpy(), 1, E)
    assert np.array_equal(perm.cpu().numpy(), r_perm)
    assert np.array_equal(pos.cpu().numpy(), r_pos)
    assert np.array_equal(counts.cpu().numpy(), r_counts)
    assert np.array_equal(offsets.cpu().numpy(), r_off)
    n_valid = int(r_off[-1])
    expect = hidden[torch.from_numpy(r_perm[:n_valid]) // k]
    assert torch.equal(rows.cpu()[:n_valid], expect), "gathered rows are not exact copies"
    assert not rows.cpu()[n_valid:].any(), "sentinel rows must be zero"


def test_permute_matches_torch_sort_histc_cumsum():
    ids = _perm_case(4096, 8, 128, 21)
    _, perm, _, counts, offsets = ops.permute_fwd(torch.empty(4096, 8, dtype=BF, device=DEV), ids.to(DEV), 1, 128,
                                                  False)
    flat = ids.reshape(-1)
    _, ref_perm = torch.sort(flat, stable=True)
    hist = torch.histc(flat.float(), bins=128, min=0, max=127)
    assert torch.equal(perm.cpu().long(), ref_perm)
    assert torch.equal(counts.cpu().long(), torch.bincount(flat, minlength=128))
    assert torch.equal(offsets.cpu(), torch.cumsum(hist, 0, dtype=torch.int32))


def test_permute_owner_buckets_give_send_splits():
    ids = _perm_case(2048, 8, 128, 22)
    _, perm, _, counts, _ = ops.permute_fwd(torch.empty(2048, 8, dtype=BF, device=DEV), ids.to(DEV), 16, 8, False)
    dest = ids.reshape(-1) // 16
    assert torch.equal(perm.cpu().long(), torch.argsort(dest, stable=True))
    assert torch.equal(counts.cpu().long(), torch.bincount(dest, minlength=8))


@pytest.mark.parametrize("divisor,nb", [(1, 64), (16, 8), (3, 5)])
def test_permute_out_of_range_ids_are_sentinels(divisor, nb):
    """Negative ids and ids past the last bucket, at divisors above 1 too: the
    bucket is floor(id / divisor), so -1 is below bucket 0 (not in it) and
    sorts with the sentinels after every real bucket, as the oracle's
    stable_permutation says."""
    g = gen(divisor * 100 + nb)
    T, k = 600, 4
    ids = torch.randint(-3 * divisor, (nb + 2) * divisor, (T, k), generator=g)
    assert (ids < 0).any() and (ids // divisor >= nb).any() and ((ids >= 0) & (ids < divisor)).any()
    hidden = torch.randn(T, 32, generator=g).to(BF)
    rows, perm, pos, counts, offsets = ops.permute_fwd(hidden.to(DEV), ids.to(DEV), divisor, nb, True)
    r_perm, r_pos, r_counts, r_off = O.stable_permutation(ids.numpy(), divisor, nb)
    assert np.array_equal(perm.cpu().numpy(), r_perm)
    assert np.array_equal(pos.cpu().numpy(), r_pos)
    assert np.array_equal(counts.cpu().numpy(), r_counts)
    assert np.array_equal(offsets.cpu().numpy(), r_off)
    n_valid = int(r_off[-1])
    assert torch.equal(rows.cpu()[:n_valid], hidden[torch.from_numpy(r_perm[:n_valid]) // k])
    assert not rows.cpu()[n_valid:].any()


def test_permute_empty_input():
    _, perm, pos, counts, offsets = ops.permute_fwd(torch.empty(0, 64, dtype=BF, device=DEV),
                                                    torch.empty(0, 8, dtype=torch.long, device=DEV), 1, 16, True)
    assert perm.numel() == 0 and counts.cpu().tolist() == [0] * 16 and offsets.cpu().tolist() == [0] * 16


# -------------------------------------------------------------- grouped GEMM


def _groups(counts):
    counts = torch.tensor(counts, dtype=torch.int64)
    return counts, torch.cumsum(counts, 0).to(torch.int32)


def _ref_fwd(a, w, counts):
    out, s = [], 0
    for e, c in enumerate(counts.tolist()):
        out.append(a[s:s + c].float() @ w[e].float().t())
        s += c
    return torch.cat(out)


GEMM_CASES = [
    ("c2like", [256, 0, 300, 1, 128, 255, 513], 1536, 2048),
    ("ragged", [7, 0, 0, 130, 64, 1], 200, 72),
    ("single", [1000], 128, 256),
    ("split", [770, 257, 33], 1280, 64),  # m-tiles of 224/224/224/98 and 160/97 rows
    ("skewed", [0, 0, 3000, 0, 1, 0, 0, 0], 1536, 128),  # one group of 12 m-tiles, the rest empty or one row
    # at least 448 rows per expert on average: the row-grouped GEMMs take the ping-pong loop
    ("ping", [900, 0, 1100, 17, 513, 2000], 1536, 2048),
    ("ping_ragged", [1700, 3, 0, 640, 70], 200, 72),  # ragged n-tile, K tail inside the third k-tile
    ("ping_shortk", [520, 480, 33], 264, 40),  # two k-tiles (one nearly empty) per tile
    # at most 288 rows per expert on average and wide outputs: 320-row tiles (exactly one and two full m-tiles)
    ("wide", [320, 319, 1, 0, 640, 100, 33], 1536, 256),
]


@pytest.mark.parametrize("name,cnt,N,K", GEMM_CASES, ids=[c[0] for c in GEMM_CASES])
def test_grouped_gemm_fwd(name, cnt, N, K):
    counts, offs = _groups(cnt)
    M = int(counts.sum()) + 5  # trailing rows past offs[-1] are not touched
    G = len(cnt)
    a = torch.randn(M, K, generator=gen(1)).to(BF)
    w = (torch.randn(G, N, K, generator=gen(2)) * 0.05).to(BF)
    c = torch.full((M, N), 7.0, dtype=BF, device=DEV)
    _lib.call("moe_grouped_gemm_fwd", (ad := a.to(DEV)).data_ptr(), (wd := w.to(DEV)).data_ptr(),
              (od := offs.to(DEV)).data_ptr(), G, M, N, K, c.data_ptr(), _lib.stream_of(c))
    torch.cuda.synchronize()
    n = int(counts.sum())
    close_bf16(c[:n], _ref_fwd(a, w, counts), f"fwd {name}", max_rel=8e-3)
    assert (c[n:].float() == 7.0).all(), "rows past offs[-1] were written"


@pytest.mark.parametrize("name,cnt,N,K", GEMM_CASES, ids=[c[0] for c in GEMM_CASES])
def test_grouped_gemm_dgrad(name, cnt, N, K):
    counts, offs = _groups(cnt)
    M = int(counts.sum())
    G = len(cnt)
    dc = torch.randn(M, N, generator=gen(3)).to(BF)
    w = (torch.randn(G, N, K, generator=gen(4)) * 0.05).to(BF)
    da = torch.empty(M, K, dtype=BF, device=DEV)
    _lib.call("moe_grouped_gemm_dgrad", (dcd := dc.to(DEV)).data_ptr(), (wd := w.to(DEV)).data_ptr(),
              (od := offs.to(DEV)).data_ptr(), G, M, N, K, da.data_ptr(), _lib.stream_of(da))
    ref, s = [], 0
    for e, c in enumerate(counts.tolist()):
        ref.append(dc[s:s + c].float() @ w[e].float())
        s += c
    close_bf16(da, torch.cat(ref), f"dgrad {name}", max_rel=8e-3)


@pytest.mark.parametrize("name,cnt,N,K", GEMM_CASES, ids=[c[0] for c in GEMM_CASES])
@pytest.mark.parametrize("accumulate,f32", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_grouped_gemm_wgrad(name, cnt, N, K, accumulate, f32):
    counts, offs = _groups(cnt)
    M = int(counts.sum())
    G = len(cnt)
    dc = torch.randn(M, N, generator=gen(5)).to(BF)
    a = torch.randn(M, K, generator=gen(6)).to(BF)
    base = torch.randn(G, N, K, generator=gen(7))
    dw = base.to(torch.float32 if f32 else BF).to(DEV)
    _lib.call("moe_grouped_gemm_wgrad", (dcd := dc.to(DEV)).data_ptr(), (ad := a.to(DEV)).data_ptr(),
              (od := offs.to(DEV)).data_ptr(), G, M, N, K, dw.data_ptr(), f32, accumulate, _lib.stream_of(dw))
    s = 0
    start = base.to(torch.float32 if f32 else BF).float()
    for e, c in enumerate(counts.tolist()):
        ref = dc[s:s + c].float().t() @ a[s:s + c].float()
        if accumulate:
            ref = ref + start[e]
        s += c
        if c == 0 and accumulate:
            assert torch.equal(dw[e].cpu().float(), start[e]), "accumulate must leave empty groups untouched"
        elif c == 0:
            assert not dw[e].cpu().float().any(), "empty group must get a zero gradient"
        else:
            close_bf16(dw[e], ref, f"wgrad {name} g{e}", max_rel=8e-3)


def _skewed_counts(name):
    g = np.random.default_rng(len(name))
    if name == "zipf200":  # one tile per group, Zipf rows, a tenth of the groups empty
        c = (3000 / np.arange(1, 201) ** 1.1).astype(np.int64)
        c[g.choice(200, 20, replace=False)] = 0
        return g.permutation(c).tolist(), 256, 192
    if name == "many1000":  # ten heavy groups among 990 of 0-20 rows: light XCD ranges touch > 64 groups
        c = g.integers(0, 21, 1000)
        c[g.choice(1000, 10, replace=False)] = g.integers(2000, 4001, 10)
        return c.tolist(), 128, 320
    if name == "ties64":  # 60 groups of equal cost between 4 heavy ones
        c = np.full(64, 96)
        c[[3, 17, 40, 63]] = 4000
        return c.tolist(), 256, 256
    return [1, 0, 5000, 2, 0, 33], 296, 264  # "ragged": ragged tiles on both sides


@pytest.mark.parametrize("name,accumulate,f32", [("zipf200", 0, 0), ("many1000", 0, 0), ("many1000", 1, 0),
                                                 ("ties64", 0, 0), ("ties64", 0, 1), ("ragged", 1, 1)])
def test_grouped_gemm_wgrad_skewed_routing(name, accumulate, f32):
    """Weight gradients under skewed row counts, where the tiles are split over
    the XCDs by cost and dealt in cost order: many groups per XCD range (more
    than 64 in the light ranges of many1000), groups of equal cost, ragged
    tiles.  Every group against an fp32 product on the GPU."""
    cnt, N, K = _skewed_counts(name)
    counts, offs = _groups(cnt)
    M, G = int(counts.sum()), len(cnt)
    dc = torch.randn(M, N, generator=gen(8)).to(BF).to(DEV)
    a = torch.randn(M, K, generator=gen(9)).to(BF).to(DEV)
    odt = torch.float32 if f32 else BF
    start = torch.randn(G, N, K, generator=gen(10)).to(odt).to(DEV)
    dw = start.clone()
    _lib.call("moe_grouped_gemm_wgrad", dc.data_ptr(), a.data_ptr(), (od := offs.to(DEV)).data_ptr(), G, M, N, K,
              dw.data_ptr(), f32, accumulate, _lib.stream_of(dw))
    ref = torch.zeros(G, N, K, device=DEV)
    s = 0
    for e, c in enumerate(cnt):
        if c:
            ref[e] = dc[s:s + c].float().t() @ a[s:s + c].float()
        s += c
    if accumulate:
        ref += start.float()
    live = counts.to(DEV) > 0
    got = dw.float()
    assert torch.isfinite(got).all()
    scale = ref.abs().amax((1, 2)).clamp_min(1e-30)
    rel = (got - ref).abs().amax((1, 2)) / scale
    cos = F.cosine_similarity(got.reshape(G, -1).double(), ref.reshape(G, -1).double(), dim=1)
    # bf16 output: one rounding of each element (2^-9 of it), two with the
    # accumulate (the fresh sum's, then the sum with the old gradient's);
    # fp32 output: the fp32 summation order alone.
    bar = 1e-4 if f32 else (1.6e-2 if accumulate else 8e-3)
    bad = live & ((rel > bar) | (cos < 0.9999))
    assert not bad.any(), f"{name}: groups {bad.nonzero().flatten().tolist()[:8]} off (max rel {float(rel[live].max()):.3e})"
    empty = ~live
    if accumulate:
        assert torch.equal(dw[empty], start[empty]), "accumulate must leave empty groups untouched"
    else:
        assert not dw[empty].any(), "empty groups must get zero gradients"
    print(f"{name}: {G} groups, {M} rows, worst rel {float(rel[live].max()):.2e}")


@pytest.mark.parametrize("cnt,I,H", [([256, 0, 300, 1, 128], 768, 2048), ([5, 64, 0, 17], 64, 96),
                                     ([600, 0, 1500, 5, 257], 768, 2048)])  # the last on the ping-pong loop
def test_swiglu_fwd_and_fused_backward(cnt, I, H):
    counts, offs = _groups(cnt)
    M = int(counts.sum())
    G = len(cnt)
    xp = torch.randn(M, H, generator=gen(8)).to(BF)
    gu = (torch.randn(G, 2 * I, H, generator=gen(9)) * 0.05).to(BF)
    dn = (torch.randn(G, H, I, generator=gen(10)) * 0.05).to(BF)
    dy = torch.randn(M, H, generator=gen(11)).to(BF)
    act = torch.empty(M, I, dtype=BF, device=DEV)
    pre = torch.empty(M, 2 * I, dtype=BF, device=DEV)
    od = offs.to(DEV)
    xpd, gud, dnd, dyd = xp.to(DEV), gu.to(DEV), dn.to(DEV), dy.to(DEV)
    s = _lib.stream_of(act)
    _lib.call("moe_grouped_gemm_swiglu_fwd", xpd.data_ptr(), gud.data_ptr(), od.data_ptr(), G, M, H, I,
              act.data_ptr(), pre.data_ptr(), s)
    ref_pre = _ref_fwd(xp, gu, counts)
    gate, up = ref_pre.chunk(2, dim=-1)
    close_bf16(pre, ref_pre, "swiglu pre", max_rel=8e-3)
    close_bf16(act, F.silu(gate) * up, "swiglu act", max_rel=8e-3)
    d_pre = torch.empty(M, 2 * I, dtype=BF, device=DEV)
    _lib.call("moe_grouped_gemm_dgrad_swiglu_bwd", dyd.data_ptr(), dnd.data_ptr(), pre.data_ptr(), od.data_ptr(),
              G, M, H, I, d_pre.data_ptr(), s)
    # reference: autograd of silu(g)*u at the saved (bf16) pre-activation
    p = pre.cpu().float().requires_grad_()
    g2, u2 = p.chunk(2, dim=-1)
    d_act, s0 = [], 0
    for e, c in enumerate(counts.tolist()):
        d_act.append(dy[s0:s0 + c].float() @ dn[e].float())
        s0 += c
    (F.silu(g2) * u2).backward(torch.cat(d_act))
    close_bf16(d_pre, p.grad, "swiglu d_pre", max_rel=1e-2)


def test_dgrad_swiglu_leaves_the_sentinel_tail_untouched():
    """Rows past offs[G-1] (sentinel routes under EP) are neither read nor
    written by the input-gradient GEMM or the SwiGLU backward: NaN poison in
    pre and d_pre there stays bit for bit, and the valid rows equal a run over
    the valid rows alone."""
    cnt, I, H, tail = [40, 0, 71, 9], 64, 96, 57
    counts, offs = _groups(cnt)
    V = int(counts.sum())
    M, G = V + tail, len(cnt)
    dn = (torch.randn(G, H, I, generator=gen(40)) * 0.05).to(BF).to(DEV)
    dy = torch.randn(M, H, generator=gen(41)).to(BF).to(DEV)
    pre = torch.randn(M, 2 * I, generator=gen(42)).to(BF).to(DEV)
    pre[V:] = float("nan")
    d_pre = torch.full((M, 2 * I), float("nan"), dtype=BF, device=DEV)
    poison = d_pre[V:].clone()
    od = offs.to(DEV)
    s = _lib.stream_of(pre)
    _lib.call("moe_grouped_gemm_dgrad_swiglu_bwd", dy.data_ptr(), dn.data_ptr(), pre.data_ptr(), od.data_ptr(),
              G, M, H, I, d_pre.data_ptr(), s)
    valid = torch.empty(V, 2 * I, dtype=BF, device=DEV)
    _lib.call("moe_grouped_gemm_dgrad_swiglu_bwd", dy.data_ptr(), dn.data_ptr(), pre.data_ptr(), od.data_ptr(),
              G, V, H, I, valid.data_ptr(), s)
    torch.cuda.synchronize()
    assert torch.equal(d_pre[V:].view(torch.int16), poison.view(torch.int16)), "sentinel rows were written"
    assert torch.equal(d_pre[:V], valid) and torch.isfinite(valid.float()).all()


# ------------------------------------------------------------------- combine


# k spans the specialised (1, 2, 4, 6, 8) and the run-time (3, 16) slot counts.
@pytest.mark.parametrize("T,k,E,H,sent", [(512, 2, 8, 256, 0.0), (1024, 8, 128, 2048, 0.0), (300, 4, 16, 72, 0.3),
                                          (700, 3, 24, 136, 0.1), (64, 16, 32, 264, 0.0), (200, 6, 64, 72, 0.2),
                                          (333, 1, 8, 520, 0.0)])
def test_combine_forward_backward(T, k, E, H, sent):
    ids = _perm_case(T, k, E, 31, sentinel_frac=sent)
    hidden = torch.randn(T, H, generator=gen(32)).to(BF)
    rows, perm, pos, counts, offsets = ops.permute_fwd(hidden.to(DEV), ids.to(DEV), 1, E, True)
    S = T * k
    y = torch.randn(S, H, generator=gen(33)).to(BF)
    scores = torch.rand(T, k, generator=gen(34))
    out = torch.empty(T, H, dtype=BF, device=DEV)
    yd, sd = y.to(DEV), scores.to(DEV)
    st = _lib.stream_of(out)
    _lib.call("moe_combine_fwd", yd.data_ptr(), pos.data_ptr(), offsets.data_ptr(), E, sd.data_ptr(), T, H, k,
              out.data_ptr(), st)
    posc = pos.cpu().long().view(T, k)
    valid = ids < E
    ref = (y.float()[posc] * (scores * valid).unsqueeze(-1)).sum(1)
    close_bf16(out, ref, "combine fwd", max_rel=8e-3)
    d_out = torch.randn(T, H, generator=gen(35)).to(BF)
    dy = torch.full((S, H), 3.0, dtype=BF, device=DEV)
    d_s = torch.empty(T * k, dtype=torch.float32, device=DEV)
    _lib.call("moe_combine_bwd", (dd := d_out.to(DEV)).data_ptr(), yd.data_ptr(), pos.data_ptr(),
              offsets.data_ptr(), E, sd.data_ptr(), T, H, k, dy.data_ptr(), d_s.data_ptr(), st)
    ref_dy = torch.zeros(S, H)
    ref_dy[posc.reshape(-1)] = (d_out.float().unsqueeze(1) * (scores * valid).unsqueeze(-1)).reshape(S, H)
    close_bf16(dy, ref_dy, "combine d_y", max_rel=8e-3)
    ref_ds = (y.float()[posc] * d_out.float().unsqueeze(1)).sum(-1) * valid
    close_bf16(d_s.view(T, k), ref_ds, "combine d_scores", max_rel=1e-3)


@pytest.mark.parametrize("k", [4, 5, 16])
def test_permute_backward_sums_routes(k):
    T, E, H = 777, 32, 136
    ids = _perm_case(T, k, E, 41, sentinel_frac=0.2)
    hidden = torch.zeros(T, H, dtype=BF, device=DEV)
    _, perm, pos, counts, offsets = ops.permute_fwd(hidden, ids.to(DEV), 1, E, False)
    dperm = torch.randn(T * k, H, generator=gen(42)).to(BF)
    d_add = torch.randn(T, H, generator=gen(43)).to(BF)
    dh = torch.empty(T, H, dtype=BF, device=DEV)
    _lib.call("moe_permute_bwd", (dp := dperm.to(DEV)).data_ptr(), pos.data_ptr(), offsets.data_ptr(), E, T, H, k,
              (da := d_add.to(DEV)).data_ptr(), dh.data_ptr(), _lib.stream_of(dh))
    posc = pos.cpu().long().view(T, k)
    ref = (dperm.float()[posc] * (ids < E).unsqueeze(-1)).sum(1) + d_add.float()
    close_bf16(dh, ref, "permute bwd", max_rel=8e-3)

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible to torch")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def close_bf16(actual, expected, name="tensor", max_rel=2e-2, min_cos=0.9999):
    """The path's floating-point bar: normwise max relative error and cosine similarity."""
    a = actual.detach().float().cpu().reshape(-1)
    b = expected.detach().float().cpu().reshape(-1)
    assert a.shape == b.shape, f"{name}: shape {tuple(a.shape)} vs {tuple(b.shape)}"
    assert torch.isfinite(a).all(), f"{name}: non-finite values"
    denom = b.abs().max().clamp_min(1e-30)
    rel = float((a - b).abs().max() / denom)
    cos = float(torch.nn.functional.cosine_similarity(a.double(), b.double(), dim=0)) if b.abs().max() > 0 else 1.0
    assert rel <= max_rel and cos >= min_cos, f"{name}: max rel err {rel:.3e} (<= {max_rel}), cosine {cos:.6f}"
    return rel, cos


def routing_check(indices, ref_indices, logits, *, expect_ties=0):
    """Bit-exact routing against the oracle: every token whose selection does
    not depend on torch.topk's (unpinned) tie order must match exactly, and the
    number of tokens excused for exact ties must be ``expect_ties`` (0 for
    continuous random logits), so that a tie detector that fires too often
    cannot make the comparison vacuous.  Returns the tie mask."""
    from oracle import moe_oracle as O

    ties = O.topk_ties(logits.detach().float().cpu(), ref_indices)
    mismatch = (indices.detach().cpu() != ref_indices.cpu()).any(dim=1)
    bad = int((mismatch & ~ties).sum())
    assert bad == 0, f"{bad} tokens routed differently from the oracle"
    assert int(ties.sum()) == expect_ties, f"{int(ties.sum())} tokens excused for exact ties, expected {expect_ties}"
    return ties

"""Expert weight gradients written into an FSDP unit's reduce-scatter bucket
on the GPU (moe_grouped_gemm_wgrad_bucket), against the oracle's packing of
the dense gradients that ops.experts_bwd produces from the same inputs
(parallel/parallel/engine/_dp_param_unit.py:395-417).  The same kernel
arithmetic writes both, so the bucket is compared bit for bit."""

import pytest
import torch

from oracle import moe_oracle as O
from parallel_amd import ops
from parallel_amd.fsdp_bucket import GradBucketLayout, experts_backward_into_bucket

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def _inputs(T, H, E, k, I, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(DEV, BF)
    logits = torch.randn(T, E, generator=g)
    logits[:, -1] -= 100.0  # the last expert gets no routes: an empty group
    scores, idx = torch.softmax(logits, -1).topk(k, dim=-1)
    gu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(DEV, BF)
    dn = (torch.randn(E, H, I, generator=g) * 0.02).to(DEV, BF)
    d_out = torch.randn(T, H, generator=g).to(DEV, BF)
    return x, idx.to(DEV), (scores / scores.sum(-1, keepdim=True)).to(DEV), gu, dn, d_out


def _layout(E, H, I, world):
    # an unrelated parameter between the two projections, as in a real unit
    return GradBucketLayout.from_named_shapes(
        [("gate_up_proj", (E, 2 * I, H)), ("router", (E, H)), ("down_proj", (E, H, I))], world)


@pytest.mark.parametrize("world,T,H,E,k,I", [(1, 96, 256, 6, 2, 128), (2, 96, 256, 6, 2, 128), (3, 96, 256, 6, 2, 128),
                                              (4, 96, 256, 6, 2, 128),
                                              # the C2 layer: 16 experts per rank, and 43 with a padded last chunk
                                              (8, 4096, 2048, 128, 8, 768), (3, 4096, 2048, 128, 8, 768)])
def test_bucket_matches_packed_dense_gradients(world, T, H, E, k, I):
    x, idx, scores, gu, dn, d_out = _inputs(T, H, E, k, I, seed=world)
    out, *saved = ops.experts_fwd(x, idx, scores, gu, dn)
    d_x, d_w, d_gu, d_dn = ops.experts_bwd(d_out, scores, gu, dn, *saved)
    layout = _layout(E, H, I, world)
    bucket = layout.new_bucket(BF, DEV)
    d_x2, d_w2 = experts_backward_into_bucket(d_out, scores, gu, dn, saved, bucket, layout)
    torch.cuda.synchronize()
    assert torch.equal(d_x2, d_x) and torch.equal(d_w2, d_w)
    assert not d_gu[-1].any(), "the empty expert's gradient is zero"
    expected = O.fsdp_pack_grads([d_gu.cpu(), None, d_dn.cpu()], world, dtype=BF,
                                 shapes=[s.shape for s in layout.slots])
    assert torch.equal(bucket.cpu(), expected)


def test_bucket_accumulates_and_leaves_padding_alone():
    T, H, E, k, I, world = 80, 256, 6, 2, 128, 4  # ceil(6/4) = 2 rows per rank: rank 3 is all padding
    x, idx, scores, gu, dn, d_out = _inputs(T, H, E, k, I, seed=11)
    out, *saved = ops.experts_fwd(x, idx, scores, gu, dn)
    _, _, d_gu, d_dn = ops.experts_bwd(d_out, scores, gu, dn, *saved)
    layout = _layout(E, H, I, world)
    start = torch.randn(world, layout.bucket_numel, generator=torch.Generator().manual_seed(5)).to(DEV, BF)
    bucket = start.clone()
    experts_backward_into_bucket(d_out, scores, gu, dn, saved, bucket, layout, accumulate=True)
    torch.cuda.synchronize()
    # torch's bf16 add of the existing bucket and the bf16 gradient
    shapes = [s.shape for s in layout.slots]
    packed = O.fsdp_pack_grads([d_gu.cpu(), None, d_dn.cpu()], world, dtype=torch.float32, shapes=shapes)
    mask = O.fsdp_pack_grads([torch.ones_like(d_gu, device="cpu"), None, torch.ones_like(d_dn, device="cpu")],
                             world, dtype=torch.float32, shapes=shapes).bool()
    expected = torch.where(mask, (start.cpu().float() + packed).to(BF), start.cpu())
    assert torch.equal(bucket.cpu(), expected)


def test_bucket_rejects_unaligned_rank_chunks():
    T, H, E, k, I = 32, 256, 4, 2, 128
    x, idx, scores, gu, dn, d_out = _inputs(T, H, E, k, I, seed=3)
    out, *saved = ops.experts_fwd(x, idx, scores, gu, dn)
    # a 5-element parameter makes bucket_numel odd: rank chunks lose 16-byte alignment
    layout = GradBucketLayout.from_named_shapes(
        [("gate_up_proj", (E, 2 * I, H)), ("down_proj", (E, H, I)), ("bias", (5,))], 2)
    bucket = layout.new_bucket(BF, DEV)
    with pytest.raises((ValueError, RuntimeError), match="aligned"):
        experts_backward_into_bucket(d_out, scores, gu, dn, saved, bucket, layout)
    with pytest.raises(ValueError):
        experts_backward_into_bucket(d_out, scores, gu, dn, saved, bucket.cpu(), layout)

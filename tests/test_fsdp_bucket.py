"""FSDP gradient-bucket layout on the CPU: the oracle's packing of a unit's
reduce-scatter input (parallel/parallel/engine/_dp_param_unit.py:200-202,
:268-277, :395-417) and the host-side layout of parallel_amd.fsdp_bucket.

The packing is pinned by what the collective does with it: after
reduce_scatter_tensor over gloo (two CPU ranks), every rank must hold, at each
parameter's offset, the sum over ranks of its own rows of that parameter
(ceil(rows / world) of them), zeros past the last row.
"""

import os

import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

from oracle import moe_oracle as O
from parallel_amd.fsdp_bucket import GradBucketLayout, pack_gradient

SHAPES = [(5, 2, 3), (3, 4), (8, 2)]


def test_layout_known_answer():
    layout, numel = O.fsdp_bucket_layout(SHAPES, 2)
    # padded rows 3, 2, 4; offsets are consecutive padded shards
    assert layout == [(3, 0, 18), (2, 18, 8), (4, 26, 8)] and numel == 34
    grads = [torch.arange(30.0).view(5, 2, 3), torch.ones(3, 4), torch.full((8, 2), 7.0)]
    b = O.fsdp_pack_grads(grads, 2)
    assert b.shape == (2, 34)
    assert torch.equal(b[0, :18], torch.arange(18.0)) and torch.equal(b[1, :12], torch.arange(18.0, 30.0))
    assert not b[1, 12:18].any(), "rows past the parameter's end stay zero"
    assert torch.equal(b[0, 18:26], torch.ones(8)) and torch.equal(b[1, 18:22], torch.ones(4))
    assert not b[1, 22:26].any()
    assert torch.equal(b[:, 26:], torch.full((2, 8), 7.0))


@pytest.mark.parametrize("world", [1, 2, 3, 4])
def test_host_layout_and_pack_match_oracle(world):
    g = torch.Generator().manual_seed(world)
    grads = [torch.randn(*s, generator=g) for s in SHAPES]
    layout = GradBucketLayout.from_named_shapes([(f"p{i}", s) for i, s in enumerate(SHAPES)], world)
    ref_layout, ref_numel = O.fsdp_bucket_layout(SHAPES, world)
    assert layout.bucket_numel == ref_numel
    assert [(s.padded_rows, s.bucket_offset, s.padded_numel) for s in layout.slots] == ref_layout
    bucket = layout.new_bucket(torch.float32, "cpu")
    for i, grad in enumerate(grads):
        pack_gradient(bucket, layout, f"p{i}", grad)
    assert torch.equal(bucket, O.fsdp_pack_grads(grads, world))


def test_layout_errors():
    with pytest.raises(ValueError):
        GradBucketLayout.from_named_shapes([("a", (4,))], 0)
    with pytest.raises(ValueError):
        GradBucketLayout.from_named_shapes([("scalar", ())], 2)
    layout = GradBucketLayout.from_named_shapes([("a", (4, 2))], 2)
    with pytest.raises(KeyError):
        layout.slot("b")
    with pytest.raises(ValueError):
        pack_gradient(layout.new_bucket(torch.float32, "cpu"), layout, "a", torch.ones(3, 2))


def _reduce_scatter_worker(rank, world, port, result):
    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    dist.init_process_group("gloo", rank=rank, world_size=world)
    try:
        g = torch.Generator().manual_seed(100 + rank)
        grads = [torch.randn(*s, generator=g) for s in SHAPES]
        bucket = O.fsdp_pack_grads(grads, world)
        out = torch.empty(bucket.shape[1])
        dist.reduce_scatter_tensor(out, bucket.reshape(-1), op=dist.ReduceOp.SUM)
        result[rank] = out
    finally:
        dist.destroy_process_group()


def test_packing_is_the_reduce_scatter_layout():
    world = 2
    result = mp.Manager().dict()
    mp.spawn(_reduce_scatter_worker, args=(world, 29611, result), nprocs=world)
    # the sum over ranks of each full gradient, regenerated in rank order
    sums = [torch.zeros(*s) for s in SHAPES]
    for r in range(world):
        g = torch.Generator().manual_seed(100 + r)
        for i, s in enumerate(SHAPES):
            sums[i] += torch.randn(*s, generator=g)
    layout, _ = O.fsdp_bucket_layout(SHAPES, world)
    for rank in range(world):
        out = result[rank]
        for total, s, (padded_rows, offset, padded_numel) in zip(sums, SHAPES, layout):
            shard = out[offset:offset + padded_numel].view(padded_rows, *s[1:])
            start = rank * padded_rows
            rows = min(padded_rows, max(s[0] - start, 0))
            assert torch.allclose(shard[:rows], total[start:start + rows], atol=1e-6)
            assert not shard[rows:].any()

"""CPU tests of the host side: the C-ABI library loads and exports every
declared symbol, argument validation raises the reference's exception types,
and there is no CPU fallback."""

import ctypes
import re

import pytest
import torch

from conftest import ROOT
from parallel_amd import (
    ExpertPartition,
    TokenDispatcher,
    load_balancing_loss_func,
    register_experts_implementation,
    sequence_parallel_load_balancing_loss,
)
from parallel_amd import _lib, ops
from parallel_amd.workloads import WORKLOADS

HEADER = ROOT / "include" / "moe_mi355x.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moe_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    syms = declared_symbols()
    assert len(syms) >= 18
    assert set(syms) == set(_lib.SIGNATURES), "ctypes signatures and header disagree"


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), f"{name} missing from {_lib.LIB_PATH}"
    assert lib.moe_abi_version() == _lib.ABI_VERSION


def test_library_size_queries_and_argument_checks_run_without_a_gpu():
    lib = _lib.load()
    assert lib.moe_permute_workspace_bytes(32768, 128) == 64 * 129 * 4  # 512-route chunks x (E + sentinel)
    # one partial row per block (16 tokens for E <= 256, else 4), as the router
    # kernels write them, plus 16 row-group sums, each 2E+1 floats
    assert lib.moe_aux_loss_workspace_bytes(4096, 128) == (256 + 16) * 257 * 4
    assert lib.moe_aux_loss_workspace_bytes(40, 8) == (3 + 16) * 17 * 4
    assert lib.moe_aux_loss_workspace_bytes(4096, 512) == (1024 + 16) * 1025 * 4
    assert lib.moe_aux_loss_workspace_bytes(1 << 20, 128) == (65536 + 16) * 257 * 4
    # one pass for E <= 256 in 16-expert tiles (no split-K partials), split-K otherwise
    assert lib.moe_router_fwd_workspace_bytes(4096, 2048, 128) == 0
    assert lib.moe_router_fwd_workspace_bytes(4096, 2048, 120) >= 4096 * 120 * 4
    assert lib.moe_router_fwd_workspace_bytes(4096, 2048, 512) >= 4096 * 512 * 4
    assert lib.moe_router_aux_fwd_workspace_bytes(4096, 2048, 128) == (256 + 16) * 257 * 4
    # invalid sizes are rejected before any HIP call
    rc = lib.moe_grouped_gemm_fwd(None, None, None, 1, 8, 8, 8, None, None)
    assert rc == _lib.MOE_ERR_INVALID
    assert b"null" in lib.moe_last_error()
    buf = ctypes.create_string_buffer(64)
    rc = lib.moe_grouped_gemm_fwd(ctypes.addressof(buf), ctypes.addressof(buf), None, 1, 8, 12, 8, None, None)
    assert rc in (_lib.MOE_ERR_UNSUPPORTED, _lib.MOE_ERR_INVALID)
    with pytest.raises(ValueError, match="top_k"):
        _lib.check(lib.moe_router_topk_fwd(None, None, None, 4, 8, 9, 1, None), "topk")


def test_ops_refuse_cpu_tensors():
    x = torch.randn(4, 16, dtype=torch.bfloat16)
    w = torch.randn(8, 16, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU only"):
        ops.router_fwd(x, w, 2, True)
    gu = torch.randn(8, 32, 16, dtype=torch.bfloat16)
    dn = torch.randn(8, 16, 16, dtype=torch.bfloat16)
    idx = torch.zeros(4, 2, dtype=torch.int64)
    with pytest.raises(ValueError, match="GPU only"):
        ops.experts(x, idx, torch.rand(4, 2), gu, dn)


def test_expert_partition_contract():
    with pytest.raises(ValueError, match="ep_size must be positive"):
        ExpertPartition(8, 0, 0)
    with pytest.raises(ValueError, match="outside the expert-parallel group"):
        ExpertPartition(8, 2, 2)
    with pytest.raises(ValueError, match="divisible"):
        ExpertPartition(6, 4, 0)
    p = ExpertPartition(num_experts=8, ep_size=2, ep_rank=1)
    assert (p.local_count, p.start, p.stop, p.global_experts) == (4, 4, 8, range(4, 8))
    # parallel tests/test_model_parallel.py:140-147
    li, ls, m = p.localize_routes(torch.tensor([[0, 6], [4, 3]]), torch.tensor([[0.2, 0.8], [0.7, 0.3]]))
    torch.testing.assert_close(li, torch.tensor([[4, 2], [0, 4]]))
    torch.testing.assert_close(ls, torch.tensor([[0.0, 0.8], [0.7, 0.0]]))
    torch.testing.assert_close(m, torch.tensor([[False, True], [True, False]]))
    with pytest.raises(ValueError, match="same shape"):
        p.localize_routes(torch.zeros(2, 2, dtype=torch.long), torch.zeros(2, 3))


def test_token_dispatcher_contract():
    d = TokenDispatcher(ExpertPartition(8, 1, 0), None)
    with pytest.raises(ValueError, match="same shape"):
        d.dispatch(torch.zeros(2, 8), torch.zeros(2, 2, dtype=torch.long), torch.zeros(2, 3))
    share = TokenDispatcher(ExpertPartition(8, 4, 2), None)
    assert (share.world_size, share.rank) == (4, 2)
    assert share._exchange_splits(torch.tensor([3, 0, 5, 1])) == ((3, 0, 5, 1), (0, 0, 5, 0))


def test_aux_loss_api_edges():
    assert load_balancing_loss_func(None, 8, 2) == 0
    assert load_balancing_loss_func(torch.zeros(4, 8), 8, 2) == 0  # not a tuple: transformers returns 0
    assert sequence_parallel_load_balancing_loss(None, num_experts=8, top_k=2, group=None) is None


def test_transformers_registry_plugin():
    assert register_experts_implementation()
    from transformers.integrations.moe import ALL_EXPERTS_FUNCTIONS

    assert "mi355x" in ALL_EXPERTS_FUNCTIONS


def test_workload_shapes():
    c2 = WORKLOADS["c2"]
    assert (c2.tokens, c2.slots, c2.hidden, c2.experts, c2.top_k, c2.intermediate) == (4096, 32768, 2048, 128, 8, 768)
    assert c2.gemm_flops() == pytest.approx(9.277e11, rel=1e-3)
    assert WORKLOADS["c4"].gemm_flops() == pytest.approx(3.711e12, rel=1e-3)
    assert WORKLOADS["c5"].gemm_flops() == pytest.approx(7.422e12, rel=1e-3)


def test_bench_tags_kernel_dispatches_by_entry_point():
    """rocprofv3 kernel names of one step -> the bench's per-entry-point tags."""
    import bench

    g = "void moe::grouped_gemm_kernel<{}, {}, {}, moe::TileCfg<{}> >(moe::GemmParams)"
    big, tall, small = "256, 256, 32, 2, 4, 5", "512, 128, 32, 4, 2, 4", "128, 128, 32, 2, 2, 5"
    names = [
        g.format(0, "true", 1, small), "void moe::router_reduce_topk_kernel<2, 8>(float const*)",
        g.format(0, "true", 2, big), g.format(0, "true", 0, big), "void moe::combine_fwd_kernel<8>(unsigned short const*)",
        "void moe::combine_bwd_kernel<8>(unsigned short const*)",
        "void moe::combine_router_bwd_kernel<8, 2>(unsigned short const*)",
        g.format(0, "false", 0, tall), "moe::swiglu_bwd_kernel(unsigned short*)", g.format(0, "false", 0, big),
        "void moe::permute_bwd_kernel<8>(unsigned short const*)", g.format(1, "false", 4, big),
        g.format(1, "false", 4, big),
        g.format(1, "false", 4, small), g.format(0, "false", 0, small),
    ]
    assert bench.tag_dispatches(names) == [
        "router_fwd", "router_fwd", "up_fwd", "down_fwd", "combine_fwd", "combine_bwd", "combine_bwd",
        "down_dgrad", "down_dgrad", "up_dgrad", "permute_bwd", "up_wgrad", "down_wgrad",
        "router_gemm_bwd", "router_gemm_bwd",
    ]


def test_size_queries_accept_empty_and_tiny_shapes():
    """Every workspace query is host arithmetic only; with no tokens or one
    token it must return (no division by a zero tile count) and never ask for
    less than the non-empty case of the same layer."""
    lib = _lib.load()
    for T in (0, 1, 7):
        for E in (1, 8, 128, 1024):
            assert lib.moe_router_fwd_workspace_bytes(T, 2048, E) >= 0
            assert lib.moe_router_aux_fwd_workspace_bytes(T, 2048, E) >= 0
            assert lib.moe_router_logits_bwd_workspace_bytes(T, 2048, E) >= 0
            assert lib.moe_aux_loss_workspace_bytes(T, E) >= 0
            assert lib.moe_permute_workspace_bytes(T * 8, E) >= 0
        assert lib.moe_rmsnorm_bwd_workspace_bytes(T, 2048) >= 0
    assert lib.moe_router_fwd_workspace_bytes(4096, 2048, 128) >= lib.moe_router_fwd_workspace_bytes(1, 2048, 128)


def test_zero_size_calls_accept_null_buffers_without_a_gpu():
    """With no rows or tokens every entry point whose work is empty returns 0
    before any HIP call, with NULL for the empty buffers (an EP rank can
    receive no rows).  The non-empty weight buffers are a host stand-in that
    is never dereferenced."""
    lib = _lib.load()
    buf = ctypes.create_string_buffer(1 << 12)
    b = ctypes.addressof(buf) + (16 - ctypes.addressof(buf) % 16) % 16
    E, H, I, k = 16, 256, 128, 4
    calls = {
        "swiglu_fwd": lambda: lib.moe_grouped_gemm_swiglu_fwd(None, b, b, E, 0, H, I, None, None, None),
        "fwd": lambda: lib.moe_grouped_gemm_fwd(None, b, b, E, 0, H, I, None, None),
        "dgrad": lambda: lib.moe_grouped_gemm_dgrad(None, b, b, E, 0, 2 * I, H, None, None),
        "dgrad_swiglu": lambda: lib.moe_grouped_gemm_dgrad_swiglu_bwd(None, b, None, b, E, 0, H, I, None, None),
        "router_fwd": lambda: lib.moe_router_fwd(None, b, None, None, None, None, None, 0, H, E, k, 1, b, 16, None),
        "topk_fwd": lambda: lib.moe_router_topk_fwd(None, None, None, 0, E, k, 1, None),
        "topk_bwd": lambda: lib.moe_router_topk_bwd(None, None, None, 0, E, k, 1, None, 0, None, None),
        "topk_bwd_bf16": lambda: lib.moe_router_topk_bwd_bf16(None, None, None, None, 0, E, k, 1, None, None),
        "combine_fwd": lambda: lib.moe_combine_fwd(None, None, None, E, None, 0, H, k, None, None),
        "combine_bwd": lambda: lib.moe_combine_bwd(None, None, None, None, E, None, 0, H, k, None, None, None),
        "combine_router_bwd": lambda: lib.moe_combine_router_bwd(None, None, None, None, E, None, 0, H, k, None, None,
                                                                 None, None, None, None, None, None, E, 1, 0, None,
                                                                 None),
        "permute_bwd": lambda: lib.moe_permute_bwd(None, None, None, E, 0, H, k, None, None, None),
        "dispatch_meta": lambda: lib.moe_dispatch_meta(None, None, None, 0, 4, k, None, None, None, None),
    }
    for name, call in calls.items():
        assert call() == _lib.MOE_OK, f"{name}: {lib.moe_last_error()}"
    # the fused combine + router top-k backward checks the router's sizes and arguments too
    assert lib.moe_combine_router_bwd(b, b, b, b, E, None, 4, H, k, b, None, b, b, None, None, None, None, 2000, 1, 0,
                                      b, None) == _lib.MOE_ERR_UNSUPPORTED
    assert lib.moe_combine_router_bwd(b, b, b, b, E, None, 4, H, 8, b, None, b, b, None, None, None, None, 4, 1, 0,
                                      b, None) == _lib.MOE_ERR_UNSUPPORTED
    assert lib.moe_combine_router_bwd(b, b, b, b, E, None, 4, H, k, b, None, b, b, None, None, b, None, E, 1, 0,
                                      b, None) == _lib.MOE_ERR_INVALID
    assert b"stats and d_aux" in lib.moe_last_error()
    assert lib.moe_combine_router_bwd(b, None, b, b, E, None, 4, H, k, b, None, b, b, None, None, None, None, E, 1, 0,
                                      b, None) == _lib.MOE_ERR_INVALID
    # a missing non-empty operand is still an error
    assert lib.moe_grouped_gemm_fwd(None, None, b, E, 0, H, I, None, None) == _lib.MOE_ERR_INVALID
    assert lib.moe_grouped_gemm_fwd(None, b, b, E, 8, H, I, None, None) == _lib.MOE_ERR_INVALID


def test_accumulate_grad_is_refused_under_torch_compile(monkeypatch):
    """accumulate_grad writes .grad from inside the backward, which tracing
    cannot see: the ops refuse it while torch.compile traces them (checked
    before any tensor reaches the library)."""
    import torch

    from parallel_amd import ops

    monkeypatch.setattr(torch.compiler, "is_compiling", lambda: True)
    x = torch.zeros(4, 8)
    with pytest.raises(RuntimeError, match="torch.compile"):
        ops.experts(x, torch.zeros(4, 2, dtype=torch.int64), torch.zeros(4, 2), torch.zeros(2, 8, 8),
                    torch.zeros(2, 8, 4), accumulate_grad=True)
    with pytest.raises(RuntimeError, match="torch.compile"):
        ops.moe_block(x, torch.zeros(2, 8), torch.zeros(2, 8, 8), torch.zeros(2, 8, 4), 2, True,
                      accumulate_grad=True)

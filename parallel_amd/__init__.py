"""parallel_amd — the Qwen3-MoE expert path of jonahsamost/parallel on MI355X (gfx950).

Router top-k softmax, stable token permutation with per-expert counts and EP
send splits, grouped SwiGLU expert GEMMs forward and backward, weighted
combine and the load-balancing aux loss, as hand-written HIP kernels behind a
C ABI (``include/moe_mi355x.h``), exposed as torch.library ops with autograd
and as drop-ins for the reference's interfaces.
"""

from .aux_loss import load_balancing_loss_func, sequence_parallel_load_balancing_loss
from .checkpoint import MoeLayerWeights, load_moe_layer
from .fsdp_bucket import GradBucketLayout, experts_backward_into_bucket, pack_gradient
from .norm_router import norm_router_aux
from .expert_parallel import (
    ExpertPartition,
    ReplicatedTokenExpertParallel,
    SequenceParallelExpertParallel,
    local_expert_range,
    verify_expert_modules,
)
from .moe import (
    EXPERTS_IMPLEMENTATION,
    Experts,
    MoeConfig,
    SparseMoeBlock,
    TopKRouter,
    mi355x_experts_forward,
    register_experts_implementation,
)
from .token_dispatch import DispatchState, TokenDispatcher, variable_all_to_all

__all__ = [
    "DispatchState",
    "EXPERTS_IMPLEMENTATION",
    "ExpertPartition",
    "Experts",
    "GradBucketLayout",
    "MoeConfig",
    "MoeLayerWeights",
    "ReplicatedTokenExpertParallel",
    "SequenceParallelExpertParallel",
    "SparseMoeBlock",
    "TokenDispatcher",
    "TopKRouter",
    "experts_backward_into_bucket",
    "load_balancing_loss_func",
    "load_moe_layer",
    "norm_router_aux",
    "pack_gradient",
    "local_expert_range",
    "mi355x_experts_forward",
    "register_experts_implementation",
    "sequence_parallel_load_balancing_loss",
    "variable_all_to_all",
    "verify_expert_modules",
]

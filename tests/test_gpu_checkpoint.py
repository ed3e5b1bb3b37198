"""The safetensors loader on the device: a small Qwen3-MoE checkpoint in the
hub layout (per-expert projections, two shards and an index) is loaded with
``load_moe_layer(device="cuda")`` for every EP rank, and the router and
expert kernels run on the loaded weights.  The reference is the CPU oracle on
the parameters transformers' own ``from_pretrained`` builds from the same
files (its load-time packing, TF conversion_mapping.py qwen2_moe rules, and
the EXPERT dim-0 placement of
parallel/parallel/engine/model_parallel/models/qwen3_moe.py:64-65,81-84)."""

import pytest
import torch

from conftest import close_bf16, routing_check
from oracle import moe_oracle as O
from parallel_amd import ExpertPartition, load_moe_layer, ops
from test_checkpoint import _hub_state, _write_sharded

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
E, H, I, K, LAYERS, T = 8, 64, 32, 2, 2, 96


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory):
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM

    cfg = Qwen3MoeConfig(
        vocab_size=32, hidden_size=H, intermediate_size=64, moe_intermediate_size=I, num_hidden_layers=LAYERS,
        num_attention_heads=2, num_key_value_heads=1, head_dim=32, num_experts=E, num_experts_per_tok=K,
        decoder_sparse_step=1, mlp_only_layers=[], norm_topk_prob=True,
    )
    torch.manual_seed(3)
    model = Qwen3MoeForCausalLM(cfg)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape).mul(0.08).to(BF).float())  # bf16-representable weights
    path = tmp_path_factory.mktemp("qwen3moe_hub_gpu")
    cfg.save_pretrained(path)
    _write_sharded(_hub_state(model), path)
    loaded = Qwen3MoeForCausalLM.from_pretrained(str(path))  # local path only
    return path, loaded


@pytest.mark.parametrize("ep_size", [1, 2])
def test_loaded_weights_run_on_the_kernels(checkpoint, ep_size):
    path, loaded = checkpoint
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(9)).to(BF)
    d_out = torch.randn(T, H, generator=torch.Generator().manual_seed(10)).to(BF)
    for layer in range(LAYERS):
        mlp = loaded.model.layers[layer].mlp
        ref_gu = mlp.experts.gate_up_proj.detach()
        ref_dn = mlp.experts.down_proj.detach()
        ref_rw = mlp.gate.weight.detach()
        logits_ref = O.router_logits(x.float(), ref_rw)
        scores_ref, idx_ref = O.topk_softmax(logits_ref, K, True)
        total = torch.zeros(T, H)
        for rank in range(ep_size):
            w = load_moe_layer(path, layer, ep_size=ep_size, ep_rank=rank, device=DEV, dtype=BF)
            assert w.gate_up_proj.is_cuda and w.gate_up_proj.shape == (E // ep_size, 2 * I, H)
            logits, scores, idx = ops.router_fwd(x.to(DEV), w.router_weight, K, True)
            routing_check(idx, idx_ref, logits_ref)
            part = ExpertPartition(E, ep_size, rank)
            li, ls, _ = part.localize_routes(idx, scores)
            gu = w.gate_up_proj.clone().requires_grad_()
            dn = w.down_proj.clone().requires_grad_()
            out = ops.experts(x.to(DEV), li, ls, gu, dn)
            out.backward(d_out.to(DEV))
            rli, rls, _ = part.localize_routes(idx_ref, scores_ref)
            gr = ref_gu[part.start:part.stop].clone().requires_grad_()
            dr = ref_dn[part.start:part.stop].clone().requires_grad_()
            want = O.experts_grouped(x.float(), rli, rls, gr, dr)
            want.backward(d_out.float())
            close_bf16(out, want, f"layer {layer} rank {rank}/{ep_size} out")
            close_bf16(gu.grad, gr.grad, f"layer {layer} rank {rank}/{ep_size} d_gate_up")
            close_bf16(dn.grad, dr.grad, f"layer {layer} rank {rank}/{ep_size} d_down")
            total += out.float().cpu()
        # the ranks' shares sum to the whole layer on transformers' weights
        full = O.experts_grouped(x.float(), idx_ref, scores_ref, ref_gu, ref_dn)
        close_bf16(total, full, f"layer {layer} sum over {ep_size} ranks")

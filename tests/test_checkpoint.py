"""Qwen3-MoE safetensors -> one rank's packed expert weights (CPU tests).

The packing is pinned against transformers' own load-time conversion of the
hub layout (per-expert gate/up/down projections -> ``gate_up_proj [E,2I,H]``,
``down_proj [E,H,I]``): a tiny model is written in the hub layout as two
shards plus an index, loaded by ``from_pretrained`` from the local directory,
and its packed parameters compared with ``load_moe_layer`` for every EP rank.
"""

import json

import pytest
import torch
from safetensors.torch import save_file

from parallel_amd.checkpoint import checkpoint_files, load_moe_layer

E, H, I, LAYERS = 4, 16, 8, 2


def _tiny_model():
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM

    cfg = Qwen3MoeConfig(
        vocab_size=32, hidden_size=H, intermediate_size=32, moe_intermediate_size=I, num_hidden_layers=LAYERS,
        num_attention_heads=2, num_key_value_heads=1, head_dim=8, num_experts=E, num_experts_per_tok=2,
        decoder_sparse_step=1, mlp_only_layers=[], norm_topk_prob=True,
    )
    torch.manual_seed(0)
    model = Qwen3MoeForCausalLM(cfg)
    with torch.no_grad():
        for p in model.parameters():
            p.normal_(0, 0.1)
    return cfg, model


def _hub_state(model):
    """The model's state in the hub layout (one tensor per expert projection)."""
    out = {}
    for name, t in model.state_dict().items():
        if name.endswith("mlp.experts.gate_up_proj"):
            base = name[: -len("gate_up_proj")]
            half = t.shape[1] // 2  # gate rows first, then up
            for e in range(t.shape[0]):
                out[f"{base}{e}.gate_proj.weight"] = t[e, :half].contiguous()
                out[f"{base}{e}.up_proj.weight"] = t[e, half:].contiguous()
        elif name.endswith("mlp.experts.down_proj"):
            base = name[: -len("down_proj")]
            for e in range(t.shape[0]):
                out[f"{base}{e}.down_proj.weight"] = t[e].contiguous()
        else:
            out[name] = t.contiguous()
    return out


def _write_sharded(state, path):
    names = sorted(state)
    half = len(names) // 2
    shards = {"model-00001-of-00002.safetensors": names[:half], "model-00002-of-00002.safetensors": names[half:]}
    weight_map = {}
    for fname, keys in shards.items():
        save_file({k: state[k] for k in keys}, str(path / fname), metadata={"format": "pt"})
        weight_map.update({k: fname for k in keys})
    (path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))


@pytest.fixture(scope="module")
def hub_checkpoint(tmp_path_factory):
    from transformers import Qwen3MoeForCausalLM

    cfg, model = _tiny_model()
    path = tmp_path_factory.mktemp("qwen3moe_hub")
    cfg.save_pretrained(path)
    state = _hub_state(model)
    assert any(".mlp.experts.3.down_proj.weight" in k for k in state), "hub layout has per-expert tensors"
    _write_sharded(state, path)
    loaded = Qwen3MoeForCausalLM.from_pretrained(str(path))  # transformers' own conversion, local path only
    return path, model, loaded


@pytest.mark.parametrize("ep_size", [1, 2, 4])
def test_loader_matches_transformers_conversion(hub_checkpoint, ep_size):
    path, model, loaded = hub_checkpoint
    for layer in range(LAYERS):
        mlp = loaded.model.layers[layer].mlp
        for rank in range(ep_size):
            w = load_moe_layer(path, layer, ep_size=ep_size, ep_rank=rank)
            lo, hi = rank * E // ep_size, (rank + 1) * E // ep_size
            assert torch.equal(w.gate_up_proj, mlp.experts.gate_up_proj.detach()[lo:hi])
            assert torch.equal(w.down_proj, mlp.experts.down_proj.detach()[lo:hi])
            assert torch.equal(w.router_weight, mlp.gate.weight.detach())
            assert torch.equal(w.norm_weight, loaded.model.layers[layer].post_attention_layernorm.weight.detach())
            assert (w.partition.start, w.partition.stop) == (lo, hi)
        # and the round trip returns the original packed parameters
        assert torch.equal(mlp.experts.gate_up_proj.detach(), model.model.layers[layer].mlp.experts.gate_up_proj.detach())


def test_gate_rows_first(hub_checkpoint):
    path, model, _ = hub_checkpoint
    files = checkpoint_files(path)
    from safetensors import safe_open

    name = "model.layers.1.mlp.experts.2.up_proj.weight"
    with safe_open(str(files[name]), framework="pt") as fh:
        up = fh.get_tensor(name)
    w = load_moe_layer(path, 1, ep_size=2, ep_rank=1)  # local experts 2, 3
    assert torch.equal(w.gate_up_proj[0, I:], up)


def test_packed_checkpoint_is_sliced(tmp_path, hub_checkpoint):
    _, model, _ = hub_checkpoint
    state = {k: v.contiguous() for k, v in model.state_dict().items()}
    save_file(state, str(tmp_path / "model.safetensors"))
    w = load_moe_layer(tmp_path / "model.safetensors", 0, ep_size=2, ep_rank=0, dtype=torch.bfloat16)
    ref = model.model.layers[0].mlp.experts
    assert w.gate_up_proj.dtype == torch.bfloat16 and w.gate_up_proj.shape == (2, 2 * I, H)
    assert torch.equal(w.gate_up_proj, ref.gate_up_proj.detach()[:2].bfloat16())
    assert torch.equal(w.down_proj, ref.down_proj.detach()[:2].bfloat16())


def test_loader_errors(hub_checkpoint, tmp_path):
    path, _, _ = hub_checkpoint
    with pytest.raises(ValueError, match="divisible"):
        load_moe_layer(path, 0, ep_size=3, ep_rank=0)
    with pytest.raises(KeyError):
        load_moe_layer(path, 7)
    with pytest.raises(FileNotFoundError):
        load_moe_layer(tmp_path, 0)

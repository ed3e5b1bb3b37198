"""Seeded synthetic workloads for the benchmark configurations (C1-C5).

Shapes follow the Qwen3-MoE configs the benchmark is quoted on.  Small inputs
come from numpy's PCG64 (stable across torch versions, so CPU and GPU runs see
identical bits); the multi-GB weight tensors of the large configs are drawn
with torch's generator on the target device.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from .moe import MoeConfig


@dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    seq: int
    hidden: int
    experts: int  # global experts
    top_k: int
    intermediate: int
    norm_topk_prob: bool = True
    aux_coef: float = 0.001
    local_experts: int | None = None  # EP share (C3)
    sources: int = 1  # EP source ranks (C3)
    zipf_alpha: float | None = None  # C3 expert draw
    logit_bias_std: float | None = None  # C4 router imbalance
    router_std: float = 0.02
    dtype: str = "bf16"

    @property
    def tokens(self) -> int:
        return self.batch * self.seq

    @property
    def slots(self) -> int:
        return self.tokens * self.top_k

    def config(self) -> MoeConfig:
        return MoeConfig(
            hidden_size=self.hidden,
            num_experts=self.local_experts or self.experts,
            num_experts_per_tok=self.top_k,
            moe_intermediate_size=self.intermediate,
            norm_topk_prob=self.norm_topk_prob,
            router_aux_loss_coef=self.aux_coef,
        )

    def gemm_flops(self, rows: int | None = None) -> float:
        """Expert GEMM FLOPs for forward + backward: 18 * rows * H * I."""
        r = self.slots if rows is None else rows
        return 18.0 * r * self.hidden * self.intermediate


WORKLOADS: dict[str, Workload] = {
    "c1": Workload("c1", 1, 512, 256, 8, 2, 128, dtype="fp32"),
    "c2": Workload("c2", 4, 1024, 2048, 128, 8, 768),
    "c3": Workload("c3", 1, 4096, 2048, 128, 8, 768, local_experts=64, sources=2, zipf_alpha=1.2),
    "c4": Workload("c4", 8, 2048, 2048, 128, 8, 768, logit_bias_std=0.5, router_std=None),
    "c5": Workload("c5", 4, 2048, 4096, 128, 8, 1536),
}


def scaled(w: Workload, tokens: int, name: str | None = None) -> Workload:
    """The same layer with fewer tokens (for parity runs against the CPU oracle)."""
    from dataclasses import replace

    return replace(w, name=name or f"{w.name}_t{tokens}", batch=1, seq=tokens)


def _np_normal(rng: np.random.Generator, shape, std: float) -> np.ndarray:
    return (rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def make_block_inputs(w: Workload, seed: int = 0, device="cpu", dtype=torch.bfloat16,
                      weights_on_device_rng: bool = False) -> dict[str, torch.Tensor]:
    """x [T,H], router weight [E,H], gate_up [E,2I,H], down [E,H,I], d_out [T,H]
    (+ logit_bias [E] for C4).  Router std 0.02, or 1/sqrt(H) when the config asks
    for unit-variance logits; expert weights N(0, 0.02); x, d_out N(0, 1)."""
    rng = np.random.default_rng(np.random.PCG64(seed))
    T, H, E, I = w.tokens, w.hidden, w.local_experts or w.experts, w.intermediate
    router_std = w.router_std if w.router_std is not None else 1.0 / np.sqrt(H)
    out = {
        "x": torch.from_numpy(_np_normal(rng, (T, H), 1.0)),
        "router_weight": torch.from_numpy(_np_normal(rng, (w.experts, H), router_std)),
        "d_out": torch.from_numpy(_np_normal(rng, (T, H), 1.0)),
    }
    if w.logit_bias_std is not None:
        out["logit_bias"] = torch.from_numpy(_np_normal(rng, (w.experts,), w.logit_bias_std))
    if weights_on_device_rng:
        g = torch.Generator(device=device)
        g.manual_seed(seed + 1)
        gu = torch.randn(E, 2 * I, H, generator=g, device=device, dtype=torch.float32).mul_(0.02).to(dtype)
        dn = torch.randn(E, H, I, generator=g, device=device, dtype=torch.float32).mul_(0.02).to(dtype)
    else:
        gu = torch.from_numpy(_np_normal(rng, (E, 2 * I, H), 0.02))
        dn = torch.from_numpy(_np_normal(rng, (E, H, I), 0.02))
    tensors = {k: v.to(device=device, dtype=dtype if k != "logit_bias" else torch.float32) for k, v in out.items()}
    tensors["gate_up_proj"] = gu.to(device=device, dtype=dtype)
    tensors["down_proj"] = dn.to(device=device, dtype=dtype)
    return tensors


def ep_receive_buffer(w: Workload, seed: int = 0, empty_local_experts: int = 4):
    """C3: one rank's receive layout for an EP group of ``w.sources`` ranks.

    Every source rank routes its tokens to ``top_k`` distinct global experts drawn
    with weight rank^-alpha over a seeded permutation of the experts (Gumbel
    top-k), with ``empty_local_experts`` of this rank's experts given weight 0.
    Scores are a renormalised softmax over random logits of the chosen experts.
    Returns numpy arrays: per-source global indices [sources, T, k] int64, scores
    [sources, T, k] f32, and the receive layout of rank 0: source-rank-major rows,
    in flat (token, k) order inside a source block (token_dispatch.py:116) —
    (row_source [R], row_token [R], row_local_expert [R], row_score [R]).
    """
    rng = np.random.default_rng(np.random.PCG64(seed + 17))
    E, El, k, T = w.experts, w.local_experts or w.experts, w.top_k, w.tokens
    ranks = np.empty(E, dtype=np.float64)
    ranks[rng.permutation(E)] = np.arange(1, E + 1, dtype=np.float64)
    weight = ranks ** (-(w.zipf_alpha or 1.0))
    weight[rng.choice(El, size=empty_local_experts, replace=False)] = 0.0
    logw = np.where(weight > 0, np.log(np.maximum(weight, 1e-300)), -np.inf)
    idx = np.empty((w.sources, T, k), dtype=np.int64)
    sc = np.empty((w.sources, T, k), dtype=np.float32)
    for s in range(w.sources):
        gumbel = -np.log(-np.log(rng.random((T, E))))
        keys = logw[None, :] + gumbel
        top = np.argsort(-keys, axis=1, kind="stable")[:, :k]
        idx[s] = top
        lg = rng.standard_normal((T, k)).astype(np.float32)
        p = np.exp(lg - lg.max(axis=1, keepdims=True))
        sc[s] = (p / p.sum(axis=1, keepdims=True)).astype(np.float32)
    rows_src, rows_tok, rows_exp, rows_sc = [], [], [], []
    for s in range(w.sources):
        flat = idx[s].reshape(-1)
        keep = np.nonzero(flat // El == 0)[0]  # owner rank 0, flat (token, k) order
        rows_src.append(np.full(keep.size, s, dtype=np.int64))
        rows_tok.append(keep // k)
        rows_exp.append(flat[keep])
        rows_sc.append(sc[s].reshape(-1)[keep])
    return idx, sc, (np.concatenate(rows_src), np.concatenate(rows_tok), np.concatenate(rows_exp),
                     np.concatenate(rows_sc))

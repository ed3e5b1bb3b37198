"""CPU oracle for the Qwen3-MoE expert path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or, for the
CPU baseline, as the thing timed on the host).  The product path
(``parallel_amd``) never imports it and has no CPU fallback.

It restates, on the CPU, the reference path's arithmetic:
  * router           TF/models/qwen3_moe/modeling_qwen3_moe.py:258-267
  * experts          TF/integrations/moe.py:377-478 (grouped form) and
                     TF/models/qwen3_moe/modeling_qwen3_moe.py:222-246 (eager form)
  * SwiGLU gate      TF/integrations/moe.py:509-521
  * aux loss         TF/models/qwen3_moe/modeling_qwen3_moe.py:514-593,
                     parallel/parallel/engine/model_parallel/sequence_parallel.py:239-280
  * EP ownership     parallel/parallel/engine/model_parallel/expert_parallel.py:12-60
  * token dispatch   parallel/parallel/engine/model_parallel/token_dispatch.py:86-174
  * block-input norm TF/models/qwen3_moe/modeling_qwen3_moe.py:294-299 (Qwen3MoeRMSNorm, the
                     post_attention_layernorm applied before the MoE block at :345)
  * FSDP grad bucket parallel/parallel/engine/_dp_param_unit.py:200-202 (padded rows),
                     :268-277 (bucket layout), :395-417 (rank-major packing of the
                     reduce-scatter input)
where TF/ is transformers (the reference pins 5.14.1, uv.lock:2274-2275; the
5.15.0 installed here is what the golden vectors were generated with).
Integer work (sort keys, permutations, counts, splits) is numpy; floating
point work is torch fp32 on the CPU with autograd for the backward.

Parity pins (tests/test_oracle.py): golden vectors written by transformers'
own Qwen3MoeSparseMoeBlock (tests/golden/), the reference's known-answer
tests for localize_routes and the zero-receive dispatch, two independent
formulations of the experts (grouped vs eager loop), balanced routing giving
aux == top_k, brute-force permutations on tiny inputs and finite differences.
The ordering of exactly tied router probabilities is implementation-defined
in torch.topk and is not pinned; the oracle and the kernels both put the
lower expert index first, and tests count ties separately.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

# ----------------------------------------------------------------- norm


def rmsnorm(hidden: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Qwen3MoeRMSNorm.forward (modeling_qwen3_moe.py:294-299): fp32 statistics,
    then weight * hs.to(input dtype) in the input dtype (autograd-capable)."""
    input_dtype = hidden.dtype
    hs = hidden.to(torch.float32)
    variance = hs.pow(2).mean(-1, keepdim=True)
    hs = hs * torch.rsqrt(variance + eps)
    return weight * hs.to(input_dtype)


def norm_router_aux(hidden, norm_weight, router_weight, top_k, *, eps, norm_topk_prob, attention_mask=None):
    """The step before the MoE block: post_attention_layernorm (:345), the router
    (:258-267, fp32 logits) and the aux loss over the same logits (:514-593)."""
    x = rmsnorm(hidden, norm_weight, eps)
    logits = router_logits(x.reshape(-1, x.shape[-1]), router_weight)
    scores, indices = topk_softmax(logits, top_k, norm_topk_prob)
    aux = load_balancing_loss((logits,), router_weight.shape[0], top_k, attention_mask)
    return x, logits, scores, indices, aux


# ----------------------------------------------------------------- router


def router_logits(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """F.linear of modeling_qwen3_moe.py:260, in fp32 (x.float() @ w.float().T)."""
    return x.float() @ weight.float().t()


def topk_softmax(logits: torch.Tensor, top_k: int, norm_topk_prob: bool):
    """softmax(dtype=float) -> topk -> optional renorm (modeling_qwen3_moe.py:261-265)."""
    probs = torch.softmax(logits, dim=-1, dtype=torch.float)
    values, indices = torch.topk(probs, top_k, dim=-1)
    if norm_topk_prob:
        values = values / values.sum(dim=-1, keepdim=True)
    return values.to(logits.dtype), indices


def topk_ties(logits: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """Tokens whose selected experts or their order depend on how torch.topk breaks
    exact ties (unpinned): two equal probabilities among the first k+1 sorted
    values, i.e. inside the top k (their order is ambiguous) or at the k-th /
    (k+1)-th boundary (the selection is ambiguous).  With k == E there is no
    boundary, but ties inside still make the order ambiguous."""
    probs = torch.softmax(logits.float(), dim=-1)
    k = indices.shape[1]
    srt = torch.sort(probs, dim=-1, descending=True).values
    last = min(k, probs.shape[1] - 1)  # adjacent pairs (i, i+1) with i < last decide the top k
    if last <= 0:
        return torch.zeros(probs.shape[0], dtype=torch.bool)
    return (srt[:, :last] == srt[:, 1:last + 1]).any(dim=1)


# --------------------------------------------------------------- permutation


def stable_permutation(ids: np.ndarray, divisor: int, num_buckets: int):
    """Stable sort of flat slots by bucket = id // divisor, sentinels (bucket >= nb) last.

    The expert sort of TF/integrations/moe.py:393 (with divisor 1) and the
    owner sort of token_dispatch.py:114-116 (stable argsort by owner rank).
    Returns (perm, pos_of_slot, counts, offsets) as int64 numpy arrays;
    counts = histc/bincount over real buckets (moe.py:401-402,
    token_dispatch.py:88-90), offsets = int32 cumsum (moe.py:403).
    """
    ids = np.asarray(ids, dtype=np.int64).reshape(-1)
    buckets = ids // divisor
    buckets = np.where((buckets < 0) | (buckets >= num_buckets), num_buckets, buckets)
    perm = np.argsort(buckets, kind="stable")
    pos = np.empty_like(perm)
    pos[perm] = np.arange(perm.size)
    counts = np.bincount(buckets, minlength=num_buckets + 1)[:num_buckets]
    offsets = np.cumsum(counts).astype(np.int32)
    return perm.astype(np.int64), pos.astype(np.int64), counts.astype(np.int64), offsets


# ------------------------------------------------------------------ experts


def _grouped_linear_loop(inputs: torch.Tensor, weight: torch.Tensor, offsets: torch.Tensor) -> torch.Tensor:
    """Per-expert inputs[rows_e] @ weight[e].T (the loop of TF integrations/moe.py:179-202,
    with weight given as [E, out, in]); rows at or beyond offsets[-1] are zero."""
    pieces = []
    start = 0
    for e, end in enumerate(offsets.tolist()):
        if end > start:
            pieces.append(inputs[start:end] @ weight[e].t())
        start = end
    tail = inputs.shape[0] - start
    if tail:
        pieces.append(inputs.new_zeros(tail, weight.shape[1]))
    if not pieces:
        return inputs.new_zeros(0, weight.shape[1])
    return torch.cat(pieces, dim=0)


def _grouped_linear_torch(inputs: torch.Tensor, weight: torch.Tensor, offsets: torch.Tensor) -> torch.Tensor:
    """F.grouped_mm with a transposed weight view (TF integrations/moe.py:331-332,368)."""
    return F.grouped_mm(inputs.to(weight.dtype), weight.transpose(-2, -1), offs=offsets)


def experts_grouped(hidden, top_k_index, top_k_weights, gate_up_proj, down_proj, *, use_grouped_mm=False,
                    compute_dtype=torch.float32):
    """grouped_mm_experts_forward (TF integrations/moe.py:377-478), restated.

    The sort is stable (torch.sort there is not; outputs do not depend on the
    in-group order).  compute_dtype float32 is the accuracy oracle; the CPU
    baseline runs the config dtype through F.grouped_mm.
    """
    num_experts = gate_up_proj.shape[0]
    T, H = hidden.shape
    k = top_k_index.shape[-1]
    h = hidden.to(compute_dtype)
    gu = gate_up_proj.to(compute_dtype)
    dn = down_proj.to(compute_dtype)
    sample_weights = top_k_weights.reshape(-1)
    expert_ids = top_k_index.reshape(-1)
    expert_ids_g, perm = torch.sort(expert_ids, stable=True)
    selected = h[perm // k]
    sample_weights_g = sample_weights[perm]
    counts = torch.histc(expert_ids_g.float(), bins=num_experts, min=0, max=num_experts - 1)
    offsets = torch.cumsum(counts, dim=0, dtype=torch.int32)
    sentinel = (expert_ids_g >= num_experts).unsqueeze(-1)
    selected = selected.masked_fill(sentinel, 0.0)
    lin = _grouped_linear_torch if use_grouped_mm else _grouped_linear_loop
    proj = lin(selected, gu, offsets)
    gate, up = proj.chunk(2, dim=-1)
    act = F.silu(gate) * up
    proj = lin(act, dn, offsets)
    weighted = proj * sample_weights_g.unsqueeze(-1)
    weighted = weighted.masked_fill(sentinel, 0.0)
    inv_perm = torch.empty_like(perm)
    inv_perm[perm] = torch.arange(perm.size(0))
    weighted = weighted[inv_perm]
    out = weighted.view(T, k, H).sum(dim=1)
    return out.to(hidden.dtype)


def experts_eager(hidden, top_k_index, top_k_weights, gate_up_proj, down_proj):
    """Qwen3MoeExperts.forward eager loop (modeling_qwen3_moe.py:222-246), fp32; sentinels skipped."""
    num_experts = gate_up_proj.shape[0]
    h = hidden.float()
    out = torch.zeros_like(h)
    for e in range(num_experts):
        tok, pos_k = torch.where(top_k_index == e)  # the (token, k) pairs routed to e
        if tok.numel() == 0:
            continue
        cur = h[tok]
        gate, up = (cur @ gate_up_proj[e].float().t()).chunk(2, dim=-1)
        y = (F.silu(gate) * up) @ down_proj[e].float().t()
        y = y * top_k_weights[tok, pos_k, None].float()
        out = out.index_add(0, tok, y)
    return out


# ----------------------------------------------------------------- aux loss


def load_balancing_loss(gate_logits, num_experts, top_k, attention_mask=None):
    """load_balancing_loss_func (modeling_qwen3_moe.py:514-593), both mask branches."""
    if isinstance(gate_logits, torch.Tensor):
        gate_logits = (gate_logits,)
    logits = torch.cat(list(gate_logits), dim=0)
    routing_weights = torch.softmax(logits, dim=-1)
    _, selected = torch.topk(routing_weights, top_k, dim=-1)
    expert_mask = F.one_hot(selected, num_experts)
    if attention_mask is None:
        tokens_per_expert = torch.mean(expert_mask.float(), dim=0)
        router_prob_per_expert = torch.mean(routing_weights, dim=0)
    else:
        b, s = attention_mask.shape
        layers = logits.shape[0] // (b * s)
        m = attention_mask[None, :, :, None, None].expand(layers, b, s, top_k, num_experts)
        m = m.reshape(-1, top_k, num_experts).float()
        tokens_per_expert = torch.sum(expert_mask.float() * m, dim=0) / torch.sum(m, dim=0)
        mp = attention_mask[None, :, :, None].expand(layers, b, s, num_experts).reshape(-1, num_experts).float()
        router_prob_per_expert = torch.sum(routing_weights * mp, dim=0) / torch.sum(mp, dim=0)
    return torch.sum(tokens_per_expert * router_prob_per_expert.unsqueeze(0)) * num_experts


# --------------------------------------------------------- EP restatements


def localize_routes(global_indices, scores, num_experts, ep_size, ep_rank):
    """ExpertPartition.localize_routes (expert_parallel.py:50-60)."""
    local_count = num_experts // ep_size
    start = ep_rank * local_count
    mask = torch.div(global_indices, local_count, rounding_mode="floor") == ep_rank
    return (global_indices - start).masked_fill(~mask, local_count), scores.masked_fill(~mask, 0), mask


def dispatch_send(hidden, global_indices, scores, local_count, ep_size):
    """Send side of TokenDispatcher.dispatch (token_dispatch.py:101-125).

    Returns (send_hidden, send_local_experts, send_scores, source_tokens, send_splits).
    """
    tokens, top_k = global_indices.shape
    flat_experts = global_indices.reshape(-1)
    flat_scores = scores.reshape(-1)
    source_tokens = torch.arange(tokens).unsqueeze(1).expand(tokens, top_k).reshape(-1)
    destinations = torch.div(flat_experts, local_count, rounding_mode="floor")
    order = torch.argsort(destinations, stable=True)
    destinations = destinations[order]
    source_tokens = source_tokens[order]
    send_splits = tuple(torch.bincount(destinations, minlength=ep_size).tolist())
    send_hidden = hidden.index_select(0, source_tokens)
    send_experts = flat_experts[order] - destinations * local_count
    send_scores = flat_scores[order]
    return send_hidden, send_experts, send_scores, source_tokens, send_splits


def combine_index_add(returned, source_tokens, num_source_tokens):
    """TokenDispatcher.combine after the exchange (token_dispatch.py:169-174)."""
    result = torch.zeros((num_source_tokens, *returned.shape[1:]), dtype=returned.dtype)
    return result.index_add(0, source_tokens, returned)


# -------------------------------------------------------------- whole block


def block_forward_backward(x, router_weight, gate_up_proj, down_proj, d_out, *, top_k, norm_topk_prob, aux_coef,
                           logit_bias=None, compute_dtype=torch.float32, use_grouped_mm=False, need_grads=True):
    """Router -> experts -> (out, aux); backward of <out, d_out> + aux_coef * aux.

    The router logits are fp32 (x.float() @ w.float().T).  Returns a dict with
    logits, scores, indices, out, aux and, when need_grads, the gradients
    dx, d_router, d_gate_up, d_down (in the dtype of the leaves).
    """
    leaves = [t.detach().clone().requires_grad_(need_grads) for t in (x, router_weight, gate_up_proj, down_proj)]
    xl, rw, gu, dn = leaves
    logits = router_logits(xl, rw)
    if logit_bias is not None:
        logits = logits + logit_bias.float()
    scores, indices = topk_softmax(logits, top_k, norm_topk_prob)
    out = experts_grouped(xl.to(compute_dtype), indices, scores, gu, dn, use_grouped_mm=use_grouped_mm,
                          compute_dtype=compute_dtype)
    aux = load_balancing_loss((logits,), router_weight.shape[0], top_k)
    res = {"logits": logits.detach(), "scores": scores.detach(), "indices": indices, "out": out.detach(),
           "aux": aux.detach()}
    if need_grads:
        loss = (out.float() * d_out.float()).sum() + aux_coef * aux
        loss.backward()
        res.update(dx=xl.grad, d_router=rw.grad, d_gate_up=gu.grad, d_down=dn.grad)
    return res


def make_leaves(x, router_weight, gate_up_proj, down_proj):
    """Detached leaf copies that require grad (for repeated timed steps)."""
    return [t.detach().clone().requires_grad_(True) for t in (x, router_weight, gate_up_proj, down_proj)]


def reference_step(leaves, d_out, *, top_k, norm_topk_prob, aux_coef, compute_dtype, use_grouped_mm=True,
                   logit_bias=None):
    """One forward + backward of the reference op sequence on existing leaves
    (grads are reset first); the step the CPU baseline times."""
    for t in leaves:
        t.grad = None
    xl, rw, gu, dn = leaves
    logits = router_logits(xl, rw)
    if logit_bias is not None:
        logits = logits + logit_bias.float()
    scores, indices = topk_softmax(logits, top_k, norm_topk_prob)
    out = experts_grouped(xl, indices, scores, gu, dn, use_grouped_mm=use_grouped_mm, compute_dtype=compute_dtype)
    aux = load_balancing_loss((logits,), rw.shape[0], top_k)
    torch.autograd.backward([out, aux], [d_out.to(out.dtype), torch.tensor(aux_coef)])
    return out


# ----------------------------------------------------------------- FSDP gradient bucket


def fsdp_bucket_layout(shapes, world_size: int):
    """Per parameter (padded_rows, bucket_offset, padded_numel), and the unit's
    bucket_numel.  padded_rows = ceil(rows / world) (_dp_param_unit.py:200);
    parameters take consecutive flat offsets in unit order (:268-277)."""
    layout, offset = [], 0
    for shape in shapes:
        padded_rows = (shape[0] + world_size - 1) // world_size
        padded_numel = padded_rows
        for size in shape[1:]:
            padded_numel *= size
        layout.append((padded_rows, offset, padded_numel))
        offset += padded_numel
    return layout, offset


def fsdp_pack_grads(grads, world_size: int, dtype=None, shapes=None):
    """The reduce-scatter input [world, bucket_numel] of one FSDP unit: rank r's
    chunk holds rows [r * padded_rows, ...) of every parameter's gradient at the
    parameter's offset, zeros elsewhere (_dp_param_unit.py:395-417).  A None
    gradient (its parameter's shape from ``shapes``) leaves its slots zero."""
    if shapes is None:
        shapes = [tuple(g.shape) for g in grads]
    layout, numel = fsdp_bucket_layout(shapes, world_size)
    first = next(g for g in grads if g is not None)
    bucket = torch.zeros(world_size, numel, dtype=dtype or first.dtype)
    for g, (padded_rows, offset, padded_numel) in zip(grads, layout):
        if g is None:
            continue
        for rank in range(world_size):
            start = rank * padded_rows
            rows = min(padded_rows, max(g.shape[0] - start, 0))
            if not rows:
                continue
            dest = bucket[rank].narrow(0, offset, padded_numel).view(padded_rows, *g.shape[1:])
            dest[:rows].copy_(g.narrow(0, start, rows))
    return bucket


"""torch.library ops over the gfx950 C-ABI kernels, with fake kernels and autograd.

Every op runs on torch's current stream of the input's device and allocates
its outputs and workspaces from the caching allocator; none synchronises with
the host.  There is no CPU implementation: CPU tensors raise ``ValueError``.

Ops (namespace ``parallel_amd``):
  router_fwd / router_bwd          router GEMM + top-k softmax (+ backward)
  router_fwd_bf16                  the same with the logits of a bf16 linear (the reference's AMP)
  router_topk                      top-k softmax of given fp32 logits
  aux_loss_fwd / aux_loss_bwd      Switch load-balancing loss
  permute_fwd                      stable sort of routed slots + row gather
  experts_fwd / experts_bwd        permute -> SwiGLU grouped GEMMs -> combine
  dispatch_fwd / dispatch_bwd      owner-rank sort for TokenDispatcher
  combine_rows_fwd / _bwd          gather-form index_add back to source tokens
  rmsnorm_fwd / rmsnorm_bwd        post_attention_layernorm of the block input (+ backward)
  router_aux_fwd                   router_fwd plus the aux loss from the same top-k
  moe_block_fwd                    router, aux loss and experts as one op (moe_block)

experts_bwd_kernels issues the expert backward's launches with a caller-chosen
weight-gradient target (fsdp_bucket uses it to write into an FSDP bucket).
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib
from ._lib import call, ptr

LIB = "parallel_amd"
BF16 = torch.bfloat16


# ---------------------------------------------------------------- validation


def _require_gpu(*tensors: Tensor | None) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError(
                f"parallel_amd kernels run on the GPU only; got a tensor on {t.device} "
                "(there is no CPU implementation)"
            )


def _require_bf16(name: str, t: Tensor) -> None:
    if t.dtype != BF16:
        raise ValueError(f"{name} must be bfloat16 for the MFMA kernels, got {t.dtype}")


def _stream(t: Tensor) -> int:
    return _lib.stream_of(t)


def _ws(nbytes: int, device) -> Tensor:
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)


def _ids64(t: Tensor) -> Tensor:
    return t.to(torch.int64).contiguous()


# ------------------------------------------------------------------- router


@torch.library.custom_op(f"{LIB}::router_topk", mutates_args=())
def router_topk(logits: Tensor, top_k: int, norm_topk_prob: bool) -> tuple[Tensor, Tensor]:
    """(scores [T,k] f32, indices [T,k] int64) of softmax(logits) (TF modeling_qwen3_moe.py:261-265)."""
    _require_gpu(logits)
    logits = logits.float().contiguous()
    T, E = logits.shape
    scores = torch.empty(T, top_k, dtype=torch.float32, device=logits.device)
    idx = torch.empty(T, top_k, dtype=torch.int64, device=logits.device)
    call("moe_router_topk_fwd", ptr(logits), ptr(scores), ptr(idx), T, E, top_k, int(norm_topk_prob),
         _stream(logits))
    return scores, idx


@router_topk.register_fake
def _(logits, top_k, norm_topk_prob):
    T = logits.shape[0]
    return logits.new_empty(T, top_k, dtype=torch.float32), logits.new_empty(T, top_k, dtype=torch.int64)


@torch.library.custom_op(f"{LIB}::router_fwd", mutates_args=())
def router_fwd(x: Tensor, weight: Tensor, top_k: int, norm_topk_prob: bool,
               logit_bias: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """Qwen3MoeTopKRouter.forward (TF modeling_qwen3_moe.py:258-267) with fp32 logits.

    ``logit_bias`` [E] (fp32, not differentiated) is added to the logits before
    the softmax; the reference router has none, the imbalanced benchmark
    harness uses it."""
    _require_gpu(x, weight)
    if x.dtype == weight.dtype == torch.float32:
        return _router_fwd_f32(x.contiguous(), weight.contiguous(), top_k, norm_topk_prob, logit_bias)
    _require_bf16("router input", x)
    _require_bf16("router weight", weight)
    x = x.contiguous()
    weight = weight.contiguous()
    T, H = x.shape
    E = weight.shape[0]
    logits = torch.empty(T, E, dtype=torch.float32, device=x.device)
    scores = torch.empty(T, top_k, dtype=torch.float32, device=x.device)
    idx = torch.empty(T, top_k, dtype=torch.int64, device=x.device)
    bias = None if logit_bias is None else logit_bias.to(device=x.device, dtype=torch.float32).contiguous()
    ws = _ws(_lib.load().moe_router_fwd_workspace_bytes(T, H, E), x.device)
    call("moe_router_fwd", ptr(x), ptr(weight), ptr(bias), ptr(logits), None, ptr(scores), ptr(idx), T, H, E, top_k,
         int(norm_topk_prob), ptr(ws), ws.numel(), _stream(x), tag="router_fwd")
    return logits, scores, idx


@router_fwd.register_fake
def _(x, weight, top_k, norm_topk_prob, logit_bias=None):
    T, E = x.shape[0], weight.shape[0]
    return (x.new_empty(T, E, dtype=torch.float32), x.new_empty(T, top_k, dtype=torch.float32),
            x.new_empty(T, top_k, dtype=torch.int64))


def _one_group(T: int, device) -> Tensor:
    """Inclusive offsets [T] of a single group (a fill kernel, no host copy)."""
    return torch.full((1,), T, dtype=torch.int32, device=device)


def _router_fwd_f32(x, weight, top_k, norm_topk_prob, logit_bias):
    """Qwen3MoeTopKRouter.forward of an fp32 module (TF modeling_qwen3_moe.py:258-267,
    F.linear in fp32): the logits GEMM on fp32 MFMA, then the top-k softmax."""
    T, H = x.shape
    E = weight.shape[0]
    if weight.shape[1] != H:
        raise ValueError(f"router weight {tuple(weight.shape)} does not match hidden {H}")
    s = _stream(x)
    logits = torch.empty(T, E, dtype=torch.float32, device=x.device)
    _f32_gemm(x, weight, _one_group(T, x.device), 1, 0, T, E, H, (H, 1), (1, H), 0, logits, (E, 1), 0, False, s,
              "router_fwd")
    if logit_bias is not None:
        logits.add_(logit_bias.to(device=x.device, dtype=torch.float32))
    scores = torch.empty(T, top_k, dtype=torch.float32, device=x.device)
    idx = torch.empty(T, top_k, dtype=torch.int64, device=x.device)
    call("moe_router_topk_fwd", ptr(logits), ptr(scores), ptr(idx), T, E, top_k, int(norm_topk_prob), s,
         tag="router_fwd")
    return logits, scores, idx


def _router_bwd_f32(x, weight, logits, indices, d_logits, d_scores, norm_topk_prob, token_weight, stats, d_aux,
                    dw_target):
    """router_bwd_kernels for fp32 modules: the fp32 logits gradient (top-k
    backward, plus the aux loss's), then dx = dL·W and dW = dLᵀ·x on fp32 MFMA."""
    T, H = x.shape
    E = weight.shape[0]
    k = indices.shape[1]
    s = _stream(x)
    if d_logits is not None:
        dl = d_logits.float().contiguous().clone()
        accumulate = 1
    else:
        dl = torch.empty(T, E, dtype=torch.float32, device=x.device)
        accumulate = 0
    if d_scores is None:
        d_scores = torch.zeros(T, k, dtype=torch.float32, device=x.device)
    call("moe_router_topk_bwd", ptr(logits), ptr(indices), ptr(d_scores.float().contiguous()), T, E, k,
         int(norm_topk_prob), ptr(dl), accumulate, None, s, tag="router_topk_bwd")
    if d_aux is not None:
        tw = None if token_weight is None else token_weight.float().contiguous()
        call("moe_aux_loss_bwd", ptr(logits), ptr(tw), ptr(stats), ptr(d_aux.float().reshape(1).contiguous()), T, E,
             ptr(dl), 1, s, tag="router_topk_bwd")
    one = _one_group(T, x.device)
    dx = torch.empty(T, H, dtype=torch.float32, device=x.device)
    _f32_gemm(dl, weight, one, 1, 0, T, H, E, (E, 1), (H, 1), 0, dx, (H, 1), 0, False, s, "router_gemm_bwd")
    fresh = dw_target is None or dw_target.dtype != torch.float32
    dw = torch.empty(E, H, dtype=torch.float32, device=x.device) if fresh else dw_target
    _f32_gemm(dl, x, one, 1, 1, E, H, T, (1, E), (H, 1), 0, dw, (H, 1), 0, not fresh, s, "router_gemm_bwd")
    if dw_target is not None and fresh:
        dw_target.add_(dw)
    return dx, (None if dw_target is not None else dw)


def router_bwd_kernels(x: Tensor, weight: Tensor, logits: Tensor, indices: Tensor, d_logits: Tensor | None,
                       d_scores: Tensor | None, norm_topk_prob: bool, token_weight: Tensor | None = None,
                       stats: Tensor | None = None, d_aux: Tensor | None = None,
                       dw_target: Tensor | None = None, bf16_logits: bool = False) -> tuple[Tensor, Tensor | None]:
    """The router backward's launches: (dx [T,H] bf16, dweight [E,H] bf16).

    d_logits is the logits' incoming gradient (fp32, may be None); with
    ``d_aux`` (and the ``stats``/``token_weight`` of router_aux_fwd) the aux
    loss's logits gradient is added in the same top-k backward pass.  With
    ``dw_target`` (the router weight's existing bf16 gradient) the weight
    gradient is added into it and None is returned in its place.  With
    ``bf16_logits`` the logits were bf16 (router_fwd_bf16) and d_logits is
    their bf16 gradient: the softmax path's gradient is rounded to bf16
    before it is added, as autograd adds a bf16 tensor's gradients.  fp32
    modules get fp32 gradients from the fp32 kernels."""
    if x.dtype == weight.dtype == torch.float32:
        return _router_bwd_f32(x.contiguous(), weight.contiguous(), logits, indices, d_logits, d_scores,
                               norm_topk_prob, token_weight, stats, d_aux, dw_target)
    x = x.contiguous()
    weight = weight.contiguous()
    T, H = x.shape
    E = weight.shape[0]
    k = indices.shape[1]
    s = _stream(x)
    d_add = None if d_logits is None else d_logits.float().contiguous()
    dl_bf16 = torch.empty(T, E, dtype=BF16, device=x.device)
    if d_scores is None:
        d_scores = torch.zeros(T, k, dtype=torch.float32, device=x.device)
    d_scores = d_scores.float().contiguous()
    # Only the bf16 d_logits feeds the GEMMs; the incoming logits gradient is
    # read, not copied.
    if bf16_logits:
        tw = None if (d_aux is None or token_weight is None) else token_weight.float().contiguous()
        da = None if d_aux is None else d_aux.float().reshape(1).contiguous()
        call("moe_router_bf16_logits_bwd", ptr(logits), ptr(indices), ptr(d_scores), ptr(d_add), ptr(tw),
             ptr(stats if d_aux is not None else None), ptr(da), T, E, k, int(norm_topk_prob), ptr(dl_bf16), s,
             tag="router_topk_bwd")
    elif d_aux is not None:
        tw = None if token_weight is None else token_weight.float().contiguous()
        da = d_aux.float().reshape(1).contiguous()
        call("moe_router_aux_bwd_bf16", ptr(logits), ptr(indices), ptr(d_scores), ptr(d_add), ptr(tw), ptr(stats),
             ptr(da), T, E, k, int(norm_topk_prob), ptr(dl_bf16), s, tag="router_topk_bwd")
    else:
        call("moe_router_topk_bwd_bf16", ptr(logits), ptr(indices), ptr(d_scores), ptr(d_add), T, E, k,
             int(norm_topk_prob), ptr(dl_bf16), s, tag="router_topk_bwd")
    return _router_gemm_bwd(x, weight, dl_bf16, dw_target)


def _router_gemm_bwd(x: Tensor, weight: Tensor, dl_bf16: Tensor,
                     dw_target: Tensor | None) -> tuple[Tensor, Tensor | None]:
    """The router linear's backward from the bf16 logits gradient: (dx [T,H]
    bf16, dweight [E,H], or None when added into ``dw_target``)."""
    T, H = x.shape
    E = weight.shape[0]
    dx = torch.empty(T, H, dtype=BF16, device=x.device)
    dw = dw_target if dw_target is not None else torch.empty(E, H, dtype=weight.dtype, device=x.device)
    ws = _ws(_lib.load().moe_router_logits_bwd_workspace_bytes(T, H, E), x.device)
    call("moe_router_logits_bwd", ptr(dl_bf16), ptr(x), ptr(weight), ptr(dx), ptr(dw), int(dw_target is not None),
         T, H, E, ptr(ws), ws.numel(), _stream(x), tag="router_gemm_bwd")
    return dx, (None if dw_target is not None else dw)


@torch.library.custom_op(f"{LIB}::router_bwd", mutates_args=())
def router_bwd(x: Tensor, weight: Tensor, logits: Tensor, indices: Tensor, d_logits: Tensor | None,
               d_scores: Tensor | None, norm_topk_prob: bool) -> tuple[Tensor, Tensor]:
    """(dx [T,H] bf16, dweight [E,H] bf16) through top-k/renorm/softmax and the router GEMM."""
    return router_bwd_kernels(x, weight, logits, indices, d_logits, d_scores, norm_topk_prob)


@router_bwd.register_fake
def _(x, weight, logits, indices, d_logits, d_scores, norm_topk_prob):
    return torch.empty_like(x), torch.empty_like(weight)


def _router_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)
    x, weight, top_k, norm, _bias = inputs
    logits, _, idx = output
    ctx.save_for_backward(x, weight, logits, idx)
    ctx.norm = norm
    ctx.mark_non_differentiable(idx)


def _router_backward(ctx, d_logits, d_scores, _d_idx):
    x, weight, logits, idx = ctx.saved_tensors
    dx, dw = router_bwd(x, weight, logits, idx, d_logits, d_scores, ctx.norm)
    return dx, dw, None, None, None


router_fwd.register_autograd(_router_backward, setup_context=_router_setup)


@torch.library.custom_op(f"{LIB}::router_fwd_bf16", mutates_args=())
def router_fwd_bf16(x: Tensor, weight: Tensor, top_k: int, norm_topk_prob: bool,
                    logit_bias: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """router_fwd with the logits of a bf16 linear, as Qwen3MoeTopKRouter computes
    them under the reference's bf16 autocast (parallel/parallel/engine/engine.py:141,
    TF modeling_qwen3_moe.py:258-267): (logits [T,E] bf16, scores [T,k] bf16,
    indices, and the same logits in fp32 for the backward).  The softmax and
    top-k run in fp32 on the bf16 logits; the scores are rounded to bf16."""
    _require_gpu(x, weight)
    _require_bf16("router input", x)
    _require_bf16("router weight", weight)
    x = x.contiguous()
    weight = weight.contiguous()
    T, H = x.shape
    E = weight.shape[0]
    dev = x.device
    logits = torch.empty(T, E, dtype=torch.float32, device=dev)
    logits_b = torch.empty(T, E, dtype=BF16, device=dev)
    scores = torch.empty(T, top_k, dtype=torch.float32, device=dev)
    idx = torch.empty(T, top_k, dtype=torch.int64, device=dev)
    bias = None if logit_bias is None else logit_bias.to(device=dev, dtype=torch.float32).contiguous()
    ws = _ws(_lib.load().moe_router_fwd_workspace_bytes(T, H, E), dev)
    call("moe_router_fwd", ptr(x), ptr(weight), ptr(bias), ptr(logits), ptr(logits_b), ptr(scores), ptr(idx), T, H,
         E, top_k, int(norm_topk_prob), ptr(ws), ws.numel(), _stream(x), tag="router_fwd")
    # scores hold bf16 values; the cast is exact
    return logits_b, scores.to(BF16), idx, logits


@router_fwd_bf16.register_fake
def _(x, weight, top_k, norm_topk_prob, logit_bias=None):
    T, E = x.shape[0], weight.shape[0]
    return (x.new_empty(T, E, dtype=BF16), x.new_empty(T, top_k, dtype=BF16),
            x.new_empty(T, top_k, dtype=torch.int64), x.new_empty(T, E, dtype=torch.float32))


def _router_bf16_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)
    x, weight, top_k, norm, _bias = inputs
    _, _, idx, logits = output
    ctx.save_for_backward(x, weight, logits, idx)
    ctx.norm = norm
    ctx.mark_non_differentiable(idx, logits)


def _router_bf16_backward(ctx, d_logits, d_scores, _d_idx, _d_logits32):
    x, weight, logits, idx = ctx.saved_tensors
    dl = None if d_logits is None else d_logits.float()
    ds = None if d_scores is None else d_scores.float()
    dx, dw = router_bwd_kernels(x, weight, logits, idx, dl, ds, ctx.norm, bf16_logits=True)
    return dx, dw, None, None, None


router_fwd_bf16.register_autograd(_router_bf16_backward, setup_context=_router_bf16_setup)


# ----------------------------------------------------------------- aux loss


@torch.library.custom_op(f"{LIB}::aux_loss_fwd", mutates_args=())
def aux_loss_fwd(logits: Tensor, token_weight: Tensor | None, num_experts: int, top_k: int) -> tuple[Tensor, Tensor]:
    """(aux scalar f32, stats [E+1] = per-expert routed counts and the token total)."""
    _require_gpu(logits, token_weight)
    logits = logits.float().contiguous()
    T, E = logits.shape
    if E != num_experts:
        raise ValueError(f"router logits have {E} experts, expected {num_experts}")
    tw = None if token_weight is None else token_weight.float().contiguous()
    aux = torch.empty((), dtype=torch.float32, device=logits.device)
    stats = torch.empty(E + 1, dtype=torch.float32, device=logits.device)
    nbytes = _lib.load().moe_aux_loss_workspace_bytes(T, E)
    ws = _ws(nbytes, logits.device)
    call("moe_aux_loss_fwd", ptr(logits), ptr(tw), T, E, top_k, ptr(aux), ptr(stats), ptr(ws), ws.numel(),
         _stream(logits), tag="aux_fwd")
    return aux, stats


@aux_loss_fwd.register_fake
def _(logits, token_weight, num_experts, top_k):
    return logits.new_empty((), dtype=torch.float32), logits.new_empty(num_experts + 1, dtype=torch.float32)


@torch.library.custom_op(f"{LIB}::aux_loss_bwd", mutates_args=())
def aux_loss_bwd(logits: Tensor, token_weight: Tensor | None, stats: Tensor, d_aux: Tensor) -> Tensor:
    logits = logits.float().contiguous()
    T, E = logits.shape
    tw = None if token_weight is None else token_weight.float().contiguous()
    d_aux = d_aux.float().reshape(1).contiguous()
    dl = torch.empty(T, E, dtype=torch.float32, device=logits.device)
    call("moe_aux_loss_bwd", ptr(logits), ptr(tw), ptr(stats), ptr(d_aux), T, E, ptr(dl), 0, _stream(logits),
         tag="aux_bwd")
    return dl


@aux_loss_bwd.register_fake
def _(logits, token_weight, stats, d_aux):
    return torch.empty_like(logits, dtype=torch.float32)


def _aux_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)
    logits, token_weight, _, _ = inputs
    _, stats = output
    ctx.save_for_backward(logits, token_weight, stats)
    ctx.logits_dtype = logits.dtype
    ctx.mark_non_differentiable(stats)


def _aux_backward(ctx, d_aux, _d_stats):
    logits, token_weight, stats = ctx.saved_tensors
    if d_aux is None:
        return None, None, None, None
    dl = aux_loss_bwd(logits, token_weight, stats, d_aux)
    return dl.to(ctx.logits_dtype), None, None, None


aux_loss_fwd.register_autograd(_aux_backward, setup_context=_aux_setup)


# ------------------------------------------- the step before: norm -> router


@torch.library.custom_op(f"{LIB}::rmsnorm_fwd", mutates_args=())
def rmsnorm_fwd(hidden: Tensor, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    """Qwen3MoeRMSNorm.forward (TF modeling_qwen3_moe.py:294-299): (x like hidden, rstd [T] f32)."""
    _require_gpu(hidden, weight)
    _require_bf16("norm input", hidden)
    _require_bf16("norm weight", weight)
    H = hidden.shape[-1]
    h2 = hidden.reshape(-1, H).contiguous()
    T = h2.shape[0]
    x = torch.empty_like(h2)
    rstd = torch.empty(T, dtype=torch.float32, device=hidden.device)
    call("moe_rmsnorm_fwd", ptr(h2), ptr(weight.contiguous()), T, H, float(eps), ptr(x), ptr(rstd),
         _stream(hidden), tag="norm_fwd")
    return x.view(hidden.shape), rstd


@rmsnorm_fwd.register_fake
def _(hidden, weight, eps):
    return torch.empty_like(hidden), hidden.new_empty(hidden.numel() // hidden.shape[-1], dtype=torch.float32)


@torch.library.custom_op(f"{LIB}::rmsnorm_bwd", mutates_args=())
def rmsnorm_bwd(dx: Tensor, hidden: Tensor, weight: Tensor, rstd: Tensor) -> tuple[Tensor, Tensor]:
    """(dhidden, dweight) of rmsnorm_fwd (autograd of TF modeling_qwen3_moe.py:294-299)."""
    H = hidden.shape[-1]
    h2 = hidden.reshape(-1, H).contiguous()
    T = h2.shape[0]
    g = dx.to(BF16).reshape(-1, H).contiguous()
    dh = torch.empty_like(h2)
    dw = torch.empty(H, dtype=BF16, device=hidden.device)
    ws = _ws(_lib.load().moe_rmsnorm_bwd_workspace_bytes(T, H), hidden.device)
    call("moe_rmsnorm_bwd", ptr(g), None, ptr(h2), ptr(weight.contiguous()), ptr(rstd), T, H, ptr(dh), ptr(dw),
         ptr(ws), ws.numel(), _stream(hidden), tag="norm_bwd")
    return dh.view(hidden.shape), dw


@rmsnorm_bwd.register_fake
def _(dx, hidden, weight, rstd):
    return torch.empty_like(hidden), torch.empty_like(weight)


def _norm_setup(ctx, inputs, output):
    hidden, weight, _eps = inputs
    _, rstd = output
    ctx.save_for_backward(hidden, weight, rstd)
    ctx.mark_non_differentiable(rstd)


def _norm_backward(ctx, dx, _drstd):
    hidden, weight, rstd = ctx.saved_tensors
    dh, dw = rmsnorm_bwd(dx, hidden, weight, rstd)
    return dh, dw, None


rmsnorm_fwd.register_autograd(_norm_backward, setup_context=_norm_setup)


@torch.library.custom_op(f"{LIB}::router_aux_fwd", mutates_args=())
def router_aux_fwd(x: Tensor, weight: Tensor, top_k: int, norm_topk_prob: bool, token_weight: Tensor | None = None,
                   logit_bias: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """router_fwd plus the Switch aux loss from the same softmax and top-k: (logits, scores, indices,
    aux scalar, stats [E+1]); aux equals aux_loss_fwd(logits, token_weight, E, top_k)."""
    return _router_aux_kernels(x, weight, top_k, norm_topk_prob, token_weight, logit_bias)


def _router_aux_kernels(x, weight, top_k, norm_topk_prob, token_weight, logit_bias, bf16_logits=False):
    """(logits f32, scores f32, indices, aux, stats), plus the bf16 logits when
    ``bf16_logits`` (``logits`` then holds their values in fp32)."""
    _require_gpu(x, weight, token_weight)
    if x.dtype == weight.dtype == torch.float32:
        if bf16_logits:
            raise ValueError("bf16 router logits need bf16 hidden states and router weight")
        # fp32 modules: the fp32 router, then the aux kernels on its logits
        logits, scores, idx = _router_fwd_f32(x.contiguous(), weight.contiguous(), top_k, norm_topk_prob, logit_bias)
        T, E = logits.shape
        tw = None if token_weight is None else token_weight.float().contiguous()
        aux = torch.empty((), dtype=torch.float32, device=x.device)
        stats = torch.empty(E + 1, dtype=torch.float32, device=x.device)
        ws = _ws(_lib.load().moe_aux_loss_workspace_bytes(T, E), x.device)
        call("moe_aux_loss_fwd", ptr(logits), ptr(tw), T, E, top_k, ptr(aux), ptr(stats), ptr(ws), ws.numel(),
             _stream(x), tag="router_fwd")
        return logits, scores, idx, aux, stats
    _require_bf16("router input", x)
    _require_bf16("router weight", weight)
    x = x.contiguous()
    weight = weight.contiguous()
    T, H = x.shape
    E = weight.shape[0]
    dev = x.device
    logits = torch.empty(T, E, dtype=torch.float32, device=dev)
    scores = torch.empty(T, top_k, dtype=torch.float32, device=dev)
    idx = torch.empty(T, top_k, dtype=torch.int64, device=dev)
    aux = torch.empty((), dtype=torch.float32, device=dev)
    stats = torch.empty(E + 1, dtype=torch.float32, device=dev)
    bias = None if logit_bias is None else logit_bias.to(device=dev, dtype=torch.float32).contiguous()
    tw = None if token_weight is None else token_weight.float().contiguous()
    logits_b = torch.empty(T, E, dtype=BF16, device=dev) if bf16_logits else None
    ws = _ws(_lib.load().moe_router_aux_fwd_workspace_bytes(T, H, E), dev)
    call("moe_router_aux_fwd", ptr(x), ptr(weight), ptr(bias), ptr(tw), ptr(logits), ptr(logits_b), ptr(scores),
         ptr(idx), T, H, E, top_k, int(norm_topk_prob), ptr(aux), ptr(stats), ptr(ws), ws.numel(), _stream(x),
         tag="router_fwd")
    if bf16_logits:
        return logits, scores, idx, aux, stats, logits_b
    return logits, scores, idx, aux, stats


@router_aux_fwd.register_fake
def _(x, weight, top_k, norm_topk_prob, token_weight=None, logit_bias=None):
    T, E = x.shape[0], weight.shape[0]
    return (x.new_empty(T, E, dtype=torch.float32), x.new_empty(T, top_k, dtype=torch.float32),
            x.new_empty(T, top_k, dtype=torch.int64), x.new_empty((), dtype=torch.float32),
            x.new_empty(E + 1, dtype=torch.float32))


def _router_aux_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)
    x, weight, top_k, norm, token_weight, _bias = inputs
    logits, _, idx, _, stats = output
    ctx.save_for_backward(x, weight, logits, idx, token_weight, stats)
    ctx.norm = norm
    ctx.mark_non_differentiable(idx, stats)


def _router_aux_backward(ctx, d_logits, d_scores, _d_idx, d_aux, _d_stats):
    x, weight, logits, idx, token_weight, stats = ctx.saved_tensors
    # The aux loss's logits gradient is formed inside the top-k backward pass.
    dx, dw = router_bwd_kernels(x, weight, logits, idx, d_logits, d_scores, ctx.norm, token_weight, stats, d_aux)
    return dx, dw, None, None, None, None


router_aux_fwd.register_autograd(_router_aux_backward, setup_context=_router_aux_setup)


# ------------------------------------------------------------------ permute


@torch.library.custom_op(f"{LIB}::permute_fwd", mutates_args=())
def permute_fwd(hidden: Tensor, ids: Tensor, divisor: int, num_buckets: int,
                gather_rows: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Stable sort of slots by ids // divisor.

    Returns (permuted rows [S,H] or empty, perm [S] int32, pos_of_slot [S] int32,
    counts [nb] int32, offsets [nb] int32); slots whose bucket is >= num_buckets
    are sentinels placed last (TF integrations/moe.py:389-437).
    """
    _require_gpu(hidden, ids)
    T = hidden.shape[0]
    H = hidden.shape[1] if hidden.dim() == 2 else 0
    if ids.dim() != 2 or ids.shape[0] != T:
        raise ValueError(f"ids must be [T, k] with T={T}, got {tuple(ids.shape)}")
    k = ids.shape[1]
    S = T * k
    dev = hidden.device
    ids = _ids64(ids)
    perm = torch.empty(S, dtype=torch.int32, device=dev)
    pos = torch.empty(S, dtype=torch.int32, device=dev)
    counts = torch.empty(num_buckets, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_buckets, dtype=torch.int32, device=dev)
    if gather_rows:
        _require_bf16("hidden", hidden)
        hidden = hidden.contiguous()
        out = torch.empty(S, H, dtype=hidden.dtype, device=dev)
    else:
        out = torch.empty(0, dtype=BF16, device=dev)
    ws = _ws(_lib.load().moe_permute_workspace_bytes(S, num_buckets), dev)
    call("moe_permute_fwd", ptr(hidden) if gather_rows else None, T, H, ptr(ids), k, divisor, num_buckets,
         ptr(out) if gather_rows else None, ptr(perm), ptr(pos), ptr(counts), ptr(offsets), ptr(ws), ws.numel(),
         _stream(ids))
    return out, perm, pos, counts, offsets


@permute_fwd.register_fake
def _(hidden, ids, divisor, num_buckets, gather_rows):
    S = ids.shape[0] * ids.shape[1]
    rows = hidden.new_empty(S, hidden.shape[1]) if gather_rows else hidden.new_empty(0)
    i32 = dict(dtype=torch.int32)
    return (rows, ids.new_empty(S, **i32), ids.new_empty(S, **i32), ids.new_empty(num_buckets, **i32),
            ids.new_empty(num_buckets, **i32))


# ------------------------------------------------------------------ experts


def _check_experts(hidden: Tensor, top_k_index: Tensor, top_k_weights: Tensor, gate_up_proj: Tensor,
                   down_proj: Tensor) -> tuple[int, int, int, int, int]:
    _require_gpu(hidden, top_k_index, top_k_weights, gate_up_proj, down_proj)
    if hidden.dim() != 2:
        raise ValueError(f"hidden states must be [tokens, hidden], got {tuple(hidden.shape)}")
    if top_k_index.shape != top_k_weights.shape or top_k_index.dim() != 2 or top_k_index.shape[0] != hidden.shape[0]:
        raise ValueError("top_k_index and top_k_weights must both be [tokens, k]")
    T, H = hidden.shape
    k = top_k_index.shape[1]
    E, I2, H2 = gate_up_proj.shape
    if H2 != H or I2 % 2 or tuple(down_proj.shape) != (E, H, I2 // 2):
        raise ValueError(
            f"expert weights do not match: gate_up_proj {tuple(gate_up_proj.shape)}, "
            f"down_proj {tuple(down_proj.shape)}, hidden {H}"
        )
    if not (hidden.dtype == gate_up_proj.dtype == down_proj.dtype == torch.float32):
        # fp32 modules take the fp32 path; everything else runs in bf16
        for name, t in (("hidden states", hidden), ("gate_up_proj", gate_up_proj), ("down_proj", down_proj)):
            _require_bf16(name, t)
    elif H % 4:
        raise ValueError(f"the fp32 expert path needs hidden % 4 == 0, got {H}")
    return T, H, k, E, I2 // 2


@torch.library.custom_op(f"{LIB}::experts_fwd", mutates_args=())
def experts_fwd(hidden: Tensor, top_k_index: Tensor, top_k_weights: Tensor, gate_up_proj: Tensor,
                down_proj: Tensor, accumulate_grad: bool = False
                ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """grouped_mm_experts_forward (TF integrations/moe.py:377-478) on gfx950.

    Returns (out [T,H], and for the backward: xp [S,H], pre [S,2I], act [S,I],
    y [S,H], pos_of_slot [S] int32, offsets [E] int32).  ``accumulate_grad``
    only changes the backward (see ``experts``).
    """
    return _experts_fwd_kernels(hidden, top_k_index, top_k_weights, gate_up_proj, down_proj)


def _f32_gemm(A, B, offs, G, mode, M, N, K, sA, sB, sBg, C, sC, sCg, accumulate, s, tag):
    """moe_f32_grouped_gemm: C(i, j) (+)= sum_r A(i, r) B(r, j), strides (sAi, sAr), (sBr, sBj), (sCi, sCj)."""
    call("moe_f32_grouped_gemm", ptr(A), ptr(B), ptr(offs), G, mode, M, N, K, sA[0], sA[1], sB[0], sB[1], sBg, ptr(C),
         sC[0], sC[1], sCg, int(accumulate), s, tag=tag)


def _wgrad_launch(dc, a, offsets, E, S, n, k, dst, accumulate, tag):
    """dW[g][n_, k_] = sum over group g's rows of dc[r, n_] a[r, k_] into dst [E, n, k]
    (bf16 or fp32; added to it with ``accumulate``): the bf16 weight-gradient
    GEMM, or for fp32 operands the fp32 grouped GEMM."""
    s = _stream(dc)
    if dc.dtype == torch.float32:
        _f32_gemm(dc, a, offsets, E, 1, n, k, S, (1, n), (k, 1), 0, dst, (k, 1), n * k, accumulate, s, tag)
    else:
        call("moe_grouped_gemm_wgrad", ptr(dc), ptr(a), ptr(offsets), E, S, n, k, ptr(dst),
             int(dst.dtype == torch.float32), int(accumulate), s, tag=tag)


def _experts_fwd_f32(hidden, ids, w, gu, dn, T, H, k, E, I):
    """The fp32 expert path (fp32 modules; TF integrations/moe.py:377-478 in fp32)."""
    S = T * k
    dev = hidden.device
    s = _stream(hidden)
    f32 = dict(dtype=torch.float32, device=dev)
    xp = torch.empty(S, H, **f32)
    perm = torch.empty(S, dtype=torch.int32, device=dev)
    pos = torch.empty(S, dtype=torch.int32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E, dtype=torch.int32, device=dev)
    ws = _ws(_lib.load().moe_permute_workspace_bytes(S, E), dev)
    # the row copy moves bytes: an fp32 row is 2H bf16-sized units
    call("moe_permute_fwd", ptr(hidden), T, 2 * H, ptr(ids), k, 1, E, ptr(xp), ptr(perm), ptr(pos), ptr(counts),
         ptr(offsets), ptr(ws), ws.numel(), s, tag="permute_fwd")
    pre = torch.empty(S, 2 * I, **f32)
    _f32_gemm(xp, gu, offsets, E, 0, S, 2 * I, H, (H, 1), (1, H), 2 * I * H, pre, (2 * I, 1), 0, False, s, "up_fwd")
    act = torch.empty(S, I, **f32)
    call("moe_f32_swiglu_fwd", ptr(pre), ptr(act), ptr(offsets), E, S, I, s, tag="up_fwd")
    y = torch.empty(S, H, **f32)
    _f32_gemm(act, dn, offsets, E, 0, S, H, I, (I, 1), (1, I), H * I, y, (H, 1), 0, False, s, "down_fwd")
    out = torch.empty(T, H, **f32)
    call("moe_f32_combine_fwd", ptr(y), ptr(pos), ptr(offsets), E, ptr(w), T, H, k, ptr(out), s, tag="combine_fwd")
    return out, xp, pre, act, y, pos, offsets


def _experts_bwd_f32(d_out, w, gu, dn, xp, pre, act, y, pos, offsets, wgrad, on_d_weights):
    T, k = w.shape
    E, I2, H = gu.shape
    I = I2 // 2
    S = T * k
    dev = d_out.device
    s = _stream(d_out)
    f32 = dict(dtype=torch.float32, device=dev)
    d_out = d_out.float().contiguous()
    dy = torch.empty(S, H, **f32)
    d_w = torch.empty(T, k, **f32)
    call("moe_f32_combine_bwd", ptr(d_out), ptr(y), ptr(pos), ptr(offsets), E, ptr(w), T, H, k, ptr(dy), ptr(d_w), s,
         tag="combine_bwd")
    d_add = on_d_weights(d_w) if on_d_weights is not None else None
    d_act = torch.empty(S, I, **f32)
    _f32_gemm(dy, dn, offsets, E, 0, S, I, H, (H, 1), (I, 1), H * I, d_act, (I, 1), 0, False, s, "down_dgrad")
    d_pre = torch.empty(S, 2 * I, **f32)
    call("moe_f32_swiglu_bwd", ptr(d_act), ptr(pre), ptr(d_pre), ptr(offsets), E, S, I, s, tag="down_dgrad")
    d_xp = torch.empty(S, H, **f32)
    _f32_gemm(d_pre, gu, offsets, E, 0, S, H, 2 * I, (2 * I, 1), (H, 1), 2 * I * H, d_xp, (H, 1), 0, False, s,
              "up_dgrad")
    d_hidden = torch.empty(T, H, **f32)
    call("moe_f32_permute_bwd", ptr(d_xp), ptr(pos), ptr(offsets), E, T, H, k, ptr(d_add), ptr(d_hidden), s,
         tag="permute_bwd")
    d_gu = wgrad("gate_up_proj", d_pre, xp, 2 * I, H)
    d_down = wgrad("down_proj", dy, act, H, I)
    return d_hidden, d_w, d_gu, d_down


def _experts_fwd_kernels(hidden, top_k_index, top_k_weights, gate_up_proj, down_proj):
    T, H, k, E, I = _check_experts(hidden, top_k_index, top_k_weights, gate_up_proj, down_proj)
    if hidden.dtype == torch.float32:
        return _experts_fwd_f32(hidden.contiguous(), _ids64(top_k_index), top_k_weights.float().contiguous(),
                                gate_up_proj.contiguous(), down_proj.contiguous(), T, H, k, E, I)
    S = T * k
    dev = hidden.device
    s = _stream(hidden)
    hidden = hidden.contiguous()
    ids = _ids64(top_k_index)
    w = top_k_weights.float().contiguous()
    gu = gate_up_proj.contiguous()
    dn = down_proj.contiguous()
    xp = torch.empty(S, H, dtype=BF16, device=dev)
    perm = torch.empty(S, dtype=torch.int32, device=dev)
    pos = torch.empty(S, dtype=torch.int32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E, dtype=torch.int32, device=dev)
    ws = _ws(_lib.load().moe_permute_workspace_bytes(S, E), dev)
    call("moe_permute_fwd", ptr(hidden), T, H, ptr(ids), k, 1, E, ptr(xp), ptr(perm), ptr(pos), ptr(counts),
         ptr(offsets), ptr(ws), ws.numel(), s, tag="permute_fwd")
    act = torch.empty(S, I, dtype=BF16, device=dev)
    pre = torch.empty(S, 2 * I, dtype=BF16, device=dev)
    call("moe_grouped_gemm_swiglu_fwd", ptr(xp), ptr(gu), ptr(offsets), E, S, H, I, ptr(act), ptr(pre), s,
         tag="up_fwd")
    y = torch.empty(S, H, dtype=BF16, device=dev)
    call("moe_grouped_gemm_fwd", ptr(act), ptr(dn), ptr(offsets), E, S, H, I, ptr(y), s, tag="down_fwd")
    out = torch.empty(T, H, dtype=BF16, device=dev)
    call("moe_combine_fwd", ptr(y), ptr(pos), ptr(offsets), E, ptr(w), T, H, k, ptr(out), s, tag="combine_fwd")
    return out, xp, pre, act, y, pos, offsets


@experts_fwd.register_fake
def _(hidden, top_k_index, top_k_weights, gate_up_proj, down_proj, accumulate_grad=False):
    T, H = hidden.shape
    S = T * top_k_index.shape[1]
    E, I2, _ = gate_up_proj.shape
    i32 = dict(dtype=torch.int32)
    return (hidden.new_empty(T, H), hidden.new_empty(S, H), hidden.new_empty(S, I2), hidden.new_empty(S, I2 // 2),
            hidden.new_empty(S, H), hidden.new_empty(S, **i32), hidden.new_empty(E, **i32))


def experts_bwd_kernels(d_out: Tensor, top_k_weights: Tensor, gate_up_proj: Tensor, down_proj: Tensor, xp: Tensor,
                        pre: Tensor, act: Tensor, y: Tensor, pos_of_slot: Tensor, offsets: Tensor,
                        wgrad, on_d_weights=None, router: dict | None = None) -> tuple[Tensor, Tensor | None, object,
                                                                                        object]:
    """The expert backward's launches; ``wgrad(name, dc, a, n, k)`` issues the
    weight gradient dW[g][n,k] = dc[rows of g]ᵀ · a[rows of g] of projection
    ``name`` ("gate_up_proj", then "down_proj") and returns whatever stands for
    it.  ``on_d_weights(d_weights)``, if given, runs as soon as the routing
    weights' gradient exists and returns a bf16 [T,H] gradient that the
    permute backward adds into d_hidden (the other path to the same input).
    With ``router`` (bf16 rows only; the routing weights are the router's
    scores and nothing else uses them) the combine backward also runs the
    router's top-k backward on the weights' gradient in the same launch
    (moe_combine_router_bwd, the bits of the two separate launches), and
    ``router["finish"](d_logits_bf16)`` returns the bf16 [T,H] gradient the
    permute backward adds; d_weights is then not formed (None).
    Returns (d_hidden [T,H], d_weights [T,k] f32, wgrad's two results)."""
    if xp.dtype == torch.float32:
        return _experts_bwd_f32(d_out, top_k_weights.float().contiguous(), gate_up_proj, down_proj, xp, pre, act, y,
                                pos_of_slot, offsets, wgrad, on_d_weights)
    T, k = top_k_weights.shape
    E, I2, H = gate_up_proj.shape
    I = I2 // 2
    S = T * k
    dev = d_out.device
    s = _stream(d_out)
    d_out = d_out.to(BF16).contiguous()
    w = top_k_weights.float().contiguous()
    dy = torch.empty(S, H, dtype=BF16, device=dev)
    if router is not None:
        d_w = None
        lg = router["logits"]
        n_e = lg.shape[1]
        dl_bf16 = torch.empty(T, n_e, dtype=BF16, device=dev)
        call("moe_combine_router_bwd", ptr(d_out), ptr(y), ptr(pos_of_slot), ptr(offsets), E, ptr(w), T, H, k, ptr(dy),
             None, ptr(lg), ptr(router["indices"]), ptr(router["d_logits"]), ptr(router["token_weight"]),
             ptr(router["stats"]), ptr(router["d_aux"]), n_e, int(router["norm"]), int(router["bf16_terms"]),
             ptr(dl_bf16), s, tag="combine_bwd")
        d_add = router["finish"](dl_bf16)
    else:
        d_w = torch.empty(T, k, dtype=torch.float32, device=dev)
        call("moe_combine_bwd", ptr(d_out), ptr(y), ptr(pos_of_slot), ptr(offsets), E, ptr(w), T, H, k, ptr(dy),
             ptr(d_w), s, tag="combine_bwd")
        d_add = on_d_weights(d_w) if on_d_weights is not None else None
    d_pre = torch.empty(S, 2 * I, dtype=BF16, device=dev)
    call("moe_grouped_gemm_dgrad_swiglu_bwd", ptr(dy), ptr(down_proj), ptr(pre), ptr(offsets), E, S, H, I,
         ptr(d_pre), s, tag="down_dgrad")
    # Each consumer runs right after its producer while the tensor is still in
    # the 256 MB last-level cache: the input-gradient GEMM reads d_pre, the
    # permute backward reads d_xp; the weight gradients (1.2 GB of writes
    # that would evict both) come last.
    d_xp = torch.empty(S, H, dtype=BF16, device=dev)
    call("moe_grouped_gemm_dgrad", ptr(d_pre), ptr(gate_up_proj), ptr(offsets), E, S, 2 * I, H, ptr(d_xp), s,
         tag="up_dgrad")
    d_hidden = torch.empty(T, H, dtype=BF16, device=dev)
    call("moe_permute_bwd", ptr(d_xp), ptr(pos_of_slot), ptr(offsets), E, T, H, k, ptr(d_add), ptr(d_hidden), s,
         tag="permute_bwd")
    d_gu = wgrad("gate_up_proj", d_pre, xp, 2 * I, H)
    d_down = wgrad("down_proj", dy, act, H, I)
    return d_hidden, d_w, d_gu, d_down


@torch.library.custom_op(f"{LIB}::experts_bwd", mutates_args=())
def experts_bwd(d_out: Tensor, top_k_weights: Tensor, gate_up_proj: Tensor, down_proj: Tensor, xp: Tensor,
                pre: Tensor, act: Tensor, y: Tensor, pos_of_slot: Tensor,
                offsets: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(d_hidden [T,H], d_weights [T,k] f32, d_gate_up_proj, d_down_proj)."""
    E = gate_up_proj.shape[0]
    S = xp.shape[0]
    params = {"gate_up_proj": gate_up_proj, "down_proj": down_proj}

    def wgrad(name, dc, a, n, k):
        dw = torch.empty_like(params[name])
        _wgrad_launch(dc, a, offsets, E, S, n, k, dw, False, "up_wgrad" if name == "gate_up_proj" else "down_wgrad")
        return dw

    return experts_bwd_kernels(d_out, top_k_weights, gate_up_proj, down_proj, xp, pre, act, y, pos_of_slot, offsets,
                               wgrad)


@experts_bwd.register_fake
def _(d_out, top_k_weights, gate_up_proj, down_proj, xp, pre, act, y, pos_of_slot, offsets):
    return (torch.empty_like(d_out), top_k_weights.new_empty(top_k_weights.shape, dtype=torch.float32),
            torch.empty_like(gate_up_proj), torch.empty_like(down_proj))


def _experts_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)
    hidden, top_k_index, top_k_weights, gate_up_proj, down_proj, accumulate_grad = inputs
    _, xp, pre, act, y, pos, offsets = output
    ctx.save_for_backward(top_k_weights, gate_up_proj, down_proj, xp, pre, act, y, pos, offsets)
    ctx.weights_dtype = top_k_weights.dtype
    ctx.hidden_dtype = hidden.dtype
    # The parameters themselves (not their saved aliases): their .grad is read at backward time.
    ctx.params = (gate_up_proj, down_proj) if accumulate_grad else None
    ctx.mark_non_differentiable(xp, pre, act, y, pos, offsets)


def _grad_target(param: Tensor) -> Tensor | None:
    """param.grad when the weight-gradient kernel can add into it in place."""
    g = param.grad if param.is_leaf else None
    if g is None or g.shape != param.shape or not g.is_contiguous() or g.device != param.device:
        return None
    return g if g.dtype in (BF16, torch.float32) else None


def _experts_backward(ctx, d_out, *_unused):
    w, gu, dn, xp, pre, act, y, pos, offsets = ctx.saved_tensors
    if d_out is None:
        return None, None, None, None, None, None
    targets = [_grad_target(p) for p in ctx.params] if ctx.params is not None else [None, None]
    if targets[0] is None and targets[1] is None:
        d_hidden, d_w, d_gu, d_dn = experts_bwd(d_out, w, gu, dn, xp, pre, act, y, pos, offsets)
    else:
        d_hidden, d_w, d_gu, d_dn = experts_bwd_accumulate(d_out, w, gu, dn, xp, pre, act, y, pos, offsets,
                                                           targets[0], targets[1])
    return d_hidden.to(ctx.hidden_dtype), None, d_w.to(ctx.weights_dtype), d_gu, d_dn, None


experts_fwd.register_autograd(_experts_backward, setup_context=_experts_setup)


def experts_bwd_accumulate(d_out, top_k_weights, gate_up_proj, down_proj, xp, pre, act, y, pos_of_slot, offsets,
                           gu_grad: Tensor | None, dn_grad: Tensor | None):
    """experts_bwd with the weight gradients added into existing gradient
    tensors by the weight-gradient kernel's accumulate epilogue (bf16: the
    fp32 sum rounded to bf16 plus the existing value, rounded again, as
    torch's bf16 add; fp32 targets add the fp32 sum).  A projection whose
    target is None gets a fresh gradient, returned as usual; the returned
    gradient of an accumulated projection is None."""
    E = gate_up_proj.shape[0]
    S = xp.shape[0]
    params = {"gate_up_proj": (gate_up_proj, gu_grad), "down_proj": (down_proj, dn_grad)}

    def wgrad(name, dc, a, n, k):
        param, target = params[name]
        tag = "up_wgrad" if name == "gate_up_proj" else "down_wgrad"
        if target is None or (dc.dtype == torch.float32 and target.dtype != torch.float32):
            dw = torch.empty_like(param)
            _wgrad_launch(dc, a, offsets, E, S, n, k, dw, False, tag)
            return dw
        _wgrad_launch(dc, a, offsets, E, S, n, k, target, True, tag)
        return None

    return experts_bwd_kernels(d_out, top_k_weights, gate_up_proj, down_proj, xp, pre, act, y, pos_of_slot, offsets,
                               wgrad)


def experts(hidden: Tensor, top_k_index: Tensor, top_k_weights: Tensor, gate_up_proj: Tensor,
            down_proj: Tensor, accumulate_grad: bool = False) -> Tensor:
    """Differentiable expert layer output [T,H] (TF integrations/moe.py:377-478 contract).

    With ``accumulate_grad`` a weight that is a leaf and already holds a
    ``.grad`` (bf16 or fp32, its shape, contiguous) gets this backward's
    weight gradient added into that tensor by the weight-gradient GEMM itself,
    instead of a separate dense gradient that autograd then adds (the
    reference's accumulation, parallel/parallel/engine/engine.py:165-178);
    the result is the same bits.  Autograd sees no gradient for such a weight,
    so its post-accumulate-grad hooks do not run: leave it off where an FSDP
    unit waits for those hooks (parallel/parallel/engine/_dp_param_unit.py:669-690).
    A weight without a ``.grad`` gets a fresh gradient as usual.

    The in-place write is invisible to autograd and to tracing: tensor grad
    hooks and post-accumulate-grad hooks of such a weight do not run, and
    under ``torch.compile`` (AOTAutograd) the option is refused."""
    _refuse_traced_accumulation(accumulate_grad, "experts")
    return experts_fwd(hidden, top_k_index, top_k_weights, gate_up_proj, down_proj, accumulate_grad)[0]


def _refuse_traced_accumulation(accumulate_grad: bool, what: str) -> None:
    """accumulate_grad writes param.grad from inside a custom op's backward,
    a side effect that torch.compile / AOTAutograd cannot trace."""
    if accumulate_grad and torch.compiler.is_compiling():
        raise RuntimeError(f"{what}(accumulate_grad=True) adds into .grad inside the backward, which torch.compile "
                           "cannot trace; use accumulate_grad=False under torch.compile")


# --------------------------------------------- the whole block in one op


@torch.library.custom_op(f"{LIB}::moe_block_fwd", mutates_args=())
def moe_block_fwd(x: Tensor, router_weight: Tensor, gate_up_proj: Tensor, down_proj: Tensor, top_k: int,
                  norm_topk_prob: bool, token_weight: Tensor | None = None, logit_bias: Tensor | None = None,
                  accumulate_grad: bool = False, bf16_logits: bool = False
                  ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                             Tensor]:
    """router_aux_fwd then experts_fwd on its routes: (out, logits, scores,
    indices, aux, stats, and experts_fwd's saved tensors).  With
    ``bf16_logits`` the logits and scores are bf16 (the router under bf16
    autocast); the experts read the scores' values."""
    if bf16_logits:
        _, scores, idx, aux, stats, logits = _router_aux_kernels(x, router_weight, top_k, norm_topk_prob,
                                                                 token_weight, logit_bias, True)
    else:
        logits, scores, idx, aux, stats = _router_aux_kernels(x, router_weight, top_k, norm_topk_prob, token_weight,
                                                              logit_bias)
    out, xp, pre, act, y, pos, offsets = _experts_fwd_kernels(x, idx, scores, gate_up_proj, down_proj)
    if bf16_logits:
        scores = scores.to(BF16)  # bf16 values: the cast is exact
    return out, logits, scores, idx, aux, stats, xp, pre, act, y, pos, offsets


@moe_block_fwd.register_fake
def _(x, router_weight, gate_up_proj, down_proj, top_k, norm_topk_prob, token_weight=None, logit_bias=None,
      accumulate_grad=False, bf16_logits=False):
    T, H = x.shape
    E = router_weight.shape[0]
    rdt = BF16 if bf16_logits else torch.float32
    router = (x.new_empty(T, E, dtype=rdt), x.new_empty(T, top_k, dtype=rdt),
              x.new_empty(T, top_k, dtype=torch.int64), x.new_empty((), dtype=torch.float32),
              x.new_empty(E + 1, dtype=torch.float32))
    out, xp, pre, act, y, pos, offsets = _experts_fake(x, top_k, gate_up_proj)
    return (out, *router, xp, pre, act, y, pos, offsets)


def _experts_fake(x, top_k, gate_up_proj):
    T, H = x.shape
    S = T * top_k
    E, I2, _ = gate_up_proj.shape
    i32 = dict(dtype=torch.int32)
    return (x.new_empty(T, H), x.new_empty(S, H), x.new_empty(S, I2), x.new_empty(S, I2 // 2), x.new_empty(S, H),
            x.new_empty(S, **i32), x.new_empty(E, **i32))


def _block_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)
    x, rw, gu, dn, top_k, norm, token_weight, _bias, accumulate_grad, bf16_logits = inputs
    _, logits, scores, idx, _, stats, xp, pre, act, y, pos, offsets = output
    ctx.save_for_backward(x, rw, gu, dn, logits, scores, idx, token_weight, stats, xp, pre, act, y, pos, offsets)
    ctx.norm = norm
    ctx.bf16_logits = bf16_logits
    ctx.x_dtype = x.dtype
    ctx.params = (rw, gu, dn) if accumulate_grad else None
    ctx.mark_non_differentiable(idx, stats, xp, pre, act, y, pos, offsets)


def _block_backward(ctx, d_out, d_logits, d_scores, _d_idx, d_aux, *_unused):
    x, rw, gu, dn, logits, scores, idx, tw, stats, xp, pre, act, y, pos, offsets = ctx.saved_tensors
    if d_out is None and d_logits is None and d_scores is None and d_aux is None:
        return (None,) * 10
    targets = [_grad_target(p) for p in ctx.params] if ctx.params is not None else [None, None, None]
    # the router's weight gradient is added in place into a .grad of its own dtype
    rw_target = targets[0] if targets[0] is not None and targets[0].dtype == rw.dtype else None
    E = gu.shape[0]
    S = xp.shape[0]
    grads = {}

    def router_backward(d_w):
        # The routing weights' gradient from the experts plus any the scores
        # received elsewhere; the router's dX then joins d_hidden inside the
        # permute backward instead of a separate add.  bf16 scores have a
        # bf16 gradient, which autograd sums in bf16 (the router kernel
        # rounds d_w itself when nothing else is added).
        if d_scores is None:
            ds = d_w
        elif ctx.bf16_logits:
            ds = (d_w.to(BF16) + d_scores.to(BF16)).float()
        else:
            ds = d_w + d_scores.float()
        lg = logits.float() if ctx.bf16_logits else logits
        dx_router, grads["router"] = router_bwd_kernels(x, rw, lg, idx, d_logits, ds, ctx.norm, tw, stats, d_aux,
                                                        rw_target, bf16_logits=ctx.bf16_logits)
        return dx_router

    params = {"gate_up_proj": (gu, targets[1]), "down_proj": (dn, targets[2])}

    def wgrad(name, dc, a, n, k):
        param, target = params[name]
        tag = "up_wgrad" if name == "gate_up_proj" else "down_wgrad"
        if target is None or (dc.dtype == torch.float32 and target.dtype != torch.float32):
            dw = torch.empty_like(param)
            _wgrad_launch(dc, a, offsets, E, S, n, k, dw, False, tag)
            return dw
        _wgrad_launch(dc, a, offsets, E, S, n, k, target, True, tag)
        return None

    if d_out is None:
        d_out = torch.zeros_like(x)
    router = None
    if d_scores is None and xp.dtype == BF16 and not (x.dtype == rw.dtype == torch.float32):
        # Nothing but the experts uses the scores: the top-k backward runs
        # inside the combine backward, on the weights' gradient it forms.
        def finish(dl_bf16):
            dx_router, grads["router"] = _router_gemm_bwd(x.contiguous(), rw.contiguous(), dl_bf16, rw_target)
            return dx_router

        with_aux = d_aux is not None
        router = dict(logits=(logits.float() if ctx.bf16_logits else logits).contiguous(), indices=idx.contiguous(),
                      d_logits=None if d_logits is None else d_logits.float().contiguous(),
                      token_weight=tw.float().contiguous() if (with_aux and tw is not None) else None,
                      stats=stats if with_aux else None,
                      d_aux=d_aux.float().reshape(1).contiguous() if with_aux else None,
                      norm=ctx.norm, bf16_terms=ctx.bf16_logits, finish=finish)
    dx, _d_w, d_gu, d_dn = experts_bwd_kernels(d_out, scores, gu, dn, xp, pre, act, y, pos, offsets, wgrad,
                                              on_d_weights=None if router is not None else router_backward,
                                              router=router)
    return dx.to(ctx.x_dtype), grads["router"], d_gu, d_dn, None, None, None, None, None, None


moe_block_fwd.register_autograd(_block_backward, setup_context=_block_setup)


def moe_block(x: Tensor, router_weight: Tensor, gate_up_proj: Tensor, down_proj: Tensor, top_k: int,
              norm_topk_prob: bool, token_weight: Tensor | None = None, logit_bias: Tensor | None = None,
              accumulate_grad: bool = False, bf16_logits: bool = False) -> tuple[Tensor, Tensor, Tensor, Tensor,
                                                                                 Tensor]:
    """Qwen3MoeSparseMoeBlock's router, experts and Switch aux loss as one op:
    (out [T,H], router_logits [T,E] fp32, scores [T,k], indices [T,k], aux).

    ``bf16_logits`` runs the router as the reference does under bf16 autocast
    (parallel/parallel/engine/engine.py:141): the logits of a bf16 linear,
    softmax, top-k and the aux loss in fp32 on them, bf16 logits and scores
    returned, and a backward that sums the logits' and scores' gradients in
    bf16, as autograd does for bf16 tensors (``router_fwd_bf16``'s
    semantics).

    The same results as ``router_aux_fwd`` followed by ``experts`` (TF
    modeling_qwen3_moe.py:249-267 and integrations/moe.py:377-478, the aux
    loss of :514-593), but the backward adds the router's input gradient to
    the experts' inside the permute backward (one rounding of the sum of
    both in fp32, where autograd rounds the experts' sum, then adds), forms
    the aux loss's logits gradient inside the top-k backward (which runs
    inside the combine backward when nothing else takes the scores'
    gradient: the same bits as the separate launch), and with
    ``accumulate_grad`` adds every weight gradient into an existing ``.grad``
    (bf16 router weight; bf16 or fp32 expert weights) in the kernels, as
    ``experts`` does for the expert weights (with the same limits: no grad
    hooks for those weights, refused under ``torch.compile``)."""
    _refuse_traced_accumulation(accumulate_grad, "moe_block")
    out, logits, scores, idx, aux = moe_block_fwd(x, router_weight, gate_up_proj, down_proj, top_k, norm_topk_prob,
                                                  token_weight, logit_bias, accumulate_grad, bf16_logits)[:5]
    return out, logits, scores, idx, aux


# ------------------------------------------------------- token dispatch ops


@torch.library.custom_op(f"{LIB}::dispatch_fwd", mutates_args=())
def dispatch_fwd(hidden: Tensor, global_indices: Tensor, scores: Tensor, local_count: int,
                 ep_size: int) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Owner-major send buffers of TokenDispatcher.dispatch (token_dispatch.py:101-125).

    Returns (send_hidden [S,H], send_experts [S] int64 (local ids),
    send_scores [S], source_tokens [S] int64, pos_of_slot [S] int32,
    counts [ep] int32 = send splits).
    """
    _require_gpu(hidden, global_indices, scores)
    _require_bf16("hidden states", hidden)
    T, H = hidden.shape
    k = global_indices.shape[1]
    S = T * k
    dev = hidden.device
    s = _stream(hidden)
    hidden = hidden.contiguous()
    ids = _ids64(global_indices)
    sc = scores.float().contiguous()
    send_hidden = torch.empty(S, H, dtype=hidden.dtype, device=dev)
    perm = torch.empty(S, dtype=torch.int32, device=dev)
    pos = torch.empty(S, dtype=torch.int32, device=dev)
    counts = torch.empty(ep_size, dtype=torch.int32, device=dev)
    offsets = torch.empty(ep_size, dtype=torch.int32, device=dev)
    ws = _ws(_lib.load().moe_permute_workspace_bytes(S, ep_size), dev)
    call("moe_permute_fwd", ptr(hidden), T, H, ptr(ids), k, local_count, ep_size, ptr(send_hidden), ptr(perm),
         ptr(pos), ptr(counts), ptr(offsets), ptr(ws), ws.numel(), s)
    send_experts = torch.empty(S, dtype=torch.int64, device=dev)
    send_scores = torch.empty(S, dtype=torch.float32, device=dev)
    source_tokens = torch.empty(S, dtype=torch.int64, device=dev)
    call("moe_dispatch_meta", ptr(ids), ptr(sc), ptr(perm), S, local_count, k, ptr(send_experts), ptr(send_scores),
         ptr(source_tokens), s)
    return send_hidden, send_experts, send_scores.to(scores.dtype), source_tokens, pos, counts


@dispatch_fwd.register_fake
def _(hidden, global_indices, scores, local_count, ep_size):
    S = global_indices.shape[0] * global_indices.shape[1]
    return (hidden.new_empty(S, hidden.shape[1]), global_indices.new_empty(S, dtype=torch.int64),
            scores.new_empty(S), global_indices.new_empty(S, dtype=torch.int64),
            global_indices.new_empty(S, dtype=torch.int32), global_indices.new_empty(ep_size, dtype=torch.int32))


def _dispatch_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)
    hidden, global_indices, scores, local_count, ep_size = inputs
    _, send_experts, _, source_tokens, pos, counts = output
    ctx.save_for_backward(pos)
    ctx.T, ctx.k = global_indices.shape
    ctx.hidden_dtype = hidden.dtype
    ctx.scores_dtype = scores.dtype
    ctx.mark_non_differentiable(send_experts, source_tokens, pos, counts)


def _dispatch_backward(ctx, d_send_hidden, _d_experts, d_send_scores, *_unused):
    (pos,) = ctx.saved_tensors
    d_hidden = d_scores = None
    if d_send_hidden is not None:
        d_hidden = combine_rows_fwd(d_send_hidden.to(BF16).contiguous(), pos, ctx.T, ctx.k).to(ctx.hidden_dtype)
    if d_send_scores is not None:
        d_scores = d_send_scores.index_select(0, pos.long()).view(ctx.T, ctx.k).to(ctx.scores_dtype)
    return d_hidden, None, d_scores, None, None


dispatch_fwd.register_autograd(_dispatch_backward, setup_context=_dispatch_setup)


@torch.library.custom_op(f"{LIB}::combine_rows_fwd", mutates_args=())
def combine_rows_fwd(rows: Tensor, pos_of_slot: Tensor, num_tokens: int, top_k: int) -> Tensor:
    """out[t] = sum_j rows[pos_of_slot[t*k+j]] — TokenDispatcher.combine's index_add in gather form."""
    _require_gpu(rows, pos_of_slot)
    _require_bf16("combined rows", rows)
    S, H = rows.shape
    if S != num_tokens * top_k or pos_of_slot.numel() != S:
        raise ValueError(f"combine expects {num_tokens}*{top_k} rows, got {S}")
    out = torch.empty(num_tokens, H, dtype=rows.dtype, device=rows.device)
    n_valid = torch.full((1,), S, dtype=torch.int32, device=rows.device)
    call("moe_combine_fwd", ptr(rows.contiguous()), ptr(pos_of_slot), ptr(n_valid), 1, None, num_tokens, H, top_k,
         ptr(out), _stream(rows))
    return out


@combine_rows_fwd.register_fake
def _(rows, pos_of_slot, num_tokens, top_k):
    return rows.new_empty(num_tokens, rows.shape[1])


@torch.library.custom_op(f"{LIB}::combine_rows_bwd", mutates_args=())
def combine_rows_bwd(d_out: Tensor, pos_of_slot: Tensor, top_k: int) -> Tensor:
    """d_rows[pos_of_slot[t*k+j]] = d_out[t]."""
    T, H = d_out.shape
    S = T * top_k
    d_rows = torch.empty(S, H, dtype=BF16, device=d_out.device)
    n_valid = torch.full((1,), S, dtype=torch.int32, device=d_out.device)
    call("moe_combine_bwd", ptr(d_out.to(BF16).contiguous()), None, ptr(pos_of_slot), ptr(n_valid), 1, None, T, H,
         top_k, ptr(d_rows), None, _stream(d_out))
    return d_rows


@combine_rows_bwd.register_fake
def _(d_out, pos_of_slot, top_k):
    return d_out.new_empty(d_out.shape[0] * top_k, d_out.shape[1])


def _combine_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)
    _, pos, _, top_k = inputs
    ctx.save_for_backward(pos)
    ctx.top_k = top_k


def _combine_backward(ctx, d_out):
    (pos,) = ctx.saved_tensors
    if d_out is None:
        return None, None, None, None
    return combine_rows_bwd(d_out, pos, ctx.top_k), None, None, None


combine_rows_fwd.register_autograd(_combine_backward, setup_context=_combine_setup)

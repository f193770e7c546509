"""Router top-k on gfx950 (one HIP kernel, ``mtx_router_topk``).

``route_topk(logits, k, scoring="sigmoid_group", ...)`` reproduces bzantium/mintext
``MoERouter.__call__`` after the gate GEMM (mintext/modules/moe.py:53-67) together with
``_group_topk_routing`` (moe.py:69-103): sigmoid scores in float32, the loss-free
``e_score_correction_bias`` added for selection only, group score = sum of the top-2
biased scores per group, top ``topk_group`` groups kept, top-k of the biased scores in the
kept groups (descending, ties to the lower expert id), weights = unbiased scores,
``w / (sum(w) + 1e-20)`` when ``norm_topk_prob``, times ``routed_scaling_factor``.

``scoring="softmax"`` is the Mixtral / Qwen3-MoE router, which the reference does not
have: top-k on the logits (the order of the float32 softmax), weights renormalised over
the top-k (or the full-softmax probabilities when ``norm_topk_prob`` is False).
"""
from __future__ import annotations

import torch

from .. import _lib as L

_SCORING = {"softmax": L.MTX_SCORING_SOFTMAX, "sigmoid_group": L.MTX_SCORING_SIGMOID_GROUP,
            "sigmoid": L.MTX_SCORING_SIGMOID_GROUP}


def _router_fwd(lg, k, scoring, b, n_group, topk_group, norm_topk_prob, routed_scaling_factor, return_scores,
                shared_expert):
    dev = lg.device
    T, E = lg.shape
    kk = k if shared_expert is None else k + 1
    idx = torch.empty((T, kk), dtype=torch.int32, device=dev)
    w = torch.empty((T, kk), dtype=torch.float32, device=dev)
    scores = torch.empty((T, E), dtype=torch.float32, device=dev) if return_scores else None
    if shared_expert is None:
        L.call("mtx_router_topk", L.ptr(lg), L.dtype_code(lg.dtype), T, E, k, _SCORING[scoring], L.ptr(b),
               n_group, topk_group, int(bool(norm_topk_prob)), float(routed_scaling_factor), L.ptr(idx), L.ptr(w),
               L.ptr(scores), L.stream(dev))
    else:
        L.call("mtx_router_topk_shared", L.ptr(lg), L.dtype_code(lg.dtype), T, E, k, _SCORING[scoring], L.ptr(b),
               n_group, topk_group, int(bool(norm_topk_prob)), float(routed_scaling_factor), int(shared_expert),
               L.ptr(idx), L.ptr(w), L.ptr(scores), L.stream(dev))
    return idx, w, scores


def router_topk_bwd(logits: torch.Tensor, topk_indices: torch.Tensor, k: int, d_topk_weights, d_scores, *,
                    scoring: str = "softmax", norm_topk_prob: bool = True,
                    routed_scaling_factor: float = 1.0) -> torch.Tensor:
    """d logits [T, E] (logits' dtype) of the router's weights and scores for fixed indices
    (``mtx_router_topk_bwd``): the VJP that jax.grad takes through MoERouter.__call__
    (mintext/modules/moe.py:52-67,101).  ``topk_indices`` [T, k] or [T, k+1] (a folded shared
    expert's constant column is ignored); ``d_topk_weights`` [T, >=k] and ``d_scores`` [T, E] may
    be None (zero)."""
    dev = L.require_device(logits, topk_indices)
    lg = logits.contiguous()
    T, E = lg.shape
    idx = topk_indices.to(torch.int32).contiguous()
    dw = None if d_topk_weights is None else d_topk_weights[:, :k].to(torch.float32).contiguous()
    ds = None if d_scores is None else d_scores.to(torch.float32).contiguous()
    dl = torch.empty((T, E), dtype=lg.dtype, device=dev)
    L.call("mtx_router_topk_bwd", L.ptr(lg), L.dtype_code(lg.dtype), T, E, k, _SCORING[scoring],
           int(bool(norm_topk_prob)), float(routed_scaling_factor), L.ptr(idx), idx.shape[1], L.ptr(dw), L.ptr(ds),
           L.ptr(dl), L.dtype_code(dl.dtype), L.stream(dev))
    return dl


class _RouterTopK(torch.autograd.Function):
    """route_topk with its VJP: gradients reach the logits (and through them the gate weight and
    the tokens) from the weights and the scores, as under jax.grad of the reference router."""

    @staticmethod
    def forward(ctx, lg, k, scoring, b, n_group, topk_group, norm, rscale, return_scores, shared_expert):
        idx, w, scores = _router_fwd(lg, k, scoring, b, n_group, topk_group, norm, rscale, return_scores,
                                     shared_expert)
        ctx.mark_non_differentiable(idx)
        ctx.save_for_backward(lg, idx)
        ctx.cfg = (k, scoring, norm, rscale)
        return (idx, w, scores) if return_scores else (idx, w)

    @staticmethod
    def backward(ctx, _gidx, gw, gscores=None):
        lg, idx = ctx.saved_tensors
        k, scoring, norm, rscale = ctx.cfg
        if gw is None and gscores is None:
            return (None,) * 10
        dl = router_topk_bwd(lg, idx, k, gw, gscores, scoring=scoring, norm_topk_prob=norm,
                             routed_scaling_factor=rscale)
        return (dl,) + (None,) * 9


def route_topk(logits: torch.Tensor, k: int, *, scoring: str = "softmax", bias: torch.Tensor | None = None,
               n_group: int = 1, topk_group: int = 1, norm_topk_prob: bool = True,
               routed_scaling_factor: float = 1.0, return_scores: bool = False, shared_expert: int | None = None):
    """Select the top-k experts per token.

    Args:
        logits: [T, E] router logits (float32 or bfloat16), i.e. the gate Linear output.
        k: experts per token.
        scoring: "softmax" or "sigmoid_group".
        bias: [E] float32 e_score_correction_bias (sigmoid_group only; None = zeros).
        shared_expert: id (>= E) of a shared expert folded into the routed weights: the
            outputs get a column k naming it with weight 1.0 (``mtx_router_topk_shared``).

    Returns:
        (topk_indices [T,k] int32, topk_weights [T,k] float32) -- [T,k+1] with a shared
        expert -- and, with return_scores, scores [T,E] float32 (sigmoid scores, or softmax
        probabilities).  Differentiable: with ``logits.requires_grad`` the weights and scores
        carry the router's VJP (``router_topk_bwd``); the bias gets no gradient.
    """
    if scoring not in _SCORING:
        raise ValueError(f"unknown scoring {scoring!r}")
    dev = L.require_device(logits)
    lg = logits
    if lg.dtype not in (torch.float32, torch.bfloat16):
        lg = lg.float()
    lg = lg.contiguous()
    b = None
    if bias is not None:
        b = bias.detach().to(device=dev, dtype=torch.float32).contiguous()
    args = (k, scoring, b, n_group, topk_group, norm_topk_prob, routed_scaling_factor, return_scores, shared_expert)
    if torch.is_grad_enabled() and lg.requires_grad:
        return _RouterTopK.apply(lg, *args)
    idx, w, scores = _router_fwd(lg, *args)
    return (idx, w, scores) if return_scores else (idx, w)


def gate_weight_linear_layout(gate_weight: torch.Tensor) -> torch.Tensor:
    """The router gate kernel [D, E] (the reference's ``kernel_axes=("embed", "mlp")`` layout,
    moe.py:30-35) -> the nn.Linear layout [E, D] that ``gate_route_topk`` reads (each expert's
    weights k-contiguous).  A load-time transform on the device (``mtx_transpose_batched``)."""
    from .expert_layout import _transpose_into

    dev = L.require_device(gate_weight)
    w = gate_weight.contiguous()
    D, E = w.shape
    out = torch.empty((E, D), dtype=w.dtype, device=dev)
    _transpose_into(w, out, 1, D, E, D * E, E, E * D, D)
    return out


def gate_supported(x: torch.Tensor, E: int) -> bool:
    """Whether ``gate_route_topk`` covers this input (bf16 tokens, D % 64 == 0, E <= 256)."""
    return x.dtype == torch.bfloat16 and x.dim() == 2 and x.shape[1] % 64 == 0 and x.shape[1] > 0 and 1 <= E <= 256


# Each 32-token workgroup of the fused kernel reads the whole gate weight, so it beats a dense
# gate GEMM + top-k only for few experts (measured: Mixtral E=8 19.6 vs 33.6 us; E=128 69 vs
# 33 us, E=256 189 vs 57 us; bench.py --study gate).
GATE_FUSED_MAX_E = 32


def gate_fused_preferred(x: torch.Tensor, E: int) -> bool:
    """Whether ``moe_block_forward`` should run the fused gate for this input."""
    return gate_supported(x, E) and E <= GATE_FUSED_MAX_E


def gate_route_topk(x: torch.Tensor, gate_weight_t: torch.Tensor, k: int, *, scoring: str = "softmax",
                    bias: torch.Tensor | None = None, n_group: int = 1, topk_group: int = 1,
                    norm_topk_prob: bool = True, routed_scaling_factor: float = 1.0,
                    shared_expert: int | None = None, return_logits: bool = False, return_scores: bool = False):
    """Router gate GEMM and top-k in one kernel (``mtx_gate_router_topk``): the gate
    ``Linear.__call__`` (mintext/modules/linear.py:123-147) -- logits = x @ W_g with f32
    accumulation and one rounding to bf16 -- followed by ``route_topk`` on those logits, with no
    [T, E] round trip through memory.

    Args:
        x: [T, D] bfloat16 tokens (D % 64 == 0).
        gate_weight_t: [E, D] bfloat16 gate weight in the nn.Linear layout
            (``gate_weight_linear_layout`` of the reference's [D, E] kernel), E <= 256.
        k, scoring, bias, n_group, topk_group, norm_topk_prob, routed_scaling_factor,
        shared_expert: as ``route_topk``.

    Returns:
        (topk_indices, topk_weights) as ``route_topk`` on the bf16 logits, then the logits
        [T, E] bfloat16 with ``return_logits`` and the scores [T, E] float32 with
        ``return_scores``.  Forward only: for gradients run the gate GEMM and ``route_topk``.
    """
    if scoring not in _SCORING:
        raise ValueError(f"unknown scoring {scoring!r}")
    if torch.is_grad_enabled() and (x.requires_grad or gate_weight_t.requires_grad):
        raise RuntimeError("gate_route_topk has no VJP; under autograd use x @ gate_weight and route_topk")
    dev = L.require_device(x, gate_weight_t)
    xc = x.contiguous()
    wt = gate_weight_t.contiguous()
    T, D = xc.shape
    E = wt.shape[0]
    if wt.shape[1] != D:
        raise ValueError(f"gate weight {tuple(wt.shape)} does not match tokens [T, {D}]")
    kk = k if shared_expert is None else k + 1
    idx = torch.empty((T, kk), dtype=torch.int32, device=dev)
    w = torch.empty((T, kk), dtype=torch.float32, device=dev)
    logits = torch.empty((T, E), dtype=torch.bfloat16, device=dev) if return_logits else None
    scores = torch.empty((T, E), dtype=torch.float32, device=dev) if return_scores else None
    b = None if bias is None else bias.to(device=dev, dtype=torch.float32).contiguous()
    L.call("mtx_gate_router_topk", L.ptr(xc), L.dtype_code(xc.dtype), L.ptr(wt.to(xc.dtype)), T, D, E, k,
           _SCORING[scoring], L.ptr(b), n_group, topk_group, int(bool(norm_topk_prob)), float(routed_scaling_factor),
           -1 if shared_expert is None else int(shared_expert), L.ptr(idx), L.ptr(w), L.ptr(logits), L.ptr(scores),
           L.stream(dev))
    out = (idx, w)
    if return_logits:
        out += (logits,)
    if return_scores:
        out += (scores,)
    return out


def update_expert_bias(bias: torch.Tensor, expert_counts: torch.Tensor, rate: float) -> torch.Tensor:
    """Loss-free load balancing of one MoE layer, in place (update_expert_biases,
    mintext/trainer.py:371-410): ``bias += rate * sign(mean(counts) - counts)``.

    ``expert_counts`` is the layer's bincount of its top-k indices (trainer.py:297-308), which
    is the ``group_sizes`` that ``route`` returns.  ``bias`` is the float32 [E]
    ``e_score_correction_bias``; it is returned for chaining.
    """
    dev = L.require_device(bias, expert_counts)
    if bias.dtype != torch.float32 or not bias.is_contiguous():
        raise TypeError("bias must be a contiguous float32 tensor (updated in place)")
    counts = expert_counts.to(torch.int32).contiguous()
    if counts.numel() != bias.numel():
        raise ValueError(f"expert_counts has {counts.numel()} entries for {bias.numel()} experts")
    L.call("mtx_expert_bias_update", L.ptr(counts), bias.numel(), float(rate), L.ptr(bias), L.stream(dev))
    return bias

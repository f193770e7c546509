"""MoE expert layer composed from the gfx950 kernels.

``moe_experts_forward`` is the composition of bzantium/mintext
``MoEExperts._forward_kernel`` (mintext/modules/moe.py:161-221): cast the expert weights to
the compute dtype (:170-171), ``route`` (:174-176), gate_up grouped GEMM (:189-192), SwiGLU
(:195-196), down grouped GEMM (:199-202), ``unroute`` (:221).  Without autograd the gate_up
GEMM and the SwiGLU run as one fused kernel.

``moe_layer_forward`` prepends the router top-k on given gate logits (moe.py:52-67) and,
optionally, a shared expert (moe.py:256-258): either evaluated as a one-group grouped GEMM
and added, or -- after the load-time ``fold_shared_expert`` -- folded into the routed GEMMs
as an always-routed extra expert with weight 1, whose output the combine adds after the
routed sum (the same sum, in the same order, as routed_out + shared_out).

Without autograd (and for the shapes the direct-to-LDS GEMM takes) the route's row gather runs
inside the gate_up GEMM: ``route_indices`` computes the permutation only and the GEMM reads
token row ``sort_indices[r] // K`` for sorted row r, so the sorted copy of the tokens is never
written (the same bits as route + GEMM).

``moe_experts_forward_fp8`` is the blockwise-fp8 variant (no reference counterpart):
activations quantised in 1x128 groups in token order, fp8 gate_up GEMM on the gathered rows
with the SwiGLU and the 1x128 re-quantisation fused, fp8 down GEMM to bf16, float32 combine.
"""
from __future__ import annotations

import torch

from .kernels.grouped_matmul import (gathered_swiglu_supported, grouped_matmul_swiglu, grouped_matmul_swiglu_gathered,
                                     grouped_matmul_vjp)
from .kernels.moe_dispatch import route, route_indices, route_quantize_fp8, unroute, unroute_add
from .kernels.router import gate_fused_preferred, gate_route_topk, gate_weight_linear_layout, route_topk
from .kernels.swiglu import swiglu_autograd


def moe_experts_forward(x: torch.Tensor, topk_indices: torch.Tensor, topk_weights: torch.Tensor,
                        gate_up: torch.Tensor, down: torch.Tensor, *, fuse_swiglu: bool | None = None,
                        gate_up_tiling=None, down_tiling=None, return_group_sizes: bool = False,
                        addend: torch.Tensor | None = None):
    """[N, D] tokens -> [N, D] in result_type(x, topk_weights) (float32 for bf16 + f32 weights).

    ``gate_up_tiling`` / ``down_tiling``: HIP tile configurations (``kernels.autotuner``), the
    counterparts of ``MoEExperts.gate_up_tiling`` / ``down_tiling`` (moe.py:189-202) that the
    reference's train.py:43-52 fills from the autotuner.  With ``return_group_sizes`` the
    result is ``(out, group_sizes)``: the per-expert token counts (the bincount of
    trainer.py:297-308) that ``route`` computed anyway.  ``addend`` ([N, D], e.g. the shared
    expert's output) is added to the combined output in the combine's own pass.
    """
    gate_up = gate_up.to(x.dtype)
    down = down.to(x.dtype)
    E = gate_up.shape[0]
    needs_grad = torch.is_grad_enabled() and (
        x.requires_grad or gate_up.requires_grad or down.requires_grad or topk_weights.requires_grad)
    if fuse_swiglu is None:
        fuse_swiglu = not needs_grad
    if fuse_swiglu and not needs_grad and gathered_swiglu_supported(x, gate_up):
        # the route's row gather runs in the gate_up GEMM's operand loads: no sorted copy
        sort_indices, group_sizes, _ = route_indices(topk_indices, E)
        inter = grouped_matmul_swiglu_gathered(x, sort_indices, topk_indices.shape[1], gate_up, group_sizes,
                                               tiling=gate_up_tiling)
    else:
        sorted_tokens, sort_indices, group_sizes = route(x, topk_indices, E)
        if fuse_swiglu:
            inter = grouped_matmul_swiglu(sorted_tokens, gate_up, group_sizes, tiling=gate_up_tiling)
        else:
            h = grouped_matmul_vjp(sorted_tokens, gate_up, group_sizes, tiling=gate_up_tiling)
            inter = swiglu_autograd(h)
    out = grouped_matmul_vjp(inter, down, group_sizes, tiling=down_tiling)
    if addend is None:
        res = unroute(out, sort_indices, topk_weights, topk_indices.shape[1])
    else:
        res = unroute_add(out, sort_indices, topk_weights, topk_indices.shape[1], addend)
    return (res, group_sizes) if return_group_sizes else res


def fold_shared_expert(gate_up: torch.Tensor, down: torch.Tensor, shared_gate_up: torch.Tensor,
                       shared_down: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Load-time transform: the shared expert appended as expert E of the routed weights.

    gate_up [E, D, 2I] + shared [D, 2I] (or [1, D, 2I]) -> [E+1, D, 2I]; down [E, I, D] +
    shared [I, D] -> [E+1, I, D].  The shared expert's intermediate size must equal the routed
    one (DeepSeek-V3: n_shared_experts = 1, moe.py:231-236); the shared gate/up columns keep the
    gate-first layout.  Done once when the weights are loaded, never per step.
    """
    E, D, two_i = gate_up.shape
    sgu = shared_gate_up.reshape(-1, *shared_gate_up.shape[-2:])
    sdn = shared_down.reshape(-1, *shared_down.shape[-2:])
    if sgu.shape != (1, D, two_i) or sdn.shape != (1, two_i // 2, D) or down.shape != (E, two_i // 2, D):
        raise ValueError(f"shared expert {tuple(shared_gate_up.shape)}/{tuple(shared_down.shape)} does not fold "
                         f"into routed experts {tuple(gate_up.shape)}/{tuple(down.shape)} (intermediate sizes differ)")
    return (torch.cat([gate_up, sgu.to(gate_up.dtype)], 0).contiguous(),
            torch.cat([down, sdn.to(down.dtype)], 0).contiguous())


def moe_layer_forward(logits: torch.Tensor | None, x: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor, *,
                      k: int, scoring: str = "softmax", bias: torch.Tensor | None = None, n_group: int = 1,
                      topk_group: int = 1, norm_topk_prob: bool = True, routed_scaling_factor: float = 1.0,
                      shared_gate_up: torch.Tensor | None = None, shared_down: torch.Tensor | None = None,
                      shared_folded: bool = False, return_expert_counts: bool = False,
                      gate_weight_t: torch.Tensor | None = None, return_scores: bool = False):
    """Router top-k + routed experts (+ shared expert) -- MoEBlock.__call__ (moe.py:240-266) after
    the gate GEMM.  Returns (out [T,D] f32, topk_indices [T,k], topk_weights [T,k]), then, with
    ``return_expert_counts``, the [E] int32 per-expert token counts (trainer.py:297-308) and, with
    ``return_scores``, the router's [T,E] f32 scores (sigmoid scores, or softmax probabilities).
    Under autograd the weights (and scores) are differentiable in the logits (``route_topk``).

    ``shared_folded``: ``gate_up`` / ``down`` come from ``fold_shared_expert`` (E routed experts
    + the shared one as expert E, ``logits`` has E columns); the shared expert then runs inside
    the routed grouped GEMMs.  With ``gate_weight_t`` ([E, D], ``gate_weight_linear_layout``)
    and ``logits=None`` the gate GEMM and the top-k run as one kernel (``gate_route_topk``).
    """
    rkw = dict(scoring=scoring, bias=bias, n_group=n_group, topk_group=topk_group, norm_topk_prob=norm_topk_prob,
               routed_scaling_factor=routed_scaling_factor)
    if logits is None:
        if gate_weight_t is None:
            raise ValueError("moe_layer_forward needs the logits or the gate weight")
        E = gate_weight_t.shape[0]

        def topk(shared_expert=None):
            return gate_route_topk(x, gate_weight_t, k, shared_expert=shared_expert, return_scores=return_scores,
                                   **rkw)
    else:
        E = logits.shape[1]

        def topk(shared_expert=None):
            return route_topk(logits, k, shared_expert=shared_expert, return_scores=return_scores, **rkw)
    if shared_folded:
        if gate_up.shape[0] != E + 1:
            raise ValueError(f"folded weights need {E + 1} experts (E routed + shared), got {gate_up.shape[0]}")
        r = topk(shared_expert=E)
        out, gs = moe_experts_forward(x, r[0], r[1], gate_up, down, return_group_sizes=True)
        idx, w = r[0][:, :k], r[1][:, :k]
    else:
        r = topk()
        idx, w = r[0], r[1]
        # the shared expert's output joins the combine's pass: routed_out + shared_out (moe.py:256-258)
        shared = None if shared_gate_up is None else shared_expert_forward(x, shared_gate_up, shared_down)
        out, gs = moe_experts_forward(x, idx, w, gate_up, down, return_group_sizes=True, addend=shared)
    res = (out, idx, w)
    if return_expert_counts:
        res += (gs[:E],)
    if return_scores:
        res += (r[2],)
    return res


def moe_block_forward(x: torch.Tensor, gate_weight: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor, *,
                      k: int, scoring: str = "sigmoid_group", bias: torch.Tensor | None = None, n_group: int = 1,
                      topk_group: int = 1, norm_topk_prob: bool = True, routed_scaling_factor: float = 1.0,
                      shared_gate_up: torch.Tensor | None = None, shared_down: torch.Tensor | None = None,
                      shared_folded: bool = False, gate_weight_t: torch.Tensor | None = None):
    """``MoEBlock.__call__`` (mintext/modules/moe.py:240-266) on [B, S, D] or [N, D] tokens.

    The router gate is ``Linear.__call__`` (mintext/modules/linear.py:123-147): a dense GEMM
    ``x @ gate_weight`` ([D, E], the reference's kernel layout) with f32 accumulation and one
    rounding to the compute dtype.  For bf16 tokens with D % 64 == 0 and few experts (E <= 32,
    where it is faster; outside autograd) it runs fused with the top-k (``gate_route_topk``) on
    the gate weight in the
    nn.Linear layout -- pass ``gate_weight_t = gate_weight_linear_layout(gate_weight)``, a
    load-time transform, to skip the per-call transpose; otherwise the GEMM is hipBLASLt's
    (``torch.matmul``) and the top-k ``route_topk``.  Returns
    ``(output [.., D] float32, {"topk_indices", "scores", "topk_weights", "expert_counts"})``: the
    reference's aux data (moe.py:262-266; ``scores`` [N, E] float32 are the sigmoid scores, or the
    softmax probabilities in softmax mode) plus the weights and the counts of trainer.py:297-308.
    Under autograd the gradient reaches ``gate_weight`` and ``x`` through the router's weights
    (moe.py:53,101), as under jax.grad of the reference block.
    """
    shape = x.shape
    xf = x.reshape(-1, shape[-1])
    E = gate_weight.shape[-1]
    needs_grad = torch.is_grad_enabled() and (x.requires_grad or gate_weight.requires_grad)
    if not needs_grad and gate_fused_preferred(xf, E):
        # gate GEMM + top-k in one kernel on the nn.Linear-layout gate weight
        if gate_weight_t is None:
            gate_weight_t = gate_weight_linear_layout(gate_weight.to(xf.dtype))
        logits = None
    else:
        logits = torch.matmul(xf, gate_weight.to(xf.dtype))
        gate_weight_t = None
    out, idx, w, counts, scores = moe_layer_forward(
        logits, xf, gate_up, down, k=k, scoring=scoring, bias=bias, n_group=n_group, topk_group=topk_group,
        norm_topk_prob=norm_topk_prob, routed_scaling_factor=routed_scaling_factor, shared_gate_up=shared_gate_up,
        shared_down=shared_down, shared_folded=shared_folded, return_expert_counts=True, gate_weight_t=gate_weight_t,
        return_scores=True)
    aux = {"topk_indices": idx, "scores": scores, "topk_weights": w, "expert_counts": counts}
    return out.reshape(*shape[:-1], out.shape[-1]), aux


def shared_expert_forward(x: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor) -> torch.Tensor:
    """Dense SwiGLU MLP (mintext/modules/linear.py:164-228 as used at moe.py:231-236) as a
    one-group grouped GEMM: gate_up [D, 2I] or [1, D, 2I], down [I, D] or [1, I, D].  Under
    autograd the gate_up GEMM and the SwiGLU run as their differentiable steps."""
    gu = gate_up.reshape(1, *gate_up.shape[-2:]).to(x.dtype)
    dn = down.reshape(1, *down.shape[-2:]).to(x.dtype)
    gs = torch.full((1,), x.shape[0], dtype=torch.int32, device=x.device)
    if torch.is_grad_enabled() and (x.requires_grad or gu.requires_grad or dn.requires_grad):
        inter = swiglu_autograd(grouped_matmul_vjp(x, gu, gs))
    else:
        inter = grouped_matmul_swiglu(x, gu, gs)
    return grouped_matmul_vjp(inter, dn, gs)


def moe_experts_forward_fp8(x: torch.Tensor, topk_indices: torch.Tensor, topk_weights: torch.Tensor,
                            gate_up_q: torch.Tensor, gate_up_scale: torch.Tensor, down_q: torch.Tensor,
                            down_scale: torch.Tensor, *, scales: str = "amax") -> torch.Tensor:
    """Blockwise-fp8 expert layer; weights from ``quantize_fp8_weights`` ([E, Kout, Kin] e4m3).
    ``scales`` is the mode the weights were quantised in and the activations are quantised in:
    "amax" (scale amax/448) or "pow2" (power-of-two scales applied by the MFMA; needs D and I of at
    least 256).  Forward only: raises under autograd when an input requires grad."""
    if torch.is_grad_enabled() and any(t.requires_grad for t in (x, topk_weights, gate_up_q, down_q)):
        raise RuntimeError("moe_experts_forward_fp8 is forward-only; run it under torch.no_grad(), or train "
                           "through moe_experts_forward or moe_experts_forward_fp8_train")
    from .kernels.fp8 import (SCALE_MODES, grouped_matmul_fp8, grouped_matmul_fp8_swiglu,
                              grouped_matmul_fp8_swiglu_gathered, quantize_fp8_rows)
    if scales not in SCALE_MODES:
        raise ValueError(f"scales must be one of {SCALE_MODES}, got {scales!r}")
    f8s = dict(scales=scales)
    E = gate_up_q.shape[0]
    T, D = x.shape
    if scales == "pow2" or (D >= 256 and T * D < 2 ** 32 and gate_up_q.shape[1] * D < 2 ** 32):
        # tokens quantised in token order; the gate_up GEMM gathers their rows (no sorted copy).  The
        # power-of-two GEMMs have no other form: shapes outside it raise from the kernels.
        xq, xs = quantize_fp8_rows(x, **f8s)
        sort_indices, group_sizes, _ = route_indices(topk_indices, E)
        yq, ys = grouped_matmul_fp8_swiglu_gathered(xq, xs, sort_indices, topk_indices.shape[1], gate_up_q,
                                                    gate_up_scale, group_sizes, **f8s)
    else:
        # 1x128 quantisation of the tokens fused into their dispatch (each row read once)
        sq, ss, sort_indices, group_sizes, _ = route_quantize_fp8(x, topk_indices, E)
        yq, ys = grouped_matmul_fp8_swiglu(sq, ss, gate_up_q, gate_up_scale, group_sizes)
    out = grouped_matmul_fp8(yq, ys, down_q, down_scale, group_sizes, **f8s)
    return unroute(out, sort_indices, topk_weights, topk_indices.shape[1])


def moe_experts_forward_fp8_train(x: torch.Tensor, topk_indices: torch.Tensor, topk_weights: torch.Tensor,
                                  gate_up: torch.Tensor, down: torch.Tensor, *, scales: str = "amax") -> torch.Tensor:
    """Differentiable blockwise-fp8 expert layer: the composition of ``moe_experts_forward``
    (route, gate_up GEMM, SwiGLU, down GEMM, combine; moe.py:161-221) with both grouped GEMMs as
    ``grouped_matmul_fp8_vjp``, so that all six GEMMs of a training step (the two forward
    products, the two dlhs and the two tgmm) run on fp8 operands.  gate_up [E, D, 2I] and down
    [E, I, D] are the master weights (reference layout), quantised on each call; x [N, D] bf16.
    Gradients reach x, topk_weights, gate_up and down.  ``scales``: "amax" (amax / 448) or "pow2"
    (power-of-two scales applied by the MFMA) in every quantisation."""
    from .kernels.fp8 import grouped_matmul_fp8_vjp

    E = gate_up.shape[0]
    sorted_tokens, sort_indices, group_sizes = route(x, topk_indices, E)
    h = grouped_matmul_fp8_vjp(sorted_tokens, gate_up, group_sizes, scales=scales)
    inter = swiglu_autograd(h)
    out = grouped_matmul_fp8_vjp(inter, down, group_sizes, scales=scales)
    return unroute(out, sort_indices, topk_weights, topk_indices.shape[1])


class CapturedLayer:
    """A MoE layer forward captured once in a HIP graph and replayed (for serving loops and
    launch-bound shapes, where per-kernel host launches dominate).

    ``fn(*inputs)`` must return a tensor or a tuple of tensors and run only device work (every
    entry point of this package does: no host synchronisation, no allocation in the C-ABI, no
    memset nodes).  ``inputs`` are the static input tensors: refill them in place (``copy_``)
    between replays.  ``replay()`` returns the static outputs, overwritten by each replay.
    """

    def __init__(self, fn, *inputs, warmup: int = 2):
        self.inputs = inputs
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(warmup):  # allocator and library state settle outside the capture
                fn(*inputs)
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph), torch.no_grad():
            self.outputs = fn(*inputs)

    def replay(self):
        self.graph.replay()
        return self.outputs

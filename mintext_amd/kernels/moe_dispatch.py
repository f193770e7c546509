"""Token routing for the MoE grouped GEMM: sort by expert, unsort + weighted combine.

Drop-in for bzantium/mintext ``mintext/kernels/moe_dispatch.py`` (same names, argument
meanings and output dtypes), with every op running as HIP kernels from
``libmintext_moe.so`` on the current stream:

* ``route`` (moe_dispatch.py:47-81): stable counting sort of ``ravel(topk_indices)`` by
  expert id, row gather ``tokens[sort_indices // K]``, bincount -- ``mtx_route``.
* ``unroute`` (moe_dispatch.py:84-111): inverse permutation and the k-ordered weighted
  sum in float32 -- ``mtx_invert_permutation`` + ``mtx_unroute``.  The output dtype is
  ``result_type(sorted_output, topk_weights)`` (float32 for bf16 outputs and f32 weights).
* ``_sort_with_vjp`` (moe_dispatch.py:21-41): row gather whose VJP is the inverse scatter.

Gradients (the reference's custom VJPs) are torch.autograd Functions over the same kernels.
"""
from __future__ import annotations

import torch

from .. import _lib as L


def _as_i32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 else t.to(torch.int32)


def _route_impl(tokens: torch.Tensor, topk_indices: torch.Tensor, num_experts: int):
    dev = L.require_device(tokens, topk_indices)
    tokens = tokens.contiguous()
    idx = _as_i32(topk_indices).contiguous()
    N, K = idx.shape
    D = tokens.shape[1]
    if tokens.shape[0] != N:
        raise ValueError(f"tokens has {tokens.shape[0]} rows, topk_indices {N}")
    M = N * K
    sorted_tokens = torch.empty((M, D), dtype=tokens.dtype, device=dev)
    sort_indices = torch.empty((M,), dtype=torch.int32, device=dev)
    group_sizes = torch.empty((num_experts,), dtype=torch.int32, device=dev)
    inverse = torch.empty((M,), dtype=torch.int32, device=dev)
    ws = L.workspace(L.query("mtx_route_workspace_size", N, K, num_experts), dev)
    L.call("mtx_route", L.ptr(tokens), L.dtype_code(tokens.dtype), L.ptr(idx), N, D, K, num_experts,
           L.ptr(sorted_tokens), L.ptr(sort_indices), L.ptr(group_sizes), L.ptr(inverse), None, None,
           L.ptr(ws), ws.numel(), L.stream(dev))
    return sorted_tokens, sort_indices, group_sizes, inverse


def route_indices(topk_indices: torch.Tensor, num_experts: int):
    """The permutation half of ``route`` (moe_dispatch.py:70-79) without moving any rows.

    Returns (sort_indices [N*K] i32, group_sizes [E] i32, inverse [N*K] i32) equal to the ones
    ``route`` returns.  For GEMMs that read the token rows through ``sort_indices`` themselves
    (``grouped_matmul_swiglu_gathered``, ``grouped_matmul_fp8_swiglu_gathered``), so that the
    sorted copy of the tokens is never written.  Forward only.
    """
    dev = L.require_device(topk_indices)
    idx = _as_i32(topk_indices).contiguous()
    N, K = idx.shape
    M = N * K
    sort_indices = torch.empty((M,), dtype=torch.int32, device=dev)
    group_sizes = torch.empty((num_experts,), dtype=torch.int32, device=dev)
    inverse = torch.empty((M,), dtype=torch.int32, device=dev)
    ws = L.workspace(L.query("mtx_route_workspace_size", N, K, num_experts), dev)
    L.call("mtx_route", None, L.dtype_code(torch.float32), L.ptr(idx), N, 0, K, num_experts, None,
           L.ptr(sort_indices), L.ptr(group_sizes), L.ptr(inverse), None, None, L.ptr(ws), ws.numel(),
           L.stream(dev))
    sort_indices._mtx_inverse = inverse
    sort_indices._mtx_version = sort_indices._version
    return sort_indices, group_sizes, inverse


def _inverse_of(sort_indices: torch.Tensor) -> torch.Tensor:
    """Inverse permutation; reuses the one route() computed when sort_indices is unchanged."""
    cached = getattr(sort_indices, "_mtx_inverse", None)
    if cached is not None and getattr(sort_indices, "_mtx_version", None) == sort_indices._version:
        return cached
    dev = L.require_device(sort_indices)
    si = _as_i32(sort_indices).contiguous()
    inv = torch.empty_like(si)
    L.call("mtx_invert_permutation", L.ptr(si), si.numel(), L.ptr(inv), L.stream(dev))
    return inv


def _combine(Y: torch.Tensor, inv: torch.Tensor, w: torch.Tensor | None, N: int, K: int,
             out_dtype: torch.dtype) -> torch.Tensor:
    dev = L.require_device(Y, inv)
    Y = Y.contiguous()
    D = Y.shape[1]
    out = torch.empty((N, D), dtype=out_dtype, device=dev)
    wc = None if w is None else w.contiguous()
    L.call("mtx_unroute", L.ptr(Y), L.dtype_code(Y.dtype), L.ptr(inv), L.ptr(wc),
           L.MTX_F32 if wc is None else L.dtype_code(wc.dtype), N, K, D, L.ptr(out),
           L.dtype_code(out_dtype), L.stream(dev))
    return out


class _Route(torch.autograd.Function):
    @staticmethod
    def forward(ctx, tokens, topk_indices, num_experts):
        sorted_tokens, sort_indices, group_sizes, inverse = _route_impl(tokens, topk_indices, num_experts)
        ctx.save_for_backward(inverse)
        ctx.nk = topk_indices.shape
        ctx.tok_dtype = tokens.dtype
        ctx.mark_non_differentiable(sort_indices, group_sizes)
        sort_indices._mtx_inverse = inverse
        sort_indices._mtx_version = sort_indices._version
        return sorted_tokens, sort_indices, group_sizes

    @staticmethod
    def backward(ctx, g_sorted, _g_si, _g_gs):
        (inverse,) = ctx.saved_tensors
        N, K = ctx.nk
        # d tokens[n] = sum_k d sorted[inverse[n*K+k]]  (repeat VJP after the sort VJP)
        dx = _combine(g_sorted, inverse, None, N, K, ctx.tok_dtype)
        return dx, None, None


def _combine_add(Y: torch.Tensor, inv: torch.Tensor, w: torch.Tensor, N: int, K: int, addend: torch.Tensor,
                 out_dtype: torch.dtype) -> torch.Tensor:
    if addend.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"addend dtype {addend.dtype} not supported")
    dev = L.require_device(Y, inv, w, addend)
    Y = Y.contiguous()
    D = Y.shape[1]
    if tuple(addend.shape) != (N, D):
        raise ValueError(f"addend shape {tuple(addend.shape)} != {(N, D)}")
    a = addend.contiguous()
    wc = w.contiguous()
    out = torch.empty((N, D), dtype=out_dtype, device=dev)
    L.call("mtx_unroute_add", L.ptr(Y), L.dtype_code(Y.dtype), L.ptr(inv), L.ptr(wc), L.dtype_code(wc.dtype), N, K, D,
           L.ptr(a), L.dtype_code(a.dtype), L.ptr(out), L.dtype_code(out_dtype), L.stream(dev))
    return out


class _Unroute(torch.autograd.Function):
    """unroute, and with an addend unroute + addend (one combine pass either way); the VJP is
    ``mtx_unroute_bwd`` for the expert outputs and weights, the identity for the addend."""

    @staticmethod
    def forward(ctx, sorted_output, sort_indices, topk_weights, K, addend=None):
        N = topk_weights.shape[0]
        inv = _inverse_of(sort_indices)
        out_dtype = torch.result_type(sorted_output, topk_weights)
        if out_dtype not in (torch.float32, torch.bfloat16):
            raise TypeError(f"unroute output dtype {out_dtype} not supported")
        w = topk_weights.contiguous()
        if addend is None:
            out = _combine(sorted_output, inv, w, N, K, out_dtype)
        else:
            out = _combine_add(sorted_output, inv, w, N, K, addend, out_dtype)
            ctx.add_dtype = addend.dtype
        ctx.save_for_backward(sorted_output, inv, w)
        ctx.K = K
        return out

    @staticmethod
    def backward(ctx, dout):
        Y, inv, w = ctx.saved_tensors
        K = ctx.K
        dev = L.require_device(dout)
        N = w.shape[0]
        D = Y.shape[1]
        dout = dout.contiguous()
        if dout.dtype not in (torch.float32, torch.bfloat16):
            dout = dout.float()
        dY = dw = None
        if ctx.needs_input_grad[0] or ctx.needs_input_grad[2]:
            dY = torch.empty_like(Y.contiguous())  # the kernel writes d sorted_output whenever it runs
            dw = torch.empty_like(w) if ctx.needs_input_grad[2] else None
            L.call("mtx_unroute_bwd", L.ptr(dout), L.dtype_code(dout.dtype), L.ptr(Y.contiguous()),
                   L.dtype_code(Y.dtype), L.ptr(inv), L.ptr(w), L.dtype_code(w.dtype), N, K, D,
                   L.ptr(dY), L.ptr(dw), L.stream(dev))
        da = None
        if len(ctx.needs_input_grad) > 4 and ctx.needs_input_grad[4]:
            da = dout.to(ctx.add_dtype)
        return dY, None, dw, None, da


class _SortWithVjp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, indices):
        dev = L.require_device(x, indices)
        x = x.contiguous()
        idx = _as_i32(indices).contiguous()
        rows = idx.numel()
        D = x.shape[1] if x.dim() > 1 else 1
        out = torch.empty((rows,) + tuple(x.shape[1:]), dtype=x.dtype, device=dev)
        L.call("mtx_gather_rows", L.ptr(x), L.dtype_code(x.dtype), x.shape[0], D, L.ptr(idx), rows, 1,
               L.ptr(out), L.stream(dev))
        ctx.save_for_backward(idx)
        ctx.xshape = x.shape
        return out

    @staticmethod
    def backward(ctx, g):
        (idx,) = ctx.saved_tensors
        dev = L.require_device(g)
        g = g.contiguous()
        D = g.shape[1] if g.dim() > 1 else 1
        # gather by argsort(indices) == scatter to indices when indices is a permutation
        dx = torch.zeros(ctx.xshape, dtype=g.dtype, device=dev)
        L.call("mtx_scatter_rows", L.ptr(g), L.dtype_code(g.dtype), idx.numel(), D, L.ptr(idx), L.ptr(dx),
               L.stream(dev))
        return dx, None


def _sort_with_vjp(x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """Gather x by indices: out[i] = x[indices[i]] (moe_dispatch.py:21-24)."""
    return _SortWithVjp.apply(x, indices)


def route(tokens: torch.Tensor, topk_indices: torch.Tensor, num_experts: int):
    """Sort tokens by expert assignment for grouped matmul (moe_dispatch.py:47-81).

    Args:
        tokens: [N, D] flattened activations (float32 / bfloat16 / float8_e4m3fn).
        topk_indices: [N, K] expert indices per token.
        num_experts: total number of experts E.

    Returns:
        sorted_tokens: [N*K, D] tokens sorted by expert (contiguous groups).
        sort_indices: [N*K] int32 stable permutation (values are flat positions n*K+k).
        group_sizes: [E] int32 number of tokens assigned to each expert.
    """
    if tokens.dtype == torch.float8_e4m3fn:
        return _route_impl(tokens, topk_indices, num_experts)[:3]
    return _Route.apply(tokens, topk_indices, int(num_experts))


def unroute(sorted_output: torch.Tensor, sort_indices: torch.Tensor, topk_weights: torch.Tensor,
            num_experts_per_tok: int) -> torch.Tensor:
    """Unsort expert outputs and apply the weighted combination (moe_dispatch.py:84-111).

    Returns [N, D] in ``result_type(sorted_output, topk_weights)``.
    """
    return _Unroute.apply(sorted_output, sort_indices, topk_weights, int(num_experts_per_tok))


def unroute_add(sorted_output: torch.Tensor, sort_indices: torch.Tensor, topk_weights: torch.Tensor,
                num_experts_per_tok: int, addend: torch.Tensor) -> torch.Tensor:
    """``unroute(...) + addend`` -- the combine followed by ``output = routed_out + shared_out``
    of MoEBlock.__call__ (mintext/modules/moe.py:256-258) -- in one pass over the rows
    (``mtx_unroute_add``; the same f32 bits as the two steps).  ``addend`` is [N, D] float32 or
    bfloat16.  Differentiable in the expert outputs, the weights and the addend.
    """
    return _Unroute.apply(sorted_output, sort_indices, topk_weights, int(num_experts_per_tok), addend)


def route_quantize_fp8(tokens: torch.Tensor, topk_indices: torch.Tensor, num_experts: int):
    """1x128 e4m3 quantisation fused into the dispatch: the results of
    ``route_with_scales(*quantize_fp8_rows(tokens), topk_indices, num_experts)`` with each
    token row read once in its compute dtype (``mtx_route_quant_fp8``).  tokens [N, D] f32/bf16,
    D % 128 == 0.  Returns (sorted_q, sorted_scales, sort_indices, group_sizes, inverse).
    """
    dev = L.require_device(tokens, topk_indices)
    x = tokens.contiguous()
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"route_quantize_fp8 needs float32 or bfloat16 tokens, got {x.dtype}")
    idx = _as_i32(topk_indices).contiguous()
    N, K = idx.shape
    D = x.shape[1]
    M = N * K
    sorted_q = torch.empty((M, D), dtype=torch.float8_e4m3fn, device=dev)
    sorted_s = torch.empty((M, D // 128), dtype=torch.float32, device=dev)
    sort_indices = torch.empty((M,), dtype=torch.int32, device=dev)
    group_sizes = torch.empty((num_experts,), dtype=torch.int32, device=dev)
    inverse = torch.empty((M,), dtype=torch.int32, device=dev)
    ws = L.workspace(L.query("mtx_route_workspace_size", N, K, num_experts), dev)
    L.call("mtx_route_quant_fp8", L.ptr(x), L.dtype_code(x.dtype), L.ptr(idx), N, D, K, num_experts,
           L.ptr(sorted_q), L.ptr(sorted_s), L.ptr(sort_indices), L.ptr(group_sizes), L.ptr(inverse),
           L.ptr(ws), ws.numel(), L.stream(dev))
    sort_indices._mtx_inverse = inverse
    sort_indices._mtx_version = sort_indices._version
    return sorted_q, sorted_s, sort_indices, group_sizes, inverse


def route_with_scales(tokens_q: torch.Tensor, token_scales: torch.Tensor, topk_indices: torch.Tensor,
                      num_experts: int):
    """fp8 dispatch: route e4m3 tokens and their [N, D/128] f32 scales in one pass.

    Returns (sorted_q, sorted_scales, sort_indices, group_sizes, inverse).
    """
    dev = L.require_device(tokens_q, token_scales, topk_indices)
    tq = tokens_q.contiguous()
    sc = token_scales.contiguous().float()
    idx = _as_i32(topk_indices).contiguous()
    N, K = idx.shape
    D = tq.shape[1]
    M = N * K
    sorted_q = torch.empty((M, D), dtype=tq.dtype, device=dev)
    sorted_s = torch.empty((M, D // 128), dtype=torch.float32, device=dev)
    sort_indices = torch.empty((M,), dtype=torch.int32, device=dev)
    group_sizes = torch.empty((num_experts,), dtype=torch.int32, device=dev)
    inverse = torch.empty((M,), dtype=torch.int32, device=dev)
    ws = L.workspace(L.query("mtx_route_workspace_size", N, K, num_experts), dev)
    L.call("mtx_route", L.ptr(tq), L.MTX_FP8E4M3, L.ptr(idx), N, D, K, num_experts, L.ptr(sorted_q),
           L.ptr(sort_indices), L.ptr(group_sizes), L.ptr(inverse), L.ptr(sc), L.ptr(sorted_s),
           L.ptr(ws), ws.numel(), L.stream(dev))
    sort_indices._mtx_inverse = inverse
    sort_indices._mtx_version = sort_indices._version
    return sorted_q, sorted_s, sort_indices, group_sizes, inverse

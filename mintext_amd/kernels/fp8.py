"""Blockwise fp8 (e4m3fn) quantisation and grouped GEMM on gfx950.

The reference has no fp8 grouped GEMM; its fp8 conventions (e4m3fn, f32 scales, f32
accumulation) follow mintext/modules/linear.py:37-57, with DeepSeek-V3 style blockwise scales:
1x128 groups per activation row and 128x128 weight blocks, scale = amax / 448.

Weights are quantised once (a load-time transform) into the k-contiguous per-expert
nn.Linear layout ``w_q [E, Kout, Kin]`` with ``w_scale [E, Kout/128, Kin/128]``.
"""
from __future__ import annotations

import torch

from .. import _lib as L


def _gs(g):
    return (g if g.dtype == torch.int32 else g.to(torch.int32)).contiguous()


# Scale modes.  "amax": scale = amax / 448 (DeepSeek-V3 blockwise).  "pow2": the power-of-two scale
# 2^ceil(log2(amax / 448)) (exponent in [-126, 127], 1 for an all-zero group): the codes are exact
# quotients and the GEMMs hand the scales' exponents to the MFMA's E8M0 block-scale operands, so a
# GEMM in this mode needs operands quantised in it (the "_p2" entry points).
SCALE_MODES = ("amax", "pow2")


def _entry(name: str, scales: str) -> str:
    if scales not in SCALE_MODES:
        raise ValueError(f"scales must be one of {SCALE_MODES}, got {scales!r}")
    return name + ("_p2" if scales == "pow2" else "")


def quantize_fp8_rows(x: torch.Tensor, *, scales: str = "amax"):
    """x [M, D] (f32/bf16) -> (xq [M, D] float8_e4m3fn, x_scale [M, D/128] f32)."""
    dev = L.require_device(x)
    x = x.contiguous()
    M, D = x.shape
    xq = torch.empty((M, D), dtype=torch.float8_e4m3fn, device=dev)
    xs = torch.empty((M, D // 128), dtype=torch.float32, device=dev)
    L.call(_entry("mtx_quant_fp8_rows", scales), L.ptr(x), L.dtype_code(x.dtype), M, D, L.ptr(xq), L.ptr(xs),
           L.stream(dev))
    return xq, xs


def quantize_fp8_weights(w: torch.Tensor, *, scales: str = "amax"):
    """w [E, Kin, Kout] (reference layout) -> (w_q [E, Kout, Kin] e4m3fn, w_scale [E, Kout/128, Kin/128])."""
    dev = L.require_device(w)
    w = w.contiguous()
    E, Kin, Kout = w.shape
    wq = torch.empty((E, Kout, Kin), dtype=torch.float8_e4m3fn, device=dev)
    ws = torch.empty((E, Kout // 128, Kin // 128), dtype=torch.float32, device=dev)
    L.call(_entry("mtx_quant_fp8_weights", scales), L.ptr(w), L.dtype_code(w.dtype), E, Kin, Kout, L.ptr(wq),
           L.ptr(ws), L.stream(dev))
    return wq, ws


def grouped_matmul_fp8(xq, x_scale, w_q, w_scale, group_sizes, *, scales: str = "amax") -> torch.Tensor:
    """out [M, Kout] bf16 = blockwise-dequantised x @ W per group, f32 accumulation."""
    gs = _gs(group_sizes)
    dev = L.require_device(xq, x_scale, w_q, w_scale, gs)
    M, Kin = xq.shape
    E, Kout, Kin2 = w_q.shape
    if Kin2 != Kin:
        raise ValueError("fp8 gmm shape mismatch")
    out = torch.empty((M, Kout), dtype=torch.bfloat16, device=dev)
    ws = L.workspace(L.query("mtx_gmm_workspace_size", M, E), dev)
    L.call(_entry("mtx_gmm_fp8", scales), L.ptr(xq.contiguous()), L.ptr(x_scale.contiguous()), L.ptr(w_q.contiguous()),
           L.ptr(w_scale.contiguous()), L.ptr(gs), M, Kin, Kout, E, L.ptr(out), L.ptr(ws), ws.numel(),
           L.stream(dev))
    return out


def grouped_matmul_fp8_swiglu(xq, x_scale, w_q, w_scale, group_sizes, *, return_bf16: bool = False,
                              scales: str = "amax"):
    """SwiGLU of the fp8 gate_up GEMM (w_q [E, 2I, Kin]) re-quantised in 1x128 groups (in the same
    scale mode as the operands).

    Returns (yq [M, I] e4m3fn, y_scale [M, I/128] f32) and, with return_bf16, y [M, I] bf16.
    """
    gs = _gs(group_sizes)
    dev = L.require_device(xq, x_scale, w_q, w_scale, gs)
    M, Kin = xq.shape
    E, two_i, Kin2 = w_q.shape
    if Kin2 != Kin or two_i % 2:
        raise ValueError("fp8 gmm+swiglu shape mismatch")
    I = two_i // 2
    yq = torch.empty((M, I), dtype=torch.float8_e4m3fn, device=dev)
    ys = torch.empty((M, I // 128), dtype=torch.float32, device=dev)
    yb = torch.empty((M, I), dtype=torch.bfloat16, device=dev) if return_bf16 else None
    ws = L.workspace(L.query("mtx_gmm_workspace_size", M, E), dev)
    L.call(_entry("mtx_gmm_fp8_swiglu", scales), L.ptr(xq.contiguous()), L.ptr(x_scale.contiguous()),
           L.ptr(w_q.contiguous()),
           L.ptr(w_scale.contiguous()), L.ptr(gs), M, Kin, I, E, L.ptr(yq), L.ptr(ys), L.ptr(yb), L.ptr(ws),
           ws.numel(), L.stream(dev))
    if return_bf16:
        return yq, ys, yb
    return yq, ys


def grouped_matmul_fp8_swiglu_gathered(xq, x_scale, sort_indices, top_k: int, w_q, w_scale, group_sizes, *,
                                       return_bf16: bool = False, scales: str = "amax"):
    """``grouped_matmul_fp8_swiglu`` on the routed rows of token-order inputs: xq [T, Kin] and
    x_scale [T, Kin/128] are ``quantize_fp8_rows(tokens)``; sorted row r is token row
    ``sort_indices[r] // top_k``, read by the GEMM's operand loads (the dispatch copy is never
    written).  Same bits as ``route_quantize_fp8`` + ``grouped_matmul_fp8_swiglu``.
    """
    gs = _gs(group_sizes)
    dev = L.require_device(xq, x_scale, sort_indices, w_q, w_scale, gs)
    si = sort_indices.to(torch.int32).contiguous()
    T, Kin = xq.shape
    E, two_i, Kin2 = w_q.shape
    M = si.numel()
    if Kin2 != Kin or two_i % 2 or top_k < 1:
        raise ValueError("fp8 gathered gmm+swiglu shape mismatch")
    I = two_i // 2
    yq = torch.empty((M, I), dtype=torch.float8_e4m3fn, device=dev)
    ys = torch.empty((M, I // 128), dtype=torch.float32, device=dev)
    yb = torch.empty((M, I), dtype=torch.bfloat16, device=dev) if return_bf16 else None
    ws = L.workspace(L.query("mtx_gmm_workspace_size", M, E), dev)
    L.call(_entry("mtx_gmm_fp8_swiglu_gathered", scales), L.ptr(xq.contiguous()), L.ptr(x_scale.contiguous()), T,
           L.ptr(si), top_k,
           L.ptr(w_q.contiguous()), L.ptr(w_scale.contiguous()), L.ptr(gs), M, Kin, I, E, L.ptr(yq), L.ptr(ys),
           L.ptr(yb), L.ptr(ws), ws.numel(), L.stream(dev))
    if return_bf16:
        return yq, ys, yb
    return yq, ys


# ---- backward: dlhs and tgmm with fp8 operands ----------------------------------------------------
# The bf16 forms are grouped_matmul.py:151-187 (dlhs) and :197-235 (tgmm); the fp8 ones keep the
# forward's conventions (e4m3fn codes, f32 scale = amax / 448 per group, or the power-of-two mode,
# ``scales="pow2"``, whose GEMMs need operands quantised in it).

def quantize_fp8_weights_t(w: torch.Tensor, *, scales: str = "amax"):
    """w [E, Kin, Kout] -> (w_qt [E, Kin, Kout] e4m3fn, w_scale_t [E, Kin/128, Kout/128]): the 128x128
    blocks and codes of ``quantize_fp8_weights`` kept in w's own layout, the operand of
    ``grouped_matmul_fp8_dlhs`` (a load-time transform beside the forward one)."""
    dev = L.require_device(w)
    w = w.contiguous()
    E, Kin, Kout = w.shape
    wq = torch.empty((E, Kin, Kout), dtype=torch.float8_e4m3fn, device=dev)
    ws = torch.empty((E, Kin // 128, Kout // 128), dtype=torch.float32, device=dev)
    L.call(_entry("mtx_quant_fp8_weights_t", scales), L.ptr(w), L.dtype_code(w.dtype), E, Kin, Kout, L.ptr(wq),
           L.ptr(ws), L.stream(dev))
    return wq, ws


def grouped_matmul_fp8_dlhs(gq, g_scale, w_qt, w_scale_t, group_sizes, *, scales: str = "amax") -> torch.Tensor:
    """dX [M, Kin] bf16 = dequant(gq) @ dequant(W[g])^T per group, f32 accumulation: the fp8 dlhs
    (``mtx_gmm_fp8_dlhs``).  gq [M, Kout] / g_scale [M, Kout/128] from ``quantize_fp8_rows`` of the
    upstream gradient; w_qt / w_scale_t from ``quantize_fp8_weights_t``."""
    gs = _gs(group_sizes)
    dev = L.require_device(gq, g_scale, w_qt, w_scale_t, gs)
    M, Kout = gq.shape
    E, Kin, Kout2 = w_qt.shape
    if Kout2 != Kout:
        raise ValueError("fp8 dlhs shape mismatch")
    dx = torch.empty((M, Kin), dtype=torch.bfloat16, device=dev)
    ws = L.workspace(L.query("mtx_gmm_workspace_size", M, E), dev)
    L.call(_entry("mtx_gmm_fp8_dlhs", scales), L.ptr(gq.contiguous()), L.ptr(g_scale.contiguous()),
           L.ptr(w_qt.contiguous()), L.ptr(w_scale_t.contiguous()), L.ptr(gs), M, Kin, Kout, E, L.ptr(dx), L.ptr(ws),
           ws.numel(), L.stream(dev))
    return dx


def quantize_fp8_grouped_t(x: torch.Tensor, group_sizes: torch.Tensor, *, blocks: bool = False,
                           scales: str = "amax"):
    """Operand of ``tgmm_fp8``: x [M, F] (f32/bf16, rows grouped by expert) quantised in chunks of
    128 consecutive rows of each expert (chunk j of expert e = its rows 128j .. 128j+127,
    zero-padded) and transposed per expert into expert-major blocks: flat codes of F*128*C bytes
    (C = ceil(M/128) + E chunk slots; expert e's block [F, 128 n_e] at byte 128*F*cb[e], cb[e] =
    chunks of the experts before it) and flat scales -- one per feature and chunk (expert e's
    [F, n_e] at F*cb[e]) or, with ``blocks``, one per 128x128 block ([F/128, n_e] at
    (F/128)*cb[e])."""
    gs = _gs(group_sizes)
    dev = L.require_device(x, gs)
    x = x.contiguous()
    M, F = x.shape
    E = gs.numel()
    C = L.query("mtx_fp8_grouped_chunks", M, E)
    xt = torch.empty((F * 128 * C,), dtype=torch.float8_e4m3fn, device=dev)
    xs = torch.empty(((F // 128) * C if blocks else F * C,), dtype=torch.float32, device=dev)
    xt._mtx_features = F
    xs._mtx_features = F
    ws = L.workspace(L.query("mtx_fp8_grouped_workspace_size", E), dev)
    L.call(_entry("mtx_quant_fp8_grouped_t", scales), L.ptr(x), L.dtype_code(x.dtype), L.ptr(gs), M, F, E,
           int(bool(blocks)), L.ptr(xt), L.ptr(xs), L.ptr(ws), ws.numel(), L.stream(dev))
    return xt, xs


def tgmm_fp8(xt, xt_scale, gt, gt_scale, group_sizes, M: int, F: int | None = None,
             N: int | None = None, *, scales: str = "amax") -> torch.Tensor:
    """dW [E, F, N] bf16 = per group dequant(x)^T @ dequant(g) with f32 accumulation (``mtx_tgmm_fp8``):
    x from ``quantize_fp8_grouped_t(x, gs)`` (per-feature chunk scales), g from
    ``quantize_fp8_grouped_t(g, gs, blocks=True)``; M = rows of x and g, F / N their columns (taken
    from the quantiser's outputs when omitted).  Empty groups give zeros.  F and N must be multiples
    of 256."""
    gs = _gs(group_sizes)
    dev = L.require_device(xt, xt_scale, gt, gt_scale, gs)
    E = gs.numel()
    F = getattr(xt, "_mtx_features", None) if F is None else F
    N = getattr(gt, "_mtx_features", None) if N is None else N
    if F is None or N is None:
        raise ValueError("tgmm_fp8 needs F and N (the feature counts of x and g)")
    C = L.query("mtx_fp8_grouped_chunks", M, E)
    if xt.numel() != F * 128 * C or gt.numel() != N * 128 * C:
        raise ValueError("tgmm_fp8: operands were not quantised with these M, F, N and group count")
    dw = torch.empty((E, F, N), dtype=torch.bfloat16, device=dev)
    ws = L.workspace(L.query("mtx_fp8_grouped_workspace_size", E), dev)
    L.call(_entry("mtx_tgmm_fp8", scales), L.ptr(xt.contiguous()), L.ptr(xt_scale.contiguous()),
           L.ptr(gt.contiguous()), L.ptr(gt_scale.contiguous()), L.ptr(gs), M, F, N, E, L.ptr(dw), L.ptr(ws),
           ws.numel(), L.stream(dev))
    return dw


# ---- differentiable form: fp8 operands in the forward and in both backward GEMMs -------------------

class _GMMFP8(torch.autograd.Function):
    """Forward: 1x128 row groups of x and 128x128 blocks of W, fp8 grouped GEMM.  Backward: the fp8
    dlhs (1x128 groups of the gradient rows against W's blocks in its own layout) and the fp8 tgmm
    (x and the gradient quantised in 128-row chunks of each expert).  The quantisations follow
    the forward's conventions (e4m3fn codes; scale = amax / 448, or power-of-two scales in every
    quantisation with ``scales="pow2"``), and the backward treats each
    quantise/dequantise pair as the identity (straight-through), as fp8 training recipes do; the
    reference's only fp8 product (the per-tensor matmul of mintext/modules/linear.py:37-57) has no
    grouped form to pin this against."""

    @staticmethod
    def forward(ctx, x, weights, group_sizes, scales):
        gs = _gs(group_sizes)
        f8s = dict(scales=scales)
        xq, xs = quantize_fp8_rows(x, **f8s)
        wq, wsc = quantize_fp8_weights(weights, **f8s)
        out = grouped_matmul_fp8(xq, xs, wq, wsc, gs, **f8s)
        ctx.save_for_backward(x, weights, gs)
        ctx.scales = scales
        return out

    @staticmethod
    def backward(ctx, grad):
        x, w, gs = ctx.saved_tensors
        f8s = dict(scales=ctx.scales)
        grad = grad.contiguous()
        dx = dw = None
        if ctx.needs_input_grad[0]:
            gq, g_s = quantize_fp8_rows(grad, **f8s)
            wqt, wst = quantize_fp8_weights_t(w, **f8s)
            dx = grouped_matmul_fp8_dlhs(gq, g_s, wqt, wst, gs, **f8s).to(x.dtype)
        if ctx.needs_input_grad[1]:
            M = x.shape[0]
            xt, xts = quantize_fp8_grouped_t(x, gs, **f8s)
            gt, gts = quantize_fp8_grouped_t(grad, gs, blocks=True, **f8s)
            dw = tgmm_fp8(xt, xts, gt, gts, gs, M, x.shape[1], grad.shape[1], **f8s).to(w.dtype)
        return dx, dw, None, None


def grouped_matmul_fp8_vjp(x: torch.Tensor, weights: torch.Tensor, group_sizes: torch.Tensor, *,
                           scales: str = "amax") -> torch.Tensor:
    """Blockwise-fp8 counterpart of ``grouped_matmul_vjp`` (grouped_matmul.py:83-190): x [M, Kin]
    and weights [E, Kin, Kout] (bf16 / f32 master values, the reference layout) are quantised on
    each call; the output is bf16 [M, Kout] and differentiable in (x, weights), both backward GEMMs
    on fp8 operands.  Kin and Kout must be multiples of 256 (the tgmm tiles).  ``scales``: "amax"
    (amax / 448) or "pow2" (power-of-two scales, applied by the MFMA) in every quantisation."""
    if x.dim() != 2 or weights.dim() != 3 or weights.shape[1] != x.shape[1]:
        raise ValueError(f"grouped_matmul_fp8_vjp: x {tuple(x.shape)} and weights {tuple(weights.shape)} do not match")
    if x.shape[1] % 256 or weights.shape[2] % 256:
        raise ValueError("grouped_matmul_fp8_vjp needs Kin and Kout multiples of 256")
    if scales not in SCALE_MODES:
        raise ValueError(f"scales must be one of {SCALE_MODES}, got {scales!r}")
    return _GMMFP8.apply(x, weights, group_sizes, scales)

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


def quantize_fp8_rows(x: torch.Tensor):
    """x [M, D] (f32/bf16) -> (xq [M, D] float8_e4m3fn, x_scale [M, D/128] f32)."""
    dev = L.require_device(x)
    x = x.contiguous()
    M, D = x.shape
    xq = torch.empty((M, D), dtype=torch.float8_e4m3fn, device=dev)
    xs = torch.empty((M, D // 128), dtype=torch.float32, device=dev)
    L.call("mtx_quant_fp8_rows", L.ptr(x), L.dtype_code(x.dtype), M, D, L.ptr(xq), L.ptr(xs), L.stream(dev))
    return xq, xs


def quantize_fp8_weights(w: torch.Tensor):
    """w [E, Kin, Kout] (reference layout) -> (w_q [E, Kout, Kin] e4m3fn, w_scale [E, Kout/128, Kin/128])."""
    dev = L.require_device(w)
    w = w.contiguous()
    E, Kin, Kout = w.shape
    wq = torch.empty((E, Kout, Kin), dtype=torch.float8_e4m3fn, device=dev)
    ws = torch.empty((E, Kout // 128, Kin // 128), dtype=torch.float32, device=dev)
    L.call("mtx_quant_fp8_weights", L.ptr(w), L.dtype_code(w.dtype), E, Kin, Kout, L.ptr(wq), L.ptr(ws),
           L.stream(dev))
    return wq, ws


def grouped_matmul_fp8(xq, x_scale, w_q, w_scale, group_sizes) -> torch.Tensor:
    """out [M, Kout] bf16 = blockwise-dequantised x @ W per group, f32 accumulation."""
    gs = _gs(group_sizes)
    dev = L.require_device(xq, x_scale, w_q, w_scale, gs)
    M, Kin = xq.shape
    E, Kout, Kin2 = w_q.shape
    if Kin2 != Kin:
        raise ValueError("fp8 gmm shape mismatch")
    out = torch.empty((M, Kout), dtype=torch.bfloat16, device=dev)
    ws = L.workspace(L.query("mtx_gmm_workspace_size", M, E), dev)
    L.call("mtx_gmm_fp8", L.ptr(xq.contiguous()), L.ptr(x_scale.contiguous()), L.ptr(w_q.contiguous()),
           L.ptr(w_scale.contiguous()), L.ptr(gs), M, Kin, Kout, E, L.ptr(out), L.ptr(ws), ws.numel(),
           L.stream(dev))
    return out


def grouped_matmul_fp8_swiglu(xq, x_scale, w_q, w_scale, group_sizes, *, return_bf16: bool = False):
    """SwiGLU of the fp8 gate_up GEMM (w_q [E, 2I, Kin]) re-quantised in 1x128 groups.

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
    L.call("mtx_gmm_fp8_swiglu", L.ptr(xq.contiguous()), L.ptr(x_scale.contiguous()), L.ptr(w_q.contiguous()),
           L.ptr(w_scale.contiguous()), L.ptr(gs), M, Kin, I, E, L.ptr(yq), L.ptr(ys), L.ptr(yb), L.ptr(ws),
           ws.numel(), L.stream(dev))
    if return_bf16:
        return yq, ys, yb
    return yq, ys


def grouped_matmul_fp8_swiglu_gathered(xq, x_scale, sort_indices, top_k: int, w_q, w_scale, group_sizes, *,
                                       return_bf16: bool = False):
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
    L.call("mtx_gmm_fp8_swiglu_gathered", L.ptr(xq.contiguous()), L.ptr(x_scale.contiguous()), T, L.ptr(si), top_k,
           L.ptr(w_q.contiguous()), L.ptr(w_scale.contiguous()), L.ptr(gs), M, Kin, I, E, L.ptr(yq), L.ptr(ys),
           L.ptr(yb), L.ptr(ws), ws.numel(), L.stream(dev))
    if return_bf16:
        return yq, ys, yb
    return yq, ys

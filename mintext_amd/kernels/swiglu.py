"""Differentiable SwiGLU ``silu(h[:, :I]) * h[:, I:]`` (mintext/modules/moe.py:195-196).

Forward ``mtx_swiglu``, backward ``mtx_swiglu_bwd`` (both HIP kernels).  The fused
gate_up GEMM + SwiGLU (``grouped_matmul_swiglu``) is used instead when no gradient is needed.
"""
from __future__ import annotations

import torch

from .. import _lib as L
from .grouped_matmul import swiglu


class _SwiGLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, h):
        out = swiglu(h)
        ctx.save_for_backward(h)
        return out

    @staticmethod
    def backward(ctx, dy):
        (h,) = ctx.saved_tensors
        dev = L.require_device(h, dy)
        h = h.contiguous()
        dy = dy.contiguous().to(h.dtype)
        M, two_i = h.shape
        dh = torch.empty_like(h)
        L.call("mtx_swiglu_bwd", L.ptr(h), L.ptr(dy), L.dtype_code(h.dtype), M, two_i // 2, L.ptr(dh),
               L.stream(dev))
        return dh


def swiglu_autograd(h: torch.Tensor) -> torch.Tensor:
    return _SwiGLU.apply(h)

"""MI355X (gfx950) implementation of the bzantium/mintext MoE hot path.

Router top-k, expert-sorted dispatch, ragged grouped GEMM (bf16 / fp32 / blockwise fp8,
fused SwiGLU, dlhs and tgmm backward) and the weighted combine, as hand-written HIP kernels
behind the C-ABI of include/mintext_moe.h.  ``mintext_amd.kernels`` mirrors the reference's
``mintext.kernels`` package; ``mintext_amd.moe`` composes the expert layer.
"""
from . import _lib
from .kernels import (grouped_matmul, grouped_matmul_swiglu, grouped_matmul_vjp, route, route_topk, tgmm,
                      unroute)

__all__ = ["route", "unroute", "grouped_matmul", "grouped_matmul_vjp", "tgmm", "route_topk",
           "grouped_matmul_swiglu", "_lib"]

"""MoE kernels: token routing and grouped matmul (mirror of mintext/kernels/__init__.py:3-6).

The reference exports route, unroute, grouped_matmul, grouped_matmul_vjp and tgmm; this
package adds route_topk (router top-k), grouped_matmul_swiglu (fused gate_up + SwiGLU),
swiglu and the blockwise-fp8 entry points in ``fp8``.
"""
from .grouped_matmul import grouped_matmul, grouped_matmul_swiglu, grouped_matmul_vjp, swiglu, tgmm
from .moe_dispatch import _sort_with_vjp, route, unroute
from .router import route_topk, update_expert_bias

__all__ = ["route", "unroute", "grouped_matmul", "grouped_matmul_vjp", "tgmm", "route_topk",
           "grouped_matmul_swiglu", "swiglu", "_sort_with_vjp", "update_expert_bias"]

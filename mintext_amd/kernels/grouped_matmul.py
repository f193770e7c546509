"""Grouped matrix multiplication x[group_i] @ weights[i] per expert, on gfx950.

Drop-in for bzantium/mintext ``mintext/kernels/grouped_matmul.py`` (same names, arguments,
output dtypes and differentiability):

* ``grouped_matmul(x, weights, group_sizes, *, tiling=None)`` (grouped_matmul.py:58-76)
* ``grouped_matmul_vjp(x, weights, group_sizes, *, tiling=(128,)*9, mosaic_fusion=True)``
  (:83-114) -- forward gmm, backward dlhs = g @ W^T and drhs = tgmm(x, g) (:151-187)
* ``tgmm(lhs, rhs, group_sizes)`` (:197-235) -- per-group x^T @ g, zeros for empty groups

``tiling`` selects the HIP tile configuration (the reference passes TPU ``ragged_dot`` tilings
to XLA): a 3-tuple ``(tm, tg, tn)`` per GEMM with ``tn == 256`` (the MFMA kernels' n-tile
width) -- ``tm`` rows per m-tile (128 or 256; other values round to the nearer), ``tg`` m-tiles
per XCD scheduling group (1..64).  ``None`` and any tuple with another ``tn`` (the reference's
TPU tilings, such as its default (128, 128, 128)) keep the shape heuristics.  The
9-tuple of ``grouped_matmul_vjp`` is padded from 3 like the reference (fwd, dlhs, tgmm; the
tgmm entry is not used).  Every tile configuration computes the same f32 sums; the results are
bit-identical unless the split tail splits different tiles, and then agree to a bf16 rounding
(``mtx_gmm_workspace_size``).  ``mosaic_fusion``
is accepted and ignored.  ``group_sizes`` never leaves the device.  Extra entry points beyond the reference: ``grouped_matmul_swiglu``
(gate_up GEMM with the SwiGLU of moe.py:195-196 fused into the epilogue) and ``swiglu``.
"""
from __future__ import annotations

import torch

from .. import _lib as L


def _gs(group_sizes: torch.Tensor) -> torch.Tensor:
    g = group_sizes if group_sizes.dtype == torch.int32 else group_sizes.to(torch.int32)
    return g.contiguous()


def _check_float(*ts):
    for t in ts:
        if t.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError(f"grouped GEMM takes float32 or bfloat16 operands, got {t.dtype}")
    if len({t.dtype for t in ts}) != 1:
        raise TypeError("grouped GEMM operands must share one dtype")


HIP_TN = 256  # n-tile width of the MFMA kernels; a tiling with another tn is a TPU hint


def _tile_args(tiling) -> tuple[int, int]:
    """(tile_m, tile_group) for the C-ABI from a (tm, tg, tn) tiling; (0, 0) = heuristics.

    Only tilings with tn == 256 (those of ``kernels.autotuner``) select a HIP configuration.
    Any other tuple is a TPU ``ragged_dot`` tiling -- e.g. the (128, 128, 128) that the
    reference passes when no tiling is configured (mintext/modules/moe.py:180-186) -- and
    leaves the shape heuristics in charge.
    """
    if tiling is None:
        return 0, 0
    t = tuple(int(v) for v in tiling)
    if len(t) < 3 or any(v <= 0 for v in t):
        raise ValueError(f"tiling must hold positive ints (tm, tg, tn), got {tiling!r}")
    if t[2] != HIP_TN:
        return 0, 0
    tm = 128 if t[0] <= 128 else 256
    tg = min(max(t[1], 1), 64)
    return tm, tg


def _gmm_fwd(x: torch.Tensor, w: torch.Tensor, gs: torch.Tensor, tiling=None) -> torch.Tensor:
    dev = L.require_device(x, w, gs)
    _check_float(x, w)
    x = x.contiguous()
    w = w.contiguous()
    M, Kin = x.shape
    E, Kin2, Kout = w.shape
    if Kin2 != Kin or gs.numel() != E:
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, weights {tuple(w.shape)}, group_sizes {gs.numel()}")
    out = torch.empty((M, Kout), dtype=x.dtype, device=dev)
    ws = L.workspace(L.query("mtx_gmm_workspace_size", M, E), dev)
    tm, tg = _tile_args(tiling)
    L.call("mtx_gmm_tiled", L.MTX_GMM_OP_FWD, L.ptr(x), L.ptr(w), L.ptr(gs), L.dtype_code(x.dtype), M, Kin, Kout,
           E, tm, tg, L.ptr(out), L.ptr(ws), ws.numel(), L.stream(dev))
    return out


def _gmm_dlhs(g: torch.Tensor, w: torch.Tensor, gs: torch.Tensor, tiling=None) -> torch.Tensor:
    dev = L.require_device(g, w, gs)
    g = g.contiguous()
    w = w.contiguous()
    if g.dtype != w.dtype:
        g = g.to(w.dtype)
    M, Kout = g.shape
    E, Kin, Kout2 = w.shape
    if Kout2 != Kout:
        raise ValueError("dlhs shape mismatch")
    dx = torch.empty((M, Kin), dtype=w.dtype, device=dev)
    ws = L.workspace(L.query("mtx_gmm_workspace_size", M, E), dev)
    tm, tg = _tile_args(tiling)
    L.call("mtx_gmm_tiled", L.MTX_GMM_OP_DLHS, L.ptr(g), L.ptr(w), L.ptr(gs), L.dtype_code(w.dtype), M, Kin, Kout,
           E, tm, tg, L.ptr(dx), L.ptr(ws), ws.numel(), L.stream(dev))
    return dx


def tgmm(lhs: torch.Tensor, rhs: torch.Tensor, group_sizes: torch.Tensor) -> torch.Tensor:
    """Transposed grouped matmul: out[i] = lhs[group_i]^T @ rhs[group_i] (grouped_matmul.py:197-235).

    Args:
        lhs: [M, K] (activations of the forward pass).
        rhs: [M, N] (upstream gradient).
        group_sizes: [E] int32.

    Returns:
        [E, K, N] per-expert weight gradients in the operand dtype; empty groups give zeros.
    """
    gs = _gs(group_sizes)
    dev = L.require_device(lhs, rhs, gs)
    _check_float(lhs, rhs)
    lhs = lhs.contiguous()
    rhs = rhs.contiguous()
    M, K = lhs.shape
    M2, N = rhs.shape
    if M2 != M:
        raise ValueError("tgmm: lhs and rhs need the same number of rows")
    E = gs.numel()
    out = torch.empty((E, K, N), dtype=lhs.dtype, device=dev)
    ws = L.workspace(L.query("mtx_gmm_workspace_size", M, E), dev)
    L.call("mtx_tgmm", L.ptr(lhs), L.ptr(rhs), L.ptr(gs), L.dtype_code(lhs.dtype), M, K, N, E, L.ptr(out),
           L.ptr(ws), ws.numel(), L.stream(dev))
    return out


class _GMM(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weights, group_sizes, tiling9):
        gs = _gs(group_sizes)
        out = _gmm_fwd(x, weights, gs, None if tiling9 is None else tiling9[0:3])
        ctx.save_for_backward(x, weights, gs)
        ctx.tiling9 = tiling9
        return out

    @staticmethod
    def backward(ctx, grad):
        x, w, gs = ctx.saved_tensors
        grad = grad.contiguous().to(w.dtype)
        t9 = ctx.tiling9
        dx = _gmm_dlhs(grad, w, gs, None if t9 is None else t9[3:6]) if ctx.needs_input_grad[0] else None
        dw = tgmm(x, grad, gs) if ctx.needs_input_grad[1] else None
        return dx, dw, None, None


def _pad_tiling(tiling) -> tuple:
    t = tuple(tiling)
    if len(t) < 9:
        base = t[:3] if len(t) >= 3 else (128, 128, 128)
        t = (base * 3)[:9]
    return t


def grouped_matmul(x: torch.Tensor, weights: torch.Tensor, group_sizes: torch.Tensor, *,
                   tiling=None) -> torch.Tensor:
    """Grouped matrix multiplication: x[group_i] @ weights[i] (grouped_matmul.py:58-76).

    Args:
        x: [M, K_in] sorted tokens (contiguous per expert).
        weights: [E, K_in, K_out].
        group_sizes: [E] int32, tokens per expert (rows past the sum are zero in the output).
        tiling: (tm, tg, tn) HIP tile configuration or None (shape heuristics); does not
            change results.

    Returns:
        [M, K_out] in x's dtype.
    """
    return _GMM.apply(x, weights, group_sizes, None if tiling is None else _pad_tiling(tiling))


def grouped_matmul_vjp(x: torch.Tensor, weights: torch.Tensor, group_sizes: torch.Tensor, *,
                       tiling=(128, 128, 128, 128, 128, 128, 128, 128, 128),
                       mosaic_fusion: bool = True) -> torch.Tensor:
    """Grouped matmul with the custom backward (grouped_matmul.py:83-114, 151-187).

    Forward: gmm.  Backward: dlhs = grad @ W^T per group, drhs = tgmm(x, grad).
    ``tiling`` (3 or 9 ints, padded like grouped_matmul.py:108-112): entries 0-2 configure the
    forward GEMM and 3-5 the dlhs GEMM as ``(tm, tg, tn)``; ``None`` keeps the heuristics.
    ``mosaic_fusion`` is accepted and ignored.
    """
    del mosaic_fusion
    return _GMM.apply(x, weights, group_sizes, None if tiling is None else _pad_tiling(tiling))


def grouped_matmul_swiglu(x: torch.Tensor, weights: torch.Tensor, group_sizes: torch.Tensor, *,
                          tiling=None) -> torch.Tensor:
    """silu(h[:, :I]) * h[:, I:] with h = grouped_matmul(x, weights) -- fused, h never stored.

    weights: [E, K_in, 2I] with the gate columns first (the fused gate_up layout of
    mintext/modules/moe.py:125-132).  Returns [M, I] in x's dtype.  Forward only.  ``tiling``:
    (tm, tg, tn) as for ``grouped_matmul``.
    """
    gs = _gs(group_sizes)
    dev = L.require_device(x, weights, gs)
    _check_float(x, weights)
    x = x.contiguous()
    w = weights.contiguous()
    M, Kin = x.shape
    E, Kin2, two_i = w.shape
    if Kin2 != Kin or two_i % 2 or gs.numel() != E:
        raise ValueError("grouped_matmul_swiglu shape mismatch")
    I = two_i // 2
    out = torch.empty((M, I), dtype=x.dtype, device=dev)
    ws = L.workspace(L.query("mtx_gmm_workspace_size", M, E), dev)
    tm, tg = _tile_args(tiling)
    L.call("mtx_gmm_tiled", L.MTX_GMM_OP_SWIGLU, L.ptr(x), L.ptr(w), L.ptr(gs), L.dtype_code(x.dtype), M, Kin, I,
           E, tm, tg, L.ptr(out), L.ptr(ws), ws.numel(), L.stream(dev))
    return out


def gathered_swiglu_supported(tokens: torch.Tensor, weights: torch.Tensor) -> bool:
    """Whether ``grouped_matmul_swiglu_gathered`` takes these operands: bf16, K_in a multiple of
    64, I a multiple of 128, 16-byte aligned, 32-bit operand offsets (the direct-to-LDS kernels)."""
    if tokens.dtype != torch.bfloat16 or weights.dtype != torch.bfloat16 or tokens.dim() != 2 or weights.dim() != 3:
        return False
    T, Kin = tokens.shape
    two_i = weights.shape[2]
    return (Kin > 0 and Kin % 64 == 0 and two_i % 256 == 0 and T * Kin * 2 < 2 ** 32 and Kin * two_i * 2 < 2 ** 32
            and tokens.is_contiguous() and weights.is_contiguous()
            and tokens.data_ptr() % 16 == 0 and weights.data_ptr() % 16 == 0)


def grouped_matmul_swiglu_gathered(tokens: torch.Tensor, sort_indices: torch.Tensor, top_k: int,
                                   weights: torch.Tensor, group_sizes: torch.Tensor, *, tiling=None) -> torch.Tensor:
    """``grouped_matmul_swiglu(route(tokens, ...)[0], weights, group_sizes)`` with the route's row
    gather done by the GEMM's operand loads: sorted row r is ``tokens[sort_indices[r] // top_k]``
    (moe_dispatch.py:67,76), read straight from the token-order tensor, so the sorted copy is
    never written.  Same bits as the two steps (with the same ``tiling``, as for
    ``grouped_matmul_swiglu``).  bf16 only; shapes outside the direct-to-LDS kernels (K_in % 64,
    I % 128) raise MtxError with status MTX_ERR_UNSUPPORTED.  Forward only.
    """
    gs = _gs(group_sizes)
    dev = L.require_device(tokens, sort_indices, weights, gs)
    _check_float(tokens, weights)
    x = tokens.contiguous()
    w = weights.contiguous()
    si = sort_indices.to(torch.int32).contiguous()
    T, Kin = x.shape
    E, Kin2, two_i = w.shape
    M = si.numel()
    if Kin2 != Kin or two_i % 2 or gs.numel() != E or top_k < 1:
        raise ValueError("grouped_matmul_swiglu_gathered shape mismatch")
    I = two_i // 2
    out = torch.empty((M, I), dtype=x.dtype, device=dev)
    ws = L.workspace(L.query("mtx_gmm_workspace_size", M, E), dev)
    tm, tg = _tile_args(tiling)
    L.call("mtx_gmm_gathered", L.MTX_GMM_OP_SWIGLU, L.ptr(x), T, L.ptr(si), top_k, L.ptr(w), L.ptr(gs),
           L.dtype_code(x.dtype), M, Kin, I, E, tm, tg, L.ptr(out), L.ptr(ws), ws.numel(), L.stream(dev))
    return out


def swiglu(h: torch.Tensor) -> torch.Tensor:
    """silu(h[:, :I]) * h[:, I:] (mintext/modules/moe.py:195-196) as one HIP kernel."""
    dev = L.require_device(h)
    _check_float(h)
    h = h.contiguous()
    M, two_i = h.shape
    I = two_i // 2
    out = torch.empty((M, I), dtype=h.dtype, device=dev)
    L.call("mtx_swiglu", L.ptr(h), L.dtype_code(h.dtype), M, I, L.ptr(out), L.stream(dev))
    return out

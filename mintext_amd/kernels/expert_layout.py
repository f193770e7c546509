"""Expert weight layouts: HF per-expert <-> fused, on the device (one HIP kernel,
``mtx_transpose_batched``).

Mirror of bzantium/mintext ``mintext/checkpoint/conversion.py``:

* ``experts_from_hf(gate, up, down)`` -- ``_import_expert_weights`` (conversion.py:80-133): HF's
  per-expert ``gate_proj.weight`` / ``up_proj.weight`` [I, D] and ``down_proj.weight`` [D, I],
  stacked over experts, become the fused ``gate_up_proj`` [E, D, 2I] (gate columns first) and
  ``down_proj`` [E, I, D] that the grouped GEMMs read;
* ``experts_from_hf_fused(gate_up_proj, down_proj)`` -- the fused-HF fallback of the same
  function (conversion.py:107-116): [E, 2I, D] / [E, D, I] transposed;
* ``experts_to_hf(gate_up, down)`` -- ``_export_expert_weights`` (conversion.py:136-166).

All three are pure data movement (bit-exact), HBM-bound: each element is read once and written
once.  Inputs and outputs are device tensors (float32 or bfloat16).
"""
from __future__ import annotations

import torch

from .. import _lib as L


def _transpose_into(src: torch.Tensor, dst: torch.Tensor, B: int, R: int, C: int, in_bs: int, in_ld: int,
                    out_bs: int, out_ld: int, src_off: int = 0, dst_off: int = 0) -> None:
    dev = L.require_device(src, dst)
    if src.dtype != dst.dtype or src.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"expert weights must be float32 or bfloat16 on both sides, got {src.dtype} -> {dst.dtype}")
    es = src.element_size()
    L.call("mtx_transpose_batched", src.data_ptr() + src_off * es, L.dtype_code(src.dtype), B, R, C, in_bs, in_ld,
           dst.data_ptr() + dst_off * es, out_bs, out_ld, L.stream(dev))


def experts_from_hf(gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """HF per-expert weights stacked over experts -> fused layout.

    Args:
        gate, up: [E, I, D] (``experts.{e}.gate_proj.weight`` / ``up_proj.weight``).
        down: [E, D, I] (``experts.{e}.down_proj.weight``).

    Returns:
        (gate_up [E, D, 2I] with gate columns first, down [E, I, D]).
    """
    gate, up, down = gate.contiguous(), up.contiguous(), down.contiguous()
    E, I, D = gate.shape
    if up.shape != (E, I, D) or down.shape != (E, D, I):
        raise ValueError(f"HF expert shapes gate {tuple(gate.shape)}, up {tuple(up.shape)}, down {tuple(down.shape)}")
    gate_up = torch.empty((E, D, 2 * I), dtype=gate.dtype, device=gate.device)
    dn = torch.empty((E, I, D), dtype=down.dtype, device=down.device)
    _transpose_into(gate, gate_up, E, I, D, I * D, D, D * 2 * I, 2 * I)
    _transpose_into(up, gate_up, E, I, D, I * D, D, D * 2 * I, 2 * I, dst_off=I)
    _transpose_into(down, dn, E, D, I, D * I, I, I * D, D)
    return gate_up, dn


def experts_from_hf_fused(gate_up_proj: torch.Tensor, down_proj: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """HF fused experts ``gate_up_proj`` [E, 2I, D], ``down_proj`` [E, D, I] -> [E, D, 2I], [E, I, D]."""
    gu, dp = gate_up_proj.contiguous(), down_proj.contiguous()
    E, two_i, D = gu.shape
    if dp.shape != (E, D, two_i // 2):
        raise ValueError(f"HF fused expert shapes {tuple(gu.shape)} / {tuple(dp.shape)}")
    I = two_i // 2
    out_gu = torch.empty((E, D, two_i), dtype=gu.dtype, device=gu.device)
    out_dn = torch.empty((E, I, D), dtype=dp.dtype, device=dp.device)
    _transpose_into(gu, out_gu, E, two_i, D, two_i * D, D, D * two_i, two_i)
    _transpose_into(dp, out_dn, E, D, I, D * I, I, I * D, D)
    return out_gu, out_dn


def experts_to_hf(gate_up: torch.Tensor, down: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fused layout -> HF per-expert weights stacked over experts: (gate [E,I,D], up [E,I,D], down [E,D,I])."""
    gu, dn = gate_up.contiguous(), down.contiguous()
    E, D, two_i = gu.shape
    I = two_i // 2
    if dn.shape != (E, I, D):
        raise ValueError(f"fused expert shapes {tuple(gu.shape)} / {tuple(dn.shape)}")
    gate = torch.empty((E, I, D), dtype=gu.dtype, device=gu.device)
    up = torch.empty((E, I, D), dtype=gu.dtype, device=gu.device)
    down_hf = torch.empty((E, D, I), dtype=dn.dtype, device=dn.device)
    _transpose_into(gu, gate, E, D, I, D * two_i, two_i, I * D, D)
    _transpose_into(gu, up, E, D, I, D * two_i, two_i, I * D, D, src_off=I)
    _transpose_into(dn, down_hf, E, I, D, I * D, D, D * I, I)
    return gate, up, down_hf

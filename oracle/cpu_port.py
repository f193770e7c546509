"""CPU restatement of the reference MoE layer forward in the reference's own arithmetic --
MEASUREMENT INFRASTRUCTURE ONLY.

Used by nothing but the ``cpu_baseline`` leg of ``bench.py`` (the float64 checker is
``oracle/moe_oracle.py``).  It runs the steps of bzantium/mintext's layer with torch on the host
CPU, in the compute dtype the reference uses (bf16 operands, f32 routing and combine):

* router: softmax over f32 logits + top-k + renormalisation (HF mixtral/modeling_mixtral.py:104-111,
  qwen3_moe:258-267), or sigmoid + bias + group-limited top-k (mintext/modules/moe.py:52-103);
* ``route``: stable argsort of the flattened indices, row gather of the K-fold repeat, bincount
  (mintext/kernels/moe_dispatch.py:47-81);
* ``ragged_dot`` per expert group (mintext/kernels/grouped_matmul.py:242-277), SwiGLU
  (mintext/modules/moe.py:195-196), ``ragged_dot`` of the down projection;
* ``unroute``: argsort of the permutation, gather, f32 einsum combine (moe_dispatch.py:84-111);
* shared expert as a dense SwiGLU MLP added to the routed output (moe.py:256-258).

JAX is not installed here or on the GPU host, so this torch restatement stands in for the JAX-CPU
one; it is timed, never checked against (the GPU path is checked against the float64 oracle).
"""
from __future__ import annotations

import torch


def router(logits: torch.Tensor, k: int, scoring: str, bias=None, n_group: int = 1, topk_group: int = 1,
           norm_topk_prob: bool = True, routed_scaling_factor: float = 1.0):
    lg = logits.float()
    if scoring == "softmax":
        p = torch.softmax(lg, dim=-1)
        w, idx = torch.topk(p, k, dim=-1)
        if norm_topk_prob:
            w = w / w.sum(-1, keepdim=True)
    else:
        s = torch.sigmoid(lg)                                        # moe.py:53
        r = s if bias is None else s + bias                          # moe.py:56
        T, E = r.shape
        if n_group > 1 and topk_group < n_group:
            g = r.reshape(T, n_group, E // n_group).topk(min(2, E // n_group), dim=-1)[0].sum(-1)  # :76-80
            gi = g.topk(topk_group, dim=-1)[1]                                                     # :83
            gm = torch.zeros(T, n_group, dtype=torch.bool).scatter_(1, gi, True)                   # :86-89
            r = r.masked_fill(~gm.repeat_interleave(E // n_group, dim=1), float("-inf"))           # :92-95
        idx = r.topk(k, dim=-1)[1]                                   # :98
        w = s.gather(1, idx)                                         # :101
        if norm_topk_prob:
            w = w / (w.sum(-1, keepdim=True) + 1e-20)                # :63-64
    return idx.to(torch.int32), w * routed_scaling_factor


def route(x: torch.Tensor, idx: torch.Tensor, E: int):
    K = idx.shape[1]
    flat = idx.reshape(-1).long()
    perm = torch.argsort(flat, stable=True)                          # moe_dispatch.py:73
    sorted_x = x[perm // K]                                          # :67, :76
    gs = torch.bincount(flat, minlength=E)                           # :79
    return sorted_x, perm, gs


def ragged_dot(x: torch.Tensor, w: torch.Tensor, gs: torch.Tensor) -> torch.Tensor:
    out = torch.zeros(x.shape[0], w.shape[2], dtype=x.dtype)
    off = 0
    for e, n in enumerate(gs.tolist()):
        if n:
            out[off:off + n] = x[off:off + n] @ w[e]
        off += n
    return out


def unroute(y: torch.Tensor, perm: torch.Tensor, w: torch.Tensor, K: int) -> torch.Tensor:
    inv = torch.argsort(perm)                                        # moe_dispatch.py:102
    u = y[inv].reshape(w.shape[0], K, -1)                            # :103-108
    return torch.einsum("nkd,nk->nd", u.float(), w.float())          # :111


def moe_layer(x, logits, gate_up, down, k: int, scoring: str, shared=None, **router_kw) -> torch.Tensor:
    """One layer forward from the gate logits (the bench's path), in x's dtype."""
    E = gate_up.shape[0]
    idx, w = router(logits, k, scoring, **router_kw)
    sx, perm, gs = route(x, idx, E)
    h = ragged_dot(sx, gate_up, gs)
    i = h.shape[1] // 2
    inter = torch.nn.functional.silu(h[:, :i]) * h[:, i:]            # moe.py:195-196
    out = unroute(ragged_dot(inter, down, gs), perm, w, k)
    if shared is not None:
        sh = x @ shared[0]
        out = out + (torch.nn.functional.silu(sh[:, :sh.shape[1] // 2]) * sh[:, sh.shape[1] // 2:]) @ shared[1]
    return out

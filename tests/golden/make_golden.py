"""Write the golden fixtures in tests/golden/*.npz from implementations independent of the
oracle (run on CPU: ``python tests/golden/make_golden.py``).

Sources of truth used here, none of them the oracle or the product:
  * routers: HF transformers 5.15 MixtralTopKRouter / Qwen3MoeTopKRouter (softmax top-k,
    renormalised) and DeepseekV3TopkRouter (sigmoid + bias, group-limited), constructed
    locally with an identity gate so that their logits are the given ones.  The DeepSeek
    router returns its top-k unsorted; the fixture stores the set ordered by descending
    biased score, ties to the lower index -- the order of lax.top_k in the reference
    (mintext/modules/moe.py:98).
  * dispatch: torch.sort(stable=True) and torch.bincount (jnp.argsort(stable=True) /
    jnp.bincount semantics of mintext/kernels/moe_dispatch.py:73,79).
  * grouped GEMMs: per-group torch float64 matmuls (the reference tests' loop references,
    tests/test_moe_kernels.py:162-273,429-479).
  * expert layer: HF MixtralExperts (float64) with the fused [E,D,2I] weights transposed to
    HF's [E,2I,D] layout (the export of mintext/checkpoint/conversion.py:137-166).
  * fp8: torch's float8_e4m3fn cast.
Inputs are regenerated from numpy PCG64 seeds where large; only expected outputs and small
inputs are stored.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent


def _rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------------------------- routers
def _hf_softmax_router(logits: np.ndarray, k: int, norm: bool):
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeTopKRouter

    T, E = logits.shape
    cfg = Qwen3MoeConfig(hidden_size=E, num_experts=E, num_experts_per_tok=k, norm_topk_prob=norm)
    r = Qwen3MoeTopKRouter(cfg)
    with torch.no_grad():
        r.weight.copy_(torch.eye(E))
        _, w, idx = r(torch.from_numpy(logits.astype(np.float32)))
    return idx.numpy().astype(np.int32), w.float().numpy()


def _hf_mixtral_router(logits: np.ndarray, k: int):
    from transformers import MixtralConfig
    from transformers.models.mixtral.modeling_mixtral import MixtralTopKRouter

    T, E = logits.shape
    cfg = MixtralConfig(hidden_size=E, num_local_experts=E, num_experts_per_tok=k)
    r = MixtralTopKRouter(cfg)
    with torch.no_grad():
        r.weight.copy_(torch.eye(E))
        _, w, idx = r(torch.from_numpy(logits.astype(np.float32)))
    return idx.numpy().astype(np.int32), w.float().numpy()


def _hf_deepseek_router(logits, bias, k, n_group, topk_group, norm, scale):
    from transformers import DeepseekV3Config
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3TopkRouter

    T, E = logits.shape
    cfg = DeepseekV3Config(hidden_size=E, n_routed_experts=E, num_experts_per_tok=k, n_group=n_group,
                           topk_group=topk_group, norm_topk_prob=norm, routed_scaling_factor=scale)
    r = DeepseekV3TopkRouter(cfg)
    with torch.no_grad():
        r.weight.copy_(torch.eye(E))
        r.e_score_correction_bias.copy_(torch.from_numpy(bias.astype(np.float32)))
        x = torch.from_numpy(logits.astype(np.float32))
        _, w, idx = r(x)
        scores = x.sigmoid()
    biased = (scores + torch.from_numpy(bias.astype(np.float32))).numpy()
    idx = idx.numpy()
    w = w.numpy()
    # order the unsorted HF top-k like lax.top_k: descending biased score, ties -> lower id
    out_i = np.empty_like(idx)
    out_w = np.empty_like(w)
    for t in range(T):
        order = sorted(range(k), key=lambda j: (-float(biased[t, idx[t, j]]), int(idx[t, j])))
        out_i[t] = idx[t, order]
        out_w[t] = w[t, order]
    return out_i.astype(np.int32), out_w, scores.numpy()


def make_routers():
    # Mixtral-like: E=8, k=2 (C1/C2 routing)
    lg = (_rng(101).standard_normal((96, 8)) * 1.3).astype(np.float32)
    mi, mw = _hf_mixtral_router(lg, 2)
    # Qwen3-like: E=128, k=8 (C4/C5 routing)
    lq = (_rng(102).standard_normal((48, 128)) * 0.9).astype(np.float32)
    qi, qw = _hf_softmax_router(lq, 8, True)
    qi_nn, qw_nn = _hf_softmax_router(lq, 8, False)
    # DeepSeek-V3-like: E=64 (8 groups of 8), top-4 groups, k=8, bias, scale 2.5
    ld = (_rng(103).standard_normal((48, 64)) * 1.5).astype(np.float32)
    bd = (_rng(104).standard_normal(64) * 1e-3).astype(np.float32)
    di, dw, ds = _hf_deepseek_router(ld, bd, 8, 8, 4, True, 2.5)
    # DeepSeek-V3 full width: E=256, 8 groups, top-4 groups, k=8
    l3 = (_rng(105).standard_normal((16, 256)) * 1.0).astype(np.float32)
    b3 = (_rng(106).standard_normal(256) * 1e-3).astype(np.float32)
    d3i, d3w, d3s = _hf_deepseek_router(l3, b3, 8, 8, 4, True, 2.5)
    np.savez_compressed(OUT / "routers.npz",
                        mixtral_logits=lg, mixtral_idx=mi, mixtral_w=mw,
                        qwen_logits=lq, qwen_idx=qi, qwen_w=qw, qwen_idx_nonorm=qi_nn, qwen_w_nonorm=qw_nn,
                        ds_logits=ld, ds_bias=bd, ds_idx=di, ds_w=dw, ds_scores=ds,
                        ds3_logits=l3, ds3_bias=b3, ds3_idx=d3i, ds3_w=d3w, ds3_scores=d3s)


def _router_grad(router, logits: np.ndarray, G: np.ndarray):
    """d/d logits of sum_k w[t,k] * G[t, idx[t,k]] through an HF router with an identity gate
    (torch autograd of HF's own forward, which runs in float32)."""
    x = torch.from_numpy(logits.astype(np.float32)).requires_grad_(True)
    _, w, idx = router(x)
    loss = (w.float() * torch.from_numpy(G).gather(1, idx.long())).sum()
    loss.backward()
    return idx.detach().numpy().astype(np.int32), x.grad.numpy().astype(np.float32)


def make_router_grads():
    """Router VJP fixtures: HF routers (softmax norm / no-norm, DeepSeek sigmoid + group-limited,
    norm / no-norm) differentiated by torch autograd, plus the scores' VJPs from torch.sigmoid /
    torch.softmax autograd (the reference differentiates jax.nn.sigmoid at moe.py:53)."""
    from transformers import DeepseekV3Config, MixtralConfig, Qwen3MoeConfig
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3TopkRouter
    from transformers.models.mixtral.modeling_mixtral import MixtralTopKRouter
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeTopKRouter

    arrays = {}

    def eye_(r, E):
        with torch.no_grad():
            r.weight.copy_(torch.eye(E))
        return r

    # Mixtral: E=8, k=2 (always renormalised)
    lg = (_rng(111).standard_normal((64, 8)) * 1.3).astype(np.float32)
    G = _rng(112).standard_normal((64, 8)).astype(np.float32)
    r = eye_(MixtralTopKRouter(MixtralConfig(hidden_size=8, num_local_experts=8, num_experts_per_tok=2)), 8)
    arrays["mixtral__idx"], arrays["mixtral__dl"] = _router_grad(r, lg, G)
    arrays["mixtral__logits"], arrays["mixtral__G"] = lg, G
    # Qwen3: E=128, k=8, norm and no-norm
    lq = (_rng(113).standard_normal((32, 128)) * 0.9).astype(np.float32)
    Gq = _rng(114).standard_normal((32, 128)).astype(np.float32)
    for norm in (True, False):
        cfg = Qwen3MoeConfig(hidden_size=128, num_experts=128, num_experts_per_tok=8, norm_topk_prob=norm)
        r = eye_(Qwen3MoeTopKRouter(cfg), 128)
        tag = "qwen_norm" if norm else "qwen_nonorm"
        arrays[f"{tag}__idx"], arrays[f"{tag}__dl"] = _router_grad(r, lq, Gq)
    arrays["qwen__logits"], arrays["qwen__G"] = lq, Gq
    # DeepSeek-V3: E=64 in 8 groups, top-4 groups, k=8, bias, x2.5, norm and no-norm
    ld = (_rng(115).standard_normal((32, 64)) * 1.5).astype(np.float32)
    bd = (_rng(116).standard_normal(64) * 1e-3).astype(np.float32)
    Gd = _rng(117).standard_normal((32, 64)).astype(np.float32)
    for norm in (True, False):
        cfg = DeepseekV3Config(hidden_size=64, n_routed_experts=64, num_experts_per_tok=8, n_group=8, topk_group=4,
                               norm_topk_prob=norm, routed_scaling_factor=2.5)
        r = eye_(DeepseekV3TopkRouter(cfg), 64)
        with torch.no_grad():
            r.e_score_correction_bias.copy_(torch.from_numpy(bd))
        tag = "ds_norm" if norm else "ds_nonorm"
        arrays[f"{tag}__idx"], arrays[f"{tag}__dl"] = _router_grad(r, ld, Gd)
    arrays["ds__logits"], arrays["ds__bias"], arrays["ds__G"] = ld, bd, Gd
    # scores: d/d logits of sum(scores * H), sigmoid and full softmax, float64
    H = _rng(118).standard_normal((32, 64))
    x = torch.from_numpy(ld.astype(np.float64)).requires_grad_(True)
    (torch.sigmoid(x) * torch.from_numpy(H)).sum().backward()
    arrays["scores__H"], arrays["scores__dl_sigmoid"] = H.astype(np.float32), x.grad.numpy()
    x = torch.from_numpy(ld.astype(np.float64)).requires_grad_(True)
    (torch.softmax(x, -1) * torch.from_numpy(H)).sum().backward()
    arrays["scores__dl_softmax"] = x.grad.numpy()
    np.savez_compressed(OUT / "router_grads.npz", **arrays)


def make_moe_block_grads():
    """HF DeepseekV3MoE (float64 experts, float32 router) differentiated by torch autograd:
    d/d(x, gate weight, routed and shared expert weights) of sum(out * G) on the shared-expert
    block fixture's inputs -- the gradients jax.grad takes through MoEBlock.__call__
    (mintext/modules/moe.py:240-266), router included."""
    from transformers import DeepseekV3Config
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3MoE

    p = moe_block_inputs()
    D, E, K, I = p["D"], p["E"], p["K"], p["I"]
    cfg = DeepseekV3Config(hidden_size=D, moe_intermediate_size=I, n_routed_experts=E, num_experts_per_tok=K,
                           n_group=p["n_group"], topk_group=p["topk_group"], routed_scaling_factor=p["scale"],
                           norm_topk_prob=True, n_shared_experts=1, hidden_act="silu")
    blk = DeepseekV3MoE(cfg).double().train()
    t64 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).double()
    with torch.no_grad():
        blk.gate.weight.copy_(t64(p["wg"].T))
        blk.gate.e_score_correction_bias.copy_(t64(p["bias"]))
        blk.experts.gate_up_proj.copy_(t64(np.swapaxes(p["gate_up"], 1, 2)))
        blk.experts.down_proj.copy_(t64(np.swapaxes(p["down"], 1, 2)))
        blk.shared_experts.gate_proj.weight.copy_(t64(p["shared_gate_up"][:, :I].T))
        blk.shared_experts.up_proj.weight.copy_(t64(p["shared_gate_up"][:, I:].T))
        blk.shared_experts.down_proj.weight.copy_(t64(p["shared_down"].T))
    G = _rng(22).standard_normal((p["T"], D))
    xt = t64(p["x"]).requires_grad_(True)
    out = blk(xt[None]).reshape(p["T"], D)
    (out * torch.from_numpy(G)).sum().backward()
    sg = torch.cat([blk.shared_experts.gate_proj.weight.grad.T, blk.shared_experts.up_proj.weight.grad.T], 1)
    np.savez_compressed(OUT / "moe_block_grads.npz", G=G, dx=xt.grad.numpy(),
                        dwg=blk.gate.weight.grad.T.numpy(),
                        dgate_up=np.swapaxes(blk.experts.gate_up_proj.grad.numpy(), 1, 2),
                        ddown=np.swapaxes(blk.experts.down_proj.grad.numpy(), 1, 2),
                        dshared_gate_up=sg.numpy(), dshared_down=blk.shared_experts.down_proj.weight.grad.T.numpy())


# --------------------------------------------------------------------------------- dispatch
def _torch_route(idx: np.ndarray, E: int):
    flat = torch.from_numpy(idx.astype(np.int64)).reshape(-1)
    perm = torch.sort(flat, stable=True).indices
    gs = torch.bincount(flat, minlength=E)[:E]
    return perm.numpy().astype(np.int32), gs.numpy().astype(np.int32)


def make_dispatch():
    cases = {}
    # the reference TestSortDispatch shape: N=32, K=2, E=4 (tests/test_moe_kernels.py:25)
    cases["rand_n32_k2_e4"] = (_rng(201).integers(0, 4, (32, 2)), 4)
    # all tokens to one expert (tests/test_moe_kernels.py:105-117)
    cases["single_expert"] = (np.zeros((8, 1), np.int64), 4)
    # experts 2,3 empty (:119-134)
    cases["empty_experts"] = (_rng(202).integers(0, 2, (8, 1)), 4)
    # Mixtral-like E=8, K=2, many tokens
    cases["rand_n1000_k2_e8"] = (np.stack([_rng(203).permutation(8)[:2] for _ in range(1000)]), 8)
    # DeepSeek-like E=256, K=8
    cases["rand_n300_k8_e256"] = (np.stack([_rng(204 + i).permutation(256)[:8] for i in range(300)]), 256)
    # heavy skew: 90% to expert 5
    sk = _rng(205).integers(0, 16, (700, 4))
    sk[_rng(206).random((700, 4)) < 0.9] = 5
    cases["skew_n700_k4_e16"] = (sk, 16)
    arrays = {}
    for name, (idx, E) in cases.items():
        perm, gs = _torch_route(idx, E)
        arrays[f"{name}__idx"] = idx.astype(np.int32)
        arrays[f"{name}__E"] = np.int32(E)
        arrays[f"{name}__perm"] = perm
        arrays[f"{name}__gs"] = gs
    np.savez_compressed(OUT / "dispatch.npz", **arrays)


# ------------------------------------------------------------------------------------- gmm
def _gmm64(x, w, gs):
    x = torch.from_numpy(x).double()
    w = torch.from_numpy(w).double()
    out = torch.zeros(x.shape[0], w.shape[2], dtype=torch.float64)
    off = 0
    for e, g in enumerate(gs):
        if g:
            out[off:off + g] = x[off:off + g] @ w[e]
        off += g
    return out.numpy()


def _tgmm64(x, g, gs):
    x = torch.from_numpy(x).double()
    g = torch.from_numpy(g).double()
    out = torch.zeros(len(gs), x.shape[1], g.shape[1], dtype=torch.float64)
    off = 0
    for e, n in enumerate(gs):
        if n:
            out[e] = x[off:off + n].T @ g[off:off + n]
        off += n
    return out.numpy()


def make_gmm():
    # group-size patterns from the reference tests (tests/test_moe_kernels.py:190-273,405-479)
    cases = {
        "uniform_e4": ([16, 16, 16, 16], 32, 16),
        "single": ([16], 8, 4),
        "gs_8_8_0_0": ([8, 8, 0, 0], 8, 4),
        "gs_15_1_0_0": ([15, 1, 0, 0], 8, 4),
        "gs_10_5_1_0": ([10, 5, 1, 0], 8, 4),
        "gs_8_0_8": ([8, 0, 8], 4, 4),
        "gs_10_3_2_1": ([10, 3, 2, 1], 8, 4),
        "ragged_mid": ([37, 0, 91, 5, 0, 123], 64, 96),
    }
    arrays = {}
    for i, (name, (gs, kin, kout)) in enumerate(cases.items()):
        r = _rng(300 + i)
        M = int(sum(gs))
        x = r.standard_normal((M, kin)).astype(np.float32)
        w = r.standard_normal((len(gs), kin, kout)).astype(np.float32)
        g = r.standard_normal((M, kout)).astype(np.float32)
        arrays[f"{name}__gs"] = np.array(gs, np.int32)
        arrays[f"{name}__x"] = x
        arrays[f"{name}__w"] = w
        arrays[f"{name}__g"] = g
        arrays[f"{name}__out"] = _gmm64(x, w, gs)
        arrays[f"{name}__dlhs"] = _gmm64(g, np.swapaxes(w, 1, 2).copy(), gs)
        arrays[f"{name}__tgmm"] = _tgmm64(x, g, gs)
    np.savez_compressed(OUT / "gmm.npz", **arrays)


# ------------------------------------------------------------------------------------- fp8
def make_fp8():
    r = _rng(401)
    vals = np.concatenate([
        r.standard_normal(4000).astype(np.float32) * 50,
        r.standard_normal(1000).astype(np.float32) * 1e-2,
        np.array([0.0, -0.0, 448, -448, 440, 2 ** -6, 2 ** -7, 2 ** -9, 3 * 2 ** -10, 2 ** -10, 0.3, 1.0,
                  1.0625, 1.125, 1.1875, 240.0, 232.0, 248.0], np.float32),
    ])
    codes = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.savez_compressed(OUT / "fp8.npz", values=vals, codes=codes)


# ------------------------------------------------------------------------- tiny MoE layer
def make_moe_tiny():
    """C1: T=256, D=128, E=8, K=2, I=256, fp32, softmax renormalised over top-k."""
    from transformers import MixtralConfig
    from transformers.models.mixtral.modeling_mixtral import MixtralSparseMoeBlock

    T, D, E, K, I = 256, 128, 8, 2, 256
    r = _rng(1)
    x = r.standard_normal((T, D)).astype(np.float32)
    wg = (r.standard_normal((D, E)) * 0.02).astype(np.float32)
    gate_up = (r.standard_normal((E, D, 2 * I)) * 0.02).astype(np.float32)
    down = (r.standard_normal((E, I, D)) * 0.02).astype(np.float32)
    cfg = MixtralConfig(hidden_size=D, intermediate_size=I, num_local_experts=E, num_experts_per_tok=K,
                        hidden_act="silu", router_jitter_noise=0.0)
    blk = MixtralSparseMoeBlock(cfg).double().eval()
    with torch.no_grad():
        blk.gate.weight.copy_(torch.from_numpy(wg.T.copy()).double())
        blk.experts.gate_up_proj.copy_(torch.from_numpy(np.swapaxes(gate_up, 1, 2).copy()).double())
        blk.experts.down_proj.copy_(torch.from_numpy(np.swapaxes(down, 1, 2).copy()).double())
        xt = torch.from_numpy(x).double()
        logits = xt @ torch.from_numpy(wg).double()
        out = blk(xt.reshape(2, 128, D)).reshape(T, D)
        _, w, idx = blk.gate(xt)
    np.savez_compressed(OUT / "moe_tiny.npz", logits=logits.float().numpy(), idx=idx.numpy().astype(np.int32),
                        w=w.numpy(), out=out.numpy())


# ------------------------------------------------- DeepSeek-style block with a shared expert
def moe_block_inputs():
    """Inputs of the shared-expert block fixture (regenerated from a PCG64 seed by the tests)."""
    T, D, E, K, I, G, TG = 64, 64, 16, 4, 32, 4, 2
    r = _rng(21)
    x = r.standard_normal((T, D)).astype(np.float32)
    wg = (r.standard_normal((D, E)) * 0.2).astype(np.float32)
    bias = (r.standard_normal(E) * 0.05).astype(np.float32)
    gate_up = (r.standard_normal((E, D, 2 * I)) * 0.05).astype(np.float32)
    down = (r.standard_normal((E, I, D)) * 0.05).astype(np.float32)
    sgu = (r.standard_normal((D, 2 * I)) * 0.05).astype(np.float32)
    sdn = (r.standard_normal((I, D)) * 0.05).astype(np.float32)
    return dict(T=T, D=D, E=E, K=K, I=I, n_group=G, topk_group=TG, scale=2.5, x=x, wg=wg, bias=bias,
                gate_up=gate_up, down=down, shared_gate_up=sgu, shared_down=sdn)


def make_moe_block_shared():
    """HF DeepseekV3MoE (float64 experts; its router computes float32 logits and scores):
    sigmoid + bias, group-limited top-4 of 16 experts, norm, x2.5, one shared expert."""
    from transformers import DeepseekV3Config
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3MoE

    p = moe_block_inputs()
    D, E, K, I = p["D"], p["E"], p["K"], p["I"]
    cfg = DeepseekV3Config(hidden_size=D, moe_intermediate_size=I, n_routed_experts=E, num_experts_per_tok=K,
                           n_group=p["n_group"], topk_group=p["topk_group"], routed_scaling_factor=p["scale"],
                           norm_topk_prob=True, n_shared_experts=1, hidden_act="silu")
    blk = DeepseekV3MoE(cfg).double().eval()
    t64 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).double()
    with torch.no_grad():
        blk.gate.weight.copy_(t64(p["wg"].T))
        blk.gate.e_score_correction_bias.copy_(t64(p["bias"]))
        blk.experts.gate_up_proj.copy_(t64(np.swapaxes(p["gate_up"], 1, 2)))
        blk.experts.down_proj.copy_(t64(np.swapaxes(p["down"], 1, 2)))
        blk.shared_experts.gate_proj.weight.copy_(t64(p["shared_gate_up"][:, :I].T))
        blk.shared_experts.up_proj.weight.copy_(t64(p["shared_gate_up"][:, I:].T))
        blk.shared_experts.down_proj.weight.copy_(t64(p["shared_down"].T))
        xt = t64(p["x"])
        logits, w, idx = blk.gate(xt)
        out = blk(xt[None]).reshape(p["T"], D)
    np.savez_compressed(OUT / "moe_block_shared.npz", logits=logits.float().numpy(),
                        idx=idx.numpy().astype(np.int32), w=w.float().numpy(), out=out.numpy())


if __name__ == "__main__":
    torch.manual_seed(0)
    make_router_grads()
    make_moe_block_grads()
    make_routers()
    make_dispatch()
    make_gmm()
    make_fp8()
    make_moe_tiny()
    make_moe_block_shared()
    for p in sorted(OUT.glob("*.npz")):
        print(p.name, p.stat().st_size)

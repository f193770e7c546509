"""GPU parity: router top-k (HIP) vs the oracle and the HF-derived fixtures.

Indices must be bit-exact.  Softmax mode selects on the logits, so its indices are exact for
any input; sigmoid mode selects on float32 scores computed on the GPU, which can differ from
numpy's sigmoid by an ulp, so its indices are checked bit-exactly against the oracle's
selection run on the GPU's own scores (the scores themselves at 1e-6 relative).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def test_softmax_router_fixtures(dev):
    from mintext_amd.kernels import route_topk

    g = golden("routers")
    for key, k in (("mixtral", 2), ("qwen", 8)):
        idx, w = route_topk(torch.from_numpy(g[f"{key}_logits"]).to(dev), k, scoring="softmax")
        np.testing.assert_array_equal(idx.cpu().numpy(), g[f"{key}_idx"])
        np.testing.assert_allclose(w.cpu().numpy(), g[f"{key}_w"], rtol=1e-5, atol=1e-7)
    idx, w = route_topk(torch.from_numpy(g["qwen_logits"]).to(dev), 8, scoring="softmax", norm_topk_prob=False)
    np.testing.assert_array_equal(idx.cpu().numpy(), g["qwen_idx_nonorm"])
    np.testing.assert_allclose(w.cpu().numpy(), g["qwen_w_nonorm"], rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("key", ["ds", "ds3"])
def test_sigmoid_group_router_fixtures(dev, key):
    from mintext_amd.kernels import route_topk

    g = golden("routers")
    idx, w, s = route_topk(torch.from_numpy(g[f"{key}_logits"]).to(dev), 8, scoring="sigmoid_group",
                           bias=torch.from_numpy(g[f"{key}_bias"]), n_group=8, topk_group=4,
                           routed_scaling_factor=2.5, return_scores=True)
    s = s.cpu().numpy()
    np.testing.assert_allclose(s, g[f"{key}_scores"], rtol=1e-6)
    oi, ow, _ = O.router_sigmoid_group(None, 8, bias=g[f"{key}_bias"], n_group=8, topk_group=4,
                                       routed_scaling_factor=2.5, scores=s)
    np.testing.assert_array_equal(idx.cpu().numpy(), oi)
    np.testing.assert_array_equal(idx.cpu().numpy(), g[f"{key}_idx"])
    np.testing.assert_allclose(w.cpu().numpy(), ow, rtol=1e-5)


@pytest.mark.parametrize("T,E,k,dt", [(16384, 128, 8, torch.bfloat16), (8192, 8, 2, torch.bfloat16),
                                      (4096, 256, 8, torch.float32), (1000, 64, 6, torch.float32),
                                      (777, 5, 3, torch.float32), (300, 1024, 8, torch.float32),
                                      (100, 3, 1, torch.float32), (64, 40, 40, torch.float32)])
def test_softmax_router_large(dev, T, E, k, dt):
    from mintext_amd.kernels import route_topk

    logits = (torch.randn(T, E, device=dev) * 1.3).to(dt)
    idx, w = route_topk(logits, k, scoring="softmax")
    lg = logits.float().cpu().numpy()
    oi, ow, _ = O.router_softmax(lg, k)
    np.testing.assert_array_equal(idx.cpu().numpy(), oi)
    np.testing.assert_allclose(w.cpu().numpy(), ow, rtol=1e-5, atol=1e-7)


def test_softmax_router_ties_lower_index_first(dev):
    from mintext_amd.kernels import route_topk

    lg = np.random.default_rng(4).integers(0, 3, (512, 16)).astype(np.float32)  # heavy ties
    idx, _ = route_topk(torch.from_numpy(lg).to(dev), 5, scoring="softmax")
    np.testing.assert_array_equal(idx.cpu().numpy(), O.topk_desc(lg, 5))


def test_deepseek_router_full_size(dev):
    """C3 routing: T=4096, E=256, 8 groups / top-4, k=8, bias, scale 2.5."""
    from mintext_amd.kernels import route_topk

    T, E = 4096, 256
    logits = torch.randn(T, E, device=dev).to(torch.bfloat16)
    bias = torch.randn(E, device=dev) * 1e-3
    idx, w, s = route_topk(logits, 8, scoring="sigmoid_group", bias=bias, n_group=8, topk_group=4,
                           routed_scaling_factor=2.5, return_scores=True)
    s = s.cpu().numpy()
    np.testing.assert_allclose(s, O.sigmoid_f32(logits.float().cpu().numpy()), rtol=1e-6)
    oi, ow, _ = O.router_sigmoid_group(None, 8, bias=bias.cpu().numpy(), n_group=8, topk_group=4,
                                       routed_scaling_factor=2.5, scores=s)
    np.testing.assert_array_equal(idx.cpu().numpy(), oi)
    np.testing.assert_allclose(w.cpu().numpy(), ow, rtol=1e-5)


def test_bias_steers_selection(dev):
    """tests/test_model.py:468-478 of the reference: bias [10,0,0,0] always selects expert 0."""
    from mintext_amd.kernels import route_topk

    idx, _ = route_topk(torch.randn(64, 4, device=dev), 2, scoring="sigmoid_group",
                        bias=torch.tensor([10.0, 0, 0, 0]), n_group=2, topk_group=1)
    assert (idx[:, 0] == 0).all()
    assert ((idx >= 0) & (idx < 4)).all()


# ---- router gate GEMM fused with the top-k -----------------------------------------------------
GATE_CASES = [
    # (T, D, E, K, scoring, n_group, topk_group, scale, with_bias, shared)
    (300, 4096, 8, 2, "softmax", 1, 1, 1.0, False, False),         # Mixtral shape
    (257, 2048, 128, 8, "softmax", 1, 1, 1.0, False, False),       # Qwen3 shape
    (130, 7168, 256, 8, "sigmoid_group", 8, 4, 2.5, True, False),  # DeepSeek-V3 shape
    (64, 64, 16, 4, "sigmoid_group", 4, 2, 2.5, True, True),       # folded shared expert column
    (33, 128, 3, 1, "softmax", 1, 1, 1.0, False, False),           # odd E, T
]


@pytest.mark.parametrize("T,D,E,K,scoring,ng,tg,scale,with_bias,shared", GATE_CASES)
def test_gate_route_topk_fused(dev, T, D, E, K, scoring, ng, tg, scale, with_bias, shared):
    """gate_route_topk: logits within one bf16 rounding of the float64 product x @ Wg, and the
    selection / weights of route_topk on those bf16 logits, bit for bit."""
    from mintext_amd.kernels import route_topk
    from mintext_amd.kernels.router import gate_route_topk, gate_weight_linear_layout

    g = torch.Generator(device=dev)
    g.manual_seed(T + E)
    x = torch.randn(T, D, device=dev, generator=g).bfloat16()
    wg = (torch.randn(D, E, device=dev, generator=g) * 0.02).bfloat16()  # reference kernel layout [D, E]
    bias = (torch.randn(E, device=dev, generator=g) * 1e-3) if with_bias else None
    kw = dict(scoring=scoring, bias=bias, n_group=ng, topk_group=tg, routed_scaling_factor=scale)
    se = E if shared else None
    wt = gate_weight_linear_layout(wg)
    assert torch.equal(wt, wg.t().contiguous())
    idx, w, lg = gate_route_topk(x, wt, K, shared_expert=se, return_logits=True, **kw)
    ref = x.double().cpu() @ wg.double().cpu()
    got = lg.double().cpu()
    assert ((got - ref).abs() <= 2.0 ** -8 * ref.abs() + 1e-4).all()
    idx2, w2, s2 = route_topk(lg, K, shared_expert=se, return_scores=True, **kw)
    assert torch.equal(idx, idx2) and torch.equal(w, w2)
    idx3, w3, s3 = gate_route_topk(x, wt, K, shared_expert=se, return_scores=True, **kw)  # deterministic
    assert torch.equal(idx, idx3) and torch.equal(w, w3)
    assert torch.equal(s3, s2)  # the scores of route_topk on the same bf16 logits, bit for bit


def test_gate_route_topk_unsupported_shapes_raise(dev):
    from mintext_amd._lib import MtxError
    from mintext_amd.kernels.router import gate_route_topk

    x = torch.randn(8, 64, device=dev)
    with pytest.raises(MtxError):
        gate_route_topk(x, torch.randn(8, 64, device=dev), 2)  # f32 tokens
    xb = x.bfloat16()
    with pytest.raises(MtxError):
        gate_route_topk(xb, torch.randn(300, 64, device=dev).bfloat16(), 2)  # E > 256


# ---- router VJP ---------------------------------------------------------------------------------
VJP_FIXTURES = [("mixtral", "mixtral", "softmax", True, 1.0), ("qwen_norm", "qwen", "softmax", True, 1.0),
                ("qwen_nonorm", "qwen", "softmax", False, 1.0), ("ds_norm", "ds", "sigmoid_group", True, 2.5),
                ("ds_nonorm", "ds", "sigmoid_group", False, 2.5)]


@pytest.mark.parametrize("tag,base,scoring,norm,scale", VJP_FIXTURES)
def test_router_bwd_matches_hf_autograd(dev, tag, base, scoring, norm, scale):
    """mtx_router_topk_bwd against torch autograd through the HF routers (float32)."""
    from mintext_amd.kernels.router import router_topk_bwd

    g = golden("router_grads")
    lg, G, idx = g[f"{base}__logits"], g[f"{base}__G"], g[f"{tag}__idx"]
    dw = np.take_along_axis(G, idx, axis=1)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    dl = router_topk_bwd(t(lg), t(idx), idx.shape[1], t(dw), None, scoring=scoring, norm_topk_prob=norm,
                         routed_scaling_factor=scale)
    assert dl.dtype == torch.float32
    ref = g[f"{tag}__dl"]
    err = np.linalg.norm(dl.cpu().numpy() - ref) / np.linalg.norm(ref)
    assert err < 1e-5


@pytest.mark.parametrize("scoring,T,E,K,ng,tg,norm,dt", [
    ("sigmoid_group", 4096, 256, 8, 8, 4, True, torch.bfloat16),   # C3 router
    ("softmax", 16384, 128, 8, 1, 1, True, torch.bfloat16),        # C4 / C5 router
    ("softmax", 8192, 8, 2, 1, 1, True, torch.float32),            # C2 router
    ("softmax", 1000, 64, 6, 1, 1, False, torch.float32),
    ("sigmoid_group", 777, 64, 8, 8, 4, False, torch.float32),
    ("softmax", 300, 1024, 8, 1, 1, True, torch.float32),
])
def test_router_bwd_matches_oracle(dev, scoring, T, E, K, ng, tg, norm, dt):
    """The router VJP (weights and scores) through autograd of route_topk against the float64
    oracle on the GPU's own indices; the logits' gradient comes back in the logits' dtype."""
    from mintext_amd.kernels import route_topk

    gen = torch.Generator(device=dev)
    gen.manual_seed(T + E)
    logits = (torch.randn(T, E, device=dev, generator=gen) * 1.3).to(dt).requires_grad_(True)
    bias = torch.randn(E, device=dev, generator=gen) * 1e-3 if scoring != "softmax" else None
    idx, w, s = route_topk(logits, K, scoring=scoring, bias=bias, n_group=ng, topk_group=tg, norm_topk_prob=norm,
                           routed_scaling_factor=2.5, return_scores=True)
    assert w.requires_grad and s.requires_grad and not idx.requires_grad
    gw = torch.randn(T, K, device=dev, generator=gen)
    gs = torch.randn(T, E, device=dev, generator=gen)
    ((w * gw).sum() + (s * gs).sum()).backward()
    assert logits.grad.dtype == dt
    ref = O.router_vjp(logits.detach().float().cpu().numpy(), idx.cpu().numpy(), gw.cpu().numpy(),
                       gs.cpu().numpy(), scoring, norm, 2.5)
    got = logits.grad.double().cpu().numpy()
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err < (1e-5 if dt == torch.float32 else 2e-2 / 4)

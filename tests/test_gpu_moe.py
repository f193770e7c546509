"""GPU parity of the composed expert layer (MoEExperts._forward_kernel, mintext/modules/moe.py:161-221)
and of the MoE layer forward on the C1 fixture (HF MixtralSparseMoeBlock in float64)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden, rel_err
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _c1_inputs():
    rng = np.random.default_rng(1)
    T, D, E, I = 256, 128, 8, 256
    x = rng.standard_normal((T, D)).astype(np.float32)
    wg = (rng.standard_normal((D, E)) * 0.02).astype(np.float32)
    gate_up = (rng.standard_normal((E, D, 2 * I)) * 0.02).astype(np.float32)
    down = (rng.standard_normal((E, I, D)) * 0.02).astype(np.float32)
    return x, wg, gate_up, down


def test_tiny_layer_fp32_matches_hf(dev):
    """C1: fp32, softmax renormalised top-2 -> out within 1e-5 of HF (float64)."""
    from mintext_amd.moe import moe_layer_forward

    g = golden("moe_tiny")
    x, _, gate_up, down = _c1_inputs()
    t = lambda a: torch.from_numpy(a).to(dev)
    out, idx, w = moe_layer_forward(t(g["logits"]), t(x), t(gate_up), t(down), k=2, scoring="softmax")
    np.testing.assert_array_equal(idx.cpu().numpy(), g["idx"])
    np.testing.assert_allclose(w.cpu().numpy(), g["w"], rtol=1e-5)
    assert out.dtype == torch.float32
    assert rel_err(out.cpu().numpy(), g["out"]) < 1e-5
    np.testing.assert_allclose(out.cpu().numpy(), g["out"], rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("fuse", [True, False])
def test_bf16_layer_matches_oracle(dev, fuse):
    from mintext_amd.kernels import route_topk
    from mintext_amd.moe import moe_experts_forward

    T, D, E, K, I = 1024, 256, 8, 2, 512
    x = torch.randn(T, D, device=dev).bfloat16()
    logits = torch.randn(T, E, device=dev)
    gate_up = (torch.randn(E, D, 2 * I, device=dev) * 0.05).bfloat16()
    down = (torch.randn(E, I, D, device=dev) * 0.05).bfloat16()
    idx, w = route_topk(logits, K)
    out = moe_experts_forward(x, idx, w, gate_up, down, fuse_swiglu=fuse)
    ref = O.moe_experts(x.float().cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy(), gate_up.float().cpu().numpy(),
                        down.float().cpu().numpy())
    assert out.dtype == torch.float32
    assert rel_err(out.cpu().numpy(), ref) < 2e-2


def test_fp8_layer_matches_oracle(dev):
    from mintext_amd.kernels import route_topk
    from mintext_amd.kernels.fp8 import quantize_fp8_weights
    from mintext_amd.moe import moe_experts_forward_fp8

    T, D, E, K, I = 1024, 512, 16, 4, 256
    x = torch.randn(T, D, device=dev).bfloat16()
    gate_up = (torch.randn(E, D, 2 * I, device=dev) * 0.05).bfloat16()
    down = (torch.randn(E, I, D, device=dev) * 0.05).bfloat16()
    idx, w = route_topk(torch.randn(T, E, device=dev), K)
    guq, gus = quantize_fp8_weights(gate_up)
    dnq, dns = quantize_fp8_weights(down)
    out = moe_experts_forward_fp8(x, idx, w, guq, gus, dnq, dns)
    u8 = lambda t: t.view(torch.uint8).cpu().numpy()
    # same quantisation points as the kernels: only f32-vs-f64 accumulation, the bf16 output
    # rounding and the resulting one-step code flips in the re-quantisation differ
    ref_q = O.moe_experts_fp8(x.float().cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy(), u8(guq), gus.cpu().numpy(),
                              u8(dnq), dns.cpu().numpy())
    assert rel_err(out.cpu().numpy(), ref_q) < 2e-2
    # against the unquantised float64 layer: each GEMM is within 6e-2 (test_gpu_fp8); the layer
    # quantises activations twice in series (x, then the SwiGLU output), so its bound is 1e-1
    ref = O.moe_experts(x.float().cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy(), gate_up.float().cpu().numpy(),
                        down.float().cpu().numpy())
    assert rel_err(out.cpu().numpy(), ref) < 1e-1


def test_block_backward_matches_oracle(dev):
    """Gradient of sum(out * g) through route -> gmm -> SwiGLU -> gmm -> unroute (fp32)."""
    from mintext_amd.moe import moe_experts_forward

    rng = np.random.default_rng(5)
    T, D, E, K, I = 64, 32, 4, 2, 16
    x = rng.standard_normal((T, D))
    gu = rng.standard_normal((E, D, 2 * I)) * 0.2
    dn = rng.standard_normal((E, I, D)) * 0.2
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    w = rng.random((T, K))
    g = rng.standard_normal((T, D))
    f = lambda a: torch.from_numpy(a.astype(np.float32)).to(dev).requires_grad_(True)
    xt, gut, dnt, wt = f(x), f(gu), f(dn), f(w)
    out = moe_experts_forward(xt, torch.from_numpy(idx).to(dev), wt, gut, dnt)
    (out * torch.from_numpy(g.astype(np.float32)).to(dev)).sum().backward()
    # float64 finite differences of the oracle layer on a few coordinates
    L = lambda xx, gg, dd, ww: float(np.sum(O.moe_experts(xx, idx, ww, gg, dd) * g))
    eps = 1e-6
    for (arr, grad, name) in ((x, xt.grad, "x"), (gu, gut.grad, "gate_up"), (dn, dnt.grad, "down"), (w, wt.grad, "w")):
        flat = arr.reshape(-1)
        for pos in np.random.default_rng(len(name)).choice(flat.size, 6, replace=False):
            p, m = arr.copy().reshape(-1), arr.copy().reshape(-1)
            p[pos] += eps
            m[pos] -= eps
            args = {"x": x, "gate_up": gu, "down": dn, "w": w}
            args[name] = p.reshape(arr.shape)
            lp = L(args["x"], args["gate_up"], args["down"], args["w"])
            args[name] = m.reshape(arr.shape)
            lm = L(args["x"], args["gate_up"], args["down"], args["w"])
            num = (lp - lm) / (2 * eps)
            np.testing.assert_allclose(grad.reshape(-1)[pos].item(), num, rtol=1e-3, atol=1e-4, err_msg=name)


# ---- shared expert folded into the routed GEMMs, expert counts, loss-free bias update -------

def _block_inputs():
    import sys

    from conftest import GOLDEN

    sys.path.insert(0, str(GOLDEN))
    from make_golden import moe_block_inputs

    return moe_block_inputs()


@pytest.mark.gpu
def test_router_topk_shared_column(dev):
    from mintext_amd.kernels import route_topk

    p = _block_inputs()
    lg = torch.from_numpy(golden("moe_block_shared")["logits"]).to(dev)
    kw = dict(scoring="sigmoid_group", bias=torch.from_numpy(p["bias"]).to(dev), n_group=p["n_group"],
              topk_group=p["topk_group"], routed_scaling_factor=p["scale"])
    idx, w = route_topk(lg, p["K"], **kw)
    idx2, w2 = route_topk(lg, p["K"], shared_expert=p["E"], **kw)
    assert idx2.shape == (p["T"], p["K"] + 1)
    assert torch.equal(idx2[:, :p["K"]], idx) and torch.equal(w2[:, :p["K"]], w)
    assert (idx2[:, p["K"]] == p["E"]).all() and (w2[:, p["K"]] == 1.0).all()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_folded_shared_expert_block(dev, dtype):
    from mintext_amd.moe import fold_shared_expert, moe_layer_forward

    p = _block_inputs()
    g = golden("moe_block_shared")
    cdt = torch.float32 if dtype == "f32" else torch.bfloat16
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(cdt)
    x, gu, dn, sgu, sdn = t(p["x"]), t(p["gate_up"]), t(p["down"]), t(p["shared_gate_up"]), t(p["shared_down"])
    lg = torch.from_numpy(g["logits"]).to(dev)
    kw = dict(k=p["K"], scoring="sigmoid_group", bias=torch.from_numpy(p["bias"]).to(dev), n_group=p["n_group"],
              topk_group=p["topk_group"], routed_scaling_factor=p["scale"])
    out_s, idx_s, w_s, cnt_s = moe_layer_forward(lg, x, gu, dn, shared_gate_up=sgu, shared_down=sdn,
                                                 return_expert_counts=True, **kw)
    gu_f, dn_f = fold_shared_expert(gu, dn, sgu, sdn)
    out_f, idx_f, w_f, cnt_f = moe_layer_forward(lg, x, gu_f, dn_f, shared_folded=True, return_expert_counts=True,
                                                 **kw)
    # same routing, same counts, same output bits as routed + shared evaluated separately
    assert torch.equal(idx_f, idx_s) and torch.equal(w_f, w_s) and torch.equal(cnt_f, cnt_s)
    assert torch.equal(out_f, out_s)
    assert np.array_equal(cnt_f.cpu().numpy(), np.bincount(idx_f.cpu().numpy().ravel(), minlength=p["E"]))
    tol = 1e-5 if dtype == "f32" else 2e-2
    assert rel_err(out_f.double().cpu().numpy(), g["out"]) < tol


@pytest.mark.gpu
@pytest.mark.parametrize("E", [8, 256, 1000])
def test_expert_bias_update_matches_oracle(dev, E):
    from mintext_amd.kernels import update_expert_bias

    rng = np.random.default_rng(E)
    counts = rng.integers(0, 3 * E, size=E).astype(np.int32)
    counts[: E // 4] = int(counts.mean())  # some experts exactly at the (integer) mean
    bias = (rng.standard_normal(E) * 0.01).astype(np.float32)
    b = torch.from_numpy(bias).to(dev)
    update_expert_bias(b, torch.from_numpy(counts).to(dev), 1e-3)
    assert np.array_equal(b.cpu().numpy(), O.expert_bias_update(counts, 1e-3, bias))


@pytest.mark.gpu
@pytest.mark.parametrize("T,E,K", [(512, 32, 8), (2048, 128, 4)])
def test_folded_shared_expert_mfma_shapes(dev, T, E, K):
    # shapes on the bf16 MFMA kernels (D, I multiples of 256 / 128): folded == separate up to the
    # f32 summation order of split-K tail tiles (the two layouts split different tiles), i.e.
    # within a bf16 rounding of each expert output.  T = 2048, E = 128: about 80 rows per expert
    # (one m-tile per scheduling group) and a shared group of 8 m-tiles, spread through the
    # tile order by the tile builder
    from mintext_amd.moe import fold_shared_expert, moe_layer_forward

    rng = np.random.default_rng(3)
    D, I = 512, 256
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev).bfloat16()
    x = t(rng.standard_normal((T, D)))
    gu, dn = t(rng.standard_normal((E, D, 2 * I)) * 0.03), t(rng.standard_normal((E, I, D)) * 0.03)
    sgu, sdn = t(rng.standard_normal((D, 2 * I)) * 0.03), t(rng.standard_normal((I, D)) * 0.03)
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).to(dev).bfloat16()
    bias = torch.from_numpy((rng.standard_normal(E) * 1e-3).astype(np.float32)).to(dev)
    kw = dict(k=K, scoring="sigmoid_group", bias=bias, n_group=8, topk_group=4, routed_scaling_factor=2.5)
    out_s, idx, w = moe_layer_forward(lg, x, gu, dn, shared_gate_up=sgu, shared_down=sdn, **kw)
    gu_f, dn_f = fold_shared_expert(gu, dn, sgu, sdn)
    out_f, idx_f, w_f = moe_layer_forward(lg, x, gu_f, dn_f, shared_folded=True, **kw)
    assert torch.equal(idx_f, idx) and torch.equal(w_f, w)
    scale = out_s.abs().max().item()
    assert ((out_f - out_s).abs() <= 2.0 ** -7 * out_s.abs() + 2.0 ** -9 * scale).all()
    f = lambda a: a.float().cpu().numpy()
    ref = O.moe_block(f(x), idx.cpu().numpy(), w.cpu().numpy(), f(gu), f(dn), f(sgu), f(sdn))
    assert rel_err(out_f.double().cpu().numpy(), ref) < 2e-2


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_moe_block_forward_with_gate(dev, dtype):
    # MoEBlock.__call__ from the tokens: hipBLASLt gate GEMM, then the HIP path; against the
    # HF DeepseekV3MoE fixture (the gate is the identity-free Linear x @ Wg)
    from mintext_amd.moe import moe_block_forward

    p = _block_inputs()
    g = golden("moe_block_shared")
    cdt = torch.float32 if dtype == "f32" else torch.bfloat16
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(cdt)
    x = t(p["x"]).reshape(2, p["T"] // 2, p["D"])
    out, aux = moe_block_forward(x, t(p["wg"]), t(p["gate_up"]), t(p["down"]), k=p["K"], scoring="sigmoid_group",
                                 bias=torch.from_numpy(p["bias"]).to(dev), n_group=p["n_group"],
                                 topk_group=p["topk_group"], routed_scaling_factor=p["scale"],
                                 shared_gate_up=t(p["shared_gate_up"]), shared_down=t(p["shared_down"]))
    assert out.shape == (2, p["T"] // 2, p["D"]) and out.dtype == torch.float32
    idx = aux["topk_indices"].cpu().numpy()
    assert np.array_equal(aux["expert_counts"].cpu().numpy(), np.bincount(idx.ravel(), minlength=p["E"]))
    if dtype == "f32":
        # f32 logits: the same expert sets as HF's router
        for r in range(p["T"]):
            assert set(idx[r].tolist()) == set(g["idx"][r].tolist())
        assert rel_err(out.reshape(p["T"], p["D"]).double().cpu().numpy(), g["out"]) < 1e-5
    else:
        # bf16 logits may flip near-ties: check against the oracle block on the GPU's own routing
        f = lambda a: a.float().cpu().numpy()
        ref = O.moe_block(f(t(p["x"])), idx, aux["topk_weights"].cpu().numpy(), f(t(p["gate_up"])), f(t(p["down"])),
                          f(t(p["shared_gate_up"])), f(t(p["shared_down"])))
        assert rel_err(out.reshape(p["T"], p["D"]).double().cpu().numpy(), ref) < 2e-2


# ---- backward of the block, router included; the aux contract ----------------------------------

def test_moe_block_backward_matches_hf_autograd(dev):
    """MoEBlock.__call__ under autograd (fp32): gradients of sum(out * G) w.r.t. the tokens, the
    gate weight (through the router's weights, moe.py:53,101), the routed and the shared expert
    weights, against torch autograd through HF DeepseekV3MoE (float64 experts, float32 router)."""
    from mintext_amd.moe import moe_block_forward

    p = _block_inputs()
    g = golden("moe_block_grads")
    leaf = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev).requires_grad_(True)
    x, wg, gu, dn = leaf(p["x"]), leaf(p["wg"]), leaf(p["gate_up"]), leaf(p["down"])
    sgu, sdn = leaf(p["shared_gate_up"]), leaf(p["shared_down"])
    out, aux = moe_block_forward(x.reshape(2, p["T"] // 2, p["D"]), wg, gu, dn, k=p["K"], scoring="sigmoid_group",
                                 bias=torch.from_numpy(p["bias"]).to(dev), n_group=p["n_group"],
                                 topk_group=p["topk_group"], routed_scaling_factor=p["scale"], shared_gate_up=sgu,
                                 shared_down=sdn)
    (out.reshape(p["T"], p["D"]) * torch.from_numpy(g["G"].astype(np.float32)).to(dev)).sum().backward()
    for got, ref, name in ((x.grad, g["dx"], "x"), (wg.grad, g["dwg"], "gate_weight"),
                           (gu.grad, g["dgate_up"], "gate_up"), (dn.grad, g["ddown"], "down"),
                           (sgu.grad, g["dshared_gate_up"], "shared_gate_up"),
                           (sdn.grad, g["dshared_down"], "shared_down")):
        assert got is not None, name
        assert rel_err(got.double().cpu().numpy(), ref) < 1e-5, name


@pytest.mark.parametrize("scoring", ["sigmoid_group", "softmax"])
@pytest.mark.parametrize("fused_gate", [False, True])
def test_moe_block_aux_scores(dev, scoring, fused_gate):
    """aux carries the reference's {"topk_indices", "scores"} (moe.py:262-266): [N, E] float32
    sigmoid scores (softmax probabilities in softmax mode) of the gate logits."""
    from mintext_amd.moe import moe_block_forward

    rng = np.random.default_rng(11)
    T, D, E, K, I = 256, 128, 16, 4, 128
    cdt = torch.bfloat16 if fused_gate else torch.float32
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev).to(cdt)
    x = t(rng.standard_normal((T, D)))
    wg = t(rng.standard_normal((D, E)) * 0.2)
    gu, dn = t(rng.standard_normal((E, D, 2 * I)) * 0.05), t(rng.standard_normal((E, I, D)) * 0.05)
    kw = dict(k=K, scoring=scoring, n_group=4 if scoring != "softmax" else 1, topk_group=2 if scoring != "softmax" else 1)
    with torch.no_grad():
        out, aux = moe_block_forward(x, wg, gu, dn, **kw)
    assert {"topk_indices", "scores"} <= set(aux)
    s = aux["scores"]
    assert s.shape == (T, E) and s.dtype == torch.float32
    # the logits the router saw: the gate GEMM's output in the compute dtype
    lg = (x.double() @ wg.double()).to(cdt).float().cpu().numpy()
    if scoring == "softmax":
        ex = np.exp(lg.astype(np.float64) - lg.max(-1, keepdims=True))
        ref = ex / ex.sum(-1, keepdims=True)
    else:
        ref = O.sigmoid_f32(lg)
    if fused_gate:  # the fused gate's logits are within one bf16 rounding of x @ Wg (checked elsewhere)
        assert np.abs(s.cpu().numpy() - ref).max() < 2e-2
    else:
        np.testing.assert_allclose(s.cpu().numpy(), ref, rtol=1e-5, atol=1e-7)
    # softmax mode: the selected experts hold the K largest of the scores returned beside them
    if scoring == "softmax":
        sn = s.cpu().numpy()
        sel = np.zeros_like(sn, bool)
        np.put_along_axis(sel, aux["topk_indices"].cpu().numpy().astype(np.int64), True, axis=1)
        assert (np.where(sel, sn, np.inf).min(1) >= np.where(sel, -np.inf, sn).max(1)).all()


@pytest.mark.parametrize("T,D,E,K,I", [(2048, 512, 8, 2, 512), (1024, 256, 32, 8, 256)])
def test_bf16_layer_autograd_mfma_matches_oracle_vjp(dev, T, D, E, K, I):
    """moe_experts_forward under autograd on the bf16 MFMA kernels (gmm fwd, dlhs, tgmm, SwiGLU
    and its VJP, route / unroute VJPs) against the oracle's float64 VJP on the same inputs."""
    from mintext_amd.kernels import route_topk
    from mintext_amd.moe import moe_experts_forward

    gen = torch.Generator(device=dev)
    gen.manual_seed(T + E)
    x = torch.randn(T, D, device=dev, generator=gen).bfloat16().requires_grad_(True)
    gu = (torch.randn(E, D, 2 * I, device=dev, generator=gen) * 0.05).bfloat16().requires_grad_(True)
    dn = (torch.randn(E, I, D, device=dev, generator=gen) * 0.05).bfloat16().requires_grad_(True)
    idx, w = route_topk(torch.randn(T, E, device=dev, generator=gen), K)
    w = w.clone().requires_grad_(True)
    G = torch.randn(T, D, device=dev, generator=gen)
    out = moe_experts_forward(x, idx, w, gu, dn)
    assert out.dtype == torch.float32
    (out * G).sum().backward()
    f = lambda a: a.detach().float().cpu().numpy()
    dx, dw, dgu, ddn = O.moe_experts_vjp(f(x), idx.cpu().numpy(), f(w), f(gu), f(dn), f(G))
    for got, ref, name in ((x.grad, dx, "x"), (w.grad, dw, "w"), (gu.grad, dgu, "gate_up"), (dn.grad, ddn, "down")):
        assert got.dtype == (torch.float32 if name == "w" else torch.bfloat16), name
        assert rel_err(f(got), ref) < 2e-2, name

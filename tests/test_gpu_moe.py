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

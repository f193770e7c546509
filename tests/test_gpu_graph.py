"""The MoE layer forward captured in a HIP graph (moe.CapturedLayer): every replay, with eager
work and synchronisations between replays, reproduces the eager result bit for bit, and a
replay after the inputs are refilled in place follows the new inputs."""
from __future__ import annotations

import numpy as np
import pytest
import torch


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,T,D,E,K,I", [("f32", 256, 128, 8, 2, 256), ("bf16", 1024, 512, 16, 4, 256)])
def test_captured_layer_replays_match_eager(dev, dtype, T, D, E, K, I):
    from mintext_amd.kernels import route_topk
    from mintext_amd.moe import CapturedLayer, moe_experts_forward

    cdt = torch.float32 if dtype == "f32" else torch.bfloat16
    g = torch.Generator(device=dev)
    g.manual_seed(T + D)
    x = torch.randn(T, D, device=dev, generator=g).to(cdt)
    logits = torch.randn(T, E, device=dev, generator=g).to(cdt)
    gu = (torch.randn(E, D, 2 * I, device=dev, generator=g) * 0.05).to(cdt)
    dn = (torch.randn(E, I, D, device=dev, generator=g) * 0.05).to(cdt)

    def layer(x_, lg_):
        idx, w = route_topk(lg_, K, scoring="softmax")
        return moe_experts_forward(x_, idx, w, gu, dn), idx

    with torch.no_grad():
        ref, ref_idx = layer(x, logits)
    cap = CapturedLayer(layer, x, logits)
    for r in range(3):
        out, idx = cap.replay()
        torch.cuda.synchronize()
        assert torch.equal(idx, ref_idx), f"replay {r}"
        assert torch.equal(out, ref), f"replay {r}"
        # eager work between replays (allocations, other kernels of this package)
        with torch.no_grad():
            layer(torch.randn_like(x.float()).to(cdt), torch.randn_like(logits.float()).to(cdt))
        torch.cuda.synchronize()
    # refill the static inputs in place: the replay follows them
    x2 = torch.randn(T, D, device=dev, generator=g).to(cdt)
    lg2 = torch.randn(T, E, device=dev, generator=g).to(cdt)
    with torch.no_grad():
        ref2, idx2 = layer(x2, lg2)
    x.copy_(x2)
    logits.copy_(lg2)
    out, idx = cap.replay()
    torch.cuda.synchronize()
    assert torch.equal(idx, idx2) and torch.equal(out, ref2)
    assert not torch.equal(ref2, ref)

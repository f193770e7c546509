"""Expert weight layout conversion on the GPU (mtx_transpose_batched) against the oracle's
restatement of mintext/checkpoint/conversion.py:80-166: bit-exact, round trips, ragged and
unaligned shapes (per-element path), and the C4/C3 shapes at full size."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O


def _rand(shape, dt, dev, rng):
    return torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(dev).to(dt)


@pytest.mark.gpu
@pytest.mark.parametrize("E,I,D", [(2, 64, 128), (3, 40, 72), (1, 7, 5), (4, 96, 200)])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_import_export_matches_oracle(dev, E, I, D, dt):
    from mintext_amd.kernels.expert_layout import experts_from_hf, experts_from_hf_fused, experts_to_hf

    rng = np.random.default_rng(E * 1000 + I + D)
    gate, up, down = _rand((E, I, D), dt, dev, rng), _rand((E, I, D), dt, dev, rng), _rand((E, D, I), dt, dev, rng)
    gu, dn = experts_from_hf(gate, up, down)
    f = lambda t: t.float().cpu().numpy()
    ogu, odn = O.experts_from_hf(f(gate), f(up), f(down))
    assert np.array_equal(f(gu), ogu) and np.array_equal(f(dn), odn)
    g2, u2, d2 = experts_to_hf(gu, dn)
    assert torch.equal(g2, gate) and torch.equal(u2, up) and torch.equal(d2, down)
    # HF fused form: gate_up_proj [E, 2I, D] = gate rows then up rows
    gu3, dn3 = experts_from_hf_fused(torch.cat([gate, up], 1), down)
    assert torch.equal(gu3, gu) and torch.equal(dn3, dn)


@pytest.mark.gpu
def test_full_size_roundtrip_and_bandwidth(dev):
    # C3 expert shapes (256 experts, D=7168, I=2048, bf16: 22.5 GB of weights) are too large to
    # hold three copies of next to the test suite's other buffers; C4's (128 x 2048 x 768) are
    # checked whole, plus a 16-expert slice of C3
    from mintext_amd.kernels.expert_layout import experts_from_hf, experts_to_hf

    rng = np.random.default_rng(5)
    for E, I, D in [(128, 768, 2048), (16, 2048, 7168)]:
        gate = _rand((E, I, D), torch.bfloat16, dev, rng)
        up = _rand((E, I, D), torch.bfloat16, dev, rng)
        down = _rand((E, D, I), torch.bfloat16, dev, rng)
        gu, dn = experts_from_hf(gate, up, down)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(3):
            experts_from_hf(gate, up, down)
        b.record()
        b.synchronize()
        ms = a.elapsed_time(b) / 3
        nbytes = 2 * 3 * E * I * D * 2
        print(f"expert import E={E} I={I} D={D}: {ms:.3f} ms, {nbytes / ms / 1e6:.0f} GB/s")
        # spot-check against the definition, then the exact round trip
        e, d, i = 3, 1000 % D, 17
        assert gu[e, d, i] == gate[e, i, d] and gu[e, d, I + i] == up[e, i, d] and dn[e, i, d] == down[e, d, i]
        g2, u2, d2 = experts_to_hf(gu, dn)
        assert torch.equal(g2, gate) and torch.equal(u2, up) and torch.equal(d2, down)
        del gate, up, down, gu, dn, g2, u2, d2

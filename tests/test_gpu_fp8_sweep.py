"""GPU parity sweep of the blockwise-fp8 grouped GEMM (the persistent kernel) over seeded random
shapes: expert counts 1-128, uniform / Zipf / ragged-with-empty group sizes, rows past
sum(group_sizes), reductions of 2-24 blocks, per-128-block magnitudes spread over 1e-3 .. 1e3
(the block-to-block rescaling), plain store and SwiGLU + re-quantisation, in both scale modes
(amax/448 and power-of-two); three larger cases give every workgroup more than two tiles, so that
tiles come from the per-XCD ticket counters.  Each case is checked against the
dequantise-then-float64 oracle (1e-2) and the unquantised float64 product (6e-2), and rows past
the groups must be zero."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_err
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _groups(rng, M, E, kind):
    if kind == "uniform":
        gs = np.full(E, M // E)
        gs[: M - gs.sum()] += 1
    elif kind == "zipf":
        p = 1.0 / np.arange(1, E + 1) ** 1.2
        gs = rng.multinomial(M, p[rng.permutation(E)] / p.sum())
    else:
        cut = np.sort(rng.integers(0, M + 1, E - 1))
        gs = np.diff(np.concatenate([[0], cut, [M]]))
        if E > 2:
            gs[1] += gs[2]
            gs[2] = 0
    return gs.astype(np.int32)


def _cases(n=16, seed=77):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        E = int(rng.choice([1, 3, 8, 32, 128]))
        M = int(rng.integers(1, 5000))
        kin = int(rng.choice([256, 384, 512, 768, 1024, 2048, 3072]))
        kout = int(rng.choice([256, 512, 768]))
        kind = str(rng.choice(["uniform", "zipf", "ragged"]))
        past = int(rng.choice([0, 0, 7, 300]))
        swiglu = bool(i % 4 == 3)
        out.append((i, E, M, kin, kout, kind, past, swiglu))
    # many tiles per workgroup (ticketed tiles): 1400-2900 tiles of 256 x 256
    out += [(n, 16, 60000, 512, 1536, "zipf", 7, False), (n + 1, 8, 40000, 768, 2048, "uniform", 0, True),
            (n + 2, 128, 50000, 256, 1536, "ragged", 300, False)]
    return out


def _u8(t):
    return t.view(torch.uint8).cpu().numpy()


@pytest.mark.parametrize("scales", ["amax", "pow2"])
@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"c{c[0]}-E{c[1]}-M{c[2]}-K{c[3]}-N{c[4]}-{c[5]}-p{c[6]}-{'swiglu' if c[7] else 'store'}")
def test_gmm_fp8_sweep(dev, case, scales):
    from mintext_amd.kernels.fp8 import grouped_matmul_fp8, grouped_matmul_fp8_swiglu, quantize_fp8_rows, \
        quantize_fp8_weights

    i, E, M, kin, kout, kind, past, swiglu = case
    rng = np.random.default_rng(300 + i)
    gs = _groups(rng, M, E, kind)
    Mt = M + past
    blk = torch.from_numpy(10.0 ** rng.uniform(-3, 3, (Mt, kin // 128))).float().to(dev)
    x = (torch.randn(Mt, kin, device=dev) * blk.repeat_interleave(128, 1)).bfloat16()
    wblk = torch.from_numpy(10.0 ** rng.uniform(-1, 1, (E, kin // 128, 1))).float().to(dev)
    w = (torch.randn(E, kin, kout, device=dev) * 0.02 * wblk.repeat_interleave(128, 1)).bfloat16()
    f8s = dict(scales=scales)
    xq, xs = quantize_fp8_rows(x, **f8s)
    wq, ws = quantize_fp8_weights(w, **f8s)
    gt = torch.from_numpy(gs).to(dev)
    deq = O.gmm_fp8(_u8(xq), xs.cpu().numpy(), _u8(wq), ws.cpu().numpy(), gs)
    if not swiglu:
        out = grouped_matmul_fp8(xq, xs, wq, ws, gt, **f8s)
        got = out.float().cpu().numpy()
        assert (out[M:] == 0).all(), "rows past sum(group_sizes) must be zero"
        assert rel_err(got, deq) < 1e-2, rel_err(got, deq)
        full = O.gmm(x.float().cpu().numpy(), w.float().cpu().numpy(), gs)
        assert rel_err(got, full) < 6e-2, rel_err(got, full)
    else:
        yq, ys, yb = grouped_matmul_fp8_swiglu(xq, xs, wq, ws, gt, return_bf16=True, **f8s)
        ref = O.swiglu(deq)
        assert rel_err(yb.float().cpu().numpy()[:M], ref[:M]) < 1e-2
        assert (yb[M:] == 0).all() and (_u8(yq)[M:] == 0).all()
        d = O.dequant_rows(_u8(yq), ys.cpu().numpy())
        assert rel_err(d[:M], ref[:M]) < 6e-2


def _cases_tgmm(n=4, seed=8080):
    """fp8 tgmm shapes of 2048 or more 256x256 tiles (the persistent kernel's range on a 256-CU
    part): experts of 0, 1-128 and thousands of rows, and group sizes summing past M."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        E = int(rng.choice([64, 128]))
        F = int(rng.choice([768, 1024, 2048]))
        N = int(rng.choice([1024, 1536, 2048]))
        while E * (F // 256) * (N // 256) < 2048:
            N += 512
        out.append((i, E, F, N, i % 2 == 1))
    return out


@pytest.mark.parametrize("scales", ["amax", "pow2"])
@pytest.mark.parametrize("case", _cases_tgmm(), ids=lambda c: f"t{c[0]}-E{c[1]}-F{c[2]}-N{c[3]}-past{int(c[4])}")
def test_tgmm_fp8_sweep_persistent_every_expert_bits(dev, case, scales):
    """Every expert's dW from the persistent fp8 tgmm has the bits of the same expert quantised and
    computed alone (a one-expert problem of few tiles, on the per-tile kernel); empty experts,
    and experts whose rows all lie past M, are zero."""
    from mintext_amd.kernels.fp8 import quantize_fp8_grouped_t, tgmm_fp8

    i, E, F, N, past = case
    rng = np.random.default_rng(600 + i)
    gs = rng.integers(0, 700, E).astype(np.int32)
    gs[rng.choice(E, E // 8, replace=False)] = 0
    small = rng.choice(np.flatnonzero(gs), 6, replace=False)
    gs[small] = rng.integers(1, 129, 6)
    gs[int(rng.integers(0, E))] = int(rng.integers(3000, 9000))
    M = int(gs.sum()) - (int(gs.sum()) // 10 if past else 0)
    x = torch.randn(M, F, device=dev).bfloat16()
    g = torch.randn(M, N, device=dev).bfloat16()
    tg = torch.from_numpy(gs).to(dev)
    f8s = dict(scales=scales)
    dw = tgmm_fp8(*quantize_fp8_grouped_t(x, tg, **f8s), *quantize_fp8_grouped_t(g, tg, blocks=True, **f8s), tg, M,
                  **f8s)
    off = np.minimum(np.concatenate([[0], np.cumsum(gs)]), M)
    for e in range(E):
        r0, r1 = int(off[e]), int(off[e + 1])
        if r1 == r0:
            assert not dw[e].any(), f"expert {e}"
            continue
        one = torch.tensor([r1 - r0], dtype=torch.int32, device=dev)
        alone = tgmm_fp8(*quantize_fp8_grouped_t(x[r0:r1], one, **f8s),
                         *quantize_fp8_grouped_t(g[r0:r1], one, blocks=True, **f8s), one, r1 - r0, **f8s)
        assert torch.equal(alone[0].view(torch.int16), dw[e].view(torch.int16)), f"expert {e}"

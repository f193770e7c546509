"""GPU parity sweep of the bf16 grouped GEMM over seeded random shapes (forward and dlhs): expert
counts 1-48, uniform / Zipf / ragged-with-empty group sizes, rows past sum(group_sizes), and
reductions on both sides of the persistent kernel's range (Kred <= 1024 runs the persistent
plain-store kernel, longer ones the per-tile kernel with its split tail).  Each case checks the
default schedule against the 128-row tiling (the same f32 sums: bit for bit when no tile is split,
else within a bf16 ulp plus the f32 cancellation error), both against the float64 oracle at
2e-2, and that rows past the groups are zero.  A second seeded set holds groups of 512 rows or
more on average with long reductions (forward, dlhs) and the fused SwiGLU: the shapes of the
one-wave-per-SIMD kernel, with its thin, partial and split-tail tiles."""
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
    else:  # ragged, with an empty group when E > 2
        cut = np.sort(rng.integers(0, M + 1, E - 1))
        gs = np.diff(np.concatenate([[0], cut, [M]]))
        if E > 2:
            gs[1] += gs[2]
            gs[2] = 0
    return gs.astype(np.int32)


def _cases(n=20, seed=2024):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        E = int(rng.choice([1, 2, 5, 8, 16, 48]))
        M = int(rng.integers(1, 3000))
        kred = int(rng.choice([128, 256, 512, 768, 1024, 1280, 2048]))
        nout = int(rng.choice([256, 512, 768]))
        kind = str(rng.choice(["uniform", "zipf", "ragged"]))
        past = int(rng.choice([0, 0, 5, 300]))
        op = "dlhs" if i % 3 == 2 else "fwd"
        out.append((i, E, M, kred, nout, kind, past, op))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"c{c[0]}-E{c[1]}-M{c[2]}-K{c[3]}-N{c[4]}-{c[5]}-p{c[6]}-{c[7]}")
def test_gmm_sweep(dev, case):
    from mintext_amd.kernels.grouped_matmul import _gmm_dlhs, _gmm_fwd

    i, E, M, kred, nout, kind, past, op = case
    rng = np.random.default_rng(100 + i)
    gs = _groups(rng, M, E, kind)
    Mt = M + past
    x = (rng.standard_normal((Mt, kred)) * 0.5).astype(np.float32)
    # forward: w [E, Kred, Nout]; dlhs: w [E, Nout, Kred] (output Nout = Kin, reduction Kred = Kout)
    wshape = (E, kred, nout) if op == "fwd" else (E, nout, kred)
    w = (rng.standard_normal(wshape) * 0.05).astype(np.float32)
    xt = torch.from_numpy(x).to(dev).bfloat16()
    wt = torch.from_numpy(w).to(dev).bfloat16()
    gt = torch.from_numpy(gs).to(dev)
    f = _gmm_fwd if op == "fwd" else _gmm_dlhs
    out = f(xt, wt, gt)
    out128 = f(xt, wt, gt, tiling=(128, 1, 256))
    assert out.shape == (Mt, nout)
    assert (out[M:] == 0).all(), "rows past sum(group_sizes) must be zero"
    xr, wr = xt.float().cpu().numpy(), wt.float().cpu().numpy()
    ref = O.gmm(xr, wr, gs) if op == "fwd" else O.gmm_dlhs(xr, wr, gs)
    for o in (out, out128):
        got = o.float().cpu().numpy()
        assert rel_err(got, ref) < 2e-2, rel_err(got, ref)
    if kred <= 1024:  # persistent kernel: whole tiles, the sums of the 128-row tiling bit for bit
        assert torch.equal(out, out128)
    else:
        d = (out.float() - out128.float()).abs()
        bound = out128.float().abs() * 2.0 ** -7 + 1e-5 * float(np.abs(ref).max() if ref.size else 1.0)
        assert bool((d <= bound).all()), (d - bound).max().item()


def _cases_large(n=12, seed=4242):
    """Shapes on the one-wave-per-SIMD kernel's side of the dispatch: groups of 512 rows or more
    on average, reductions past the persistent kernel's 1024 (forward, dlhs) and any reduction
    for the fused SwiGLU (which always takes that kernel at this mean)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        op = ("fwd", "dlhs", "swiglu")[i % 3]
        E = int(rng.choice([1, 2, 3, 4, 6, 8]))
        M = E * int(rng.integers(512, 2400)) + int(rng.integers(0, 256))
        kred = int(rng.choice([512, 768, 1152, 2304] if op == "swiglu" else [1056, 1152, 1536, 2048, 2304, 3072]))
        nout = int(rng.choice([256, 512, 768, 1024, 1536]))
        kind = str(rng.choice(["uniform", "zipf", "ragged"]))
        past = int(rng.choice([0, 7, 256]))
        out.append((i, E, M, kred, nout, kind, past, op))
    return out


@pytest.mark.parametrize("case", _cases_large(), ids=lambda c: f"c{c[0]}-E{c[1]}-M{c[2]}-K{c[3]}-N{c[4]}-{c[5]}-p{c[6]}-{c[7]}")
def test_gmm_sweep_large_groups(dev, case):
    from mintext_amd.kernels.grouped_matmul import _gmm_dlhs, _gmm_fwd, grouped_matmul_swiglu

    i, E, M, kred, nout, kind, past, op = case
    rng = np.random.default_rng(500 + i)
    gs = _groups(rng, M, E, kind)
    Mt = M + past
    x = (rng.standard_normal((Mt, kred)) * 0.5).astype(np.float32)
    wshape = (E, nout, kred) if op == "dlhs" else (E, kred, nout)
    w = (rng.standard_normal(wshape) * 0.05).astype(np.float32)
    xt = torch.from_numpy(x).to(dev).bfloat16()
    wt = torch.from_numpy(w).to(dev).bfloat16()
    gt = torch.from_numpy(gs).to(dev)
    f = {"fwd": _gmm_fwd, "dlhs": _gmm_dlhs}.get(op)
    if f is None:
        out = grouped_matmul_swiglu(xt, wt, gt)
        out128 = grouped_matmul_swiglu(xt, wt, gt, tiling=(128, 1, 256))
    else:
        out = f(xt, wt, gt)
        out128 = f(xt, wt, gt, tiling=(128, 1, 256))
    ncols = nout // 2 if op == "swiglu" else nout
    assert out.shape == (Mt, ncols)
    assert (out[M:] == 0).all(), "rows past sum(group_sizes) must be zero"
    xr, wr = xt.float().cpu().numpy(), wt.float().cpu().numpy()
    if op == "dlhs":
        ref = O.gmm_dlhs(xr, wr, gs)
    else:
        ref = O.gmm(xr, wr, gs)
        if op == "swiglu":
            ref = O.swiglu(ref)
    for o in (out, out128):
        got = o.float().cpu().numpy()
        assert rel_err(got[:M], ref[:M]) < 2e-2, rel_err(got[:M], ref[:M])
    if op == "swiglu":  # whole tiles (no split tail on this path): the 128-row tiling's bits
        assert torch.equal(out, out128)
    else:
        d = (out.float() - out128.float()).abs()
        bound = out128.float().abs() * 2.0 ** -7 + 1e-5 * float(np.abs(ref).max())
        assert bool((d <= bound).all()), (d - bound).max().item()


def _cases_tgmm(n=6, seed=9090):
    """tgmm shapes of 2048 or more 256x256 tiles (the persistent kernel's range on a 256-CU part):
    experts of 0, 1-95 and thousands of rows, and group sizes summing past M."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        E = int(rng.choice([64, 96, 128]))
        K = int(rng.choice([768, 1024, 2048]))
        N = int(rng.choice([1024, 1536, 2048]))
        while E * (K // 256) * (N // 256) < 2048:
            N += 512
        past = i % 3 == 2
        out.append((i, E, K, N, past))
    return out


@pytest.mark.parametrize("case", _cases_tgmm(), ids=lambda c: f"t{c[0]}-E{c[1]}-K{c[2]}-N{c[3]}-past{int(c[4])}")
def test_tgmm_sweep_persistent_every_expert_bits(dev, case):
    """Every expert's dW from the persistent tgmm has the bits of the same expert computed alone
    (a one-expert problem of few tiles, on the per-tile kernel); empty experts are zero."""
    from mintext_amd.kernels import tgmm

    i, E, K, N, past = case
    rng = np.random.default_rng(500 + i)
    gs = rng.integers(0, 600, E).astype(np.int32)
    gs[rng.choice(E, E // 8, replace=False)] = 0
    small = rng.choice(np.flatnonzero(gs), 6, replace=False)
    gs[small] = rng.integers(1, 96, 6)
    gs[int(rng.integers(0, E))] = int(rng.integers(3000, 9000))
    M = int(gs.sum()) - (int(gs.sum()) // 10 if past else 0)
    x = torch.randn(M, K, device=dev).bfloat16()
    g = torch.randn(M, N, device=dev).bfloat16()
    out = tgmm(x, g, torch.from_numpy(gs).to(dev))
    off = np.minimum(np.concatenate([[0], np.cumsum(gs)]), M)
    for e in range(E):
        r0, r1 = int(off[e]), int(off[e + 1])
        if r1 == r0:
            assert not out[e].any(), f"expert {e}"
            continue
        alone = tgmm(x[r0:r1], g[r0:r1], torch.tensor([r1 - r0], dtype=torch.int32, device=dev))
        assert torch.equal(alone[0].view(torch.int16), out[e].view(torch.int16)), f"expert {e}"

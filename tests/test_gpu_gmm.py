"""GPU parity: grouped GEMM forward / fused SwiGLU / dlhs / tgmm (HIP) vs the oracle.

Tolerances (north star): fp32 path 1e-5 relative against float64; bf16 path 2e-2 relative
against a float64 reference computed from the same bf16-rounded operands.  Shapes cover the
reference tests (tests/test_moe_kernels.py:140-490) on the exact-fp32 path, and the MFMA
tilings (256- and 128-row tiles, 256- and 128-column tiles) with ragged, empty and skewed
groups on the bf16 path.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden, rel_err, tile_list_workspace_bytes
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def _close(got, ref, rtol):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert rel_err(got, ref) < rtol, rel_err(got, ref)
    scale = np.abs(ref).max() if ref.size else 1.0
    np.testing.assert_allclose(got, ref, rtol=rtol, atol=rtol * scale)


# --------------------------------------------------------------------- exact fp32 fixtures
def test_gmm_fp32_golden(dev):
    from mintext_amd.kernels import grouped_matmul, grouped_matmul_vjp, tgmm

    g = golden("gmm")
    for n in sorted({k.split("__")[0] for k in g.files}):
        gs, x, w, gr = g[f"{n}__gs"], g[f"{n}__x"], g[f"{n}__w"], g[f"{n}__g"]
        out = grouped_matmul(_t(x, dev), _t(w, dev), _t(gs, dev))
        _close(out.cpu().numpy(), g[f"{n}__out"], 1e-5)
        out2 = grouped_matmul_vjp(_t(x, dev), _t(w, dev), _t(gs, dev), tiling=(64, 64, 64))
        assert torch.equal(out, out2)
        tg = tgmm(_t(x, dev), _t(gr, dev), _t(gs, dev))
        _close(tg.cpu().numpy(), g[f"{n}__tgmm"], 1e-5)
        empty = np.flatnonzero(gs == 0)
        assert (tg[torch.from_numpy(empty).to(dev)] == 0).all()
        xt = _t(x, dev).requires_grad_(True)
        wt = _t(w, dev).requires_grad_(True)
        grouped_matmul_vjp(xt, wt, _t(gs, dev)).backward(_t(gr, dev))
        _close(xt.grad.cpu().numpy(), g[f"{n}__dlhs"], 1e-5)
        _close(wt.grad.cpu().numpy(), g[f"{n}__tgmm"], 1e-5)


def test_gmm_rows_past_group_sum_are_zero(dev):
    from mintext_amd.kernels import grouped_matmul

    x = torch.randn(300, 64, device=dev)
    w = torch.randn(3, 64, 32, device=dev)
    gs = torch.tensor([100, 0, 150], dtype=torch.int32, device=dev)
    out = grouped_matmul(x, w, gs)
    assert (out[250:] == 0).all()
    xb, wb = x.bfloat16(), torch.randn(3, 64, 256, device=dev).bfloat16()
    outb = grouped_matmul(xb, wb, gs)
    assert (outb[250:] == 0).all()
    _close(outb[:250].float().cpu().numpy(), O.gmm(xb.float().cpu().numpy(), wb.float().cpu().numpy(), [100, 0, 150])[:250],
           2e-2)


def test_gmm_finite_difference(dev):
    """tests/test_moe_kernels.py:209-231,358-403 (dx and dW by central differences)."""
    from mintext_amd.kernels import grouped_matmul_vjp

    torch.manual_seed(0)
    x = torch.randn(8, 4, device=dev, dtype=torch.float32)
    w = torch.randn(2, 4, 4, device=dev)
    gs = torch.tensor([4, 4], dtype=torch.int32, device=dev)
    xg = x.clone().requires_grad_(True)
    wg = w.clone().requires_grad_(True)
    grouped_matmul_vjp(xg, wg, gs).sum().backward()
    eps = 1e-3
    for i in range(4):
        for j in range(4):
            xp, xm = x.clone(), x.clone()
            xp[i, j] += eps
            xm[i, j] -= eps
            num = (grouped_matmul_vjp(xp, w, gs).sum() - grouped_matmul_vjp(xm, w, gs).sum()).item() / (2 * eps)
            np.testing.assert_allclose(xg.grad[i, j].item(), num, rtol=0.02, atol=1e-4)
    for e in range(2):
        for i in range(2):
            for j in range(2):
                wp, wm = w.clone(), w.clone()
                wp[e, i, j] += eps
                wm[e, i, j] -= eps
                num = (grouped_matmul_vjp(x, wp, gs).sum() - grouped_matmul_vjp(x, wm, gs).sum()).item() / (2 * eps)
                np.testing.assert_allclose(wg.grad[e, i, j].item(), num, rtol=0.02, atol=1e-4)


# ----------------------------------------------------------------------------- bf16 MFMA
def _groups(rng, M, E, kind):
    if kind == "uniform":
        gs = np.full(E, M // E)
        gs[: M - gs.sum()] += 1
    elif kind == "skew":
        p = 1.0 / np.arange(1, E + 1) ** 1.2
        p = p[rng.permutation(E)]
        gs = rng.multinomial(M, p / p.sum())
        gs[rng.integers(0, E)] = 0
        gs[0] += M - gs.sum()
    else:  # ragged with empties
        cut = np.sort(rng.integers(0, M + 1, E - 1))
        gs = np.diff(np.concatenate([[0], cut, [M]]))
        gs[1] = gs[1] + gs[2]
        gs[2] = 0
    return gs.astype(np.int32)


BF16_SHAPES = [
    # (M, E, Kin, Kout, groups)  -- tiles: M/E >= 192 -> 256-row tiles, else 128-row
    (2048, 4, 256, 512, "uniform"),
    (2048, 8, 128, 768, "ragged"),
    (1500, 16, 192, 256, "skew"),
    (640, 8, 64, 384, "ragged"),  # Kout % 256 != 0 -> 128-column tiles
    (96, 3, 64, 256, "ragged"),
]


@pytest.mark.parametrize("M,E,Kin,Kout,kind", BF16_SHAPES)
def test_gmm_bf16_mfma(dev, M, E, Kin, Kout, kind):
    from mintext_amd.kernels import grouped_matmul
    from mintext_amd.kernels.grouped_matmul import _gmm_dlhs

    rng = np.random.default_rng(M + Kin)
    gs = _groups(rng, M, E, kind)
    x = torch.randn(M, Kin, device=dev).bfloat16()
    w = (torch.randn(E, Kin, Kout, device=dev) * 0.05).bfloat16()
    out = grouped_matmul(x, w, _t(gs, dev))
    assert out.dtype == torch.bfloat16
    xr, wr = x.float().cpu().numpy(), w.float().cpu().numpy()
    _close(out.float().cpu().numpy(), O.gmm(xr, wr, gs), 2e-2)
    # dlhs (reduction over Kout; output Kin columns)
    gr = torch.randn(M, Kout, device=dev).bfloat16()
    dx = _gmm_dlhs(gr, w, _t(gs, dev))
    _close(dx.float().cpu().numpy(), O.gmm_dlhs(gr.float().cpu().numpy(), wr, gs), 2e-2)


def test_gmm_short_last_tiles(dev):
    """Groups of whole 256-row tiles plus a last tile of 1..128 rows (and single, empty and
    one-row groups): every row computed once, for the forward, the fused SwiGLU and dlhs."""
    from mintext_amd.kernels import grouped_matmul, grouped_matmul_swiglu
    from mintext_amd.kernels.grouped_matmul import _gmm_dlhs

    gs = np.array([257, 287, 544, 356, 383, 384, 200, 0, 1, 2049], np.int32)  # tails 1..127, 128, single
    M, E, Kin, Kout = int(gs.sum()), len(gs), 128, 512
    x = torch.randn(M, Kin, device=dev).bfloat16()
    w = (torch.randn(E, Kin, Kout, device=dev) * 0.05).bfloat16()
    xr, wr = x.float().cpu().numpy(), w.float().cpu().numpy()
    ref = O.gmm(xr, wr, gs)
    out = grouped_matmul(x, w, _t(gs, dev)).float().cpu().numpy()
    _close(out, ref, 2e-2)
    # per-row check: a dropped or doubly written row would show as a row-wise outlier
    row_err = np.abs(out - ref).max(1) / (np.abs(ref).max(1) + 1e-6)
    assert row_err.max() < 5e-2, int(np.argmax(row_err))
    y = grouped_matmul_swiglu(x, w, _t(gs, dev)).float().cpu().numpy()
    _close(y, O.swiglu(ref), 2e-2)
    gr = torch.randn(M, Kout, device=dev).bfloat16()
    dx = _gmm_dlhs(gr, w, _t(gs, dev))
    _close(dx.float().cpu().numpy(), O.gmm_dlhs(gr.float().cpu().numpy(), wr, gs), 2e-2)


@pytest.mark.parametrize("M,E,Kin,I,kind", [(2048, 4, 256, 256, "uniform"), (1000, 8, 128, 384, "ragged"),
                                            (300, 5, 64, 128, "skew")])
def test_gmm_swiglu_fused(dev, M, E, Kin, I, kind):
    from mintext_amd.kernels import grouped_matmul_swiglu

    rng = np.random.default_rng(I + M)
    gs = _groups(rng, M, E, kind)
    for dt, tol in ((torch.bfloat16, 2e-2), (torch.float32, 1e-5)):
        x = torch.randn(M, Kin, device=dev).to(dt)
        w = (torch.randn(E, Kin, 2 * I, device=dev) * 0.1).to(dt)
        y = grouped_matmul_swiglu(x, w, _t(gs, dev))
        ref = O.swiglu(O.gmm(x.float().cpu().numpy(), w.float().cpu().numpy(), gs))
        _close(y.float().cpu().numpy(), ref, tol)


@pytest.mark.parametrize("M,E,K,N,kind", [(2048, 4, 256, 512, "uniform"), (1700, 8, 128, 256, "skew"),
                                          (900, 6, 256, 128, "ragged"),
                                          # 256x256 direct-to-LDS path: ragged tails, empty groups
                                          (1000, 8, 512, 256, "ragged"), (5000, 16, 256, 768, "skew"),
                                          (333, 3, 256, 256, "ragged")])
def test_tgmm_bf16_mfma(dev, M, E, K, N, kind):
    from mintext_amd.kernels import tgmm

    rng = np.random.default_rng(K + N + M)
    gs = _groups(rng, M, E, kind)
    x = torch.randn(M, K, device=dev).bfloat16()
    g = torch.randn(M, N, device=dev).bfloat16()
    out = tgmm(x, g, _t(gs, dev))
    ref = O.tgmm(x.float().cpu().numpy(), g.float().cpu().numpy(), gs)
    _close(out.float().cpu().numpy(), ref, 2e-2)
    for e in np.flatnonzero(gs == 0):
        assert (out[int(e)] == 0).all()


@pytest.mark.parametrize("past_m", [False, True])
def test_tgmm_bf16_persistent_matches_per_tile(dev, past_m):
    """2048 tiles (E=64, 2048 x 1024 per expert) take the persistent tgmm, whose ring runs across
    tiles and restarts around experts of fewer than three 32-row stages: empty experts (and, with
    group sizes summing past M, experts whose rows are all dropped) give zeros, the result is
    within 2e-2 of float64, and each checked expert's dW has the bits of the same expert computed
    alone (a one-expert problem of 32 tiles, which takes the per-tile kernel)."""
    from mintext_amd.kernels import tgmm

    E, K, N = 64, 2048, 1024
    rng = np.random.default_rng(64)
    gs = rng.integers(0, 400, E).astype(np.int32)
    gs[::9] = 0
    gs[[1, 2, 4, 6, 8]] = [1, 32, 33, 64, 95]  # one, one, two, two and three stages
    gs[3] = 2500                               # a long tile early in the order
    M = int(gs.sum()) - (3000 if past_m else 0)
    x = torch.randn(M, K, device=dev).bfloat16()
    g = torch.randn(M, N, device=dev).bfloat16()
    out = tgmm(x, g, _t(gs, dev))
    off = np.minimum(np.concatenate([[0], np.cumsum(gs)]), M)
    rows = off[1:] - off[:-1]
    assert past_m == bool((rows < gs).any())
    for e in np.flatnonzero(rows == 0):
        assert (out[int(e)] == 0).all()
    ref = O.tgmm(x.float().cpu().numpy(), g.float().cpu().numpy(), rows.astype(np.int32))
    _close(out.float().cpu().numpy(), ref, 2e-2)
    for e in (1, 2, 3, 4, 6, 8, int(np.flatnonzero(rows)[-1])):
        r0, r1 = int(off[e]), int(off[e + 1])
        alone = tgmm(x[r0:r1], g[r0:r1], _t(np.array([r1 - r0], np.int32), dev))
        assert torch.equal(alone[0].view(torch.int16), out[e].view(torch.int16)), f"expert {e}"


def test_gmm_bf16_sampled_mixtral_shape(dev):
    """C2 gate_up shape (M=16384, Kin=4096, Kout=28672, E=8): sampled rows/columns vs float64."""
    from mintext_amd.kernels import grouped_matmul_swiglu

    M, E, D, I = 16384, 8, 4096, 14336
    rng = np.random.default_rng(2)
    gs = _groups(rng, M, E, "uniform")
    gs[3] += 37
    gs[5] -= 37
    x = torch.randn(M, D, device=dev).bfloat16()
    w = (torch.randn(E, D, 2 * I, device=dev) * 0.02).bfloat16()
    y = grouped_matmul_swiglu(x, w, _t(gs, dev))
    off = np.concatenate([[0], np.cumsum(gs)])
    rows = np.sort(rng.choice(M, 48, replace=False))
    cols = np.sort(rng.choice(I, 40, replace=False))
    xs = x[torch.from_numpy(rows).to(dev)].float().cpu().numpy().astype(np.float64)
    ref = np.empty((rows.size, cols.size))
    for i, r in enumerate(rows):
        e = int(np.searchsorted(off, r, side="right") - 1)
        we = w[e].float()
        gate = we[:, torch.from_numpy(cols).to(dev)].cpu().numpy().astype(np.float64)
        up = we[:, torch.from_numpy(cols + I).to(dev)].cpu().numpy().astype(np.float64)
        ref[i] = O.silu(xs[i] @ gate) * (xs[i] @ up)
    got = y[torch.from_numpy(rows).to(dev)][:, torch.from_numpy(cols).to(dev)].float().cpu().numpy()
    _close(got, ref, 2e-2)


def test_gmm_bf16_sampled_deepseek_shape(dev):
    """C3 shapes (E=256, ~128 rows per expert): gate_up+SwiGLU and down, sampled rows vs float64."""
    from mintext_amd.kernels import grouped_matmul, grouped_matmul_swiglu

    M, E, D, I = 32768, 256, 7168, 2048
    rng = np.random.default_rng(3)
    gs = rng.multinomial(M, np.full(E, 1.0 / E)).astype(np.int32)
    gs[7] = 0
    gs[8] += M - gs.sum()
    x = torch.randn(M, D, device=dev).bfloat16()
    wgu = (torch.randn(E, D, 2 * I, device=dev) * 0.006).bfloat16()
    y = grouped_matmul_swiglu(x, wgu, _t(gs, dev))
    wd = (torch.randn(E, I, D, device=dev) * 0.006).bfloat16()
    o = grouped_matmul(y, wd, _t(gs, dev))
    off = np.concatenate([[0], np.cumsum(gs)])
    rows = np.sort(rng.choice(M, 24, replace=False))
    cols = np.sort(rng.choice(I, 32, replace=False))
    ocols = np.sort(rng.choice(D, 32, replace=False))
    tc, toc = torch.from_numpy(cols).to(dev), torch.from_numpy(ocols).to(dev)
    ref_y = np.empty((rows.size, cols.size))
    ref_o = np.empty((rows.size, ocols.size))
    for i, r in enumerate(rows):
        e = int(np.searchsorted(off, r, side="right") - 1)
        xr = x[int(r)].double().cpu().numpy()
        gate = wgu[e][:, tc].double().cpu().numpy()
        up = wgu[e][:, tc + I].double().cpu().numpy()
        ref_y[i] = O.silu(xr @ gate) * (xr @ up)
        ref_o[i] = y[int(r)].double().cpu().numpy() @ wd[e][:, toc].double().cpu().numpy()
    tr = torch.from_numpy(rows).to(dev)
    _close(y[tr][:, tc].float().cpu().numpy(), ref_y, 2e-2)
    _close(o[tr][:, toc].float().cpu().numpy(), ref_o, 2e-2)


def test_tgmm_bf16_sampled_qwen3_shape(dev):
    """C5 tgmm shape (M=131072, K=2048, N=1536, E=128, Zipf-skewed groups): sampled blocks vs float64."""
    from mintext_amd.kernels import tgmm

    M, E, K, N = 131072, 128, 2048, 1536
    rng = np.random.default_rng(5)
    gs = _groups(rng, M, E, "skew")
    x = torch.randn(M, K, device=dev).bfloat16()
    g = torch.randn(M, N, device=dev).bfloat16()
    out = tgmm(x, g, _t(gs, dev))
    off = np.concatenate([[0], np.cumsum(gs)])
    experts = [int(np.argmax(gs)), int(np.argmin(gs)), int(rng.integers(0, E)), int(rng.integers(0, E))]
    ks = np.sort(rng.choice(K, 24, replace=False))
    ns = np.sort(rng.choice(N, 24, replace=False))
    for e in experts:
        r0, r1 = int(off[e]), int(off[e + 1])
        xs = x[r0:r1][:, torch.from_numpy(ks).to(dev)].float().cpu().numpy().astype(np.float64)
        gsm = g[r0:r1][:, torch.from_numpy(ns).to(dev)].float().cpu().numpy().astype(np.float64)
        ref = xs.T @ gsm
        got = out[e][torch.from_numpy(ks).to(dev)][:, torch.from_numpy(ns).to(dev)].float().cpu().numpy()
        if r1 == r0:
            assert (got == 0).all()
        else:
            _close(got, ref, 2e-2)


# --------------------------------------------------------------- split tail (256-row tiles)
SPLIT_SHAPES = [
    # (group sizes, Kin, Kout): per-XCD tile counts whose last round is sparse, so the tail
    # tiles run as k-pieces: 8 x 2080 rows, 1 n-tile -> 9 tiles per XCD, each in 3 pieces;
    # 4 groups of ~9.5k rows (one empty), 2 n-tiles -> 37 tiles per XCD, the last 5 in 4 pieces
    ([2080] * 8, 1024, 256),
    ([9472, 0, 9500, 9444 + 9472], 256, 512),
    ([300, 5, 257, 0, 1], 2048, 256),
]


@pytest.mark.parametrize("op", ["fwd", "dlhs"])
@pytest.mark.parametrize("gs,Kin,Kout", SPLIT_SHAPES)
def test_gmm_split_tail_matches_whole_tiles(dev, gs, Kin, Kout, op):
    """The split tail (full workspace) against whole tiles (workspace without the partials
    region) and the float64 oracle: same values to bf16 rounding, deterministic bits."""
    from mintext_amd import _lib as L

    rng = np.random.default_rng(len(gs) + Kin)
    gs = np.asarray(gs, np.int32)
    M, E = int(gs.sum()) + 7, len(gs)  # 7 rows past the groups -> zeros
    if op == "fwd":
        x = rng.standard_normal((M, Kin)).astype(np.float32)
        w = (rng.standard_normal((E, Kin, Kout)) * 0.05).astype(np.float32)
        n_red, n_out = Kin, Kout
    else:  # dx = g @ w^T: the reduction runs over Kout
        x = rng.standard_normal((M, Kout)).astype(np.float32)
        w = (rng.standard_normal((E, Kin, Kout)) * 0.05).astype(np.float32)
        n_red, n_out = Kout, Kin
    xb, wb = _t(x, dev, torch.bfloat16), _t(w, dev, torch.bfloat16)
    g = _t(gs, dev)
    full = L.query("mtx_gmm_workspace_size", M, E)
    st = L.stream(dev)
    name = "mtx_gmm" if op == "fwd" else "mtx_gmm_dlhs"

    def run(ws_bytes):
        ws = L.workspace(full, dev)
        out = torch.full((M, n_out), float("nan"), dtype=torch.bfloat16, device=dev)
        L.call(name, xb.data_ptr(), wb.data_ptr(), g.data_ptr(), L.dtype_code(torch.bfloat16), M, Kin, Kout, E,
               out.data_ptr(), ws.data_ptr(), ws_bytes, st)
        torch.cuda.synchronize()
        return out

    split, split2 = run(full), run(full)
    whole = run(full - (64 << 20))  # tile lists only: every tile runs whole
    assert torch.equal(split, split2)
    xf, wf = xb.float().cpu().numpy(), wb.float().cpu().numpy()
    ref = O.gmm(xf, wf, gs) if op == "fwd" else O.gmm_dlhs(xf, wf, gs)
    assert ref.shape == (M, n_out) and n_red > 0
    for out in (split, whole):
        assert (out[int(gs.sum()):] == 0).all()
        _close(out.float().cpu().numpy(), ref, 2e-2)
    # both round f32 sums of the same products, added in another order: a bf16 ulp apart at
    # most, plus the f32 summation error where the sum cancels
    d = (split.float() - whole.float()).abs()
    bound = whole.float().abs() * 2.0 ** -7 + 1e-5 * float(np.abs(ref).max())
    assert (d <= bound).all(), (d - bound).max().item()


@pytest.mark.parametrize("dtype,M", [("bf16", 300_000), ("f32", 70_000)])
def test_gmm_more_zero_tiles_than_threads(dev, dtype, M):
    """Rows past sum(group_sizes) spanning more zero tiles than the tile builder's 1024 threads
    (256-row tiles on the bf16 path, 64-row tiles on the f32 path) all come out as zeros."""
    from mintext_amd.kernels import grouped_matmul, tgmm
    from mintext_amd.kernels.grouped_matmul import _gmm_dlhs

    cdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    gs = np.array([100, 0, 57], np.int32)
    x = torch.randn(M, 64, device=dev).to(cdt)
    w = (torch.randn(3, 64, 256, device=dev) * 0.1).to(cdt)
    g = _t(gs, dev)
    out = grouped_matmul(x, w, g)
    assert (out[157:] == 0).all()
    tol = 2e-2 if dtype == "bf16" else 1e-5
    _close(out[:157].float().cpu().numpy(), O.gmm(x[:157].float().cpu().numpy(), w.float().cpu().numpy(), gs)[:157], tol)
    dy = torch.randn(M, 256, device=dev).to(cdt)
    dx = _gmm_dlhs(dy, w, g, None)
    assert (dx[157:] == 0).all()
    dw = tgmm(x, dy, g)
    ref = O.tgmm(x[:157].float().cpu().numpy(), dy[:157].float().cpu().numpy(), gs)
    _close(dw.float().cpu().numpy(), ref, tol)


def test_gmm_group_sizes_past_m_are_clipped(dev):
    """Group sizes summing past M (up to INT32_MAX) keep the first M rows: the oracle's
    cumulative offsets clipped to M."""
    from mintext_amd.kernels import grouped_matmul

    M = 600
    gs = np.array([2**31 - 1, 5, 7], np.int32)
    for cdt, tol in ((torch.bfloat16, 2e-2), (torch.float32, 1e-5)):
        x = torch.randn(M, 64, device=dev).to(cdt)
        w = (torch.randn(3, 64, 256, device=dev) * 0.1).to(cdt)
        out = grouped_matmul(x, w, _t(gs, dev))
        _close(out.float().cpu().numpy(), O.gmm(x.float().cpu().numpy(), w.float().cpu().numpy(), gs), tol)


@pytest.mark.parametrize("T,K,E,D,I", [(512, 2, 8, 256, 256), (1000, 8, 64, 512, 128), (300, 3, 5, 128, 384)])
def test_gmm_swiglu_gathered_equals_route_then_gmm(dev, T, K, E, D, I):
    """The route's row gather inside the gate_up GEMM's operand loads gives the bits of
    route + grouped_matmul_swiglu, and route_indices the route's permutation and sizes."""
    from mintext_amd.kernels import route
    from mintext_amd.kernels.grouped_matmul import grouped_matmul_swiglu, grouped_matmul_swiglu_gathered
    from mintext_amd.kernels.moe_dispatch import route_indices

    rng = np.random.default_rng(T + E)
    idx = _t(rng.integers(0, E, (T, K)).astype(np.int32), dev)
    x = torch.randn(T, D, device=dev).bfloat16()
    w = (torch.randn(E, D, 2 * I, device=dev) * 0.05).bfloat16()
    st, si, gs = route(x, idx, E)
    si2, gs2, inv2 = route_indices(idx, E)
    assert torch.equal(si, si2) and torch.equal(gs, gs2)
    assert torch.equal(inv2.long(), torch.argsort(si2.long()))
    from mintext_amd.kernels.moe_dispatch import _inverse_of

    assert _inverse_of(si2) is inv2  # the combine reuses the route's inverse
    ref = grouped_matmul_swiglu(st, w, gs)
    out = grouped_matmul_swiglu_gathered(x, si2, K, w, gs2)
    assert torch.equal(out, ref)


def test_gmm_gathered_fwd_op_and_unsupported_shapes(dev):
    """mtx_gmm_gathered's plain forward op equals grouped_matmul on the routed rows: bit for bit
    with a tile-list workspace (every tile whole, as in grouped_matmul's persistent kernel for this
    short reduction), within one bf16 rounding with the full workspace (whose split tail sums a
    tile's k-pieces in another association); shapes outside the direct-to-LDS kernels are refused
    with MTX_ERR_UNSUPPORTED."""
    from mintext_amd import _lib as L
    from mintext_amd.kernels import grouped_matmul, route
    from mintext_amd.kernels.grouped_matmul import grouped_matmul_swiglu_gathered
    from mintext_amd.kernels.moe_dispatch import route_indices

    T, K, E, D, N = 700, 2, 6, 256, 512
    rng = np.random.default_rng(5)
    idx = _t(rng.integers(0, E, (T, K)).astype(np.int32), dev)
    x = torch.randn(T, D, device=dev).bfloat16()
    w = (torch.randn(E, D, N, device=dev) * 0.05).bfloat16()
    st, si, gs = route(x, idx, E)
    ref = grouped_matmul(st, w, gs)
    M = T * K
    for ws_bytes in (tile_list_workspace_bytes(M, E), L.query("mtx_gmm_workspace_size", M, E)):
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        ws = L.workspace(ws_bytes, dev)
        L.call("mtx_gmm_gathered", L.MTX_GMM_OP_FWD, L.ptr(x), T, L.ptr(si), K, L.ptr(w), L.ptr(gs),
               L.dtype_code(torch.bfloat16), M, D, N, E, 0, 0, L.ptr(out), L.ptr(ws), ws.numel(), L.stream(dev))
        if ws_bytes == tile_list_workspace_bytes(M, E):
            assert torch.equal(out, ref)
        else:  # a bf16 ulp apart at most, plus the f32 summation error where the sum cancels
            bound = ref.float().abs() * 2.0 ** -7 + 1e-5 * float(ref.float().abs().max())
            assert bool(((out.float() - ref.float()).abs() <= bound).all())
    for tiling in ((128, 2, 256), (256, 1, 256)):  # explicit tilings (the autotuner's space)
        from mintext_amd.kernels.grouped_matmul import grouped_matmul_swiglu

        wg = (torch.randn(E, D, 2 * 128, device=dev) * 0.05).bfloat16()
        si3, gs3, _ = route_indices(idx, E)
        got = grouped_matmul_swiglu_gathered(x, si3, K, wg, gs3, tiling=tiling)
        assert torch.equal(got, grouped_matmul_swiglu(st, wg, gs, tiling=tiling)), tiling
    si2, gs2, _ = route_indices(idx, E)
    w_odd = (torch.randn(E, D, 2 * 64, device=dev) * 0.05).bfloat16()  # I = 64: not a 128 multiple
    with pytest.raises(L.MtxError) as ei:
        grouped_matmul_swiglu_gathered(x, si2, K, w_odd, gs2)
    assert ei.value.status == L.MTX_ERR_UNSUPPORTED
    xf = torch.randn(T, D, device=dev)  # f32 tokens: no gathered path
    with pytest.raises(L.MtxError) as ei:
        grouped_matmul_swiglu_gathered(xf, si2, K, w.float()[:, :, :256].contiguous(), gs2)
    assert ei.value.status == L.MTX_ERR_UNSUPPORTED


def test_gathered_paths_on_empty_inputs(dev):
    """No tokens: the permutation-only route and both gathered GEMMs return empty results."""
    from mintext_amd.kernels.fp8 import grouped_matmul_fp8_swiglu_gathered, quantize_fp8_rows, quantize_fp8_weights
    from mintext_amd.kernels.grouped_matmul import grouped_matmul_swiglu_gathered
    from mintext_amd.kernels.moe_dispatch import route_indices

    E, K, D, I = 4, 2, 256, 128
    idx = torch.zeros(0, K, dtype=torch.int32, device=dev)
    si, gs, inv = route_indices(idx, E)
    assert si.numel() == 0 and inv.numel() == 0 and gs.cpu().tolist() == [0] * E
    x = torch.zeros(0, D, device=dev).bfloat16()
    w = torch.randn(E, D, 2 * I, device=dev).bfloat16()
    assert grouped_matmul_swiglu_gathered(x, si, K, w, gs).shape == (0, I)
    xq, xs = quantize_fp8_rows(x)
    wq, wsc = quantize_fp8_weights(w)
    yq, ys = grouped_matmul_fp8_swiglu_gathered(xq, xs, si, K, wq, wsc, gs)
    assert yq.shape == (0, I) and ys.shape == (0, 1)
    from mintext_amd.kernels import route
    from mintext_amd.moe import moe_experts_forward

    st, si0, gs0 = route(x, idx, E)
    assert st.shape == (0, D) and si0.numel() == 0 and gs0.cpu().tolist() == [0] * E
    down = torch.randn(E, I, D, device=dev).bfloat16()
    out = moe_experts_forward(x, idx, torch.zeros(0, K, device=dev), w, down)
    assert out.shape == (0, D)



def test_gmm_bf16_operand_beyond_32bit_offsets(dev):
    """An A operand of 4 GiB (2^21 rows x 1024 bf16): byte offsets past 32 bits take the
    register-staged MFMA kernel; sampled rows of every group against float64."""
    from mintext_amd.kernels import grouped_matmul

    M, Kin, Kout, E = 1 << 21, 1024, 256, 3
    gs = np.array([700001, 0, M - 700001], np.int32)
    x = torch.empty(M, Kin, dtype=torch.bfloat16, device=dev)
    x.normal_()
    w = (torch.randn(E, Kin, Kout, device=dev) * 0.03).bfloat16()
    out = grouped_matmul(x, w, _t(gs, dev))
    rng = np.random.default_rng(9)
    rows = np.unique(np.concatenate([[0, 700000, 700001, M - 1], rng.integers(0, M, 40)]))
    off = np.concatenate([[0], np.cumsum(gs)])
    tr = torch.from_numpy(rows).to(dev)
    xs = x[tr].double().cpu().numpy()
    got = out[tr].double().cpu().numpy()
    ref = np.stack([xs[i] @ w[int(np.searchsorted(off, r, side="right") - 1)].double().cpu().numpy()
                    for i, r in enumerate(rows)])
    _close(got, ref, 2e-2)
    del x, out
    torch.cuda.empty_cache()

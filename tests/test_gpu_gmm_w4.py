"""GPU parity of the one-wave-per-SIMD grouped GEMM (the 256-row tile path for groups that average
at least 512 rows): every tile form it has -- whole 256-row tiles, partial tiles of 129-255 rows
(full form, rows past the group masked), thin tiles of 1-128 rows (1-4 row blocks), split-tail
pieces, zero tiles for rows past the groups and (SwiGLU) scheduling groups of 8-10 m-tiles -- for
the plain forward, the fused SwiGLU, dlhs and the gathered gate_up.  With whole tiles each
element is the MFMA sequence of the other bf16 kernels, so the results equal the 128-row tiling
bit for bit; all are checked against the float64 oracle at the bf16 bound (2e-2)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_err, tile_list_workspace_bytes
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

OPS = {"fwd": 0, "swiglu": 1, "dlhs": 2}

# group sizes (mean >= 512): remainders past whole 256-row tiles cover every thin form (1-32,
# 33-64, 65-96, 97-128 rows), the partial full form (129-255) and exact multiples; one empty group
GROUPS = [
    [769, 808, 838, 868, 896],
    [897, 1024, 1000, 1279, 0, 1025, 768 + 255],
    [2048 + 14, 2048 + 77, 1984, 2125, 2019, 2058, 2063, 2048],
    # mean >= 8 x 256 (scheduling groups aligned to experts): one or two m-tiles past a group of
    # 8 stay in it (groups of 9 and 10), three go to the end of the list
    [2048 + 300, 2048 + 600, 2048 + 513, 1800, 2500, 2048, 2048 + 256],
]


def _run_tiled(dev, op, x, w, g, M, Kin, Kout, E, tile_m, ws_bytes):
    from mintext_amd import _lib as L

    ws = L.workspace(L.query("mtx_gmm_workspace_size", M, E), dev)
    ncols = Kin if op == "dlhs" else Kout
    out = torch.full((M, ncols), float("nan"), dtype=torch.bfloat16, device=dev)
    L.call("mtx_gmm_tiled", OPS[op], x.data_ptr(), w.data_ptr(), g.data_ptr(), L.dtype_code(torch.bfloat16), M, Kin,
           Kout, E, tile_m, 0, out.data_ptr(), ws.data_ptr(), ws_bytes, L.stream(dev))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("op", ["fwd", "swiglu", "dlhs"])
@pytest.mark.parametrize("gi", range(len(GROUPS)))
def test_w4_tile_forms_match_128_row_tiling(dev, op, gi):
    from mintext_amd import _lib as L

    gs = np.asarray(GROUPS[gi], np.int32)
    E = len(gs)
    M = int(gs.sum()) + 300  # two zero tiles past the groups
    Kred, N = 1280, 512      # 40 ring stages (the per-tile kernels), two 256-column tiles
    rng = np.random.default_rng(7 + gi)
    if op == "dlhs":  # dx [M, Kin] = g [M, Kout] @ w[e]^T, w [E, Kin, Kout]
        Kin, Kout = N, Kred
        x = rng.standard_normal((M, Kout)).astype(np.float32)
        w = (rng.standard_normal((E, Kin, Kout)) * 0.05).astype(np.float32)
    else:
        Kin, Kout = Kred, (N // 2 if op == "swiglu" else N)
        x = rng.standard_normal((M, Kin)).astype(np.float32)
        w = (rng.standard_normal((E, Kin, N)) * 0.05).astype(np.float32)
    xb = torch.from_numpy(x).to(dev).bfloat16()
    wb = torch.from_numpy(w).to(dev).bfloat16()
    g = torch.from_numpy(gs).to(dev)
    whole_ws = tile_list_workspace_bytes(M, E)
    full_ws = L.query("mtx_gmm_workspace_size", M, E)
    whole = _run_tiled(dev, op, xb, wb, g, M, Kin, Kout, E, 256, whole_ws)
    t128 = _run_tiled(dev, op, xb, wb, g, M, Kin, Kout, E, 128, whole_ws)
    split = _run_tiled(dev, op, xb, wb, g, M, Kin, Kout, E, 256, full_ws)
    split2 = _run_tiled(dev, op, xb, wb, g, M, Kin, Kout, E, 256, full_ws)
    assert torch.equal(whole, t128), "256-row whole tiles must give the 128-row tiling's bits"
    assert torch.equal(split, split2), "the split tail is deterministic"
    used = int(gs.sum())
    for out in (whole, split):
        assert (out[used:] == 0).all(), "rows past sum(group_sizes) must be zero"
    xf, wf = xb.float().cpu().numpy(), wb.float().cpu().numpy()
    if op == "fwd":
        ref = O.gmm(xf, wf, gs)
    elif op == "dlhs":
        ref = O.gmm_dlhs(xf, wf, gs)
    else:
        ref = O.swiglu(O.gmm(xf, wf, gs))
    for out in (whole, split):
        got = out.float().cpu().numpy()
        assert rel_err(got[:used], ref[:used]) < 2e-2, rel_err(got[:used], ref[:used])
    # split pieces sum the same products in another association: a bf16 ulp apart at most,
    # plus the f32 summation error where the sum cancels
    d = (split.float() - whole.float()).abs()
    bound = whole.float().abs() * 2.0 ** -7 + 1e-5 * float(np.abs(ref).max())
    assert (d <= bound).all(), (d - bound).max().item()


@pytest.mark.parametrize("T,K,E", [(2100, 2, 8), (1500, 3, 4)])
def test_w4_gathered_swiglu_equals_route_then_gmm(dev, T, K, E):
    """The gathered gate_up on the one-wave-per-SIMD kernel (mean group >= 512 rows) gives the
    bits of route + grouped_matmul_swiglu."""
    from mintext_amd.kernels import route
    from mintext_amd.kernels.grouped_matmul import grouped_matmul_swiglu, grouped_matmul_swiglu_gathered
    from mintext_amd.kernels.moe_dispatch import route_indices

    D, I = 1280, 384
    rng = np.random.default_rng(T)
    idx = torch.from_numpy(rng.integers(0, E, (T, K)).astype(np.int32)).to(dev)
    x = torch.randn(T, D, device=dev).bfloat16()
    w = (torch.randn(E, D, 2 * I, device=dev) * 0.05).bfloat16()
    st, si, gs = route(x, idx, E)
    si2, gs2, _ = route_indices(idx, E)
    assert (T * K) // E >= 512
    ref = grouped_matmul_swiglu(st, w, gs)
    out = grouped_matmul_swiglu_gathered(x, si2, K, w, gs2)
    assert torch.equal(out, ref)
    refo = O.swiglu(O.gmm(st.float().cpu().numpy(), w.float().cpu().numpy(), gs.cpu().numpy()))
    assert rel_err(out.float().cpu().numpy(), refo) < 2e-2


@pytest.mark.parametrize("op", ["fwd", "swiglu", "dlhs"])
@pytest.mark.parametrize("gi", [0, 3])
def test_w4_n_tiles_split_over_xcds_match_128_row_tiling(dev, op, gi):
    """A number of n-tiles that is a multiple of 8 (the plain forward's XCD split of the n-tiles;
    for the SwiGLU, with GROUPS[3], its merged scheduling groups): the bits of the 128-row tiling
    and the float64 oracle at the bf16 bound."""
    from mintext_amd import _lib as L

    gs = np.asarray(GROUPS[gi], np.int32)
    E = len(gs)
    M = int(gs.sum()) + 300
    N = 2048  # eight 256-column n-tiles (fwd, dlhs) / eight 128-column SwiGLU tiles
    rng = np.random.default_rng(11 + gi)
    if op == "dlhs":  # dx [M, Kin] = g [M, Kout] @ w[e]^T: Kin = N output columns
        Kin, Kout = N, 512
        x = rng.standard_normal((M, Kout)).astype(np.float32)
        w = (rng.standard_normal((E, Kin, Kout)) * 0.05).astype(np.float32)
    else:
        Kin, Kout = 512, (N // 2 if op == "swiglu" else N)
        x = rng.standard_normal((M, Kin)).astype(np.float32)
        w = (rng.standard_normal((E, Kin, N)) * 0.05).astype(np.float32)
    x = torch.from_numpy(x).to(dev).bfloat16()
    w = torch.from_numpy(w).to(dev).bfloat16()
    g = torch.from_numpy(gs).to(dev)
    whole_ws = tile_list_workspace_bytes(M, E)
    full_ws = L.query("mtx_gmm_workspace_size", M, E)
    whole = _run_tiled(dev, op, x, w, g, M, Kin, Kout, E, 256, whole_ws)
    t128 = _run_tiled(dev, op, x, w, g, M, Kin, Kout, E, 128, whole_ws)
    split = _run_tiled(dev, op, x, w, g, M, Kin, Kout, E, 256, full_ws)
    assert torch.equal(whole, t128), "256-row whole tiles must give the 128-row tiling's bits"
    used = int(gs.sum())
    assert (whole[used:] == 0).all() and (split[used:] == 0).all()
    xf, wf = x.float().cpu().numpy(), w.float().cpu().numpy()
    ref = O.gmm_dlhs(xf, wf, gs) if op == "dlhs" else O.gmm(xf, wf, gs)
    if op == "swiglu":
        ref = O.swiglu(ref)
    for out in (whole, split):
        assert rel_err(out.float().cpu().numpy()[:used], ref[:used]) < 2e-2

"""mtx_gmm_tiled_noalloc (the grouped GEMM without a caller workspace, for callers that cannot
allocate) against mtx_gmm_tiled, both called through the C-ABI: bit for bit against the workspace
entry point given a tile-list-only workspace (the same whole-tile schedule), within the dtype's
tolerance against the full workspace (split tail) and against the float64 oracle.  Two calls in a
row on one device, the second smaller, so the second reuses the device array the first wrote."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import rel_err, tile_list_workspace_bytes
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


_tile_list_bytes = tile_list_workspace_bytes


def _groups(rng, M, E):
    cut = np.sort(rng.integers(0, M + 1, E - 1))
    gs = np.diff(np.concatenate([[0], cut, [M]])).astype(np.int32)
    gs[E // 2] += gs[1]
    gs[1] = 0  # an empty group
    return gs


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("op", ["fwd", "swiglu", "dlhs"])
def test_noalloc_gmm_matches_workspace_entry_point(dev, dtype, op):
    from mintext_amd import _lib as L

    lib = L.lib()
    code = {"fwd": L.MTX_GMM_OP_FWD, "swiglu": L.MTX_GMM_OP_SWIGLU, "dlhs": L.MTX_GMM_OP_DLHS}[op]
    stream = L.stream(dev)
    # bf16 kernel forms, each call smaller than the one before it on that form: reductions of 2304
    # (beyond the persistent kernel's 32 stages) with >= 512 rows per expert on average (one-wave-
    # per-SIMD kernel) and then fewer (8-wave per-tile kernel), both with split tails under the full
    # workspace; then the persistent short-reduction kernel; then 128-row tiles
    shapes = [(4096, 4, 2304, 2304), (3000, 8, 2304, 2304), (8192, 6, 512, 768), (1000, 3, 256, 384)]
    for call, (M, E, Kin, Kout) in enumerate(shapes):
        rng = np.random.default_rng(call * 10 + len(op))
        gs = _groups(rng, M, E)
        a_cols = Kout if op == "dlhs" else Kin
        out_cols = Kin if op == "dlhs" else Kout
        n_w = 2 * Kout if op == "swiglu" else Kout
        x = torch.randn(M, a_cols, device=dev).to(dtype)
        w = (torch.randn(E, Kin, n_w, device=dev) * 0.05).to(dtype)
        g = torch.from_numpy(gs).to(dev)
        outs = {}
        for kind in ("noalloc", "tiles", "full"):
            out = torch.full((M, out_cols), float("nan"), device=dev).to(dtype)
            if kind == "noalloc":
                rc = lib.mtx_gmm_tiled_noalloc(code, x.data_ptr(), w.data_ptr(), g.data_ptr(), L.dtype_code(dtype),
                                               M, Kin, Kout, E, 0, 0, out.data_ptr(), stream)
            else:
                nb = _tile_list_bytes(M, E) if kind == "tiles" else lib.mtx_gmm_workspace_size(M, E)
                ws = torch.empty(nb, dtype=torch.uint8, device=dev)
                rc = lib.mtx_gmm_tiled(code, x.data_ptr(), w.data_ptr(), g.data_ptr(), L.dtype_code(dtype), M, Kin,
                                       Kout, E, 0, 0, out.data_ptr(), ws.data_ptr(), nb, stream)
            assert rc == L.MTX_OK, (kind, rc)
            outs[kind] = out
        torch.cuda.synchronize()
        assert torch.equal(outs["noalloc"], outs["tiles"]), f"call {call}: noalloc != tile-list workspace"
        tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
        f = lambda t: t.double().cpu().numpy()
        assert rel_err(f(outs["noalloc"]), f(outs["full"])) < tol
        xa, wa = f(x), f(w)
        if op == "fwd":
            ref = O.gmm(xa, wa, gs)
        elif op == "swiglu":
            ref = O.swiglu(O.gmm(xa, wa, gs))
        else:
            ref = O.gmm_dlhs(xa, wa, gs)
        assert rel_err(f(outs["noalloc"]), ref) < tol


def test_noalloc_gmm_rejects_sizes_beyond_its_array(dev):
    from mintext_amd import _lib as L

    lib = L.lib()
    P = None
    assert lib.mtx_gmm_tiled_noalloc(0, P, P, P, 1, (1 << 20) + 1, 64, 256, 8, 0, 0, P, P) == L.MTX_ERR_UNSUPPORTED
    assert lib.mtx_gmm_tiled_noalloc(0, P, P, P, 1, 1024, 64, 256, 1025, 0, 0, P, P) == L.MTX_ERR_UNSUPPORTED
    assert lib.mtx_gmm_tiled_noalloc(0, P, P, P, 1, -1, 64, 256, 8, 0, 0, P, P) == L.MTX_ERR_ARG

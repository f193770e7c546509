"""GPU parity: route / unroute / _sort_with_vjp (HIP, through the C-ABI) vs the oracle.

Integer outputs (sort_indices, group_sizes, the gathered rows) must be bit-exact; the f32
combine is checked at 1e-5 relative.  Mirrors tests/test_moe_kernels.py:22-134 of the reference.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden, rel_err
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def test_route_matches_golden_fixtures(dev):
    from mintext_amd.kernels import route

    g = golden("dispatch")
    for n in sorted({k.split("__")[0] for k in g.files}):
        idx, E = g[f"{n}__idx"], int(g[f"{n}__E"])
        N, K = idx.shape
        x = np.random.default_rng(0).standard_normal((N, 64)).astype(np.float32)
        for dt in (torch.float32, torch.bfloat16):
            st, si, gs = route(_t(x, dev, dt), _t(idx, dev), E)
            np.testing.assert_array_equal(si.cpu().numpy(), g[f"{n}__perm"], err_msg=n)
            np.testing.assert_array_equal(gs.cpu().numpy(), g[f"{n}__gs"], err_msg=n)
            ref = torch.from_numpy(x).to(dt)[torch.from_numpy(g[f"{n}__perm"].astype(np.int64) // K)]
            assert torch.equal(st.cpu(), ref), n


@pytest.mark.parametrize("N,K,E,D", [(16384, 8, 128, 2048), (4096, 8, 256, 512), (8192, 2, 8, 4096), (3, 1, 1, 8)])
def test_route_large_bit_exact(dev, N, K, E, D):
    from mintext_amd.kernels import route

    rng = np.random.default_rng(N + E)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(min(N, 64))]) if K > 1 else rng.integers(0, E, (N, K))
    if K > 1:
        idx = np.concatenate([idx, rng.integers(0, E, (N - idx.shape[0], K))])  # duplicates allowed too
    x = torch.randn(N, D, device=dev, dtype=torch.bfloat16)
    st, si, gs = route(x, _t(idx.astype(np.int32), dev), E)
    perm = np.argsort(idx.ravel(), kind="stable")
    np.testing.assert_array_equal(si.cpu().numpy(), perm)
    np.testing.assert_array_equal(gs.cpu().numpy(), np.bincount(idx.ravel(), minlength=E))
    assert torch.equal(st, x[torch.from_numpy(perm // K).to(dev)])


@pytest.mark.parametrize("N,K,E", [(384, 3, 31), (900, 4, 9), (2048, 2, 8), (2049, 2, 8), (18432, 1, 1),
                                   (18433, 1, 1), (5, 8, 2), (2500, 3, 31), (32768, 2, 32), (40000, 1, 17)])
def test_route_few_experts_bit_exact(dev, N, K, E):
    """E <= 32 and ids x (E+1) <= 36864 take the one-workgroup sort (bucket tables of 9, 17
    and 33 entries; the cases at the limit and one id past it), larger products the chunked
    sort.  Ragged sizes, about 1% out-of-range ids (sorted last, uncounted)."""
    from mintext_amd.kernels.moe_dispatch import _route_impl

    rng = np.random.default_rng(N * 7 + E)
    idx = rng.integers(0, E, (N, K)).astype(np.int32)
    bad = rng.random((N, K)) < 0.01
    idx[bad] = rng.choice(np.array([-3, E, E + 5], np.int32), bad.sum())
    x = torch.randn(N, 64, device=dev, dtype=torch.bfloat16)
    st, si, gs, inv = _route_impl(x, _t(idx, dev), E)
    key = np.where((idx >= 0) & (idx < E), idx, E).ravel()
    perm = np.argsort(key, kind="stable")
    np.testing.assert_array_equal(si.cpu().numpy(), perm)
    np.testing.assert_array_equal(inv.cpu().numpy(), np.argsort(perm))
    np.testing.assert_array_equal(gs.cpu().numpy(), np.bincount(key, minlength=E + 1)[:E])
    assert torch.equal(st, x[torch.from_numpy(perm // K).to(dev)])


@pytest.mark.parametrize("N,K,E", [(70000, 2, 1023), (5000, 8, 600), (300000, 1, 64), (1, 1, 1023), (777, 5, 200),
                                   (0, 8, 128)])
def test_route_chunked_bit_exact(dev, N, K, E):
    """The two-launch counting sort with its count-table cap (at most 16384 entries: 16 chunks at
    E = 1023, chunks of many ids), ragged chunk counts (the table's zero pad columns), one id, no
    ids (group sizes still written as zeros), about 1% out-of-range ids (sorted last)."""
    from mintext_amd.kernels.moe_dispatch import _route_impl

    rng = np.random.default_rng(N * 3 + E)
    idx = rng.integers(0, E, (N, K)).astype(np.int32)
    bad = rng.random((N, K)) < 0.01
    idx[bad] = rng.choice(np.array([-1, E, E + 9], np.int32), bad.sum())
    x = torch.randn(N, 64, device=dev, dtype=torch.bfloat16)
    st, si, gs, inv = _route_impl(x, _t(idx, dev), E)
    key = np.where((idx >= 0) & (idx < E), idx, E).ravel()
    perm = np.argsort(key, kind="stable")
    np.testing.assert_array_equal(si.cpu().numpy(), perm)
    np.testing.assert_array_equal(inv.cpu().numpy(), np.argsort(perm))
    np.testing.assert_array_equal(gs.cpu().numpy(), np.bincount(key, minlength=E + 1)[:E])
    assert torch.equal(st, x[torch.from_numpy(perm // K).to(dev)])


@pytest.mark.parametrize("nbytes", [16, 4096 * 16 + 48, 37 << 20])
@pytest.mark.parametrize("variant", [0x00, 0x41, 0x81, 0xF0, 0x21])
def test_stream_copy(dev, nbytes, variant):
    from mintext_amd import _lib as L

    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=dev)
    dst = torch.zeros_like(src)
    L.call("mtx_stream_copy", L.ptr(src), L.ptr(dst), nbytes, variant, 0 if variant & 0x40 else 7, L.stream(dev))
    assert torch.equal(dst, src)


def test_route_out_of_range_ids_sorted_last(dev):
    from mintext_amd.kernels import route

    idx = np.array([[1, 7], [0, -1], [2, 1], [9, 0]], np.int32)  # E = 4: 7, -1, 9 invalid
    x = np.arange(4 * 8, dtype=np.float32).reshape(4, 8)
    st, si, gs = route(_t(x, dev), _t(idx, dev), 4)
    _, perm, gso = O.route(x, idx, 4)
    np.testing.assert_array_equal(si.cpu().numpy(), perm)
    np.testing.assert_array_equal(gs.cpu().numpy(), gso)
    assert gs.sum().item() == 5


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_unroute_matches_oracle(dev, dt):
    from mintext_amd.kernels import route, unroute

    rng = np.random.default_rng(3)
    N, D, K, E = 1000, 200, 4, 16
    idx = np.stack([rng.permutation(E)[:K] for _ in range(N)]).astype(np.int32)
    y = rng.standard_normal((N * K, D)).astype(np.float32)
    w = rng.random((N, K)).astype(np.float32)
    _, si, _ = route(_t(rng.standard_normal((N, D)).astype(np.float32), dev), _t(idx, dev), E)
    yt = _t(y, dev, dt)
    out = unroute(yt, si, _t(w, dev), K)
    assert out.dtype == torch.float32  # result_type(bf16, f32) = f32 as in moe_dispatch.py:111
    ref = O.unroute(yt.float().cpu().numpy(), si.cpu().numpy(), w, K)
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    # without route's cached inverse (fresh sort_indices tensor)
    out2 = unroute(yt, si.clone(), _t(w, dev), K)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("ydt,adt", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                     (torch.float32, torch.bfloat16), (torch.float32, torch.float32)])
@pytest.mark.parametrize("N,K,D", [(513, 2, 512), (300, 8, 1024), (77, 3, 198)])
def test_unroute_add_equals_two_steps(dev, ydt, adt, N, K, D):
    """unroute_add = unroute + addend (routed_out + shared_out, moe.py:256-258), bit for bit,
    on the row-wise (bf16, K <= 8), vectorised and scalar (D % 8 != 0) combine kernels."""
    from mintext_amd.kernels import route, unroute
    from mintext_amd.kernels.moe_dispatch import unroute_add

    rng = np.random.default_rng(N + K)
    E = 16
    idx = np.stack([rng.permutation(E)[:K] for _ in range(N)]).astype(np.int32)
    _, si, _ = route(_t(rng.standard_normal((N, D)).astype(np.float32), dev), _t(idx, dev), E)
    y = _t(rng.standard_normal((N * K, D)).astype(np.float32), dev, ydt)
    w = _t(rng.random((N, K)).astype(np.float32), dev)
    a = _t(rng.standard_normal((N, D)).astype(np.float32), dev, adt)
    out = unroute_add(y, si, w, K, a)
    ref = unroute(y, si, w, K) + a.to(torch.float32)
    assert out.dtype == torch.float32
    assert torch.equal(out, ref)


def test_route_unroute_gradients(dev):
    """tests/test_moe_kernels.py:69-103: grad of sum(unroute(route(x))) and finite differences."""
    from mintext_amd.kernels import route, unroute

    rng = np.random.default_rng(42)
    N, D, K, E = 32, 64, 2, 4
    x = _t(rng.standard_normal((N, D)).astype(np.float32), dev).requires_grad_(True)
    idx = _t(rng.integers(0, E, (N, K)).astype(np.int32), dev)
    w = _t(rng.random((N, K)).astype(np.float32), dev).requires_grad_(True)

    def fn(tok, ww):
        st, si, _ = route(tok, idx, E)
        return unroute(st, si, ww, K).sum()

    loss = fn(x, w)
    loss.backward()
    # closed form: d/dx = sum_k w[n,k]; d/dw[n,k] = sum_d x[n,d]
    np.testing.assert_allclose(x.grad.cpu().numpy(), np.repeat(w.detach().cpu().numpy().sum(1, keepdims=True), D, 1),
                               rtol=1e-6)
    np.testing.assert_allclose(w.grad.cpu().numpy(), np.repeat(x.detach().cpu().numpy().sum(1, keepdims=True), K, 1),
                               rtol=1e-5, atol=1e-5)
    eps = 1e-3
    xr = x.detach()
    for i, j in [(0, 0), (5, 7), (31, 63), (17, 30)]:
        xp, xm = xr.clone(), xr.clone()
        xp[i, j] += eps
        xm[i, j] -= eps
        num = (fn(xp, w.detach()) - fn(xm, w.detach())).item() / (2 * eps)
        np.testing.assert_allclose(x.grad[i, j].item(), num, rtol=0.02, atol=1e-4)


def test_unroute_backward_matches_oracle(dev):
    from mintext_amd.kernels import route, unroute

    rng = np.random.default_rng(8)
    N, D, K, E = 300, 96, 3, 8
    idx = np.stack([rng.permutation(E)[:K] for _ in range(N)]).astype(np.int32)
    _, si, _ = route(_t(np.zeros((N, D), np.float32), dev), _t(idx, dev), E)
    y = _t(rng.standard_normal((N * K, D)).astype(np.float32), dev).requires_grad_(True)
    w = _t(rng.random((N, K)).astype(np.float32), dev).requires_grad_(True)
    g = rng.standard_normal((N, D)).astype(np.float32)
    out = unroute(y, si, w, K)
    out.backward(_t(g, dev))
    perm = si.cpu().numpy()
    inv = O.invert_permutation(perm)
    Y = y.detach().cpu().numpy()
    W = w.detach().cpu().numpy()
    dY = np.empty_like(Y)
    dY[inv] = (W.reshape(-1, 1) * np.repeat(g, K, axis=0))
    dW = np.einsum("nkd,nd->nk", Y[inv].reshape(N, K, D), g)
    np.testing.assert_allclose(y.grad.cpu().numpy(), dY, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(w.grad.cpu().numpy(), dW, rtol=1e-5, atol=1e-4)


def test_single_and_empty_expert_edge_cases(dev):
    """tests/test_moe_kernels.py:105-134."""
    from mintext_amd.kernels import route, unroute

    x = torch.randn(8, 16, device=dev)
    st, si, gs = route(x, torch.zeros(8, 1, dtype=torch.int32, device=dev), 4)
    assert gs.cpu().tolist() == [8, 0, 0, 0]
    out = unroute(st, si, torch.ones(8, 1, device=dev), 1)
    assert torch.equal(out, x)
    idx = torch.randint(0, 2, (8, 1), device=dev, dtype=torch.int32)
    st, si, gs = route(x, idx, 4)
    assert gs[2].item() == 0 and gs[3].item() == 0 and gs.sum().item() == 8
    assert torch.isfinite(unroute(st, si, torch.ones(8, 1, device=dev), 1)).all()


def test_sort_with_vjp(dev):
    from mintext_amd.kernels import _sort_with_vjp

    x = torch.randn(50, 12, device=dev, requires_grad=True)
    p = torch.randperm(50, device=dev).to(torch.int32)
    y = _sort_with_vjp(x, p)
    assert torch.equal(y, x.detach()[p.long()])
    g = torch.randn(50, 12, device=dev)
    y.backward(g)
    expect = torch.empty_like(g)
    expect[p.long()] = g
    assert torch.equal(x.grad, expect)


_F32, _BF16 = torch.float32, torch.bfloat16


@pytest.mark.parametrize("N,K,D,ydt,gdt,wdt", [(257, 1, 512, _BF16, _F32, _F32), (300, 2, 1024, _BF16, _F32, _F32),
                                               (129, 3, 264, _F32, _F32, _F32), (64, 8, 2048, _BF16, _F32, _F32),
                                               (65, 9, 512, _BF16, _F32, _F32), (70, 2, 100, _BF16, _F32, _F32),
                                               (200, 2, 512, _BF16, _BF16, _BF16), (100, 8, 256, _BF16, _BF16, _F32),
                                               (90, 4, 136, _F32, _BF16, _BF16),
                                               (50, 8, 1800, _BF16, _F32, _F32)])  # lanes with 1 or 2 chunks
def test_unroute_bwd_vector_and_scalar_forms(dev, N, K, D, ydt, gdt, wdt):
    """mtx_unroute_bwd (the layer's combine output and router weights as dout / w, in f32 or bf16):
    d_sorted bit-exact against the f32 products of the inputs rounded to the row dtype, d_w against
    a float64 sum (rounded to bf16 when w is bf16).  D % 8 == 0 with K <= 8 runs the 16-byte vector
    kernel; K = 9 and D = 100 the scalar one."""
    from mintext_amd import _lib as L
    from mintext_amd.kernels import route

    rng = np.random.default_rng(N * 31 + K)
    E = max(K, 8)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(N)]).astype(np.int32)
    _, si, _ = route(_t(np.zeros((N, 8), np.float32), dev), _t(idx, dev), E)
    inv = O.invert_permutation(si.cpu().numpy()).astype(np.int32)
    Y = _t(rng.standard_normal((N * K, D)).astype(np.float32), dev, ydt)
    wt = _t(rng.random((N, K)).astype(np.float32), dev, wdt)
    gt = _t(rng.standard_normal((N, D)).astype(np.float32), dev, gdt)
    w = wt.float().cpu().numpy()  # the values the kernel reads, as f32
    g = gt.float().cpu().numpy()
    dY = torch.full_like(Y, 7.0)
    dw = torch.full((N, K), 7.0, dtype=wdt, device=dev)
    it = _t(inv, dev)
    L.call("mtx_unroute_bwd", L.ptr(gt), L.dtype_code(gdt), L.ptr(Y), L.dtype_code(ydt), L.ptr(it), L.ptr(wt),
           L.dtype_code(wdt), N, K, D, L.ptr(dY), L.ptr(dw), L.stream(dev))
    torch.cuda.synchronize()
    want = torch.empty((N * K, D), dtype=torch.float32)
    want[torch.from_numpy(inv).long()] = torch.from_numpy(np.repeat(w.reshape(-1, 1), D, 1) * np.repeat(g, K, axis=0))
    assert torch.equal(dY.cpu(), want.to(ydt))
    Yn = Y.float().cpu().numpy().astype(np.float64)
    dw_ref = np.einsum("nkd,nd->nk", Yn[inv].reshape(N, K, D), g.astype(np.float64))
    rtol = 1e-5 if wdt == _F32 else 2.0 ** -8  # bf16 d_w: one rounding of the f32 sum
    np.testing.assert_allclose(dw.float().cpu().numpy(), dw_ref, rtol=rtol, atol=1e-4 * np.sqrt(D))


@pytest.mark.parametrize("M,I", [(300, 8), (257, 768), (64, 2048), (33, 2056), (40, 12)])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_swiglu_vector_form_same_bits_as_scalar(dev, M, I, dt):
    """mtx_swiglu / mtx_swiglu_bwd: the 16-byte vector kernels (I % 8 == 0, aligned rows) give the
    bits of the scalar kernels, which run on a copy of the same data one element past a 16-byte
    boundary; both within
    rounding of the float64 oracle.  I = 12 runs the scalar kernels only."""
    from mintext_amd import _lib as L

    rng = np.random.default_rng(M + I)
    h_np = (rng.standard_normal((M, 2 * I)) * 4).astype(np.float32)
    dy_np = rng.standard_normal((M, I)).astype(np.float32)

    def at_offset(a):  # the same values at a data pointer one element past a 16-byte boundary
        flat = torch.empty(a.numel() + 8, dtype=dt, device=dev)
        v = flat[1:1 + a.numel()].view(a.shape)
        v.copy_(a)
        return v

    h = _t(h_np, dev, dt)
    dy = _t(dy_np, dev, dt)
    outs = []
    for hh, dd in ((h, dy), (at_offset(h), at_offset(dy))):
        y = torch.empty((M, I), dtype=dt, device=dev)
        dh = torch.empty((M, 2 * I), dtype=dt, device=dev)
        L.call("mtx_swiglu", L.ptr(hh), L.dtype_code(dt), M, I, L.ptr(y), L.stream(dev))
        L.call("mtx_swiglu_bwd", L.ptr(hh), L.ptr(dd), L.dtype_code(dt), M, I, L.ptr(dh), L.stream(dev))
        outs.append((y, dh))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    tol = 1e-5 if dt == torch.float32 else 2e-2
    hf, dyf = h.float().cpu().numpy(), dy.float().cpu().numpy()
    assert rel_err(outs[0][0].float().cpu().numpy(), O.swiglu(hf)) < tol
    assert rel_err(outs[0][1].float().cpu().numpy(), O.swiglu_bwd(hf, dyf)) < tol

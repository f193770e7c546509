"""GPU parity of the blockwise-fp8 backward (dlhs and tgmm with e4m3 operands; the bf16 forms are
grouped_matmul.py:151-187 and :197-235): quantisers bit-exact against the oracle, the GEMMs within
1e-2 of the dequantised float64 oracle and 6e-2 of the unquantised product, empty and skewed groups,
the C5 backward shapes at full size; in both scale modes (amax/448 and power-of-two)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_err
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _u8(t):
    return t.view(torch.uint8).cpu().numpy()


def _zipf_groups(rng, M, E, empty=(1,)):
    p = 1.0 / np.arange(1, E + 1) ** 1.2
    gs = rng.multinomial(M, p[rng.permutation(E)] / p.sum()).astype(np.int32)
    for e in empty:
        gs[(e + 1) % E] += gs[e]
        gs[e] = 0
    return gs


SCALES = ["amax", "pow2"]


@pytest.mark.parametrize("scales", SCALES)
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_quant_weights_t_bit_exact(dev, dt, scales):
    from mintext_amd.kernels.fp8 import quantize_fp8_weights, quantize_fp8_weights_t

    w = (torch.randn(3, 256, 384, device=dev) * 0.02).to(dt)
    w[1, :128, :128] = 0  # an all-zero block -> scale 1
    q, s = quantize_fp8_weights_t(w, scales=scales)
    oq, os_ = O.quant_fp8_weights_t(w.float().cpu().numpy(), scales=scales)
    assert np.array_equal(_u8(q), oq) and np.array_equal(s.cpu().numpy(), os_)
    # the same blocks as the forward's prepack
    qf, sf = quantize_fp8_weights(w, scales=scales)
    assert torch.equal(q.view(torch.uint8), qf.view(torch.uint8).transpose(1, 2)) and torch.equal(s, sf.transpose(1, 2))


@pytest.mark.parametrize("scales", SCALES)
@pytest.mark.parametrize("blocks", [False, True])
@pytest.mark.parametrize("M,F,E", [(1000, 256, 6), (4095, 512, 16), (129, 128, 3), (5000, 768, 64)])
def test_quant_grouped_t_bit_exact(dev, blocks, M, F, E, scales):
    from mintext_amd.kernels.fp8 import quantize_fp8_grouped_t

    rng = np.random.default_rng(M + F)
    gs = _zipf_groups(rng, M - 7, E)  # 7 rows past sum(group_sizes): not quantised
    x = (torch.randn(M, F, device=dev) * torch.rand(1, F, device=dev) * 5).bfloat16()
    xt, xs = quantize_fp8_grouped_t(x, _t(gs, dev), blocks=blocks, scales=scales)
    oq, os_ = O.quant_fp8_grouped_t(x.float().cpu().numpy(), gs, blocks, scales=scales)
    _, cb = O.fp8_group_chunks(gs, M)
    used = int(cb[-1])
    assert np.array_equal(_u8(xt)[:128 * F * used], oq[:128 * F * used])
    nf = F // 128 if blocks else F
    assert np.array_equal(xs.cpu().numpy()[:nf * used], os_[:nf * used])


@pytest.mark.parametrize("scales", SCALES)
@pytest.mark.parametrize("M,Kin,Kout,E", [(2000, 256, 384, 6), (3000, 768, 2048, 16), (700, 2048, 1536, 4)])
def test_gmm_fp8_dlhs(dev, M, Kin, Kout, E, scales):
    from mintext_amd.kernels.fp8 import grouped_matmul_fp8_dlhs, quantize_fp8_rows, quantize_fp8_weights_t

    rng = np.random.default_rng(M)
    gs = _zipf_groups(rng, M, E)
    g = torch.randn(M, Kout, device=dev).bfloat16()
    w = (torch.randn(E, Kin, Kout, device=dev) * 0.02).bfloat16()
    gq, gsc = quantize_fp8_rows(g, scales=scales)
    wq, ws = quantize_fp8_weights_t(w, scales=scales)
    dx = grouped_matmul_fp8_dlhs(gq, gsc, wq, ws, _t(gs, dev), scales=scales)
    assert dx.dtype == torch.bfloat16 and dx.shape == (M, Kin)
    got = dx.float().cpu().numpy()
    ref_q = O.gmm_fp8_dlhs(_u8(gq), gsc.cpu().numpy(), _u8(wq), ws.cpu().numpy(), gs)
    assert rel_err(got, ref_q) < 1e-2
    ref = O.gmm_dlhs(g.float().cpu().numpy(), w.float().cpu().numpy(), gs)
    assert rel_err(got, ref) < 6e-2


@pytest.mark.parametrize("scales", SCALES)
@pytest.mark.parametrize("M,F,N,E", [(2000, 256, 256, 6), (5000, 768, 2048, 16), (3000, 2048, 1536, 8),
                                     (300, 256, 512, 40)])
def test_tgmm_fp8(dev, M, F, N, E, scales):
    from mintext_amd.kernels.fp8 import quantize_fp8_grouped_t, tgmm_fp8

    rng = np.random.default_rng(M + E)
    gs = _zipf_groups(rng, M, E, empty=(0, E // 2))
    x = torch.randn(M, F, device=dev).bfloat16()
    g = torch.randn(M, N, device=dev).bfloat16()
    tg = _t(gs, dev)
    xt, xs = quantize_fp8_grouped_t(x, tg, scales=scales)
    gt, gsc = quantize_fp8_grouped_t(g, tg, blocks=True, scales=scales)
    dw = tgmm_fp8(xt, xs, gt, gsc, tg, M, scales=scales)
    assert dw.dtype == torch.bfloat16 and dw.shape == (E, F, N)
    got = dw.float().cpu().numpy()
    for e in np.flatnonzero(gs == 0):
        assert not got[e].any()
    ref_q = O.tgmm_fp8(_u8(xt), xs.cpu().numpy(), _u8(gt), gsc.cpu().numpy(), gs, M, F, N)
    assert rel_err(got, ref_q) < 1e-2
    ref = O.tgmm(x.float().cpu().numpy(), g.float().cpu().numpy(), gs)
    assert rel_err(got, ref) < 6e-2


@pytest.mark.parametrize("scales", SCALES)
def test_tgmm_fp8_persistent_matches_per_tile(dev, scales):
    """2048 tiles (E=64, 1024 x 2048 per expert) take the persistent kernel, whose ring runs across
    tiles and restarts around experts of one chunk: empty experts give zeros, the result is within
    1e-2 of the dequantised oracle, and each checked expert's dW has the bits of the same expert
    computed alone (a one-expert problem of few tiles, which takes the per-tile kernel)."""
    from mintext_amd.kernels.fp8 import quantize_fp8_grouped_t, tgmm_fp8

    E, F, N = 64, 1024, 2048
    rng = np.random.default_rng(2048)
    gs = _zipf_groups(rng, 9000, E, empty=(0, 5, 40))
    gs[[7, 9, 11]] = [1, 128, 129]  # one chunk (two), two chunks
    gs[3] += 3000                   # a long tile early in the order
    M = int(gs.sum())
    x = torch.randn(M, F, device=dev).bfloat16()
    g = torch.randn(M, N, device=dev).bfloat16()
    f8s = dict(scales=scales)
    dw = tgmm_fp8(*quantize_fp8_grouped_t(x, _t(gs, dev), **f8s),
                  *quantize_fp8_grouped_t(g, _t(gs, dev), blocks=True, **f8s), _t(gs, dev), M, **f8s)
    got = dw.float().cpu().numpy()
    for e in np.flatnonzero(gs == 0):
        assert not got[e].any()
    xt, xs = quantize_fp8_grouped_t(x, _t(gs, dev), **f8s)
    gt, gsc = quantize_fp8_grouped_t(g, _t(gs, dev), blocks=True, **f8s)
    ref_q = O.tgmm_fp8(_u8(xt), xs.cpu().numpy(), _u8(gt), gsc.cpu().numpy(), gs, M, F, N)
    assert rel_err(got, ref_q) < 1e-2
    off = np.concatenate([[0], np.cumsum(gs)])
    for e in (3, 7, 9, 11, int(np.argmax(gs)), int(np.flatnonzero(gs)[-1])):
        r0, r1 = int(off[e]), int(off[e + 1])
        one = _t(np.array([r1 - r0], np.int32), dev)
        alone = tgmm_fp8(*quantize_fp8_grouped_t(x[r0:r1], one, **f8s),
                         *quantize_fp8_grouped_t(g[r0:r1], one, blocks=True, **f8s), one, r1 - r0, **f8s)
        assert torch.equal(alone[0].view(torch.int16), dw[e].view(torch.int16)), f"expert {e}"


@pytest.mark.timeout(600)
@pytest.mark.parametrize("scales", SCALES)
def test_fp8_backward_c5_full_size(dev, scales):
    """The C5 backward shapes (M=131072, D=2048, I=768, E=128, the bench's Zipf(1.2) routing) with
    fp8 operands: dlhs of both expert GEMMs on sampled rows, tgmm of both on sampled blocks."""
    import bench
    from mintext_amd.kernels import route, route_topk
    from mintext_amd.kernels.fp8 import (grouped_matmul_fp8_dlhs, quantize_fp8_grouped_t, quantize_fp8_rows,
                                         quantize_fp8_weights_t, tgmm_fp8)

    cfg = bench.CONFIGS["qwen3_bwd"]
    T, D, E, K, I = cfg["T"], cfg["D"], cfg["E"], cfg["K"], cfg["I"]
    M = T * K
    with torch.no_grad():
        x, logits, gate_up, down, _, g = bench.layer_inputs("qwen3_bwd", dev)
        idx, _ = route_topk(logits, K)
        st, _, gs = route(x, idx, E)
        gy = torch.randn(M, D, device=dev, generator=g).bfloat16()    # d out of the down GEMM
        gh = torch.randn(M, 2 * I, device=dev, generator=g).bfloat16()  # d out of the gate_up GEMM
        y = torch.randn(M, I, device=dev, generator=g).bfloat16()      # the down GEMM's input
        f8s = dict(scales=scales)
        dnq, dns = quantize_fp8_weights_t(down, **f8s)
        guq, gus = quantize_fp8_weights_t(gate_up, **f8s)
        a = grouped_matmul_fp8_dlhs(*quantize_fp8_rows(gy, **f8s), dnq, dns, gs, **f8s)   # [M, I]
        b = grouped_matmul_fp8_dlhs(*quantize_fp8_rows(gh, **f8s), guq, gus, gs, **f8s)   # [M, D]
        c = tgmm_fp8(*quantize_fp8_grouped_t(y, gs, **f8s), *quantize_fp8_grouped_t(gy, gs, blocks=True, **f8s), gs, M,
                     **f8s)  # [E, I, D]
        d = tgmm_fp8(*quantize_fp8_grouped_t(st, gs, **f8s), *quantize_fp8_grouped_t(gh, gs, blocks=True, **f8s), gs,
                     M, **f8s)  # [E, D, 2I]
    gsh = gs.cpu().numpy()
    off = np.concatenate([[0], np.cumsum(gsh)])
    rng = np.random.default_rng(61)
    nz = np.flatnonzero(gsh)
    experts = np.unique(np.concatenate([[int(np.argmax(gsh)), int(nz[np.argmin(gsh[nz])])],
                                        rng.choice(nz, 6, replace=False)]))
    h = lambda t: t.float().cpu().numpy().astype(np.float64)
    for e in experts:
        r0, r1 = int(off[e]), int(off[e + 1])
        rows = np.unique(np.concatenate([[r0, r1 - 1], rng.integers(r0, r1, 6)]))
        tr = torch.from_numpy(rows).to(dev)
        assert rel_err(h(a[tr]), h(gy[tr]) @ h(down[e]).T) < 6e-2, f"dlhs down, expert {e}"
        assert rel_err(h(b[tr]), h(gh[tr]) @ h(gate_up[e]).T) < 6e-2, f"dlhs gate_up, expert {e}"
        ks, ns = np.sort(rng.choice(I, 16, replace=False)), np.sort(rng.choice(D, 16, replace=False))
        ref_c = h(y[r0:r1][:, torch.from_numpy(ks).to(dev)]).T @ h(gy[r0:r1][:, torch.from_numpy(ns).to(dev)])
        got_c = h(c[int(e)][torch.from_numpy(ks).to(dev)][:, torch.from_numpy(ns).to(dev)])
        assert rel_err(got_c, ref_c) < 6e-2, f"tgmm down, expert {e}"
        kd, nd = np.sort(rng.choice(D, 16, replace=False)), np.sort(rng.choice(2 * I, 16, replace=False))
        ref_d = h(st[r0:r1][:, torch.from_numpy(kd).to(dev)]).T @ h(gh[r0:r1][:, torch.from_numpy(nd).to(dev)])
        got_d = h(d[int(e)][torch.from_numpy(kd).to(dev)][:, torch.from_numpy(nd).to(dev)])
        assert rel_err(got_d, ref_d) < 6e-2, f"tgmm gate_up, expert {e}"


@pytest.mark.parametrize("scales", SCALES)
def test_gmm_fp8_vjp_matches_kernels_and_oracle(dev, scales):
    """grouped_matmul_fp8_vjp: the forward and both gradients are bit for bit the fp8 kernels on the
    quantised operands (rows / 128x128 blocks / 128-row chunks), and within 6e-2 of the float64
    product and VJP of the unquantised operands; an empty group gets a zero weight gradient."""
    from mintext_amd.kernels.fp8 import (grouped_matmul_fp8, grouped_matmul_fp8_dlhs, grouped_matmul_fp8_vjp,
                                         quantize_fp8_grouped_t, quantize_fp8_rows, quantize_fp8_weights,
                                         quantize_fp8_weights_t, tgmm_fp8)

    rng = np.random.default_rng(5)
    M, Kin, Kout, E = 3000, 512, 768, 12
    gs = _zipf_groups(rng, M, E)
    tg = _t(gs, dev)
    x = torch.randn(M, Kin, device=dev).bfloat16().requires_grad_(True)
    w = (torch.randn(E, Kin, Kout, device=dev) * 0.02).bfloat16().requires_grad_(True)
    G = torch.randn(M, Kout, device=dev).bfloat16()
    f8s = dict(scales=scales)
    out = grouped_matmul_fp8_vjp(x, w, tg, **f8s)
    out.backward(G)
    assert out.dtype == torch.bfloat16 and x.grad.dtype == torch.bfloat16 and w.grad.dtype == torch.bfloat16
    with torch.no_grad():
        ref_out = grouped_matmul_fp8(*quantize_fp8_rows(x, **f8s), *quantize_fp8_weights(w, **f8s), tg, **f8s)
        ref_dx = grouped_matmul_fp8_dlhs(*quantize_fp8_rows(G, **f8s), *quantize_fp8_weights_t(w, **f8s), tg, **f8s)
        ref_dw = tgmm_fp8(*quantize_fp8_grouped_t(x, tg, **f8s), *quantize_fp8_grouped_t(G, tg, blocks=True, **f8s),
                          tg, M, **f8s)
    assert torch.equal(out, ref_out) and torch.equal(x.grad, ref_dx) and torch.equal(w.grad, ref_dw)
    f = lambda t: t.detach().float().cpu().numpy()
    assert rel_err(f(out), O.gmm(f(x), f(w), gs)) < 6e-2
    assert rel_err(f(x.grad), O.gmm_dlhs(f(G), f(w), gs)) < 6e-2
    assert rel_err(f(w.grad), O.tgmm(f(x), f(G), gs)) < 6e-2
    for e in np.flatnonzero(gs == 0):
        assert not w.grad[e].any()


@pytest.mark.parametrize("scales", SCALES)
@pytest.mark.parametrize("T,D,E,K,I", [(1024, 512, 16, 4, 256), (2048, 256, 8, 2, 512)])
def test_fp8_layer_training_matches_oracle_vjp(dev, T, D, E, K, I, scales):
    """moe_experts_forward_fp8_train (all six GEMMs on fp8 operands) against the float64 forward
    and VJP of the unquantised layer.  Each fp8 GEMM is within 6e-2 of its unquantised product
    (test above); the layer and its gradients pass through two of them in series (the output:
    x, then the SwiGLU output quantised; dx: the down and gate_up dlhs), so the bound is 1e-1, as
    for the fp8 inference layer (test_gpu_moe.py)."""
    from mintext_amd.kernels import route_topk
    from mintext_amd.moe import moe_experts_forward_fp8_train

    gen = torch.Generator(device=dev)
    gen.manual_seed(T + E)
    x = torch.randn(T, D, device=dev, generator=gen).bfloat16().requires_grad_(True)
    gu = (torch.randn(E, D, 2 * I, device=dev, generator=gen) * 0.05).bfloat16().requires_grad_(True)
    dn = (torch.randn(E, I, D, device=dev, generator=gen) * 0.05).bfloat16().requires_grad_(True)
    idx, w = route_topk(torch.randn(T, E, device=dev, generator=gen), K)
    w = w.clone().requires_grad_(True)
    G = torch.randn(T, D, device=dev, generator=gen)
    out = moe_experts_forward_fp8_train(x, idx, w, gu, dn, scales=scales)
    assert out.dtype == torch.float32
    (out * G).sum().backward()
    f = lambda a: a.detach().float().cpu().numpy()
    ref = O.moe_experts(f(x), idx.cpu().numpy(), f(w), f(gu), f(dn))
    errs = {"out": rel_err(f(out), ref)}
    dx, dw, dgu, ddn = O.moe_experts_vjp(f(x), idx.cpu().numpy(), f(w), f(gu), f(dn), f(G))
    for got, r, name in ((x.grad, dx, "x"), (w.grad, dw, "w"), (gu.grad, dgu, "gate_up"), (dn.grad, ddn, "down")):
        errs[name] = rel_err(f(got), r)
    print("fp8 training layer rel errors", {k: round(v, 4) for k, v in errs.items()})
    assert all(v < 1e-1 for v in errs.values()), errs


def test_tgmm_fp8_p2_chunks_of_very_different_magnitude(dev):
    """Power-of-two mode: neighbouring 128-row chunks of an expert whose scales are 2^100 and more
    apart (a normal chunk, a chunk of values near 1e-33 with a subnormal-range scale, an all-zero
    chunk, then normal again) -- the accumulators stay in true units, so dW is finite and within
    1e-2 of the dequantised float64 product and 6e-2 of the unquantised one.  The dlhs of the same
    rows goes through the forward kernel's power-of-two mode."""
    from mintext_amd.kernels.fp8 import (grouped_matmul_fp8_dlhs, quantize_fp8_grouped_t, quantize_fp8_rows,
                                         quantize_fp8_weights_t, tgmm_fp8)

    gs = np.array([512, 0, 384], np.int32)
    M, F, N = int(gs.sum()), 256, 512
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    x = torch.randn(M, F, device=dev, generator=gen)
    g = torch.randn(M, N, device=dev, generator=gen)
    x[128:256] *= 1e-33   # chunk 1 of expert 0: scale near 2^-117
    g[128:256] *= 1e-30
    x[256:384] = 0        # chunk 2: scale 1
    x[512 + 128:512 + 256] *= 3e-28
    tg = _t(gs, dev)
    xt, xs = quantize_fp8_grouped_t(x, tg, scales="pow2")
    gt, gsc = quantize_fp8_grouped_t(g, tg, blocks=True, scales="pow2")
    dw = tgmm_fp8(xt, xs, gt, gsc, tg, M, scales="pow2")
    got = dw.float().cpu().numpy()
    assert np.isfinite(got).all() and not got[1].any()
    ref_q = O.tgmm_fp8(_u8(xt), xs.cpu().numpy(), _u8(gt), gsc.cpu().numpy(), gs, M, F, N)
    assert rel_err(got, ref_q) < 1e-2
    assert rel_err(got, O.tgmm(x.cpu().numpy(), g.cpu().numpy(), gs)) < 6e-2
    w = torch.randn(3, F, N, device=dev, generator=gen) * 0.02
    gq, gsc2 = quantize_fp8_rows(g, scales="pow2")
    wq, ws = quantize_fp8_weights_t(w, scales="pow2")
    dx = grouped_matmul_fp8_dlhs(gq, gsc2, wq, ws, tg, scales="pow2").float().cpu().numpy()
    assert np.isfinite(dx).all()
    ref_dx = O.gmm_fp8_dlhs(_u8(gq), gsc2.cpu().numpy(), _u8(wq), ws.cpu().numpy(), gs)
    assert rel_err(dx, ref_dx) < 1e-2

"""GPU parity at the benchmark's full sizes, on exactly the flows ``bench.py`` times.

Each test builds the inputs of one bench config with ``bench.layer_inputs`` (same seeds, same
shapes), runs the layer through the product API and through the bench's step sequence (which
must agree bit for bit), and checks sampled rows of every stage against the float64 oracle:

* C2 (Mixtral, bf16): router -> permutation -> gate_up + SwiGLU on the gathered token rows ->
  down (K_in = 14336) -> combine;
* C3 (DeepSeek-V3, bf16): sigmoid group-limited router, the routed GEMMs, the shared expert and
  the combine with the shared output added in its pass (``unroute_add``);
* C4 (Qwen3, fp8): token-order 1x128 quantiser -> fp8 gate_up + SwiGLU + re-quantisation on the
  gathered rows -> fp8 down at K_in = 768 -> combine;
* C5 (Qwen3 backward, bf16, Zipf-skewed loads): dlhs of both expert GEMMs and both tgmm.
* the study of the layer's HBM-bound backward kernels (``bench.py --study dispatch-bwd``, C2 /
  C3 / C4 shapes): the combine and route VJPs, SwiGLU and its VJP.

Sampled rows cover every expert's first and last rows (partial m-tiles) and random interior
rows; tolerances are the north-star ones (bf16 2e-2, fp8 6e-2 against the unquantised product
and 1e-2 against the dequantised one, f32 combine 1e-5), written at each check.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_err
from oracle import moe_oracle as O

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]


def _bench():
    import bench

    return bench


def _host(t) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def _u8(t) -> np.ndarray:
    return t.view(torch.uint8).cpu().numpy()


def _rows_of(gs: np.ndarray, rng, per_expert: int, experts=None) -> np.ndarray:
    """First, last and random rows of each (non-empty) expert in the grouped layout."""
    off = np.concatenate([[0], np.cumsum(gs)])
    experts = range(len(gs)) if experts is None else experts
    rows = []
    for e in experts:
        a, b = int(off[e]), int(off[e + 1])
        if b == a:
            continue
        rows += [a, b - 1] + list(rng.integers(a, b, per_expert))
    return np.unique(np.asarray(rows, np.int64))


def _expert_of(gs, rows):
    off = np.concatenate([[0], np.cumsum(gs)])
    return np.searchsorted(off, rows, side="right") - 1


def _flow_bf16(x, idx, w, gate_up, down, K, shared=None):
    """The bench's step (bench.py run(), gathered): permutation, gathered gate_up + SwiGLU,
    down, combine (+ the separate shared expert's output added in the combine's pass)."""
    from mintext_amd.kernels import grouped_matmul_vjp, unroute
    from mintext_amd.kernels.grouped_matmul import grouped_matmul_swiglu_gathered
    from mintext_amd.kernels.moe_dispatch import route_indices, unroute_add
    from mintext_amd.moe import shared_expert_forward

    si, gs, inv = route_indices(idx, gate_up.shape[0])
    inter = grouped_matmul_swiglu_gathered(x, si, K, gate_up, gs)
    o = grouped_matmul_vjp(inter, down, gs)
    sh = None if shared is None else shared_expert_forward(x, shared[0], shared[1])
    out = unroute(o, si, w, K) if sh is None else unroute_add(o, si, w, K, sh)
    return dict(si=si, gs=gs, inv=inv, inter=inter, o=o, sh=sh, out=out)


def _check_bf16_layer(f, x, idx, w, gate_up, down, K, rows, tokens, shared=None):
    """Stage-by-stage checks of a bf16 layer run ``f`` (the dict of _flow_bf16) on sampled rows."""
    si = f["si"].cpu().numpy().astype(np.int64)
    gs = f["gs"].cpu().numpy()
    ex = _expert_of(gs, rows)
    xh = _host(x[torch.from_numpy(si[rows] // K).to(x.device)])
    inter_g = _host(f["inter"][torch.from_numpy(rows).to(x.device)])
    o_g = _host(f["o"][torch.from_numpy(rows).to(x.device)])
    ref_inter = np.empty_like(inter_g)
    ref_o = np.empty_like(o_g)
    ref_o_chain = np.empty_like(o_g)
    for e in np.unique(ex):
        sel = np.flatnonzero(ex == e)
        wgu = _host(gate_up[int(e)])
        wdn = _host(down[int(e)])
        ref_inter[sel] = O.swiglu(xh[sel] @ wgu)                  # gate_up + SwiGLU, float64
        ref_o[sel] = inter_g[sel] @ wdn                           # down on the GPU's own intermediate
        ref_o_chain[sel] = ref_inter[sel] @ wdn                   # down on the float64 intermediate
    assert rel_err(inter_g, ref_inter) < 2e-2, "gate_up + SwiGLU (bf16)"
    assert rel_err(o_g, ref_o) < 2e-2, "down GEMM (bf16)"
    # combine on the sampled tokens: f32 sum of the GPU's own expert rows, against float64
    inv = f["inv"].cpu().numpy().astype(np.int64)
    wt = w.detach().cpu().numpy().astype(np.float64)
    rows_t = inv[(tokens[:, None] * K + np.arange(K)[None, :]).ravel()]
    o_t = _host(f["o"][torch.from_numpy(rows_t).to(x.device)]).reshape(len(tokens), K, -1)
    ref_out = np.einsum("tkd,tk->td", o_t, wt[tokens])
    if shared is not None:
        sh_g = _host(f["sh"][torch.from_numpy(tokens).to(x.device)])
        ref_out = ref_out + sh_g
        # the shared expert itself against float64
        xt = _host(x[torch.from_numpy(tokens).to(x.device)])
        ref_sh = O.swiglu(xt @ _host(shared[0][0])) @ _host(shared[1][0])
        assert rel_err(sh_g, ref_sh) < 2e-2, "shared expert (bf16)"
    out_t = _host(f["out"][torch.from_numpy(tokens).to(x.device)])
    assert rel_err(out_t, ref_out) < 1e-5, "combine (f32)"
    return ref_o_chain


def _sample_tokens(si, rows, K, n, rng):
    """Tokens of some sampled rows (so their expert rows are in the float64 chain), at most n."""
    toks = np.unique(si[rows] // K)
    return np.sort(rng.choice(toks, min(n, toks.size), replace=False))


def test_c2_mixtral_layer_full_size(dev):
    """C2 at T=8192, D=4096, E=8, K=2, I=14336: the headline flow, stage by stage."""
    from mintext_amd.kernels import grouped_matmul_swiglu, route, route_topk
    from mintext_amd.moe import moe_experts_forward

    B = _bench()
    cfg = B.CONFIGS["mixtral"]
    K = cfg["K"]
    with torch.no_grad():
        x, logits, gate_up, down, _, _ = B.layer_inputs("mixtral", dev)
        idx, w = route_topk(logits, K, **B.router_kwargs("mixtral"))
        f = _flow_bf16(x, idx, w, gate_up, down, K)
        # the product API runs the same flow: same bits
        assert torch.equal(moe_experts_forward(x, idx, w, gate_up, down), f["out"])
        # the gathered gate_up reads the rows route() would copy: same bits at full size
        st, si2, gs2 = route(x, idx, cfg["E"])
        assert torch.equal(si2, f["si"]) and torch.equal(gs2, f["gs"])
        assert torch.equal(grouped_matmul_swiglu(st, gate_up, gs2), f["inter"])
    oi, _, _ = O.router_softmax(logits.float().cpu().numpy(), K)
    assert np.array_equal(idx.cpu().numpy(), oi)
    rng = np.random.default_rng(21)
    gs = f["gs"].cpu().numpy()
    rows = _rows_of(gs, rng, 6)
    si = f["si"].cpu().numpy().astype(np.int64)
    tokens = _sample_tokens(si, rows, K, 16, rng)
    # end to end on tokens whose both rows are in the sample: rebuild the sample from the tokens
    inv = f["inv"].cpu().numpy().astype(np.int64)
    rows = np.unique(np.concatenate([rows, inv[(tokens[:, None] * K + np.arange(K)).ravel()]]))
    ref_o = _check_bf16_layer(f, x, idx, w, gate_up, down, K, rows, tokens)
    pos = {int(r): i for i, r in enumerate(rows)}
    wt = w.cpu().numpy().astype(np.float64)
    ref = np.stack([sum(wt[t, k] * ref_o[pos[int(inv[t * K + k])]] for k in range(K)) for t in tokens])
    assert rel_err(_host(f["out"][torch.from_numpy(tokens).to(dev)]), ref) < 2e-2, "layer end to end (bf16)"


def test_c3_deepseek_layer_full_size(dev):
    """C3 at T=4096, D=7168, E=256 (+1 shared), K=8, I=2048: sigmoid group-limited router, the
    routed GEMMs, the shared expert and its addition in the combine's pass."""
    from mintext_amd.kernels import route_topk
    from mintext_amd.moe import moe_layer_forward

    B = _bench()
    cfg = B.CONFIGS["deepseek"]
    K, E = cfg["K"], cfg["E"]
    rkw = B.router_kwargs("deepseek")
    with torch.no_grad():
        x, logits, gate_up, down, shared, _ = B.layer_inputs("deepseek", dev)
        idx, w, s = route_topk(logits, K, return_scores=True, **rkw)
        f = _flow_bf16(x, idx, w, gate_up, down, K, shared=shared)
        out_api, idx_api, w_api = moe_layer_forward(logits, x, gate_up, down, k=K, shared_gate_up=shared[0],
                                                    shared_down=shared[1], **rkw)
        assert torch.equal(idx_api, idx) and torch.equal(w_api, w)
        assert torch.equal(out_api, f["out"])
    # routing bit-exact given the GPU's own f32 scores (the scores at 1e-6)
    sh = s.cpu().numpy()
    np.testing.assert_allclose(sh, O.sigmoid_f32(logits.float().cpu().numpy()), rtol=1e-6)
    oi, ow, _ = O.router_sigmoid_group(None, K, n_group=cfg["n_group"], topk_group=cfg["topk_group"],
                                       routed_scaling_factor=cfg["scale"], scores=sh)
    assert np.array_equal(idx.cpu().numpy(), oi)
    np.testing.assert_allclose(w.cpu().numpy(), ow, rtol=1e-5)
    rng = np.random.default_rng(31)
    si = f["si"].cpu().numpy().astype(np.int64)
    inv = f["inv"].cpu().numpy().astype(np.int64)
    tokens = np.sort(rng.choice(cfg["T"], 6, replace=False))
    rows = inv[(tokens[:, None] * K + np.arange(K)).ravel()]
    gs = f["gs"].cpu().numpy()
    # plus the first and last rows of a few experts (partial m-tiles)
    rows = np.unique(np.concatenate([rows, _rows_of(gs, rng, 0, experts=rng.choice(E, 6, replace=False))]))
    ref_o = _check_bf16_layer(f, x, idx, w, gate_up, down, K, rows, tokens, shared=shared)
    pos = {int(r): i for i, r in enumerate(rows)}
    wt = w.cpu().numpy().astype(np.float64)
    xt = _host(x[torch.from_numpy(tokens).to(dev)])
    ref_sh = O.swiglu(xt @ _host(shared[0][0])) @ _host(shared[1][0])
    ref = np.stack([sum(wt[t, k] * ref_o[pos[int(inv[t * K + k])]] for k in range(K)) for t in tokens]) + ref_sh
    assert rel_err(_host(f["out"][torch.from_numpy(tokens).to(dev)]), ref) < 2e-2, "layer end to end (bf16)"


@pytest.mark.parametrize("scales", ["amax", "pow2"])
def test_c4_qwen3_fp8_layer_full_size(dev, scales):
    """C4 at T=16384, D=2048, E=128, K=8, I=768 in blockwise fp8 (amax/448 and power-of-two scales):
    quantiser codes bit-exact, gate_up + SwiGLU and the K_in = 768 down GEMM against the dequantised
    float64 oracle (1e-2) and the unquantised one (6e-2; the down GEMM against the product of the
    GPU's own bf16 SwiGLU output with the unquantised weights), combine 1e-5, the layer 1e-1 (two
    quantisations in series)."""
    from mintext_amd.kernels import route_topk, unroute
    from mintext_amd.kernels.fp8 import (grouped_matmul_fp8, grouped_matmul_fp8_swiglu_gathered, quantize_fp8_rows,
                                         quantize_fp8_weights)
    from mintext_amd.kernels.moe_dispatch import route_indices
    from mintext_amd.moe import moe_experts_forward_fp8

    B = _bench()
    cfg = B.CONFIGS["qwen3_fp8"]
    K, E, I = cfg["K"], cfg["E"], cfg["I"]
    with torch.no_grad():
        x, logits, gate_up, down, _, _ = B.layer_inputs("qwen3_fp8", dev)
        idx, w = route_topk(logits, K, **B.router_kwargs("qwen3_fp8"))
        f8s = dict(scales=scales)
        guq, gus = quantize_fp8_weights(gate_up, **f8s)
        dnq, dns = quantize_fp8_weights(down, **f8s)
        # the bench's step
        xq, xs = quantize_fp8_rows(x, **f8s)
        si, gs, inv = route_indices(idx, E)
        yq, ys, yb = grouped_matmul_fp8_swiglu_gathered(xq, xs, si, K, guq, gus, gs, return_bf16=True, **f8s)
        o = grouped_matmul_fp8(yq, ys, dnq, dns, gs, **f8s)
        out = unroute(o, si, w, K)
        assert torch.equal(moe_experts_forward_fp8(x, idx, w, guq, gus, dnq, dns, **f8s), out)
        yq2, ys2 = grouped_matmul_fp8_swiglu_gathered(xq, xs, si, K, guq, gus, gs, **f8s)
        assert torch.equal(_u8t(yq2), _u8t(yq)) and torch.equal(ys2, ys)
    oi, _, _ = O.router_softmax(logits.float().cpu().numpy(), K)
    assert np.array_equal(idx.cpu().numpy(), oi)
    rng = np.random.default_rng(41)
    gsh = gs.cpu().numpy()
    sih = si.cpu().numpy().astype(np.int64)
    invh = inv.cpu().numpy().astype(np.int64)
    tokens = np.sort(rng.choice(cfg["T"], 8, replace=False))
    big, small = int(np.argmax(gsh)), int(np.argmin(np.where(gsh > 0, gsh, 1 << 30)))
    experts = np.unique(np.concatenate([[big, small], rng.choice(E, 10, replace=False)]))
    rows = np.unique(np.concatenate([invh[(tokens[:, None] * K + np.arange(K)).ravel()],
                                     _rows_of(gsh, rng, 2, experts=experts)]))
    tr = torch.from_numpy(rows).to(dev)
    tok = sih[rows] // K
    # quantiser: codes and scales of the sampled tokens bit for bit
    oq, os_ = O.quant_fp8_rows(x[torch.from_numpy(tok).to(dev)].float().cpu().numpy(), scales=scales)
    assert np.array_equal(_u8(xq[torch.from_numpy(tok).to(dev)]), oq)
    assert np.array_equal(xs[torch.from_numpy(tok).to(dev)].cpu().numpy(), os_)
    ex = _expert_of(gsh, rows)
    xdq = O.dequant_rows(oq, os_)
    x64 = _host(x[torch.from_numpy(tok).to(dev)])
    yb_g, o_g = _host(yb[tr]), _host(o[tr])
    yq_g, ys_g = _u8(yq[tr]), ys[tr].cpu().numpy()
    ref_y, ref_y_unq, ref_o, ref_o_unq, ref_o_yb = (np.empty_like(yb_g), np.empty_like(yb_g), np.empty_like(o_g),
                                                    np.empty_like(o_g), np.empty_like(o_g))
    for e in np.unique(ex):
        sel = np.flatnonzero(ex == e)
        e = int(e)
        wgu = O.dequant_weights(_u8(guq[e])[None], gus[e].cpu().numpy()[None])[0]
        wdn = O.dequant_weights(_u8(dnq[e])[None], dns[e].cpu().numpy()[None])[0]
        ref_y[sel] = O.swiglu(xdq[sel] @ wgu)
        ref_y_unq[sel] = O.swiglu(x64[sel] @ _host(gate_up[e]))
        ref_o[sel] = O.dequant_rows(yq_g[sel], ys_g[sel]) @ wdn    # down at K_in = 768 on the GPU's codes
        ref_o_unq[sel] = ref_y_unq[sel] @ _host(down[e])
        ref_o_yb[sel] = yb_g[sel] @ _host(down[e])                 # the GPU's own SwiGLU output, unquantised W
    assert rel_err(yb_g, ref_y) < 1e-2, "fp8 gate_up + SwiGLU vs dequantised oracle"
    assert rel_err(yb_g, ref_y_unq) < 6e-2, "fp8 gate_up + SwiGLU vs unquantised"
    # the re-quantised intermediate: within e4m3's half-ulp of the SwiGLU output
    assert rel_err(O.dequant_rows(yq_g, ys_g), ref_y) < 4e-2, "SwiGLU re-quantisation"
    assert rel_err(o_g, ref_o) < 1e-2, "fp8 down (K_in=768) vs dequantised oracle"
    assert rel_err(o_g, ref_o_yb) < 6e-2, "fp8 down (K_in=768) vs bf16 SwiGLU output x unquantised down"
    assert rel_err(o_g, ref_o_unq) < 1e-1, "fp8 down vs unquantised chain"
    wt = w.cpu().numpy().astype(np.float64)
    o_t = _host(o[torch.from_numpy(invh[(tokens[:, None] * K + np.arange(K)).ravel()]).to(dev)])
    ref_out = np.einsum("tkd,tk->td", o_t.reshape(len(tokens), K, -1), wt[tokens])
    out_t = _host(out[torch.from_numpy(tokens).to(dev)])
    assert rel_err(out_t, ref_out) < 1e-5, "combine (f32)"
    pos = {int(r): i for i, r in enumerate(rows)}
    ref = np.stack([sum(wt[t, k] * ref_o_unq[pos[int(invh[t * K + k])]] for k in range(K)) for t in tokens])
    assert rel_err(out_t, ref) < 1e-1, "fp8 layer end to end vs unquantised"


def _u8t(t):
    return t.view(torch.uint8)


@pytest.mark.parametrize("loads", ["bench", "emptied"])
def test_c5_qwen3_backward_full_size(dev, loads):
    """C5 at M=131072 with Zipf(1.2)-skewed loads: dlhs of both expert GEMMs on sampled rows and
    tgmm of both on sampled blocks, against float64.  ``bench``: the bench's routing (its
    popularity bias gives 58..13462 rows per expert, no empty group); ``emptied``: the same rows
    with the first, an interior and the last expert's rows handed to a neighbour, so that empty
    groups sit at both ends and between loaded ones (empty groups give zero tgmm blocks,
    grouped_matmul.py:197-235)."""
    from mintext_amd.kernels import grouped_matmul_swiglu, route, route_topk, tgmm
    from mintext_amd.kernels.grouped_matmul import _gmm_dlhs

    B = _bench()
    cfg = B.CONFIGS["qwen3_bwd"]
    T, D, E, K, I = cfg["T"], cfg["D"], cfg["E"], cfg["K"], cfg["I"]
    M = T * K
    with torch.no_grad():
        x, logits, gate_up, down, _, g = B.layer_inputs("qwen3_bwd", dev)
        idx, _ = route_topk(logits, K)
        st, si, gs = route(x, idx, E)
        gsh = gs.cpu().numpy().copy()
        # the skew of the bench's routing: the most popular expert takes over 8x the mean
        assert gsh.max() >= 8 * gsh.mean() and gsh.min() < gsh.mean() / 8
        if loads == "emptied":
            for e in (0, 41, E - 1):  # first, interior and last expert; rows go to a neighbour
                nb = e + 1 if e + 1 < E else e - 1
                gsh[nb] += gsh[e]
                gsh[e] = 0
            assert (gsh == 0).sum() == 3 and gsh.sum() == M
            gs = torch.from_numpy(gsh).to(dev)
        y = grouped_matmul_swiglu(st, gate_up, gs)
        gy = torch.randn(M, D, device=dev, generator=g).bfloat16()
        gh = torch.randn(M, 2 * I, device=dev, generator=g).bfloat16()
        a = _gmm_dlhs(gy, down, gs)       # d inter   [M, I]
        b = _gmm_dlhs(gh, gate_up, gs)    # d x       [M, D]
        c = tgmm(y, gy, gs)               # d down    [E, I, D]
        d = tgmm(st, gh, gs)              # d gate_up [E, D, 2I]
    rng = np.random.default_rng(51)
    nz = np.flatnonzero(gsh)
    experts = np.unique(np.concatenate([[int(np.argmax(gsh)), int(nz[np.argmin(gsh[nz])])],
                                        rng.choice(nz, 14, replace=False)]))
    rows = _rows_of(gsh, rng, 3, experts=experts)
    tr = torch.from_numpy(rows).to(dev)
    ex = _expert_of(gsh, rows)
    gy_h, gh_h = _host(gy[tr]), _host(gh[tr])
    a_g, b_g = _host(a[tr]), _host(b[tr])
    ref_a, ref_b = np.empty_like(a_g), np.empty_like(b_g)
    for e in np.unique(ex):
        sel = np.flatnonzero(ex == e)
        ref_a[sel] = gy_h[sel] @ _host(down[int(e)]).T
        ref_b[sel] = gh_h[sel] @ _host(gate_up[int(e)]).T
    assert rel_err(a_g, ref_a) < 2e-2, "dlhs of the down GEMM"
    assert rel_err(b_g, ref_b) < 2e-2, "dlhs of the gate_up GEMM"
    off = np.concatenate([[0], np.cumsum(gsh)])
    ks, ns = np.sort(rng.choice(I, 24, replace=False)), np.sort(rng.choice(D, 24, replace=False))
    kd, nd = np.sort(rng.choice(D, 24, replace=False)), np.sort(rng.choice(2 * I, 24, replace=False))
    check = list(experts[:6]) + [int(e) for e in np.flatnonzero(gsh == 0)]
    for e in check:
        r0, r1 = int(off[e]), int(off[e + 1])
        if r1 == r0:
            assert (c[e] == 0).all() and (d[e] == 0).all(), f"empty expert {e}"
            continue
        got_c = _host(c[e][torch.from_numpy(ks).to(dev)][:, torch.from_numpy(ns).to(dev)])
        got_d = _host(d[e][torch.from_numpy(kd).to(dev)][:, torch.from_numpy(nd).to(dev)])
        ref_c = _host(y[r0:r1][:, torch.from_numpy(ks).to(dev)]).T @ _host(gy[r0:r1][:, torch.from_numpy(ns).to(dev)])
        ref_d = _host(st[r0:r1][:, torch.from_numpy(kd).to(dev)]).T @ _host(gh[r0:r1][:, torch.from_numpy(nd).to(dev)])
        assert rel_err(got_c, ref_c) < 2e-2, f"tgmm (down) expert {e}"
        assert rel_err(got_d, ref_d) < 2e-2, f"tgmm (gate_up) expert {e}"


@pytest.mark.parametrize("cfg", ["mixtral", "deepseek", "qwen3"])
def test_dispatch_bwd_study_flows_full_size(dev, cfg):
    """The calls ``bench.py --study dispatch-bwd`` times, at its shapes: the combine VJP
    (mtx_unroute_bwd, f32 dout and weights, bf16 rows) with d_sorted bit-exact over the whole
    array against f32 products rounded to bf16 and d_weights within 1e-5 (plus a sqrt(D)-scaled
    absolute term) of float64 on sampled tokens; the route VJP (mtx_unroute, unit weights, bf16)
    within one bf16 rounding (plus the f32 sum's own rounding) of float64 on sampled tokens; SwiGLU and its VJP (bf16) bit-identical
    between the 16-byte vector kernels and the scalar kernels over the whole array (the scalar
    ones on a copy one element past a 16-byte boundary) and within 2e-2 of the oracle on sampled
    rows."""
    from mintext_amd import _lib as L

    c = _bench().DISPATCH_BWD_CONFIGS[cfg]
    N, K, D, I = c["N"], c["K"], c["D"], c["I"]
    M = N * K
    st = L.stream(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    inv = torch.randperm(M, device=dev, generator=g).int()
    w = torch.rand(N, K, device=dev, generator=g)
    dout = torch.randn(N, D, device=dev, generator=g)
    Y = torch.randn(M, D, device=dev, generator=g).bfloat16()
    dY = torch.empty_like(Y)
    dw = torch.empty_like(w)
    dx = torch.empty(N, D, dtype=torch.bfloat16, device=dev)
    L.call("mtx_unroute_bwd", L.ptr(dout), L.MTX_F32, L.ptr(Y), L.MTX_BF16, L.ptr(inv), L.ptr(w), L.MTX_F32,
           N, K, D, L.ptr(dY), L.ptr(dw), st)
    L.call("mtx_unroute", L.ptr(Y), L.MTX_BF16, L.ptr(inv), None, L.MTX_F32, N, K, D, L.ptr(dx), L.MTX_BF16, st)
    torch.cuda.synchronize()
    invc = inv.long().cpu()
    want = torch.empty(M, D, dtype=torch.float32)
    want[invc] = (w.cpu().reshape(-1, 1) * dout.cpu().repeat_interleave(K, dim=0))
    assert torch.equal(dY.cpu(), want.to(torch.bfloat16))
    del want
    rng = np.random.default_rng(0)
    toks = np.unique(np.concatenate([[0, N - 1], rng.integers(0, N, 254)]))
    rows = invc.reshape(N, K)[toks]                           # [t, K] sorted rows of each sampled token
    Yt = _host(Y[rows.reshape(-1).to(dev)]).reshape(len(toks), K, D)
    dw_ref = np.einsum("tkd,td->tk", Yt, _host(dout[torch.from_numpy(toks).to(dev)]))
    np.testing.assert_allclose(_host(dw[torch.from_numpy(toks).to(dev)]), dw_ref, rtol=1e-5, atol=1e-5 * np.sqrt(D))
    dx_ref = Yt.sum(axis=1)
    got = _host(dx[torch.from_numpy(toks).to(dev)])
    # one bf16 rounding of the f32 sum of K bf16 values (the f32 sum itself exact but for
    # operands whose exponents differ by more than f32's mantissa allows)
    bound = 2.0 ** -8 * np.abs(dx_ref) + K * 2.0 ** -22 * np.abs(Yt).max(axis=1)
    assert np.all(np.abs(got - dx_ref) <= bound)
    del inv, w, dout, Y, dY, dw, dx

    h = torch.randn(M, 2 * I, device=dev, generator=g).bfloat16()
    dy = torch.randn(M, I, device=dev, generator=g).bfloat16()

    def at_offset(a):
        flat = torch.empty(a.numel() + 8, dtype=a.dtype, device=dev)
        v = flat[1:1 + a.numel()].view(a.shape)
        v.copy_(a)
        return v

    outs = []
    for hh, dd in ((h, dy), (at_offset(h), at_offset(dy))):
        y = torch.empty(M, I, dtype=torch.bfloat16, device=dev)
        dh = torch.empty(M, 2 * I, dtype=torch.bfloat16, device=dev)
        L.call("mtx_swiglu", L.ptr(hh), L.MTX_BF16, M, I, L.ptr(y), st)
        L.call("mtx_swiglu_bwd", L.ptr(hh), L.ptr(dd), L.MTX_BF16, M, I, L.ptr(dh), st)
        outs.append((y, dh))
        del hh, dd
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    sr = torch.from_numpy(np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, 126)]))).to(dev)
    hs, dys = _host(h[sr]), _host(dy[sr])
    assert rel_err(_host(outs[0][0][sr]), O.swiglu(hs)) < 2e-2
    assert rel_err(_host(outs[0][1][sr]), O.swiglu_bwd(hs, dys)) < 2e-2

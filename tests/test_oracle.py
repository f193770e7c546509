"""Pin the CPU oracle (oracle/moe_oracle.py) before trusting it as the GPU checker.

Each oracle function is checked against something that does not share its code: golden
fixtures written by tests/golden/make_golden.py from HF transformers, torch.sort(stable=True)
and torch float64 matmuls; brute force on tiny inputs; closed forms and invariants.  A check
that merely re-types the oracle's formula is avoided; each comparison is chosen so that a
plausible slip (dropped bias, wrong tie order, transposed operand, unstable sort, wrong
group offset) fails it.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from conftest import golden, rel_err
from oracle import moe_oracle as O


# ---------------------------------------------------------------------------- number formats
def test_bf16_round_matches_torch():
    x = np.random.default_rng(0).standard_normal(50000).astype(np.float32) * 30
    x = np.concatenate([x, np.float32([0, -0.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, 65504, 3.4e38])])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.bf16_round(x), ref)


def test_e4m3_encode_matches_torch_fixture():
    g = golden("fp8")
    np.testing.assert_array_equal(O.e4m3_encode(g["values"]), g["codes"])


def test_e4m3_decode_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = O.e4m3_decode(codes)
    both_nan = np.isnan(ref) & np.isnan(got)
    np.testing.assert_array_equal(got[~both_nan], ref[~both_nan])
    # every finite code round-trips
    fin = ~np.isnan(ref)
    np.testing.assert_array_equal(O.e4m3_encode(ref[fin]), codes[fin])


def test_e4m3_saturates():
    assert O.e4m3_encode(np.float32([1000.0]))[0] == 0x7E
    assert O.e4m3_encode(np.float32([-470.0]))[0] == 0xFE


# --------------------------------------------------------------------------------- routers
def test_topk_ties_go_to_lower_index_bruteforce():
    rng = np.random.default_rng(1)
    vals = rng.integers(0, 3, size=(200, 6)).astype(np.float32)  # many ties
    got = O.topk_desc(vals, 3)
    for t in range(vals.shape[0]):
        brute = sorted(range(6), key=lambda e: (-vals[t, e], e))[:3]
        assert list(got[t]) == brute


def test_softmax_router_matches_hf_mixtral():
    g = golden("routers")
    idx, w, _ = O.router_softmax(g["mixtral_logits"], 2)
    np.testing.assert_array_equal(idx, g["mixtral_idx"])
    np.testing.assert_allclose(w, g["mixtral_w"], rtol=1e-6, atol=1e-7)


def test_softmax_router_matches_hf_qwen3():
    g = golden("routers")
    idx, w, _ = O.router_softmax(g["qwen_logits"], 8)
    np.testing.assert_array_equal(idx, g["qwen_idx"])
    np.testing.assert_allclose(w, g["qwen_w"], rtol=1e-6, atol=1e-7)
    idx2, w2, _ = O.router_softmax(g["qwen_logits"], 8, norm_topk_prob=False)
    np.testing.assert_array_equal(idx2, g["qwen_idx_nonorm"])
    np.testing.assert_allclose(w2, g["qwen_w_nonorm"], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("key", ["ds", "ds3"])
def test_sigmoid_group_router_matches_hf_deepseek(key):
    g = golden("routers")
    idx, w, s = O.router_sigmoid_group(g[f"{key}_logits"], 8, bias=g[f"{key}_bias"], n_group=8, topk_group=4,
                                       norm_topk_prob=True, routed_scaling_factor=2.5)
    # sigmoid bits differ by a few ulp across libms; selection below is still exact
    np.testing.assert_allclose(s, g[f"{key}_scores"], rtol=5e-7, atol=0)
    np.testing.assert_array_equal(idx, g[f"{key}_idx"])
    np.testing.assert_allclose(w, g[f"{key}_w"], rtol=1e-6)


def test_group_limited_selection_bruteforce():
    """Tiny E: enumerate group choices explicitly (moe.py:76-98 read as a definition)."""
    rng = np.random.default_rng(7)
    E, ng, tg, k = 8, 4, 2, 3
    for _ in range(200):
        s = rng.random((1, E)).astype(np.float32)
        s[0, rng.integers(0, E)] = s[0, rng.integers(0, E)]  # occasional ties
        b = (rng.standard_normal(E) * 0.05).astype(np.float32)
        idx, _ = O.select_sigmoid_group(s, b, k, ng, tg)
        r = (s[0] + b).astype(np.float32)
        gsc = [float(np.float32(sorted(r[2 * q:2 * q + 2])[-1]) + np.float32(sorted(r[2 * q:2 * q + 2])[-2]))
               for q in range(ng)]
        groups = sorted(range(ng), key=lambda q: (-np.float32(gsc[q]), q))[:tg]
        cand = [e for e in range(E) if e // 2 in groups]
        best = sorted(cand, key=lambda e: (-r[e], e))[:k]
        assert list(idx[0]) == best


def test_bias_steers_selection():
    """The reference's router test: bias [10,0,0,0] makes expert 0 always selected (test_model.py:468-478)."""
    lg = np.random.default_rng(3).standard_normal((32, 4)).astype(np.float32)
    idx, _, _ = O.router_sigmoid_group(lg, 2, bias=np.float32([10, 0, 0, 0]), n_group=2, topk_group=1)
    assert (idx[:, 0] == 0).all()


# ------------------------------------------------------------------------------ router VJP
@pytest.mark.parametrize("case", [("mixtral", "mixtral", "softmax", True, 1.0), ("qwen_norm", "qwen", "softmax", True, 1.0),
                                  ("qwen_nonorm", "qwen", "softmax", False, 1.0),
                                  ("ds_norm", "ds", "sigmoid_group", True, 2.5),
                                  ("ds_nonorm", "ds", "sigmoid_group", False, 2.5)])
def test_router_vjp_matches_hf_autograd(case):
    """d logits of sum_k w[t,k] G[t, idx[t,k]]: torch autograd through the HF routers (float32)."""
    tag, base, scoring, norm, scale = case
    g = golden("router_grads")
    lg, G, idx = g[f"{base}__logits"], g[f"{base}__G"], g[f"{tag}__idx"]
    if scoring == "softmax":
        ours, _, _ = O.router_softmax(lg, idx.shape[1], norm, scale)
    else:
        ours, _, _ = O.router_sigmoid_group(lg, idx.shape[1], g["ds__bias"], 8, 4, norm, scale)
    for t in range(lg.shape[0]):  # HF's DeepSeek top-k is unsorted: same sets
        assert set(ours[t].tolist()) == set(idx[t].tolist())
    dw = np.take_along_axis(G, idx, axis=1)
    dl = O.router_vjp(lg, idx, dw, None, scoring, norm, scale)
    assert rel_err(dl, g[f"{tag}__dl"]) < 2e-6
    # the selection is not differentiated: unselected experts of a renormalised softmax get 0
    if scoring == "softmax" and norm:
        mask = np.ones_like(dl, bool)
        np.put_along_axis(mask, idx, False, axis=1)
        assert np.abs(dl[mask]).max() == 0.0 and np.abs(g[f"{tag}__dl"][mask]).max() < 1e-6


@pytest.mark.parametrize("scoring", ["sigmoid_group", "softmax"])
def test_router_vjp_scores_term_matches_torch_autograd(scoring):
    g = golden("router_grads")
    lg, H = g["ds__logits"].astype(np.float64), g["scores__H"].astype(np.float64)
    idx = np.zeros((lg.shape[0], 1), np.int32)
    dl = O.router_vjp(lg, idx, None, H, scoring, True, 1.0)
    ref = g["scores__dl_sigmoid"] if scoring == "sigmoid_group" else g["scores__dl_softmax"]
    assert rel_err(dl, ref) < 1e-7  # the fixture used H before its float32 storage rounding


@pytest.mark.parametrize("scoring,norm", [("softmax", True), ("softmax", False), ("sigmoid_group", True),
                                          ("sigmoid_group", False)])
def test_router_vjp_central_differences(scoring, norm):
    """The closed form against central differences of the weights/scores restatement."""
    rng = np.random.default_rng(7)
    T, E, k = 6, 12, 3
    lg = rng.standard_normal((T, E))
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    dw, ds = rng.standard_normal((T, k)), rng.standard_normal((T, E))
    f = lambda l: sum(float((a * b).sum()) for a, b in zip(O.router_weights_given_idx(l, idx, scoring, norm, 2.5),
                                                             (dw, ds)))
    num = np.zeros((T, E))
    h = 1e-6
    for t, e in itertools.product(range(T), range(E)):
        p, m = lg.copy(), lg.copy()
        p[t, e] += h
        m[t, e] -= h
        num[t, e] = (f(p) - f(m)) / (2 * h)
    # scores enter with unit weight (no routed scaling), weights with the scaling factor
    dl = O.router_vjp(lg, idx, dw, ds, scoring, norm, 2.5)
    assert np.abs(dl - num).max() < 1e-7


def test_moe_block_vjp_matches_hf_deepseek_autograd():
    """Block backward, router included: HF DeepseekV3MoE (float64 experts, float32 router) under
    torch autograd on the shared-expert fixture's inputs."""
    p, g = _block_inputs(), golden("moe_block_grads")
    r = O.moe_block_vjp(p["x"], p["wg"], p["gate_up"], p["down"], g["G"], k=p["K"], bias=p["bias"],
                        n_group=p["n_group"], topk_group=p["topk_group"], routed_scaling_factor=p["scale"],
                        shared_gate_up=p["shared_gate_up"], shared_down=p["shared_down"])
    assert rel_err(r["dx"], g["dx"]) < 1e-6
    assert rel_err(r["d_gate_weight"], g["dwg"]) < 1e-6
    # HF's routed weights are float32: every routed term carries their 1e-7 rounding
    assert rel_err(r["d_gate_up"], g["dgate_up"]) < 1e-6
    assert rel_err(r["d_down"], g["ddown"]) < 1e-6
    assert rel_err(r["d_shared_gate_up"], g["dshared_gate_up"]) < 1e-12
    assert rel_err(r["d_shared_down"], g["dshared_down"]) < 1e-12
    # the router's term is a real part of dx and the only source of the gate weight's gradient
    assert np.abs(g["dwg"]).max() > 1e-2


# -------------------------------------------------------------------------------- dispatch
def _dispatch_cases():
    g = golden("dispatch")
    names = sorted({k.split("__")[0] for k in g.files})
    return g, names


def test_route_matches_torch_stable_sort_fixtures():
    g, names = _dispatch_cases()
    for n in names:
        idx, E = g[f"{n}__idx"], int(g[f"{n}__E"])
        K = idx.shape[1]
        x = np.arange(idx.shape[0] * 3, dtype=np.float32).reshape(idx.shape[0], 3)
        st, perm, gs = O.route(x, idx, E)
        np.testing.assert_array_equal(perm, g[f"{n}__perm"], err_msg=n)
        np.testing.assert_array_equal(gs, g[f"{n}__gs"], err_msg=n)
        np.testing.assert_array_equal(st, x[g[f"{n}__perm"] // K])


def test_counting_sort_equals_numpy_stable_argsort():
    rng = np.random.default_rng(11)
    for E in (1, 3, 8, 129, 256):
        keys = rng.integers(0, E, 5000)
        np.testing.assert_array_equal(O.stable_counting_sort(keys, E), np.argsort(keys, kind="stable"))


def test_route_invariants_reference_tests():
    """tests/test_moe_kernels.py:47-60: sum(gs) == N*K and expert ids non-decreasing."""
    rng = np.random.default_rng(5)
    idx = rng.integers(0, 4, (32, 2))
    _, perm, gs = O.route(np.zeros((32, 1)), idx, 4)
    assert gs.sum() == 64
    assert (np.diff(idx.ravel()[perm]) >= 0).all()
    # stability: within one expert the flat positions ascend
    e_sorted = idx.ravel()[perm]
    for e in range(4):
        assert (np.diff(perm[e_sorted == e]) > 0).all()


def test_unroute_closed_form():
    """unroute(route(x)) with weights w gives sum_k w[n,k] * x[n] (combine of K copies)."""
    rng = np.random.default_rng(6)
    N, D, K, E = 50, 7, 3, 5
    x = rng.standard_normal((N, D))
    idx = np.stack([rng.permutation(E)[:K] for _ in range(N)])
    w = rng.random((N, K))
    st, perm, _ = O.route(x, idx, E)
    np.testing.assert_allclose(O.unroute(st, perm, w, K), x * w.sum(1, keepdims=True), rtol=1e-12)
    np.testing.assert_allclose(O.unroute_f32(st, perm, w, K), x * w.sum(1, keepdims=True), rtol=1e-5)


def test_invert_permutation_is_argsort():
    p = np.random.default_rng(8).permutation(1000)
    np.testing.assert_array_equal(O.invert_permutation(p), np.argsort(p))


# ------------------------------------------------------------------------------------- gmm
def _gmm_cases():
    g = golden("gmm")
    return g, sorted({k.split("__")[0] for k in g.files})


def test_gmm_dlhs_tgmm_match_torch_fixtures():
    g, names = _gmm_cases()
    for n in names:
        gs, x, w, gr = g[f"{n}__gs"], g[f"{n}__x"], g[f"{n}__w"], g[f"{n}__g"]
        np.testing.assert_allclose(O.gmm(x, w, gs), g[f"{n}__out"], rtol=1e-12, atol=1e-12, err_msg=n)
        np.testing.assert_allclose(O.gmm_dlhs(gr, w, gs), g[f"{n}__dlhs"], rtol=1e-12, atol=1e-12, err_msg=n)
        np.testing.assert_allclose(O.tgmm(x, gr, gs), g[f"{n}__tgmm"], rtol=1e-12, atol=1e-12, err_msg=n)


def test_tgmm_empty_group_exact_zero():
    x = np.ones((16, 4))
    g = np.ones((16, 4))
    out = O.tgmm(x, g, [8, 0, 8])
    assert (out[1] == 0).all() and (out[0] == 8).all()


def test_gmm_rows_past_group_sum_are_zero():
    out = O.gmm(np.ones((10, 3)), np.ones((2, 3, 2)), [4, 3])
    assert (out[7:] == 0).all() and (out[:7] == 3).all()


def test_gmm_vjp_identities():
    """<gmm(x,W), g> = <x, dlhs(g,W)> = sum_e <W_e, tgmm(x,g)_e> (adjointness pins both VJPs)."""
    rng = np.random.default_rng(9)
    gs = [5, 0, 7, 3]
    x = rng.standard_normal((15, 6))
    W = rng.standard_normal((4, 6, 4))
    g = rng.standard_normal((15, 4))
    lhs = np.sum(O.gmm(x, W, gs) * g)
    assert np.isclose(lhs, np.sum(x * O.gmm_dlhs(g, W, gs)), rtol=1e-12)
    assert np.isclose(lhs, np.sum(W * O.tgmm(x, g, gs)), rtol=1e-12)


def test_swiglu_and_bwd():
    rng = np.random.default_rng(10)
    h = rng.standard_normal((5, 8))
    y = O.swiglu(h)
    np.testing.assert_allclose(y, h[:, :4] / (1 + np.exp(-h[:, :4])) * h[:, 4:], rtol=1e-14)
    dy = rng.standard_normal((5, 4))
    dh = O.swiglu_bwd(h, dy)
    eps = 1e-6
    for i, j in itertools.product(range(5), range(8)):
        hp, hm = h.copy(), h.copy()
        hp[i, j] += eps
        hm[i, j] -= eps
        num = np.sum((O.swiglu(hp) - O.swiglu(hm)) * dy) / (2 * eps)
        assert abs(num - dh[i, j]) < 1e-6


# ------------------------------------------------------------------------------------- fp8
def test_quant_rows_roundtrip_bound():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((16, 512)).astype(np.float32) * 3
    q, s = O.quant_fp8_rows(x)
    assert q.dtype == np.uint8 and s.shape == (16, 4)
    # the group max maps exactly to +-448
    amax_codes = np.abs(O.e4m3_decode(q).reshape(16, 4, 128)).max(-1)
    np.testing.assert_array_equal(amax_codes, 448.0)
    # e4m3 has 3 mantissa bits: relative error <= 2^-4 per normal element
    deq = O.dequant_rows(q, s)
    big = np.abs(x) > 2.0 ** -6 * s.repeat(128, axis=1)
    assert (np.abs(deq - x)[big] <= np.abs(x)[big] * 2.0 ** -4 + 1e-12).all()


def test_quant_weights_layout_and_dequant():
    rng = np.random.default_rng(13)
    w = rng.standard_normal((2, 256, 384)).astype(np.float32) * 0.02
    wq, ws = O.quant_fp8_weights(w)
    assert wq.shape == (2, 384, 256) and ws.shape == (2, 3, 2)
    # block (e=1, kin-block 1, kout-block 2) scale is its amax / 448
    assert np.isclose(ws[1, 2, 1], np.abs(w[1, 128:256, 256:384]).max() / 448.0, rtol=1e-7)
    # transposed layout: wq[e, n, k] encodes w[e, k, n]
    np.testing.assert_array_equal(wq[0, 5, 7], O.e4m3_encode(np.float32(w[0, 7, 5] / ws[0, 0, 0])))
    assert rel_err(O.dequant_weights(wq, ws), w) < 0.04


def test_p2_scale_closed_form_and_codes_match_torch():
    """The power-of-two scale against the float64 closed form 2^ceil(log2(amax/448)) (clamped to
    [2^-126, 2^127], 1 for amax 0) over many binades and at the binade edges, the invariant that the
    scaled group maximum lies in (224, 448], and the codes against torch's e4m3 cast of x / scale."""
    rng = np.random.default_rng(21)
    amax = (10.0 ** rng.uniform(-35, 37, 20000)).astype(np.float32)
    edges = np.float32(448.0) * np.ldexp(np.float32(1.0), np.arange(-120, 120)).astype(np.float32)
    amax = np.concatenate([amax, edges, np.nextafter(edges, np.float32(np.inf)), np.nextafter(edges, np.float32(0)),
                           np.array([0.0, 1e-40, 1e-45, 3.0e38], np.float32)])
    s = O.p2_scale(amax)
    with np.errstate(divide="ignore"):
        e = np.ceil(np.log2(amax.astype(np.float64) / 448.0))
    ref = np.where(amax == 0, 1.0, np.ldexp(1.0, np.clip(np.where(amax > 0, e, 0), -126, 127).astype(np.int64)))
    np.testing.assert_array_equal(s.astype(np.float64), ref)
    normal = (amax > 448.0 * 2.0 ** -126) & (amax < 448.0 * 2.0 ** 127)
    q = amax[normal].astype(np.float64) / s[normal]
    assert (q > 224.0).all() and (q <= 448.0).all()
    x = (rng.standard_normal((8, 384)) * 10.0 ** rng.uniform(-20, 20, (8, 1))).astype(np.float32)
    x[3, :128] = 0
    codes, sc = O.quant_fp8_rows(x, scales="pow2")
    np.testing.assert_array_equal(sc[3, 0], np.float32(1.0))
    div = torch.from_numpy(x.reshape(8, 3, 128) / sc[..., None])
    tq = div.to(torch.float8_e4m3fn).view(torch.uint8).numpy().reshape(8, 384)
    np.testing.assert_array_equal(codes, tq)
    w = (rng.standard_normal((2, 256, 384)) * 0.02).astype(np.float32)
    wq, ws = O.quant_fp8_weights(w, scales="pow2")
    blk = np.abs(w.reshape(2, 2, 128, 3, 128)).max(axis=(2, 4))  # [E, Kin/128, Kout/128]
    np.testing.assert_array_equal(ws, np.swapaxes(O.p2_scale(blk), 1, 2))
    assert rel_err(O.dequant_weights(wq, ws), w) < 0.04


def test_gmm_fp8_equals_dequantised_gmm():
    rng = np.random.default_rng(14)
    gs = [40, 0, 88]
    x = rng.standard_normal((128, 256)).astype(np.float32)
    w = (rng.standard_normal((3, 256, 128)) * 0.05).astype(np.float32)
    xq, xs = O.quant_fp8_rows(x)
    wq, ws = O.quant_fp8_weights(w)
    got = O.gmm_fp8(xq, xs, wq, ws, gs)
    assert rel_err(got, O.gmm(x, w, gs)) < 6e-2


# ---------------------------------------------------------------------------- composition
def test_tiny_moe_layer_matches_hf_mixtral():
    """C1 (T=256, D=128, E=8, K=2, I=256): oracle router + experts == HF MixtralSparseMoeBlock (float64)."""
    g = golden("moe_tiny")
    rng = np.random.default_rng(1)
    T, D, E, I = 256, 128, 8, 256
    x = rng.standard_normal((T, D)).astype(np.float32)
    rng.standard_normal((D, E))  # gate weights (the fixture stores the logits)
    gate_up = (rng.standard_normal((E, D, 2 * I)) * 0.02).astype(np.float32)
    down = (rng.standard_normal((E, I, D)) * 0.02).astype(np.float32)
    idx, w, _ = O.router_softmax(g["logits"], 2)
    np.testing.assert_array_equal(idx, g["idx"])
    out = O.moe_experts(x, idx, w, gate_up, down)
    np.testing.assert_allclose(out, g["out"], rtol=1e-5, atol=1e-7)


def _block_inputs():
    import sys

    sys.path.insert(0, str(__import__("conftest").GOLDEN))
    from make_golden import moe_block_inputs

    return moe_block_inputs()


def test_moe_block_with_shared_expert_matches_hf_deepseek():
    # HF DeepseekV3MoE (routed experts + shared expert), float64 experts, float32 router
    p, g = _block_inputs(), golden("moe_block_shared")
    idx, w, _ = O.router_sigmoid_group(g["logits"], p["K"], bias=p["bias"], n_group=p["n_group"],
                                       topk_group=p["topk_group"], routed_scaling_factor=p["scale"])
    # HF returns its top-k unsorted: same set, same weight per expert
    for t in range(p["T"]):
        hf = dict(zip(g["idx"][t].tolist(), g["w"][t].tolist()))
        ours = dict(zip(idx[t].tolist(), w[t].tolist()))
        assert set(hf) == set(ours)
        for e in hf:
            assert abs(hf[e] - ours[e]) <= 1e-6 * abs(hf[e])
    out = O.moe_block(p["x"], idx, w, p["gate_up"], p["down"], p["shared_gate_up"], p["shared_down"])
    assert rel_err(out, g["out"]) < 1e-6
    # the shared expert is a real term: without it the output differs
    assert rel_err(O.moe_experts(p["x"], idx, w, p["gate_up"], p["down"]), g["out"]) > 1e-2


def test_folded_shared_expert_equals_block():
    # the shared expert as an always-routed extra expert (weight 1) gives the block's output
    p = _block_inputs()
    g = golden("moe_block_shared")
    idx, w, _ = O.router_sigmoid_group(g["logits"], p["K"], bias=p["bias"], n_group=p["n_group"],
                                       topk_group=p["topk_group"], routed_scaling_factor=p["scale"])
    E = p["E"]
    idx_f = np.concatenate([idx, np.full((p["T"], 1), E, np.int32)], 1)
    w_f = np.concatenate([w, np.ones((p["T"], 1), np.float32)], 1)
    gu_f = np.concatenate([p["gate_up"], p["shared_gate_up"][None]], 0)
    dn_f = np.concatenate([p["down"], p["shared_down"][None]], 0)
    folded = O.moe_experts(p["x"], idx_f, w_f, gu_f, dn_f)
    assert rel_err(folded, g["out"]) < 1e-6


def test_expert_bias_update_known_answers():
    rate = 0.001
    # mean 2: under-used experts (1, 0) go up, over-used (3, 4) go down
    got = O.expert_bias_update([3, 1, 0, 4], rate, [0.5, 0.5, 0.5, 0.5])
    assert np.array_equal(got, np.float32([0.5 - 0.001, 0.5 + 0.001, 0.5 + 0.001, 0.5 - 0.001]))
    # balanced load: unchanged (sign(0) == 0)
    assert np.array_equal(O.expert_bias_update([5, 5, 5], 0.1, [1.0, -2.0, 0.0]), np.float32([1.0, -2.0, 0.0]))
    # fractional mean 1.5
    assert np.array_equal(O.expert_bias_update([1, 2], 1.0, [0.0, 0.0]), np.float32([1.0, -1.0]))


def test_expert_layout_conversion_closed_form():
    # conversion.py:80-166 on a hand-checkable case: gate_up[e, d, i] = gate[e, i, d] (i < I) and
    # up[e, i - I, d] (i >= I); down_f[e, i, d] = down[e, d, i]; export inverts import
    E, I, D = 3, 4, 5
    gate = np.arange(E * I * D, dtype=np.float32).reshape(E, I, D)
    up = -np.arange(E * I * D, dtype=np.float32).reshape(E, I, D) - 1
    down = np.arange(E * D * I, dtype=np.float32).reshape(E, D, I) * 10
    gu, dn = O.experts_from_hf(gate, up, down)
    assert gu.shape == (E, D, 2 * I) and dn.shape == (E, I, D)
    for e, d, i in itertools.product(range(E), range(D), range(2 * I)):
        assert gu[e, d, i] == (gate[e, i, d] if i < I else up[e, i - I, d])
    for e, i, d in itertools.product(range(E), range(I), range(D)):
        assert dn[e, i, d] == down[e, d, i]
    g2, u2, d2 = O.experts_to_hf(gu, dn)
    assert np.array_equal(g2, gate) and np.array_equal(u2, up) and np.array_equal(d2, down)
    # the fused layout feeds the expert layer exactly like HF's per-expert matmuls (SwiGLU MLP)
    x = np.random.default_rng(0).standard_normal((7, D))
    h = x @ gu[1].astype(np.float64)
    hf = np.concatenate([x @ gate[1].T.astype(np.float64), x @ up[1].T.astype(np.float64)], -1)
    assert np.allclose(h, hf)


def test_planted_mistake_is_caught():
    """A transposed-operand slip in the GEMM (a plausible bug) fails the fixture comparison."""
    g = golden("gmm")
    gs, x, w = g["uniform_e4__gs"], g["uniform_e4__x"], g["uniform_e4__w"]
    wrong = O.gmm(x, w[::-1], gs)  # experts in reversed order
    assert rel_err(wrong, g["uniform_e4__out"]) > 0.5


# ------------------------------------------------------------------------ fp8 backward operands
@pytest.mark.parametrize("scales", ["amax", "pow2"])
def test_quant_weights_t_is_the_forward_blocks_in_w_layout(scales):
    """The dlhs weight operand: the forward's 128x128 blocks (pinned through quant_fp8_weights
    against torch's e4m3 cast, in both scale modes) with codes in w's own layout; dequantised it is
    within half an e4m3 step of w everywhere."""
    w = (np.random.default_rng(3).standard_normal((2, 256, 384)) * 0.05).astype(np.float32)
    q, s = O.quant_fp8_weights_t(w, scales=scales)
    qf, sf = O.quant_fp8_weights(w, scales=scales)
    assert q.shape == (2, 256, 384) and s.shape == (2, 2, 3)
    assert np.array_equal(q, np.swapaxes(qf, 1, 2)) and np.array_equal(s, np.swapaxes(sf, 1, 2))
    deq = O.e4m3_decode(q).astype(np.float64) * np.repeat(np.repeat(s, 128, 1), 128, 2)
    assert np.all(np.abs(deq - w) <= np.abs(w) * 2.0 ** -4 + np.repeat(np.repeat(s, 128, 1), 128, 2) * 2.0 ** -9)


def test_gmm_fp8_dlhs_equals_dequantised_dlhs():
    rng = np.random.default_rng(4)
    gs = np.array([100, 0, 37, 123], np.int32)
    M, Kin, Kout = int(gs.sum()) + 4, 256, 384
    g = rng.standard_normal((M, Kout)).astype(np.float32)
    w = (rng.standard_normal((4, Kin, Kout)) * 0.05).astype(np.float32)
    gq, gsc = O.quant_fp8_rows(g)
    wq, ws = O.quant_fp8_weights_t(w)
    got = O.gmm_fp8_dlhs(gq, gsc, wq, ws, gs)
    wd = O.e4m3_decode(wq).astype(np.float64) * np.repeat(np.repeat(ws, 128, 1), 128, 2)  # [E,Kin,Kout]
    ref = O.gmm_dlhs(O.dequant_rows(gq, gsc), wd, gs)  # g @ W^T per group (torch-pinned)
    assert rel_err(got, ref) < 1e-12
    # against the unquantised product: two e4m3 quantisations
    assert rel_err(got, O.gmm_dlhs(g, w, gs)) < 6e-2


@pytest.mark.parametrize("scales", ["amax", "pow2"])
@pytest.mark.parametrize("blocks", [False, True])
def test_quant_grouped_t_chunks_equal_row_and_block_quantisers(blocks, scales):
    """Each expert-aligned chunk of the transposed operand is quant_fp8_rows (1x128 along the
    transposed row) or, with blocks, quant_fp8_weights (128x128) of that zero-padded chunk, in the
    same scale mode, stored in expert-major blocks."""
    rng = np.random.default_rng(5)
    gs = np.array([130, 0, 5, 256, 0, 77], np.int32)
    M, F = int(gs.sum()) + 9, 256
    x = (rng.standard_normal((M, F)) * rng.uniform(0.01, 10, (1, F))).astype(np.float32)
    xt, xs = O.quant_fp8_grouped_t(x, gs, blocks, scales=scales)
    off, cb = O.fp8_group_chunks(gs, M)
    assert int(cb[-1]) == sum(-(-int(g) // 128) for g in gs)
    nf = F // 128 if blocks else F
    for e in range(len(gs)):
        ne = int(cb[e + 1] - cb[e])
        blk = xt[128 * F * int(cb[e]):128 * F * int(cb[e + 1])].reshape(F, 128 * ne)
        sce = xs[nf * int(cb[e]):nf * int(cb[e + 1])].reshape(nf, ne)
        for j in range(ne):
            r0 = int(off[e]) + 128 * j
            chunk = np.zeros((128, F), np.float32)
            rows = x[r0:min(r0 + 128, int(off[e + 1]))]
            chunk[: len(rows)] = rows
            if blocks:
                q, s = O.quant_fp8_weights(chunk[None], scales=scales)  # [1, F, 128] codes, [1, F/128, 1] scales
                assert np.array_equal(blk[:, 128 * j:128 * (j + 1)], q[0]) and np.array_equal(sce[:, j], s[0, :, 0])
            else:
                q, s = O.quant_fp8_rows(np.ascontiguousarray(chunk.T), scales=scales)
                assert np.array_equal(blk[:, 128 * j:128 * (j + 1)], q) and np.array_equal(sce[:, j], s[:, 0])
    # round trip within the e4m3 bound, padding dropped
    d = O.dequant_grouped_t(xt, xs, gs, M, F, blocks)
    used = int(gs.sum())
    assert rel_err(d[:used], x[:used]) < 4e-2 and not d[used:].any()


def test_tgmm_fp8_equals_dequantised_tgmm_and_empty_groups_are_zero():
    rng = np.random.default_rng(6)
    gs = np.array([300, 0, 1, 200], np.int32)
    M, F, N = int(gs.sum()), 256, 256
    x, g = rng.standard_normal((M, F)).astype(np.float32), rng.standard_normal((M, N)).astype(np.float32)
    xt, xs = O.quant_fp8_grouped_t(x, gs, False)
    gt, gsc = O.quant_fp8_grouped_t(g, gs, True)
    got = O.tgmm_fp8(xt, xs, gt, gsc, gs, M, F, N)
    ref = O.tgmm(O.dequant_grouped_t(xt, xs, gs, M, F, False), O.dequant_grouped_t(gt, gsc, gs, M, N, True), gs)
    assert rel_err(got, ref) < 1e-12
    assert not got[1].any()
    assert rel_err(got, O.tgmm(x, g, gs)) < 6e-2

"""CPU oracle of the bzantium/mintext MoE hot path -- TEST INFRASTRUCTURE ONLY.

This module is the checker for the HIP kernels.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it; the product package
(``mintext_amd``) never does.  It restates, in numpy, the reference algorithm of each
function on the hot path, citing the reference file:line it follows (paths relative to the
reference repository root).  Integer outputs (indices, permutations, group sizes, fp8
codes) are exact; floating-point outputs are computed in float64 unless a function states
otherwise.

Pinning (what checks each function, beyond restating it): see tests/test_oracle.py --
golden fixtures written by tests/golden/make_golden.py from independent implementations
(HF transformers routers and experts, torch.sort(stable=True), torch float64 matmul, torch's
float8_e4m3fn cast), brute force on tiny inputs and closed-form invariants.
"""
from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------------------------
# number formats
# ---------------------------------------------------------------------------------------------


def bf16_round(x) -> np.ndarray:
    """float32 -> nearest bfloat16 (RNE), returned as float32 values.  NaN stays NaN."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(x)
    out[nan] = np.nan
    return out


def bf16_bits(x) -> np.ndarray:
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


E4M3_MAX = 448.0


def e4m3_encode(x) -> np.ndarray:
    """float32 -> OCP e4m3fn code (uint8), round-to-nearest-even, saturating at +-448.

    Format: 1 sign, 4 exponent bits (bias 7), 3 mantissa bits, no infinities, S.1111.111
    = NaN; exponent field 0 holds subnormals m * 2^-9.
    """
    x = np.asarray(x, dtype=np.float32)
    sign = np.signbit(x).astype(np.uint8) << 7
    a = np.abs(x).astype(np.float64)
    out = np.zeros(x.shape, dtype=np.uint8)
    nan = np.isnan(x)
    sat = (a >= E4M3_MAX) & ~nan
    sub = (a < 2.0 ** -6) & ~nan
    # subnormal: m = rne(a / 2^-9) in [0, 8]
    m_sub = np.rint(a * 512.0)  # np.rint is round-half-even
    out = np.where(sub, m_sub.astype(np.uint8), out)
    # normal: a = 2^e * (1 + f/8)
    norm = ~(sub | sat | nan)
    e = np.floor(np.log2(np.where(norm, a, 1.0)))
    # guard log2 rounding at exact powers of two
    e = np.where(norm & (2.0 ** e > a), e - 1, e)
    e = np.where(norm & (2.0 ** (e + 1) <= a), e + 1, e)
    frac = np.where(norm, a / 2.0 ** e - 1.0, 0.0) * 8.0
    f = np.rint(frac)
    carry = f >= 8
    f = np.where(carry, 0, f)
    e = np.where(carry, e + 1, e)
    code = ((e + 7).astype(np.int64) << 3) | f.astype(np.int64)
    code = np.where(code > 0x7E, 0x7E, code)  # rounding up past 448 saturates
    out = np.where(norm, code.astype(np.uint8), out)
    out = np.where(sat, np.uint8(0x7E), out)
    out = np.where(nan, np.uint8(0x7F), out)
    return (out | sign).astype(np.uint8)


def e4m3_decode(q) -> np.ndarray:
    q = np.asarray(q, dtype=np.uint8)
    s = np.where(q & 0x80, -1.0, 1.0)
    e = ((q >> 3) & 0xF).astype(np.int64)
    m = (q & 7).astype(np.float64)
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e - 7).astype(np.float64))
    val = np.where((e == 0xF) & (m == 7), np.nan, val)
    return (s * val).astype(np.float32)


# ---------------------------------------------------------------------------------------------
# router top-k   (mintext/modules/moe.py:41-103; softmax router: HF mixtral/qwen3_moe routers)
# ---------------------------------------------------------------------------------------------


def topk_desc(values: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest entries per row, descending, ties to the lower index.

    This is the order lax.top_k returns (moe.py:79,83,98).  Restated as a stable sort on the
    negated values: np.lexsort keys (index, -value) -> primary -value, secondary index.
    """
    values = np.asarray(values)
    T, E = values.shape
    idx = np.arange(E)
    out = np.empty((T, k), dtype=np.int32)
    for t in range(T):
        order = np.lexsort((idx, -values[t].astype(np.float64)))
        out[t] = order[:k]
    return out


def sigmoid_f32(logits) -> np.ndarray:
    """jax.nn.sigmoid(float32(logits)) as 1 / (1 + exp(-x)) in float32 (moe.py:53)."""
    x = np.asarray(logits, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (np.float32(1.0) / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def select_sigmoid_group(scores: np.ndarray, bias, k: int, n_group: int, topk_group: int):
    """Expert selection of MoERouter._group_topk_routing (moe.py:69-103) given float32 scores.

    Returns (topk_indices [T,k] int32, masked routing scores [T,E] float32).
    Exact given the float32 scores: the only arithmetic is s + bias and a + b of the two
    largest per group, both single float32 roundings.
    """
    s = np.asarray(scores, dtype=np.float32)
    T, E = s.shape
    b = np.zeros(E, np.float32) if bias is None else np.asarray(bias, np.float32)
    r = (s + b).astype(np.float32)  # moe.py:56
    if n_group > 1 and topk_group < n_group:
        epg = E // n_group
        grouped = r.reshape(T, n_group, epg)  # moe.py:76
        top2 = -np.sort(-grouped, axis=-1)[..., : min(2, epg)]  # moe.py:79
        gscore = top2[..., 0].copy()
        if top2.shape[-1] == 2:
            gscore = (top2[..., 0] + top2[..., 1]).astype(np.float32)  # moe.py:80
        gsel = topk_desc(gscore, topk_group)  # moe.py:83
        gmask = np.zeros((T, n_group), dtype=bool)
        gmask[np.arange(T)[:, None], gsel] = True  # moe.py:86-89
        emask = np.repeat(gmask, epg, axis=1)  # moe.py:92
        r = np.where(emask, r, np.float32(-np.inf)).astype(np.float32)  # moe.py:95
    return topk_desc(r, k), r


def router_sigmoid_group(logits, k: int, bias=None, n_group: int = 1, topk_group: int = 1,
                         norm_topk_prob: bool = True, routed_scaling_factor: float = 1.0, scores=None):
    """MoERouter.__call__ after the gate GEMM (moe.py:52-67).

    ``scores`` may be passed in (float32) to reproduce the selection on given scores.
    Returns (idx int32 [T,k], weights float64 [T,k], scores float32 [T,E]).
    """
    s = sigmoid_f32(logits) if scores is None else np.asarray(scores, np.float32)
    idx, _ = select_sigmoid_group(s, bias, k, n_group, topk_group)
    w = np.take_along_axis(s.astype(np.float64), idx, axis=1)  # moe.py:101
    if norm_topk_prob:
        w = w / (w.sum(-1, keepdims=True) + 1e-20)  # moe.py:63-64
    w = w * routed_scaling_factor  # moe.py:66
    return idx, w, s


def router_softmax(logits, k: int, norm_topk_prob: bool = True, routed_scaling_factor: float = 1.0):
    """Softmax top-k router (HF mixtral/modeling_mixtral.py:104-111, qwen3_moe:258-267).

    Selection on the float32 logits (softmax is monotone); weights in float64:
    exp(l - lmax) / sum_topk exp(l - lmax) when renormalised, else the softmax probability.
    Returns (idx int32 [T,k], weights float64 [T,k], probs float64 [T,E]).
    """
    lg = np.asarray(logits, dtype=np.float32)
    idx = topk_desc(lg, k)
    l64 = lg.astype(np.float64)
    ex = np.exp(l64 - l64.max(-1, keepdims=True))
    probs = ex / ex.sum(-1, keepdims=True)
    top = np.take_along_axis(ex, idx, axis=1)
    if norm_topk_prob:
        w = top / top.sum(-1, keepdims=True)
    else:
        w = np.take_along_axis(probs, idx, axis=1)
    return idx, w * routed_scaling_factor, probs


def router_weights_given_idx(logits, topk_indices, scoring: str = "softmax", norm_topk_prob: bool = True,
                             routed_scaling_factor: float = 1.0):
    """The router's weights and scores as functions of the logits for FIXED indices, in float64:
    sigmoid mode ``take_along_axis(sigmoid(l), idx)`` (moe.py:53,101), ``/ (sum + 1e-20)``
    (moe.py:63-64), ``* scale`` (moe.py:66); softmax mode the renormalised top-k softmax or the
    full-softmax probability (HF mixtral/modeling_mixtral.py:104-111, qwen3_moe:258-267).
    Returns (weights [T,k], scores [T,E]).  The forward whose derivative ``router_vjp`` is."""
    lg = np.asarray(logits, dtype=np.float64)
    idx = np.asarray(topk_indices)
    if scoring == "softmax":
        ex = np.exp(lg - lg.max(-1, keepdims=True))
        scores = ex / ex.sum(-1, keepdims=True)
        top = np.take_along_axis(ex, idx, axis=1)
        w = top / top.sum(-1, keepdims=True) if norm_topk_prob else np.take_along_axis(scores, idx, axis=1)
    else:
        scores = 1.0 / (1.0 + np.exp(-lg))
        w = np.take_along_axis(scores, idx, axis=1)
        if norm_topk_prob:
            w = w / (w.sum(-1, keepdims=True) + 1e-20)
    return w * routed_scaling_factor, scores


def router_vjp(logits, topk_indices, d_weights, d_scores=None, scoring: str = "softmax",
               norm_topk_prob: bool = True, routed_scaling_factor: float = 1.0) -> np.ndarray:
    """d logits [T,E] float64 of <weights, d_weights> + <scores, d_scores> for fixed indices --
    the gradient jax.grad takes through MoERouter.__call__ (moe.py:52-67,101); the top-k
    selection and the bias carry none.  Chain rule through ``router_weights_given_idx``:
    d w_k / d l_e = c * (dS_k/dl_e), with the selection's Jacobian written per mode below."""
    lg = np.asarray(logits, dtype=np.float64)
    idx = np.asarray(topk_indices)
    T, E = lg.shape
    c = float(routed_scaling_factor)
    g = np.zeros((T, idx.shape[1])) if d_weights is None else np.asarray(d_weights, np.float64)
    rows = np.arange(T)[:, None]
    dl = np.zeros((T, E))
    if scoring == "softmax":
        ex = np.exp(lg - lg.max(-1, keepdims=True))
        p = ex / ex.sum(-1, keepdims=True)
        if norm_topk_prob:
            top = np.take_along_axis(ex, idx, axis=1)
            u = top / top.sum(-1, keepdims=True)               # softmax over the selected logits
            np.add.at(dl, (rows, idx), c * u * (g - (g * u).sum(-1, keepdims=True)))
        else:
            pk = np.take_along_axis(p, idx, axis=1)            # w_k = c p_{i_k}
            np.add.at(dl, (rows, idx), c * g * pk)
            dl -= c * p * (g * pk).sum(-1, keepdims=True)
        if d_scores is not None:
            ds = np.asarray(d_scores, np.float64)
            dl += p * (ds - (ds * p).sum(-1, keepdims=True))
    else:
        s = 1.0 / (1.0 + np.exp(-lg))
        sk = np.take_along_axis(s, idx, axis=1)
        if norm_topk_prob:
            den = sk.sum(-1, keepdims=True) + 1e-20
            dsk = c * (g - (g * sk).sum(-1, keepdims=True) / den) / den
        else:
            dsk = c * g
        np.add.at(dl, (rows, idx), dsk * sk * (1.0 - sk))
        if d_scores is not None:
            dl += np.asarray(d_scores, np.float64) * s * (1.0 - s)
    return dl


# ---------------------------------------------------------------------------------------------
# dispatch / combine   (mintext/kernels/moe_dispatch.py)
# ---------------------------------------------------------------------------------------------


def stable_counting_sort(keys: np.ndarray, num_buckets: int) -> np.ndarray:
    """Stable argsort of small non-negative integer keys (counting sort).

    Equals jnp.argsort(keys, stable=True) (moe_dispatch.py:73) for keys in [0, num_buckets).
    """
    keys = np.asarray(keys, dtype=np.int64).ravel()
    counts = np.bincount(keys, minlength=num_buckets)
    start = np.concatenate([[0], np.cumsum(counts)[:-1]])
    perm = np.empty(keys.size, dtype=np.int32)
    nxt = start.copy()
    for p, kk in enumerate(keys):
        perm[nxt[kk]] = p
        nxt[kk] += 1
    return perm


def route(tokens, topk_indices, num_experts: int):
    """route (moe_dispatch.py:47-81): (sorted_tokens [N*K,D], sort_indices [N*K], group_sizes [E]).

    Expert ids outside [0,E) go to a trailing bucket and are not counted (the kernels'
    documented behaviour; the reference does not define it).
    """
    idx = np.asarray(topk_indices, dtype=np.int64)
    N, K = idx.shape
    flat = idx.ravel()  # moe_dispatch.py:70
    key = np.where((flat < 0) | (flat >= num_experts), num_experts, flat)
    perm = stable_counting_sort(key, num_experts + 1)  # :73
    tokens = np.asarray(tokens)
    sorted_tokens = tokens[perm // K]  # repeat (:67) then gather (:76)
    gs = np.bincount(key, minlength=num_experts + 1)[:num_experts].astype(np.int32)  # :79
    return sorted_tokens, perm, gs


def invert_permutation(perm) -> np.ndarray:
    perm = np.asarray(perm, dtype=np.int64)
    inv = np.empty(perm.size, dtype=np.int32)
    inv[perm] = np.arange(perm.size, dtype=np.int32)  # == argsort(perm) (moe_dispatch.py:102)
    return inv


def unroute(sorted_output, sort_indices, topk_weights, k: int) -> np.ndarray:
    """unroute (moe_dispatch.py:84-111) in float64: out[n] = sum_k w[n,k] Y[inv[n*K+k]]."""
    Y = np.asarray(sorted_output, dtype=np.float64)
    inv = invert_permutation(sort_indices)
    w = np.asarray(topk_weights, dtype=np.float64)
    N = w.shape[0]
    u = Y[inv].reshape(N, k, -1)  # :103-108
    return np.einsum("nkd,nk->nd", u, w)  # :111


def unroute_f32(sorted_output, sort_indices, topk_weights, k: int) -> np.ndarray:
    """unroute with float32 arithmetic, k ascending (the fp32 path's rounding model)."""
    Y = np.asarray(sorted_output, dtype=np.float32)
    inv = invert_permutation(sort_indices)
    w = np.asarray(topk_weights, dtype=np.float32)
    N = w.shape[0]
    u = Y[inv].reshape(N, k, -1)
    acc = np.zeros((N, u.shape[-1]), dtype=np.float32)
    for kk in range(k):
        acc = (acc + w[:, kk : kk + 1] * u[:, kk]).astype(np.float32)
    return acc


# ---------------------------------------------------------------------------------------------
# grouped GEMM   (mintext/kernels/grouped_matmul.py)
# ---------------------------------------------------------------------------------------------


def group_offsets(group_sizes, M: int) -> np.ndarray:
    gs = np.maximum(np.asarray(group_sizes, dtype=np.int64), 0)
    off = np.concatenate([[0], np.cumsum(gs)])
    return np.minimum(off, M)


def gmm(x, w, group_sizes) -> np.ndarray:
    """ragged_dot (grouped_matmul.py:58-76, 242-277) in float64; rows past sum(gs) are 0."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    M = x.shape[0]
    off = group_offsets(group_sizes, M)
    out = np.zeros((M, w.shape[2]))
    for e in range(w.shape[0]):
        a, b = off[e], off[e + 1]
        if b > a:
            out[a:b] = x[a:b] @ w[e]
    return out


def gmm_dlhs(g, w, group_sizes) -> np.ndarray:
    """dlhs = ragged_dot(g, swapaxes(W,1,2)) (grouped_matmul.py:162-176), float64."""
    return gmm(g, np.swapaxes(np.asarray(w, np.float64), 1, 2), group_sizes)


def tgmm(x, g, group_sizes) -> np.ndarray:
    """tgmm (grouped_matmul.py:197-235) as per-group x^T g in float64; empty group -> 0."""
    x = np.asarray(x, dtype=np.float64)
    g = np.asarray(g, dtype=np.float64)
    M = x.shape[0]
    E = np.asarray(group_sizes).size
    off = group_offsets(group_sizes, M)
    out = np.zeros((E, x.shape[1], g.shape[1]))
    for e in range(E):
        a, b = off[e], off[e + 1]
        if b > a:
            out[e] = x[a:b].T @ g[a:b]
    return out


def silu(x):
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(over="ignore"):  # exp(-x) = inf for x < -709: x / inf is the limit, -0
        return x / (1.0 + np.exp(-x))


def swiglu(h) -> np.ndarray:
    """gate, up = split(h, 2, -1); silu(gate) * up (mintext/modules/moe.py:195-196)."""
    h = np.asarray(h, dtype=np.float64)
    i = h.shape[-1] // 2
    return silu(h[..., :i]) * h[..., i:]


def swiglu_bwd(h, dy) -> np.ndarray:
    h = np.asarray(h, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)
    i = h.shape[-1] // 2
    g, u = h[..., :i], h[..., i:]
    s = 1.0 / (1.0 + np.exp(-g))
    return np.concatenate([dy * u * s * (1 + g * (1 - s)), dy * g * s], axis=-1)


# ---------------------------------------------------------------------------------------------
# blockwise fp8 (no reference counterpart; conventions of mintext/modules/linear.py:37-57)
# ---------------------------------------------------------------------------------------------


def p2_scale(amax) -> np.ndarray:
    """Power-of-two quantisation scale: the smallest 2^e, e in [-126, 127], with amax / 2^e <= 448
    (1 when amax == 0).  No reference counterpart: the scale mode whose exponents the MFMA's E8M0
    block-scale operands apply (DeepSeek-V3 likewise restricts some fp8 scaling factors to integral
    powers of 2).  With amax = m 2^E (frexp, m in [0.5, 1)) and 448 = 0.875 2^9, the least e with
    m 2^E <= 0.875 2^(9+e) is E - 9, plus 1 when m > 0.875.  Non-finite amax (not produced by
    finite data) follows the kernels' exponent-field rule: 2^120, or 2^121 for a NaN payload
    above 0x600000."""
    a = np.asarray(amax, dtype=np.float32)
    m, E = np.frexp(np.where(np.isfinite(a), a, 1.0).astype(np.float64))
    e = E.astype(np.int64) - 9 + (m > 0.875)
    bits = a.view(np.uint32)
    e = np.where(np.isfinite(a), e, 120 + ((bits & 0x7FFFFF) > 0x600000))
    e = np.clip(e, -126, 127)
    s = np.ldexp(np.float64(1.0), e).astype(np.float32)
    return np.where(a == 0, np.float32(1.0), s).astype(np.float32)


def _scale_of(amax, scales: str) -> np.ndarray:
    if scales == "pow2":
        return p2_scale(amax)
    if scales != "amax":
        raise ValueError(f"unknown scale mode {scales!r}")
    s = (np.asarray(amax, np.float32) / np.float32(E4M3_MAX)).astype(np.float32)
    return np.where(s == 0, np.float32(1.0), s).astype(np.float32)


def quant_fp8_rows(x, group: int = 128, scales: str = "amax"):
    """1 x 128 groups: scale = amax/448 (1 if amax == 0), or with scales="pow2" the power-of-two
    p2_scale(amax); q = RNE(x / scale) in float32 (exact quotients for a power-of-two scale)."""
    x = np.asarray(x, dtype=np.float32)
    M, D = x.shape
    g = x.reshape(M, D // group, group)
    amax = np.abs(g).max(-1)
    s = _scale_of(amax, scales)
    q = e4m3_encode((g / s[..., None]).astype(np.float32)).reshape(M, D)
    return q, s


def quant_fp8_weights(w, block: int = 128, scales: str = "amax"):
    """128 x 128 blocks over (Kin, Kout) of w [E,Kin,Kout]; returns the k-contiguous
    transposed codes wq [E,Kout,Kin] and scales ws [E,Kout/128,Kin/128] (amax/448 or, with
    scales="pow2", p2_scale of the block's amax)."""
    w = np.asarray(w, dtype=np.float32)
    E, Kin, Kout = w.shape
    blk = w.reshape(E, Kin // block, block, Kout // block, block)
    amax = np.abs(blk).max(axis=(2, 4))  # [E, Kin/128, Kout/128]
    s = _scale_of(amax, scales)
    q = e4m3_encode((blk / s[:, :, None, :, None]).astype(np.float32)).reshape(E, Kin, Kout)
    return np.ascontiguousarray(np.swapaxes(q, 1, 2)), np.ascontiguousarray(np.swapaxes(s, 1, 2))


def dequant_rows(q, s, group: int = 128) -> np.ndarray:
    q = e4m3_decode(q).astype(np.float64)
    M, D = q.shape
    return (q.reshape(M, D // group, group) * np.asarray(s, np.float64)[..., None]).reshape(M, D)


def dequant_weights(wq, ws, block: int = 128) -> np.ndarray:
    """wq [E,Kout,Kin], ws [E,Kout/128,Kin/128] -> W [E,Kin,Kout] float64 (reference layout)."""
    q = e4m3_decode(wq).astype(np.float64)
    E, Kout, Kin = q.shape
    blk = q.reshape(E, Kout // block, block, Kin // block, block) * np.asarray(ws, np.float64)[:, :, None, :, None]
    return np.swapaxes(blk.reshape(E, Kout, Kin), 1, 2)


def gmm_fp8(xq, xs, wq, ws, group_sizes) -> np.ndarray:
    """Blockwise-fp8 grouped GEMM = dequantise, then float64 gmm."""
    return gmm(dequant_rows(xq, xs), dequant_weights(wq, ws), group_sizes)


def quant_fp8_weights_t(w, block: int = 128, scales: str = "amax"):
    """The 128 x 128 blocks of ``quant_fp8_weights`` with the codes kept in w's own layout:
    (wq [E,Kin,Kout], ws [E,Kin/128,Kout/128]) -- the weight operand of the fp8 dlhs, whose
    reduction is Kout (grouped_matmul.py:162-176 with swapaxes(W,1,2) in fp8)."""
    q, sc = quant_fp8_weights(w, block, scales)
    return np.ascontiguousarray(np.swapaxes(q, 1, 2)), np.ascontiguousarray(np.swapaxes(sc, 1, 2))


def gmm_fp8_dlhs(gq, gs_, wq_t, ws_t, group_sizes) -> np.ndarray:
    """fp8 dlhs dX = dY @ W^T per group: dequantise dY (1x128 rows) and W (codes in W's layout),
    then float64 (grouped_matmul.py:162-176)."""
    g = dequant_rows(gq, gs_)
    # wq_t [E,Kin,Kout] with scales [E,Kin/128,Kout/128] is the forward format of W^T
    w_t = dequant_weights(wq_t, ws_t)  # [E, Kout, Kin]  (= (W^T)^T in the reference layout)
    return gmm(g, w_t, group_sizes)


def fp8_group_chunks(group_sizes, M: int, block: int = 128):
    """Expert-aligned 128-row chunks: (row offsets [E+1] clamped to M, chunk bases [E+1])."""
    off = group_offsets(group_sizes, M)
    nch = (np.diff(off) + block - 1) // block
    cb = np.concatenate([[0], np.cumsum(nch)]).astype(np.int64)
    return off, cb


def quant_fp8_grouped_t(x, group_sizes, blocks: bool, C: int | None = None, block: int = 128,
                        scales: str = "amax"):
    """The tgmm operands: x [M,F] quantised in expert-aligned chunks of 128 rows (chunk j of expert
    e = its rows 128j .. 128j+127, zero past the expert) and transposed per expert, in expert-major
    blocks: returns flat codes (expert e's block [F, 128 n_e] at offset 128*F*cb[e], n_e = its
    chunks) and flat scales -- one per feature and chunk ([F, n_e] at F*cb[e], ``blocks`` False,
    1 x 128 along the transposed row) or one per 128 features and chunk ([F/128, n_e] at
    (F/128)*cb[e], ``blocks`` True, 128 x 128).  scale = amax/448 (1 if 0) or, with scales="pow2",
    p2_scale(amax); q = RNE(x / scale).
    C (chunk slots allocated) defaults to ceil(M/128) + E; slots past the groups stay 0."""
    x = np.asarray(x, dtype=np.float32)
    M, F = x.shape
    E = len(group_sizes)
    off, cb = fp8_group_chunks(group_sizes, M, block)
    C = int(-(-M // block) + E) if C is None else C
    nf = F // block if blocks else F
    xt = np.zeros(F * block * C, np.uint8)
    xs = np.zeros(nf * C, np.float32)
    for e in range(E):
        ne = int(cb[e + 1] - cb[e])
        if ne == 0:
            continue
        rows = np.zeros((ne * block, F), np.float32)
        rows[: int(off[e + 1] - off[e])] = x[int(off[e]):int(off[e + 1])]
        t = rows.T.reshape(F, ne, block)  # [F, chunk, row]
        if blocks:
            amax = np.abs(t.reshape(F // block, block, ne, block)).max(axis=(1, 3))  # [F/128, ne]
        else:
            amax = np.abs(t).max(-1)  # [F, ne]
        sc = _scale_of(amax.astype(np.float32), scales)
        sfull = np.repeat(sc, block, axis=0) if blocks else sc  # [F, ne]
        q = e4m3_encode((t / sfull[:, :, None]).astype(np.float32))
        xt[block * F * int(cb[e]):block * F * int(cb[e + 1])] = q.reshape(-1)
        xs[nf * int(cb[e]):nf * int(cb[e + 1])] = sc.reshape(-1)
    return xt, xs


def dequant_grouped_t(xt, xs, group_sizes, M: int, F: int, blocks: bool, block: int = 128):
    """Inverse of ``quant_fp8_grouped_t``: the [M, F] float64 rows (zero-padding dropped)."""
    off, cb = fp8_group_chunks(group_sizes, M, block)
    nf = F // block if blocks else F
    q = e4m3_decode(np.asarray(xt)).astype(np.float64)
    out = np.zeros((M, F))
    for e in range(len(group_sizes)):
        ne = int(cb[e + 1] - cb[e])
        if ne == 0:
            continue
        t = q[block * F * int(cb[e]):block * F * int(cb[e + 1])].reshape(F, ne * block)
        sc = np.asarray(xs[nf * int(cb[e]):nf * int(cb[e + 1])], np.float64).reshape(nf, ne)
        sfull = np.repeat(np.repeat(sc, block, axis=0) if blocks else sc, block, axis=1)  # [F, ne*128]
        n = int(off[e + 1] - off[e])
        out[int(off[e]):int(off[e + 1])] = (t * sfull)[:, :n].T
    return out


def tgmm_fp8(xt, xts, gt, gts, group_sizes, M: int, F: int, N: int) -> np.ndarray:
    """fp8 tgmm: dequantise both transposed operands (x with per-feature chunk scales, g with
    128 x 128 block scales), then the float64 per-group x^T g (grouped_matmul.py:197-235)."""
    return tgmm(dequant_grouped_t(xt, xts, group_sizes, M, F, False),
                dequant_grouped_t(gt, gts, group_sizes, M, N, True), group_sizes)


# ---------------------------------------------------------------------------------------------
# composition  (MoEExperts._forward_kernel, mintext/modules/moe.py:161-221)
# ---------------------------------------------------------------------------------------------


def moe_experts(x, topk_indices, topk_weights, gate_up, down) -> np.ndarray:
    """route -> gmm(gate_up) -> SwiGLU -> gmm(down) -> unroute, all in float64."""
    E = np.asarray(gate_up).shape[0]
    k = np.asarray(topk_indices).shape[1]
    sorted_tokens, perm, gs = route(np.asarray(x, np.float64), topk_indices, E)
    h = gmm(sorted_tokens, gate_up, gs)
    y = gmm(swiglu(h), down, gs)
    return unroute(y, perm, topk_weights, k)


def moe_experts_fp8(x, topk_indices, topk_weights, gu_q, gu_s, dn_q, dn_s) -> np.ndarray:
    """The blockwise-fp8 expert layer with the kernels' quantisation points: x quantised in
    1x128 groups, routed with its scales, fp8 gate_up GEMM, SwiGLU, re-quantisation of the
    SwiGLU output in 1x128 groups, fp8 down GEMM rounded to bf16, float64 combine."""
    k = np.asarray(topk_indices).shape[1]
    E = np.asarray(gu_q).shape[0]
    xq, xs = quant_fp8_rows(np.asarray(x, np.float32))
    sq, perm, gs = route(xq, topk_indices, E)
    ss = xs[perm // k]
    y = swiglu(gmm_fp8(sq, ss, gu_q, gu_s, gs)).astype(np.float32)
    yq, ys = quant_fp8_rows(y)
    o = bf16_round(gmm_fp8(yq, ys, dn_q, dn_s, gs).astype(np.float32))
    return unroute(o, perm, topk_weights, k)


def moe_block(x, topk_indices, topk_weights, gate_up, down, shared_gate_up=None, shared_down=None) -> np.ndarray:
    """MoEBlock.__call__ after the router (mintext/modules/moe.py:246-266): routed experts plus,
    when given, the shared expert MLP (moe.py:231-236, linear.py:164-228) on the same tokens,
    output = routed_out + shared_out, float64.  shared_gate_up [D, 2I'] (gate columns first),
    shared_down [I', D]."""
    out = moe_experts(x, topk_indices, topk_weights, gate_up, down)
    if shared_gate_up is not None:
        x64 = np.asarray(x, np.float64)
        h = x64 @ np.asarray(shared_gate_up, np.float64).reshape(x64.shape[1], -1)
        out = out + swiglu(h) @ np.asarray(shared_down, np.float64).reshape(-1, x64.shape[1])
    return out


def moe_experts_vjp(x, topk_indices, topk_weights, gate_up, down, dout):
    """VJP of ``moe_experts`` (MoEExperts._forward_kernel, moe.py:161-221, under jax.grad with
    the custom VJPs of grouped_matmul.py:151-187 and moe_dispatch.py:33-38,102-111) in float64.
    Returns (dx [N,D], d_topk_weights [N,K], d_gate_up [E,D,2I], d_down [E,I,D])."""
    k = np.asarray(topk_indices).shape[1]
    E = np.asarray(gate_up).shape[0]
    x64 = np.asarray(x, np.float64)
    N, D = x64.shape
    xs, perm, gs = route(x64, topk_indices, E)
    h = gmm(xs, gate_up, gs)
    inter = swiglu(h)
    y = gmm(inter, down, gs)
    inv = invert_permutation(perm)
    g = np.asarray(dout, np.float64)
    w = np.asarray(topk_weights, np.float64)
    yk = y[inv].reshape(N, k, -1)
    d_w = np.einsum("nkd,nd->nk", yk, g)                    # einsum VJP (moe_dispatch.py:111)
    dy = np.empty_like(y)
    dy[inv] = (w[:, :, None] * g[:, None, :]).reshape(N * k, -1)  # gather VJP (:102-108)
    d_inter = gmm_dlhs(dy, down, gs)
    d_down = tgmm(inter, dy, gs)
    dh = swiglu_bwd(h, d_inter)
    dxs = gmm_dlhs(dh, gate_up, gs)
    d_gate_up = tgmm(xs, dh, gs)
    dx = np.zeros((N, D))
    np.add.at(dx, perm // k, dxs)                           # sort + repeat VJP (:33-38, :67)
    return dx, d_w, d_gate_up, d_down


def moe_block_vjp(x, gate_weight, gate_up, down, dout, *, k: int, scoring: str = "sigmoid_group", bias=None,
                  n_group: int = 1, topk_group: int = 1, norm_topk_prob: bool = True,
                  routed_scaling_factor: float = 1.0, shared_gate_up=None, shared_down=None):
    """VJP of MoEBlock.__call__ (moe.py:240-266) from the tokens, router included, in float64:
    logits = x @ W_g (linear.py:123-147), router with its weights differentiated for fixed
    indices (``router_vjp``), routed experts (``moe_experts_vjp``), shared expert MLP.  The
    selection runs on the float32 logits (as the reference's f32 router does).
    Returns a dict with dx, d_gate_weight [D,E], d_gate_up, d_down and, with a shared expert,
    d_shared_gate_up [D,2I'], d_shared_down [I',D]."""
    x64 = np.asarray(x, np.float64)
    wg = np.asarray(gate_weight, np.float64)
    logits = x64 @ wg
    lg32 = logits.astype(np.float32)
    if scoring == "softmax":
        idx, w, _ = router_softmax(lg32, k, norm_topk_prob, routed_scaling_factor)
    else:
        idx, w, _ = router_sigmoid_group(lg32, k, bias, n_group, topk_group, norm_topk_prob, routed_scaling_factor)
    w, _ = router_weights_given_idx(logits, idx, scoring, norm_topk_prob, routed_scaling_factor)
    dx, d_w, d_gu, d_dn = moe_experts_vjp(x64, idx, w, gate_up, down, dout)
    dl = router_vjp(logits, idx, d_w, None, scoring, norm_topk_prob, routed_scaling_factor)
    out = {"d_gate_up": d_gu, "d_down": d_dn, "d_gate_weight": x64.T @ dl}
    dx = dx + dl @ wg.T
    if shared_gate_up is not None:
        D = x64.shape[1]
        sgu = np.asarray(shared_gate_up, np.float64).reshape(D, -1)
        sdn = np.asarray(shared_down, np.float64).reshape(-1, D)
        g = np.asarray(dout, np.float64)
        h = x64 @ sgu
        d_inter = g @ sdn.T
        out["d_shared_down"] = swiglu(h).T @ g
        dh = swiglu_bwd(h, d_inter)
        out["d_shared_gate_up"] = x64.T @ dh
        dx = dx + dh @ sgu.T
    out["dx"] = dx
    out["topk_indices"] = idx
    return out


def expert_bias_update(expert_counts, rate: float, bias) -> np.ndarray:
    """update_expert_biases (mintext/trainer.py:371-410) for one layer, float32 as under JAX with
    x64 disabled: avg = float32(sum(counts)) / float32(E); bias + sign(avg - counts) * rate."""
    c = np.asarray(expert_counts, np.int64)
    E = c.shape[-1]
    avg = np.float32(c.sum()) / np.float32(E)
    direction = np.sign(avg - c.astype(np.float32)).astype(np.float32)
    return (np.asarray(bias, np.float32) + direction * np.float32(rate)).astype(np.float32)


# ---------------------------------------------------------------------------------------------
# expert weight layouts  (mintext/checkpoint/conversion.py:80-166)
# ---------------------------------------------------------------------------------------------


def experts_from_hf(gate, up, down):
    """_import_expert_weights (conversion.py:80-133) on stacked per-expert HF weights:
    gate_up[e] = concatenate([gate[e].T, up[e].T], -1), down_f[e] = down[e].T."""
    gate, up, down = (np.asarray(a) for a in (gate, up, down))
    gate_up = np.stack([np.concatenate([gate[e].T, up[e].T], axis=-1) for e in range(gate.shape[0])])
    return gate_up, np.stack([down[e].T for e in range(down.shape[0])])


def experts_to_hf(gate_up, down):
    """_export_expert_weights (conversion.py:136-166): (gate [E,I,D], up [E,I,D], down [E,D,I])."""
    gate_up, down = np.asarray(gate_up), np.asarray(down)
    i = gate_up.shape[2] // 2
    gate = np.stack([gate_up[e, :, :i].T for e in range(gate_up.shape[0])])
    up = np.stack([gate_up[e, :, i:].T for e in range(gate_up.shape[0])])
    return gate, up, np.stack([down[e].T for e in range(down.shape[0])])

"""GPU parity of the power-of-two-scale fp8 mode ("pow2": scale 2^ceil(log2(amax/448)), the MFMA's
E8M0 block-scale operands apply it): quantisers bit-exact against the oracle, including the clamp
of the exponent to [-126, 127]; the grouped GEMMs (plain, SwiGLU + re-quantisation, gathered)
within 1e-2 of the dequantised float64 oracle and 6e-2 of the unquantised product; rows past the
groups are zero; the gathered gate_up gives the bits of route + GEMM."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_err
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
P2 = dict(scales="pow2")


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _u8(t):
    return t.view(torch.uint8).cpu().numpy()


def _is_pow2(s):
    s = np.asarray(s, np.float32)
    return ((s.view(np.uint32) & 0x7FFFFF) == 0).all() and (s > 0).all()


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_quant_rows_p2_bit_exact(dev, dt):
    from mintext_amd.kernels.fp8 import quantize_fp8_rows

    x = (torch.randn(333, 1024, device=dev) * 3).float()
    x[5, :128] = 0                       # all-zero group -> scale 1
    x[7, 200] = 1e-6                     # subnormal code after scaling
    x[9, 256:384] = 448.0                # amax exactly 448 x 2^0 -> scale 1, codes 448
    x[10, 384:512] = 449.0               # just above -> scale 2
    x[11, 512:640] *= 1e30               # large exponents
    if dt == torch.float32:
        x[12, 640:768] = 1e-39           # subnormal amax -> exponent clamped to -126
        x[13, 768:896] *= 1e-36
    x = x.to(dt)
    q, s = quantize_fp8_rows(x, **P2)
    oq, os_ = O.quant_fp8_rows(x.float().cpu().numpy(), scales="pow2")
    np.testing.assert_array_equal(s.cpu().numpy(), os_)
    np.testing.assert_array_equal(_u8(q), oq)
    assert _is_pow2(s.cpu().numpy())
    if dt == torch.float32:
        assert float(s[12, 5]) == 2.0 ** -126


def test_quant_weights_p2_bit_exact(dev):
    from mintext_amd.kernels.fp8 import quantize_fp8_weights

    w = (torch.randn(3, 256, 384, device=dev) * 0.02).bfloat16()
    w[1, :128, 128:256] = 0  # all-zero block -> scale 1
    wq, ws = quantize_fp8_weights(w, **P2)
    oq, os_ = O.quant_fp8_weights(w.float().cpu().numpy(), scales="pow2")
    np.testing.assert_array_equal(ws.cpu().numpy(), os_)
    np.testing.assert_array_equal(_u8(wq), oq)
    assert _is_pow2(ws.cpu().numpy())


def _groups(rng, M, E):
    cut = np.sort(rng.integers(0, M + 1, E - 1))
    gs = np.diff(np.concatenate([[0], cut, [M]])).astype(np.int32)
    gs[min(1, E - 1)] += gs[0]
    gs[0] = 0
    return gs


@pytest.mark.parametrize("M,E,Kin,Kout", [(1024, 4, 512, 512), (700, 8, 256, 256), (2000, 16, 768, 768),
                                           (1500, 6, 2048, 256), (600, 3, 3072, 512),
                                           (20000, 8, 512, 2048)])  # more tiles than workgroups
def test_gmm_fp8_p2(dev, M, E, Kin, Kout):
    from mintext_amd.kernels.fp8 import grouped_matmul_fp8, quantize_fp8_rows, quantize_fp8_weights

    rng = np.random.default_rng(M + 1)
    gs = _groups(rng, M, E)
    Mt = M + 37  # rows past sum(group_sizes) -> zeros
    # per-row, per-128-block magnitudes over 1e-3 .. 1e3: every lane of an MFMA carries its own
    # row scale, so a wrong lane -> row mapping of the scale operand shows
    blk = torch.from_numpy(10.0 ** rng.uniform(-3, 3, (Mt, Kin // 128))).float().to(dev)
    x = (torch.randn(Mt, Kin, device=dev) * blk.repeat_interleave(128, 1)).bfloat16()
    wblk = torch.from_numpy(10.0 ** rng.uniform(-1, 1, (E, Kin // 128, Kout // 128))).float().to(dev)
    w = (torch.randn(E, Kin, Kout, device=dev) * 0.02
         * wblk.repeat_interleave(128, 1).repeat_interleave(128, 2)).bfloat16()
    xq, xs = quantize_fp8_rows(x, **P2)
    wq, ws = quantize_fp8_weights(w, **P2)
    out = grouped_matmul_fp8(xq, xs, wq, ws, _t(gs, dev), **P2)
    assert out.dtype == torch.bfloat16
    tot = int(gs.sum())
    assert (out[tot:] == 0).all()
    got = out.float().cpu().numpy()[:tot]
    deq = O.gmm_fp8(_u8(xq), xs.cpu().numpy(), _u8(wq), ws.cpu().numpy(), gs)[:tot]
    assert rel_err(got, deq) < 1e-2, rel_err(got, deq)
    ref = O.gmm(x.float().cpu().numpy(), w.float().cpu().numpy(), gs)[:tot]
    assert rel_err(got, ref) < 6e-2, rel_err(got, ref)


@pytest.mark.parametrize("M,E,Kin,I", [(1024, 4, 256, 256), (900, 8, 512, 384), (2048, 8, 2048, 768),
                                       (12000, 8, 1024, 768)])
def test_gmm_fp8_swiglu_p2(dev, M, E, Kin, I):
    from mintext_amd.kernels.fp8 import grouped_matmul_fp8_swiglu, quantize_fp8_rows, quantize_fp8_weights

    rng = np.random.default_rng(I + 3)
    gs = _groups(rng, M, E)
    x = torch.randn(M, Kin, device=dev).bfloat16()
    w = (torch.randn(E, Kin, 2 * I, device=dev) * 0.05).bfloat16()
    xq, xs = quantize_fp8_rows(x, **P2)
    wq, ws = quantize_fp8_weights(w, **P2)
    yq, ys, yb = grouped_matmul_fp8_swiglu(xq, xs, wq, ws, _t(gs, dev), return_bf16=True, **P2)
    tot = int(gs.sum())
    ref = O.swiglu(O.gmm_fp8(_u8(xq), xs.cpu().numpy(), _u8(wq), ws.cpu().numpy(), gs))[:tot]
    assert rel_err(yb.float().cpu().numpy()[:tot], ref) < 1e-2
    # the fused re-quantisation: power-of-two 1x128 scales, the group maximum over its scale in
    # (224, 448], so its code in [224, 448] (224 < v < 232 rounds to 224), or an all-zero group
    # with scale 1; the dequantised output within 6e-2
    ysn = ys.cpu().numpy()[:tot]
    assert _is_pow2(ysn)
    deq = O.dequant_rows(_u8(yq), ys.cpu().numpy())[:tot]
    assert rel_err(deq, ref) < 6e-2
    amax = np.abs(O.e4m3_decode(_u8(yq))[:tot].reshape(tot, I // 128, 128)).max(-1)
    assert (((amax >= 224.0) & (amax <= 448.0)) | (ysn == 1.0)).all()
    # scales: the oracle's pow2 scale of the group maxima of the kernel's own bf16 output, up to
    # the bf16 rounding of those maxima (one binade at most)
    yb_max = np.abs(yb.float().cpu().numpy()[:tot].reshape(tot, I // 128, 128)).max(-1)
    ratio = ysn / O.p2_scale(yb_max.astype(np.float32))
    assert np.isin(ratio, [0.5, 1.0, 2.0]).all()


@pytest.mark.parametrize("T,K,E,D,I", [(512, 2, 8, 256, 256), (1000, 8, 64, 512, 128), (4000, 8, 16, 2048, 768)])
def test_gmm_fp8_swiglu_gathered_p2_equals_route(dev, T, K, E, D, I):
    """The gathered pow2 gate_up (token-order codes read through the permutation) gives the bits
    of the same GEMM on the routed copy of the codes and scales."""
    from mintext_amd.kernels.fp8 import (grouped_matmul_fp8_swiglu, grouped_matmul_fp8_swiglu_gathered,
                                         quantize_fp8_rows, quantize_fp8_weights)
    from mintext_amd.kernels.moe_dispatch import route_indices, route_with_scales

    rng = np.random.default_rng(T + E)
    idx = _t(rng.integers(0, E, (T, K)).astype(np.int32), dev)
    x = torch.randn(T, D, device=dev).bfloat16()
    w = (torch.randn(E, D, 2 * I, device=dev) * 0.05).bfloat16()
    xq, xs = quantize_fp8_rows(x, **P2)
    wq, ws = quantize_fp8_weights(w, **P2)
    sq, ss, si, gs, _ = route_with_scales(xq, xs, idx, E)
    si2, gs2, _ = route_indices(idx, E)
    assert torch.equal(si, si2) and torch.equal(gs, gs2)
    yq1, ys1 = grouped_matmul_fp8_swiglu(sq, ss, wq, ws, gs, **P2)
    yq2, ys2 = grouped_matmul_fp8_swiglu_gathered(xq, xs, si2, K, wq, ws, gs2, **P2)
    assert torch.equal(ys1, ys2)
    assert torch.equal(yq1.view(torch.uint8), yq2.view(torch.uint8))


def test_gmm_fp8_p2_extreme_block_scale_ratios(dev):
    """Neighbouring 128-k blocks of one row whose scales differ by up to 2^100 (a normal block, a
    block near 1e-33, a normal block; an all-zero block, then tiny ones): the power-of-two mode
    applies each block's exponents on the MFMA's E8M0 operands and accumulates in true units, so
    nothing is rescaled between blocks and nothing overflows.  Checked against the dequantised
    float64 oracle row by row (each row's own scale of magnitude)."""
    from mintext_amd.kernels.fp8 import grouped_matmul_fp8, quantize_fp8_rows, quantize_fp8_weights

    M, E, Kin, Kout = 512, 2, 512, 256
    gs = np.array([200, 312], np.int32)
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    x = torch.randn(M, Kin, device=dev, generator=g)
    blk = torch.ones(M, Kin // 128, device=dev)
    blk[0::2, 1] = 1e-33                        # normal, tiny, normal, normal
    blk[1::2, 0] = 0.0                          # zero, then tiny blocks only
    blk[1::2, 1:] = torch.tensor([1e-30, 3e-28, 1e-31], device=dev)
    x = (x * blk.repeat_interleave(128, 1)).bfloat16()
    w = (torch.randn(E, Kin, Kout, device=dev, generator=g) * 0.02).bfloat16()
    xq, xs = quantize_fp8_rows(x, **P2)
    wq, ws = quantize_fp8_weights(w, **P2)
    out = grouped_matmul_fp8(xq, xs, wq, ws, _t(gs, dev), **P2)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    deq = O.gmm_fp8(_u8(xq), xs.cpu().numpy(), _u8(wq), ws.cpu().numpy(), gs)
    for rows in (slice(0, None, 2), slice(1, None, 2)):
        assert rel_err(got[rows], deq[rows]) < 1e-2, rel_err(got[rows], deq[rows])
    assert np.abs(got[1::2]).max() < 1e-25 and np.abs(got[1::2]).max() > 1e-29


def test_gmm_fp8_p2_short_k_unsupported(dev):
    from mintext_amd import _lib as L
    from mintext_amd.kernels.fp8 import grouped_matmul_fp8, quantize_fp8_rows, quantize_fp8_weights

    x = torch.randn(300, 128, device=dev).bfloat16()
    w = (torch.randn(2, 128, 256, device=dev) * 0.05).bfloat16()
    xq, xs = quantize_fp8_rows(x, **P2)
    wq, ws = quantize_fp8_weights(w, **P2)
    with pytest.raises(L.MtxError):
        grouped_matmul_fp8(xq, xs, wq, ws, _t(np.array([100, 200], np.int32), dev), **P2)


def test_layer_forward_pow2_and_unsupported_width(dev):
    """moe_experts_forward_fp8(scales="pow2") equals its steps (pow2 quantiser, gathered SwiGLU GEMM,
    down GEMM, combine) bit for bit and stays within 1e-1 of the unquantised float64 layer; a width
    below 256 raises (the power-of-two GEMMs need K >= 256); an unknown mode raises ValueError."""
    from mintext_amd import _lib as L
    from mintext_amd.kernels import unroute
    from mintext_amd.kernels.fp8 import (grouped_matmul_fp8, grouped_matmul_fp8_swiglu_gathered, quantize_fp8_rows,
                                         quantize_fp8_weights)
    from mintext_amd.kernels.moe_dispatch import route_indices
    from mintext_amd.moe import moe_experts_forward_fp8

    rng = np.random.default_rng(11)
    T, K, E, D, I = 700, 4, 8, 512, 256
    idx = _t(np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32), dev)
    w = _t(rng.random((T, K)).astype(np.float32), dev)
    x = torch.randn(T, D, device=dev).bfloat16()
    gu = (torch.randn(E, D, 2 * I, device=dev) * 0.05).bfloat16()
    dn = (torch.randn(E, I, D, device=dev) * 0.05).bfloat16()
    with torch.no_grad():
        guq, gus = quantize_fp8_weights(gu, **P2)
        dnq, dns = quantize_fp8_weights(dn, **P2)
        out = moe_experts_forward_fp8(x, idx, w, guq, gus, dnq, dns, **P2)
        xq, xs = quantize_fp8_rows(x, **P2)
        si, gs, _ = route_indices(idx, E)
        yq, ys = grouped_matmul_fp8_swiglu_gathered(xq, xs, si, K, guq, gus, gs, **P2)
        ref = unroute(grouped_matmul_fp8(yq, ys, dnq, dns, gs, **P2), si, w, K)
        assert torch.equal(out, ref)
        xh, ih, wh = x.double().cpu().numpy(), idx.cpu().numpy(), w.double().cpu().numpy()
        guh, dnh = gu.double().cpu().numpy(), dn.double().cpu().numpy()
        want = np.zeros((T, D))
        for k in range(K):
            for e in range(E):
                sel = np.flatnonzero(ih[:, k] == e)
                want[sel] += wh[sel, k:k + 1] * (O.swiglu(xh[sel] @ guh[e]) @ dnh[e])
        assert rel_err(out.double().cpu().numpy(), want) < 1e-1
        xs_ = torch.randn(T, 128, device=dev).bfloat16()
        g2q, g2s = quantize_fp8_weights((torch.randn(E, 128, 2 * I, device=dev) * 0.05).bfloat16(), **P2)
        d2q, d2s = quantize_fp8_weights((torch.randn(E, I, 128, device=dev) * 0.05).bfloat16(), **P2)
        with pytest.raises(L.MtxError):
            moe_experts_forward_fp8(xs_, idx, w, g2q, g2s, d2q, d2s, **P2)
        with pytest.raises(ValueError):
            moe_experts_forward_fp8(x, idx, w, guq, gus, dnq, dns, scales="e8m0")

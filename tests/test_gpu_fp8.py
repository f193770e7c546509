"""GPU parity: blockwise fp8 quantisers (bit-exact codes and scales) and the fp8 grouped GEMM
(6e-2 relative against the unquantised float64 product, 1e-2 against the dequantised one)."""
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


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_quant_rows_bit_exact(dev, dt):
    from mintext_amd.kernels.fp8 import quantize_fp8_rows

    x = (torch.randn(333, 1024, device=dev) * 3).to(dt)
    x[5, :128] = 0  # all-zero group -> scale 1
    x[7, 200] = 1e-6  # subnormal after scaling
    q, s = quantize_fp8_rows(x)
    oq, os_ = O.quant_fp8_rows(x.float().cpu().numpy())
    np.testing.assert_array_equal(s.cpu().numpy(), os_)
    np.testing.assert_array_equal(_u8(q), oq)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N,K,E,D", [(16384, 8, 128, 2048), (1000, 2, 8, 384), (5, 3, 4, 128)])
def test_route_quantize_fp8_equals_quant_then_route(dev, dt, N, K, E, D):
    """The fused quantise-and-dispatch gives the bits of quantize_fp8_rows + route_with_scales
    (codes, scales, permutation, group sizes, inverse), and the codes/scales match the oracle."""
    from mintext_amd.kernels.fp8 import quantize_fp8_rows
    from mintext_amd.kernels.moe_dispatch import route_quantize_fp8, route_with_scales

    rng = np.random.default_rng(N + D)
    idx = _t(rng.integers(0, E, (N, K)).astype(np.int32), dev)
    x = (torch.randn(N, D, device=dev) * 3).to(dt)
    x[N // 2, :128] = 0  # all-zero group -> scale 1
    q1, s1, p1, g1, i1 = route_quantize_fp8(x, idx, E)
    xq, xs = quantize_fp8_rows(x)
    q2, s2, p2, g2, i2 = route_with_scales(xq, xs, idx, E)
    assert torch.equal(p1, p2) and torch.equal(g1, g2) and torch.equal(i1, i2)
    assert torch.equal(s1, s2)
    assert torch.equal(q1.view(torch.uint8), q2.view(torch.uint8))
    rows = np.argsort(idx.cpu().numpy().ravel(), kind="stable") // K
    sel = np.unique(np.linspace(0, N * K - 1, 64).astype(np.int64))
    oq, os_ = O.quant_fp8_rows(x.float().cpu().numpy()[rows[sel]])
    np.testing.assert_array_equal(_u8(q1)[sel], oq)
    np.testing.assert_array_equal(s1.cpu().numpy()[sel], os_)


def test_quant_weights_bit_exact(dev):
    from mintext_amd.kernels.fp8 import quantize_fp8_weights

    w = (torch.randn(3, 256, 384, device=dev) * 0.02).bfloat16()
    wq, ws = quantize_fp8_weights(w)
    oq, os_ = O.quant_fp8_weights(w.float().cpu().numpy())
    np.testing.assert_array_equal(ws.cpu().numpy(), os_)
    np.testing.assert_array_equal(_u8(wq), oq)


def _groups(rng, M, E):
    cut = np.sort(rng.integers(0, M + 1, E - 1))
    gs = np.diff(np.concatenate([[0], cut, [M]])).astype(np.int32)
    gs[min(1, E - 1)] += gs[0]
    gs[0] = 0
    return gs


@pytest.mark.parametrize("M,E,Kin,Kout", [(1024, 4, 512, 512), (700, 8, 256, 256), (2000, 16, 128, 768),
                                           (1500, 6, 2048, 256), (600, 3, 3072, 512), (400, 2, 3200, 256),
                                           (20000, 8, 512, 2048)])  # more tiles than workgroups
def test_gmm_fp8(dev, M, E, Kin, Kout):
    from mintext_amd.kernels.fp8 import grouped_matmul_fp8, quantize_fp8_rows, quantize_fp8_weights

    rng = np.random.default_rng(M)
    gs = _groups(rng, M, E)
    # per-128-block magnitudes spread over 1e-3 .. 1e3 exercise the block-to-block rescaling
    blk = torch.from_numpy(10.0 ** rng.uniform(-3, 3, (M, Kin // 128))).float().to(dev)
    x = (torch.randn(M, Kin, device=dev) * blk.repeat_interleave(128, 1)).bfloat16()
    wblk = torch.from_numpy(10.0 ** rng.uniform(-1, 1, (E, Kin // 128, 1))).float().to(dev)
    w = (torch.randn(E, Kin, Kout, device=dev) * 0.02 * wblk.repeat_interleave(128, 1)).bfloat16()
    xq, xs = quantize_fp8_rows(x)
    wq, ws = quantize_fp8_weights(w)
    out = grouped_matmul_fp8(xq, xs, wq, ws, _t(gs, dev))
    assert out.dtype == torch.bfloat16
    got = out.float().cpu().numpy()
    deq = O.gmm_fp8(_u8(xq), xs.cpu().numpy(), _u8(wq), ws.cpu().numpy(), gs)
    assert rel_err(got, deq) < 1e-2
    assert rel_err(got, O.gmm(x.float().cpu().numpy(), w.float().cpu().numpy(), gs)) < 6e-2
    tot = int(gs.sum())
    assert (out[tot:] == 0).all()


@pytest.mark.parametrize("swiglu", [False, True])
def test_gmm_fp8_tiny_block_scales(dev, swiglu):
    """Every other row scaled by 1e-33 (1x128 scales near 2e-36, block-to-block ratios of order 1):
    the product of such a scale and a weight-block scale (~2e-4) is below the f32 normal range, so
    the kernels never form it (block-to-block factor (sa_c/sa_n)*(sb_c/sb_n), final scale applied
    factor by factor).  The outputs stay finite and match the dequantised oracle."""
    from mintext_amd.kernels.fp8 import (grouped_matmul_fp8, grouped_matmul_fp8_swiglu, quantize_fp8_rows,
                                         quantize_fp8_weights)

    rng = np.random.default_rng(11)
    M, E, Kin, Kout = 1024, 4, 512, 512
    gs = _groups(rng, M, E)
    blk = np.ones((M, Kin // 128))
    blk[::2] = 1e-33
    x = (torch.randn(M, Kin, device=dev) * torch.from_numpy(blk).float().to(dev).repeat_interleave(128, 1)).bfloat16()
    w = (torch.randn(E, Kin, Kout, device=dev) * 0.02).bfloat16()
    xq, xs = quantize_fp8_rows(x)
    assert float(xs.min()) < 1e-35  # the tiny blocks really have tiny scales
    wq, ws = quantize_fp8_weights(w)
    tg = _t(gs, dev)
    deq = O.gmm_fp8(_u8(xq), xs.cpu().numpy(), _u8(wq), ws.cpu().numpy(), gs)
    if swiglu:
        yq, ys, yb = grouped_matmul_fp8_swiglu(xq, xs, wq, ws, tg, return_bf16=True)
        tot = int(gs.sum())
        got = yb.float().cpu().numpy()[:tot]
        ref = O.swiglu(deq)[:tot]
        assert np.isfinite(got).all() and np.isfinite(ys.cpu().numpy()).all() and rel_err(got, ref) < 1e-2
    else:
        out = grouped_matmul_fp8(xq, xs, wq, ws, tg).float().cpu().numpy()
        assert np.isfinite(out).all() and rel_err(out, deq) < 1e-2


@pytest.mark.parametrize("M,E,Kin,I", [(1024, 4, 256, 256), (900, 8, 512, 384), (2048, 8, 2048, 768),
                                       (12000, 8, 1024, 768)])
def test_gmm_fp8_swiglu_requant(dev, M, E, Kin, I):
    from mintext_amd.kernels.fp8 import grouped_matmul_fp8_swiglu, quantize_fp8_rows, quantize_fp8_weights

    rng = np.random.default_rng(I)
    gs = _groups(rng, M, E)
    x = torch.randn(M, Kin, device=dev).bfloat16()
    w = (torch.randn(E, Kin, 2 * I, device=dev) * 0.05).bfloat16()
    xq, xs = quantize_fp8_rows(x)
    wq, ws = quantize_fp8_weights(w)
    yq, ys, yb = grouped_matmul_fp8_swiglu(xq, xs, wq, ws, _t(gs, dev), return_bf16=True)
    ref = O.swiglu(O.gmm_fp8(_u8(xq), xs.cpu().numpy(), _u8(wq), ws.cpu().numpy(), gs))
    tot = int(gs.sum())
    assert rel_err(yb.float().cpu().numpy()[:tot], ref[:tot]) < 1e-2
    # the fused re-quantisation is the 1x128 quantiser applied to the f32 SwiGLU values:
    # compare with quantising the bf16 copy (codes may differ by one step where the bf16
    # rounding moved a value across a code boundary)
    deq = O.dequant_rows(_u8(yq), ys.cpu().numpy())
    assert rel_err(deq[:tot], ref[:tot]) < 6e-2
    amax = np.abs(O.e4m3_decode(_u8(yq))[:tot].reshape(tot, I // 128, 128)).max(-1)
    assert ((amax == 448.0) | (ys.cpu().numpy()[:tot] == 1.0)).all()


@pytest.mark.parametrize("Kin", [128, 512])
def test_gmm_fp8_rows_past_group_sum(dev, Kin):
    """Rows past sum(group_sizes) come out as zeros even when their inputs hold NaN codes."""
    from mintext_amd.kernels.fp8 import (grouped_matmul_fp8, grouped_matmul_fp8_swiglu, quantize_fp8_rows,
                                         quantize_fp8_weights)

    M, E, N, I = 1000, 4, 512, 256
    rng = np.random.default_rng(Kin)
    gs = np.array([300, 0, 350, 250], np.int32)  # sum 900 < M
    x = torch.randn(M, Kin, device=dev).bfloat16()
    xq, xs = quantize_fp8_rows(x)
    xq[900:] = 0x7F  # e4m3fn NaN
    w = (torch.randn(E, Kin, N, device=dev) * 0.05).bfloat16()
    wq, ws = quantize_fp8_weights(w)
    out = grouped_matmul_fp8(xq, xs, wq, ws, _t(gs, dev))
    assert (out[900:] == 0).all()
    assert torch.isfinite(out.float()).all()
    deq = O.gmm_fp8(_u8(xq)[:900], xs.cpu().numpy()[:900], _u8(wq), ws.cpu().numpy(), gs)
    assert rel_err(out.float().cpu().numpy()[:900], deq) < 1e-2
    w2 = (torch.randn(E, Kin, 2 * I, device=dev) * 0.05).bfloat16()
    wq2, ws2 = quantize_fp8_weights(w2)
    yq, ys, yb = grouped_matmul_fp8_swiglu(xq, xs, wq2, ws2, _t(gs, dev), return_bf16=True)
    assert (yq[900:] == 0).all() and (yb[900:] == 0).all() and (ys[900:] == 1.0).all()


def test_gmm_fp8_more_zero_tiles_than_threads(dev):
    """Unused rows spanning more than 1024 zero tiles of 256 rows come out as zeros."""
    from mintext_amd.kernels.fp8 import grouped_matmul_fp8, quantize_fp8_rows, quantize_fp8_weights

    M, E, Kin, N = 270_000, 2, 256, 256
    gs = np.array([300, 200], np.int32)
    x = torch.randn(M, Kin, device=dev).bfloat16()
    xq, xs = quantize_fp8_rows(x)
    w = (torch.randn(E, Kin, N, device=dev) * 0.05).bfloat16()
    wq, ws = quantize_fp8_weights(w)
    out = grouped_matmul_fp8(xq, xs, wq, ws, _t(gs, dev))
    assert (out[500:] == 0).all()
    deq = O.gmm_fp8(_u8(xq)[:500], xs.cpu().numpy()[:500], _u8(wq), ws.cpu().numpy(), gs)
    assert rel_err(out.float().cpu().numpy()[:500], deq) < 1e-2


@pytest.mark.parametrize("T,K,E,D,I", [(2048, 8, 128, 2048, 768), (1000, 2, 8, 256, 128), (333, 3, 5, 512, 256)])
def test_gmm_fp8_swiglu_gathered_equals_route_quant(dev, T, K, E, D, I):
    """Quantising the tokens in token order and gathering their rows inside the fp8 gate_up GEMM
    gives the bits of the fused quantise-and-dispatch followed by the fp8 gate_up GEMM."""
    from mintext_amd.kernels.fp8 import (grouped_matmul_fp8_swiglu, grouped_matmul_fp8_swiglu_gathered,
                                         quantize_fp8_rows, quantize_fp8_weights)
    from mintext_amd.kernels.moe_dispatch import route_indices, route_quantize_fp8

    rng = np.random.default_rng(T + D)
    idx = _t(rng.integers(0, E, (T, K)).astype(np.int32), dev)
    x = torch.randn(T, D, device=dev).bfloat16()
    wq, wsc = quantize_fp8_weights((torch.randn(E, D, 2 * I, device=dev) * 0.02).bfloat16())
    sq, ss, si, gs, _ = route_quantize_fp8(x, idx, E)
    yq1, ys1, yb1 = grouped_matmul_fp8_swiglu(sq, ss, wq, wsc, gs, return_bf16=True)
    xq, xs = quantize_fp8_rows(x)
    si2, gs2, _ = route_indices(idx, E)
    yq2, ys2, yb2 = grouped_matmul_fp8_swiglu_gathered(xq, xs, si2, K, wq, wsc, gs2, return_bf16=True)
    assert torch.equal(yq1.view(torch.uint8), yq2.view(torch.uint8))
    assert torch.equal(ys1, ys2) and torch.equal(yb1, yb2)


def test_gmm_fp8_swiglu_gathered_short_k_unsupported(dev):
    from mintext_amd import _lib as L
    from mintext_amd.kernels.fp8 import grouped_matmul_fp8_swiglu_gathered, quantize_fp8_rows, quantize_fp8_weights
    from mintext_amd.kernels.moe_dispatch import route_indices

    T, K, E, D, I = 200, 2, 4, 128, 128  # K_in = 128 < 256: only the non-persistent kernels take it
    idx = _t(np.random.default_rng(0).integers(0, E, (T, K)).astype(np.int32), dev)
    xq, xs = quantize_fp8_rows(torch.randn(T, D, device=dev).bfloat16())
    wq, wsc = quantize_fp8_weights((torch.randn(E, D, 2 * I, device=dev) * 0.02).bfloat16())
    si, gs, _ = route_indices(idx, E)
    with pytest.raises(L.MtxError) as ei:
        grouped_matmul_fp8_swiglu_gathered(xq, xs, si, K, wq, wsc, gs)
    assert ei.value.status == L.MTX_ERR_UNSUPPORTED


def test_gmm_fp8_operand_beyond_32bit_offsets(dev):
    """fp8 codes of 4 GiB (2^21 rows x 2048): byte offsets past 32 bits take the register-staged
    fp8 kernel; sampled rows against the dequantised float64 product."""
    from mintext_amd.kernels.fp8 import grouped_matmul_fp8, quantize_fp8_weights

    M, Kin, Kout, E = 1 << 21, 2048, 256, 2
    gs = np.array([1234567, M - 1234567], np.int32)
    codes = torch.randint(0, 127, (M, Kin), dtype=torch.uint8, device=dev)  # magnitudes 0..448, no NaN code
    codes |= torch.randint(0, 2, (M, Kin), dtype=torch.uint8, device=dev) << 7
    xq = codes.view(torch.float8_e4m3fn)
    xs = torch.rand(M, Kin // 128, device=dev) * 0.1 + 0.01
    wq, ws = quantize_fp8_weights((torch.randn(E, Kin, Kout, device=dev) * 0.03).bfloat16())
    out = grouped_matmul_fp8(xq, xs, wq, ws, _t(gs, dev))
    rng = np.random.default_rng(10)
    rows = np.unique(np.concatenate([[0, 1234566, 1234567, M - 1], rng.integers(0, M, 40)]))
    tr = torch.from_numpy(rows).to(dev)
    xd = O.dequant_rows(_u8(xq[tr]), xs[tr].cpu().numpy())
    wd = O.dequant_weights(_u8(wq), ws.cpu().numpy())
    ref = np.stack([xd[i] @ wd[0 if r < 1234567 else 1] for i, r in enumerate(rows)])
    assert rel_err(out[tr].float().cpu().numpy(), ref) < 1e-2
    del xq, out
    torch.cuda.empty_cache()

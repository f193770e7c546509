"""GPU parity of the fp8 quantisers on inputs built to stress the division by the scale: every
value sits on, or a few ulps beside, an e4m3 value or a rounding midpoint of its group's scale;
the inputs hold signed zeros and subnormals; and the block scales span 2^-135 .. 2^110, so both the
four-instruction quotient (scales in [2^-64, 2^100]) and the IEEE division it falls back to run.
Codes and scales must equal the oracle's (numpy float32 division, RNE encoding) bit for bit.

Construction: the matrix is cut into 128 x 128 blocks with a scale S each; the block's diagonal
holds exactly 448 S, so every 1 x 128 row group, every 128 x 1 column chunk and the block itself
have amax 448 S and the kernels' scale amax / 448 is S exactly; the other values are t * S, t an
e4m3 value or the midpoint of two neighbouring ones, moved by -2 .. 2 ulps."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

# the positive e4m3 values below 448 and the midpoints between neighbours (all exact in float32)
_VALS = np.unique(O.e4m3_decode(np.arange(0, 0x7E, dtype=np.uint8)).astype(np.float64))
_TARGETS = np.concatenate([_VALS, (_VALS[:-1] + _VALS[1:]) / 2])
_TARGETS = _TARGETS[_TARGETS <= 432.0]
# block scale exponents: subnormal, below / at the lower bound of the fast quotient, ordinary, at /
# above its upper bound
_EXPS = [-135, -80, -65, -64, -40, -20, -5, 0, 10, 30, 60, 99, 100, 110]


def _block_scale(rng, bf16: bool) -> float:
    e = int(rng.choice(_EXPS))
    # mantissa bits: <= 3 for bf16 (t * S then stays exact in bf16's 8 bits), <= 20 for f32
    # (448 S exact); the lower bound block gets a mantissa above 1 so that it takes the fast path
    nb = 3 if bf16 else 20
    m = 1.0 + int(rng.integers(0, 2 ** nb)) / 2.0 ** nb
    if e == -64 and m == 1.0:
        m = 1.5
    return float(np.ldexp(m, e))


def _adversarial(rng, rows: int, cols: int, bf16: bool) -> np.ndarray:
    assert rows % 128 == 0 and cols % 128 == 0
    x = np.zeros((rows, cols), np.float32)
    for bi in range(rows // 128):
        for bj in range(cols // 128):
            s = _block_scale(rng, bf16)
            t = rng.choice(_TARGETS, (128, 128)) * rng.choice([-1.0, 1.0], (128, 128))
            v = (t * s).astype(np.float32)
            if bf16:  # exact in bf16; ulp steps of bf16 (the low 16 bits stay zero)
                step = rng.integers(-2, 3, (128, 128)).astype(np.int32) << 16
            else:
                step = rng.integers(-2, 3, (128, 128)).astype(np.int32)
            vi = v.view(np.int32) + np.where(v != 0, step, 0).astype(np.int32)
            v = vi.view(np.float32)
            v = np.where(np.abs(v) <= np.float32(448.0 * s), v, np.float32(0.0)).astype(np.float32)
            # signed zeros and subnormals (their quotients are below every e4m3 step)
            z = rng.random((128, 128))
            v[z < 0.02] = np.float32(-0.0)
            sub = (z > 0.98) & (448.0 * s > 1e-30)
            v[sub] = np.float32(1e-40) * rng.choice([-1.0, 1.0], int(sub.sum())).astype(np.float32)
            np.fill_diagonal(v, np.float32(448.0 * s) * rng.choice([-1.0, 1.0], 128).astype(np.float32))
            x[bi * 128:(bi + 1) * 128, bj * 128:(bj + 1) * 128] = v
    if bf16:  # the construction already lies on the bf16 grid (subnormal 1e-40 rounds)
        x = torch.from_numpy(x).bfloat16().float().numpy()
    return x


def _dev_tensor(x: np.ndarray, dev, bf16: bool) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    return t.bfloat16() if bf16 else t


def _u8(t):
    return t.view(torch.uint8).cpu().numpy()


@pytest.mark.parametrize("bf16", [False, True])
def test_quant_rows_edges(dev, bf16):
    from mintext_amd.kernels.fp8 import quantize_fp8_rows

    rng = np.random.default_rng(11 + bf16)
    x = _adversarial(rng, 512, 768, bf16)
    q, s = quantize_fp8_rows(_dev_tensor(x, dev, bf16))
    oq, os_ = O.quant_fp8_rows(x)
    np.testing.assert_array_equal(s.cpu().numpy(), os_)
    np.testing.assert_array_equal(_u8(q), oq)


@pytest.mark.parametrize("bf16", [False, True])
def test_route_quantize_fp8_edges(dev, bf16):
    from mintext_amd.kernels.moe_dispatch import route_quantize_fp8

    rng = np.random.default_rng(23 + bf16)
    N, D, K, E = 384, 512, 4, 16
    x = _adversarial(rng, N, D, bf16)
    idx = torch.from_numpy(rng.integers(0, E, (N, K)).astype(np.int32)).to(dev)
    q, s, perm, gs, inv = route_quantize_fp8(_dev_tensor(x, dev, bf16), idx, E)
    rows = perm.cpu().numpy().astype(np.int64) // K
    oq, os_ = O.quant_fp8_rows(x[rows])
    np.testing.assert_array_equal(s.cpu().numpy(), os_)
    np.testing.assert_array_equal(_u8(q), oq)


@pytest.mark.parametrize("bf16", [False, True])
def test_quant_weights_edges(dev, bf16):
    from mintext_amd.kernels.fp8 import quantize_fp8_weights, quantize_fp8_weights_t

    rng = np.random.default_rng(37 + bf16)
    w = np.stack([_adversarial(rng, 256, 384, bf16) for _ in range(2)])
    wt = _dev_tensor(w, dev, bf16)
    wq, ws = quantize_fp8_weights(wt)
    oq, os_ = O.quant_fp8_weights(w)
    np.testing.assert_array_equal(ws.cpu().numpy(), os_)
    np.testing.assert_array_equal(_u8(wq), oq)
    wq, ws = quantize_fp8_weights_t(wt)
    oq, os_ = O.quant_fp8_weights_t(w)
    np.testing.assert_array_equal(ws.cpu().numpy(), os_)
    np.testing.assert_array_equal(_u8(wq), oq)


@pytest.mark.parametrize("blocks", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
def test_quant_grouped_t_edges(dev, bf16, blocks):
    from mintext_amd.kernels.fp8 import quantize_fp8_grouped_t

    rng = np.random.default_rng(41 + 2 * bf16 + blocks)
    gs = np.array([128, 0, 256, 128], np.int32)  # chunks aligned with the 128-row blocks
    x = _adversarial(rng, int(gs.sum()), 384, bf16)
    xt, xs = quantize_fp8_grouped_t(_dev_tensor(x, dev, bf16), torch.from_numpy(gs).to(dev), blocks=blocks)
    oq, os_ = O.quant_fp8_grouped_t(x, gs, blocks)
    _, cb = O.fp8_group_chunks(gs, len(x))
    used, F = int(cb[-1]), x.shape[1]  # chunk slots past the groups are not written
    nf = F // 128 if blocks else F
    np.testing.assert_array_equal(xs.cpu().numpy()[:nf * used], os_[:nf * used])
    np.testing.assert_array_equal(_u8(xt)[:128 * F * used], oq[:128 * F * used])

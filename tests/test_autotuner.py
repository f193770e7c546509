"""Autotuner (mintext_amd/kernels/autotuner.py): the reference's TestAutotuner
(tests/test_moe_kernels.py:639-716) restated on the HIP tile-configuration space, host-side
tiling handling, and -- on the GPU -- that every candidate tiling reproduces the heuristic
configuration's output bits and that autotune_moe tunes and caches."""
from __future__ import annotations

import json

import numpy as np
import pytest

from mintext_amd.kernels.autotuner import (MoETuningConfig, MoETuningResult, _cache_key, _generate_candidates,
                                           _load_cache, _save_cache, autotune_moe)
from mintext_amd.kernels.grouped_matmul import _pad_tiling, _tile_args


def _pow2(v: int) -> bool:
    return v > 0 and v & (v - 1) == 0


def test_candidate_generation():
    # same call as test_moe_kernels.py:643-651
    candidates = _generate_candidates(M=256, K=128, N=64)
    assert len(candidates) > 0
    for c in candidates:
        assert len(c) == 3
        assert all(_pow2(v) for v in c)


def test_candidates_cover_hip_space():
    c = _generate_candidates(M=16384, K=4096, N=28672, E=8)   # Mixtral gate_up: 2048 rows per expert
    assert {t[0] for t in c} == {128, 256}
    assert {t[1] for t in c if t[0] == 256} == {1, 2, 4, 8}
    assert {t[1] for t in c if t[0] == 128} == {1, 2, 4, 8, 16}
    assert all(t[2] == 256 for t in c)
    # ~128 rows per expert (DeepSeek shape): one m-tile per group only
    assert _generate_candidates(M=32768, K=7168, N=4096, E=256) == [(128, 1, 256), (256, 1, 256)]


def test_cache_save_load(tmp_path):
    config = MoETuningConfig(num_experts=8, hidden_size=256, moe_intermediate_size=512, num_experts_per_tok=2,
                             batch_seq_tokens=1024, dtype="bfloat16")
    key = _cache_key(config)
    result = MoETuningResult(gate_up_tiling=(128, 64, 256), down_tiling=(64, 128, 128), backend="ragged_dot",
                             throughput_gflops=42.0)
    _save_cache(str(tmp_path), key, result)
    loaded = _load_cache(str(tmp_path), key)
    assert loaded is not None
    assert loaded.gate_up_tiling == (128, 64, 256)
    assert loaded.down_tiling == (64, 128, 128)
    assert loaded.backend == "ragged_dot"
    assert loaded.throughput_gflops == 42.0
    # the file format of the reference (autotuner.py:75-86)
    data = json.loads((tmp_path / f"moe_tune_{key}.json").read_text())
    assert data == {"gate_up_tiling": [128, 64, 256], "down_tiling": [64, 128, 128], "backend": "ragged_dot",
                    "throughput_gflops": 42.0}


def test_cache_invalidation(tmp_path):
    c1 = MoETuningConfig(num_experts=8, hidden_size=256, moe_intermediate_size=512, num_experts_per_tok=2,
                         batch_seq_tokens=1024)
    c2 = MoETuningConfig(num_experts=16, hidden_size=256, moe_intermediate_size=512, num_experts_per_tok=2,
                         batch_seq_tokens=1024)
    k1, k2 = _cache_key(c1), _cache_key(c2)
    assert k1 != k2 and len(k1) == 64
    _save_cache(str(tmp_path), k1, MoETuningResult(None, None, "ragged_dot", 0.0))
    assert _load_cache(str(tmp_path), k2) is None
    got = _load_cache(str(tmp_path), k1)
    assert got is not None and got.gate_up_tiling is None and got.down_tiling is None


def test_corrupt_cache_is_ignored(tmp_path):
    (tmp_path / "moe_tune_abc.json").write_text("{not json")
    assert _load_cache(str(tmp_path), "abc") is None
    (tmp_path / "moe_tune_def.json").write_text(json.dumps({"gate_up_tiling": None}))
    assert _load_cache(str(tmp_path), "def") is None


def test_result_fields():
    r = MoETuningResult(gate_up_tiling=(128, 64, 256), down_tiling=None, backend="ragged_dot",
                        throughput_gflops=50.0)
    assert r.gate_up_tiling == (128, 64, 256)
    assert r.down_tiling is None
    assert r.backend == "ragged_dot"
    assert r.throughput_gflops == 50.0


def test_cached_result_needs_no_gpu(tmp_path):
    config = MoETuningConfig(num_experts=4, hidden_size=128, moe_intermediate_size=256, num_experts_per_tok=2,
                             batch_seq_tokens=64)
    r = MoETuningResult((256, 2, 256), (128, 1, 256), "hip-gfx950", 123.0)
    _save_cache(str(tmp_path), _cache_key(config), r)
    assert autotune_moe(config, cache_dir=str(tmp_path)) == r


def test_tile_args_mapping():
    assert _tile_args(None) == (0, 0)
    assert _tile_args((256, 8, 256)) == (256, 8)
    assert _tile_args((64, 1, 256)) == (128, 1)       # tm rounds to the nearer supported value
    assert _tile_args((512, 128, 256)) == (256, 64)   # tg clamps to 64
    # TPU tilings (tn != 256), e.g. the reference's default (128, 128, 128): heuristics
    assert _tile_args((128, 128, 128)) == (0, 0)
    assert _tile_args((256, 512, 512)) == (0, 0)
    with pytest.raises(ValueError):
        _tile_args((0, 1, 256))
    # 3 -> 9 padding of grouped_matmul.py:108-112
    assert _pad_tiling((256, 4, 256)) == (256, 4, 256) * 3
    assert _pad_tiling(tuple(range(1, 10))) == tuple(range(1, 10))


# ---- GPU -------------------------------------------------------------------------------------

def _groups(rng, M, E, skew=False):
    if skew:
        p = rng.dirichlet(np.full(E, 0.3))
        g = rng.multinomial(M, p)
    else:
        g = rng.multinomial(M, np.full(E, 1.0 / E))
    return g.astype(np.int32)


def _same_sums(got, ref, tag):
    """Same f32 sums up to summation order, each rounded once to bf16: tile configurations
    whose 256-row schedule splits tail tiles along K add the k-pieces in another order, so
    outputs agree to a bf16 rounding (plus the f32 error where a sum cancels), not bit for bit.
    Each configuration is deterministic."""
    import torch

    d = (got.float() - ref.float()).abs()
    bound = ref.float().abs() * 2.0 ** -7 + 1e-4 * ref.float().abs().max()
    assert (d <= bound).all(), (tag, (d - bound).max().item())


@pytest.mark.gpu
@pytest.mark.parametrize("skew", [False, True])
def test_every_tiling_gives_the_same_sums(dev, skew):
    import torch

    from mintext_amd.kernels.grouped_matmul import (_gmm_dlhs, grouped_matmul, grouped_matmul_swiglu)

    rng = np.random.default_rng(7 + skew)
    M, K, N, E = 2048, 512, 1024, 4
    gs = torch.from_numpy(_groups(rng, M - 37, E, skew)).to(dev)   # 37 rows past sum(gs)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(dev).bfloat16()
    w = torch.from_numpy((rng.standard_normal((E, K, N)) * 0.05).astype(np.float32)).to(dev).bfloat16()
    g = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(dev).bfloat16()
    ref_f = grouped_matmul(x, w, gs)
    ref_s = grouped_matmul_swiglu(x, w, gs)
    ref_d = _gmm_dlhs(g, w, gs)
    cands = _generate_candidates(M, K, N, E) + [(128, 64, 256), (256, 64, 256)]
    for t in cands:
        for got, ref in ((grouped_matmul(x, w, gs, tiling=t), ref_f),
                         (grouped_matmul_swiglu(x, w, gs, tiling=t), ref_s), (_gmm_dlhs(g, w, gs, t), ref_d)):
            _same_sums(got, ref, t)
        assert torch.equal(grouped_matmul(x, w, gs, tiling=t), grouped_matmul(x, w, gs, tiling=t)), t
    # and the heuristic result is the grouped product (bf16 tolerance vs float64)
    xs, ws_, fs = x.double().cpu().numpy(), w.double().cpu().numpy(), ref_f.double().cpu().numpy()
    off = np.concatenate([[0], np.cumsum(gs.cpu().numpy())])
    for e in range(E):
        a, b = off[e], off[e + 1]
        if b > a:
            ref = xs[a:b] @ ws_[e]
            assert np.linalg.norm(fs[a:b] - ref) / np.linalg.norm(ref) < 2e-2
    assert not fs[off[-1]:].any()


@pytest.mark.gpu
def test_grouped_matmul_vjp_with_tiling_matches_default(dev):
    import torch

    from mintext_amd.kernels.grouped_matmul import grouped_matmul_vjp

    rng = np.random.default_rng(11)
    M, K, N, E = 1024, 256, 512, 4
    gs = torch.from_numpy(_groups(rng, M, E)).to(dev)
    x0 = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(dev).bfloat16()
    w0 = torch.from_numpy((rng.standard_normal((E, K, N)) * 0.05).astype(np.float32)).to(dev).bfloat16()
    outs = []
    for tiling in [(128,) * 9, (128, 2, 256, 256, 1, 256, 128, 128, 128), None]:
        x = x0.clone().requires_grad_(True)
        w = w0.clone().requires_grad_(True)
        y = grouped_matmul_vjp(x, w, gs, tiling=tiling)
        y.float().square().sum().backward()
        outs.append((y.detach(), x.grad, w.grad))
    for other in outs[1:]:
        _same_sums(other[0], outs[0][0], "y")
        for a, b in zip(outs[0][1:], other[1:]):  # gradients of a loss of y: relative norm
            assert (torch.linalg.vector_norm((a - b).float()) / torch.linalg.vector_norm(b.float())).item() < 2e-3


@pytest.mark.gpu
def test_autotune_moe_tunes_and_caches(dev, tmp_path):
    config = MoETuningConfig(num_experts=4, hidden_size=256, moe_intermediate_size=512, num_experts_per_tok=2,
                             batch_seq_tokens=1024, dtype="bfloat16")
    r = autotune_moe(config, cache_dir=str(tmp_path), max_trials=4, warmup_iters=1, bench_iters=2)
    assert r.backend == "hip-gfx950"
    assert r.throughput_gflops > 0
    for t in (r.gate_up_tiling, r.down_tiling):
        assert t is None or (len(t) == 3 and all(_pow2(v) for v in t))
    assert _load_cache(str(tmp_path), _cache_key(config)) == r


def test_reference_default_tiling_keeps_heuristics():
    from mintext_amd.kernels.grouped_matmul import _pad_tiling

    # grouped_matmul_vjp's default and the reference's "no tiling configured" value
    for t in [(128,) * 9, _pad_tiling((128, 128, 128))]:
        assert _tile_args(t[0:3]) == (0, 0) and _tile_args(t[3:6]) == (0, 0)

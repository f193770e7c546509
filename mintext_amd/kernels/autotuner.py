"""Autotuner for the MoE grouped GEMMs on gfx950, with a disk cache.

Mirror of bzantium/mintext ``mintext/kernels/autotuner.py`` (same names, dataclasses, cache
key recipe and JSON file format, pinned by ``tests/test_moe_kernels.py:643-716``).  The search
space is the HIP kernels' own tile configuration instead of TPU ``ragged_dot`` tilings:

* ``tm`` -- rows per m-tile: 128 (4 waves, two workgroups per CU) or 256 (8 waves, one per CU);
* ``tg`` -- m-tiles per scheduling group: consecutive tiles of one XCD sweep ``tg`` m-tiles
  before moving to the next n-tile, which sets how x and weight tiles are re-read through L2;
* ``tn`` -- columns per n-tile, always 256 (the MFMA kernels' only width).

A tiling is the tuple ``(tm, tg, tn)``; ``grouped_matmul(..., tiling=...)`` and
``grouped_matmul_vjp`` take it directly.  Every tiling computes the same f32 sums (outputs
agree to a bf16 rounding, bit for bit where the kernels' split tail splits the same tiles),
so tuning only trades time.  Candidates are timed with HIP events on the current stream.

Reference: ``MoETuningConfig`` / ``MoETuningResult`` (autotuner.py:18-36), ``_cache_key``
(:39-55), ``_load_cache`` / ``_save_cache`` (:58-86), ``_generate_candidates`` (:89-104),
``autotune_moe`` (:177-310).
"""
from __future__ import annotations

import hashlib
import json
import logging
from dataclasses import dataclass
from pathlib import Path

logger = logging.getLogger(__name__)

BACKEND = "hip-gfx950"


@dataclass
class MoETuningConfig:
    """Problem dimensions for MoE autotuning (autotuner.py:18-26)."""
    num_experts: int
    hidden_size: int
    moe_intermediate_size: int
    num_experts_per_tok: int
    batch_seq_tokens: int  # B * S
    dtype: str = "bfloat16"


@dataclass
class MoETuningResult:
    """Best tilings found (autotuner.py:29-36): ``(tm, tg, tn)`` tuples or None (heuristics)."""
    gate_up_tiling: tuple[int, ...] | None
    down_tiling: tuple[int, ...] | None
    backend: str
    throughput_gflops: float


def _device_identity() -> tuple[str, str]:
    """(platform, device kind) for the cache key; the CPU when no ROCm device is visible."""
    try:
        import torch

        if torch.cuda.is_available():
            props = torch.cuda.get_device_properties(0)
            return "rocm", f"{props.name}:{getattr(props, 'gcnArchName', '')}"
    except Exception:  # pragma: no cover - torch import problems surface elsewhere
        pass
    return "cpu", "cpu"


def _cache_key(config: MoETuningConfig) -> str:
    """SHA256 of the config fields + platform + device kind (autotuner.py:39-55)."""
    platform, device_kind = _device_identity()
    key_data = {
        "num_experts": config.num_experts,
        "hidden_size": config.hidden_size,
        "moe_intermediate_size": config.moe_intermediate_size,
        "num_experts_per_tok": config.num_experts_per_tok,
        "batch_seq_tokens": config.batch_seq_tokens,
        "dtype": config.dtype,
        "platform": platform,
        "device_kind": device_kind,
    }
    return hashlib.sha256(json.dumps(key_data, sort_keys=True).encode()).hexdigest()


def _load_cache(cache_dir: str, key: str) -> MoETuningResult | None:
    """The cached result for ``key``, or None when absent or unreadable (autotuner.py:58-72)."""
    path = Path(cache_dir) / f"moe_tune_{key}.json"
    if not path.exists():
        return None
    try:
        data = json.loads(path.read_text())
        return MoETuningResult(
            gate_up_tiling=tuple(data["gate_up_tiling"]) if data["gate_up_tiling"] else None,
            down_tiling=tuple(data["down_tiling"]) if data["down_tiling"] else None,
            backend=data["backend"],
            throughput_gflops=data["throughput_gflops"],
        )
    except (json.JSONDecodeError, KeyError, TypeError):
        return None


def _save_cache(cache_dir: str, key: str, result: MoETuningResult) -> None:
    """Write ``result`` as ``moe_tune_<key>.json`` (autotuner.py:75-86 format)."""
    path = Path(cache_dir) / f"moe_tune_{key}.json"
    path.parent.mkdir(parents=True, exist_ok=True)
    data = {
        "gate_up_tiling": list(result.gate_up_tiling) if result.gate_up_tiling else None,
        "down_tiling": list(result.down_tiling) if result.down_tiling else None,
        "backend": result.backend,
        "throughput_gflops": result.throughput_gflops,
    }
    path.write_text(json.dumps(data, indent=2))


def _generate_candidates(M: int, K: int, N: int, E: int = 1) -> list[tuple[int, int, int]]:
    """HIP tile configurations ``(tm, tg, tn)`` worth timing for an [M,K] x [E,K,N] grouped GEMM.

    tm in {128, 256}; tg a power of two from 1 up to the m-tiles of a mean group (at least 1,
    at most 16); tn = 256.  Every entry is a power of two (as autotuner.py:89-104).  K and N do
    not restrict the space: shapes the MFMA tiling does not cover fall back to other kernels
    whatever the tiling.
    """
    del K, N
    out = []
    mean_rows = max(1, M // max(E, 1))
    for tm in (128, 256):
        if tm > max(128, 2 * M):
            continue
        tiles_per_group = max(1, -(-mean_rows // tm))
        tg = 1
        while tg <= min(16, max(1, tiles_per_group)):
            out.append((tm, tg, 256))
            tg *= 2
    return out


def _event_time_ms(fn, warmup_iters: int, bench_iters: int) -> float:
    import torch

    for _ in range(warmup_iters):
        fn()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(bench_iters):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / bench_iters


def _benchmark_tiling(x, weights, group_sizes, tiling, warmup_iters: int, bench_iters: int) -> float:
    """GFLOP/s of ``grouped_matmul(x, weights, group_sizes, tiling=tiling)`` (autotuner.py:107-140)."""
    from .grouped_matmul import grouped_matmul

    ms = _event_time_ms(lambda: grouped_matmul(x, weights, group_sizes, tiling=tiling), warmup_iters, bench_iters)
    M, K_in = x.shape
    K_out = weights.shape[2]
    return 2.0 * M * K_in * K_out / (ms * 1e-3) / 1e9


def _uniform_group_sizes(M: int, E: int, device):
    """Near-uniform expert loads, as the reference tunes with (autotuner.py:236-241)."""
    import torch

    base, rem = divmod(M, E)
    return torch.tensor([base + (1 if i < rem else 0) for i in range(E)], dtype=torch.int32, device=device)


def _tune_one(x, w, gs, candidates, warmup_iters, bench_iters, name):
    """Best (tiling, GFLOP/s) among the heuristic configuration (None) and ``candidates``.

    Every configuration is timed twice, in forward then reverse order, and keeps its better
    run, so that clock ramp-up and thermal drift do not favour the configurations timed last.
    """
    configs = [None] + list(candidates)
    score = {i: 0.0 for i in range(len(configs))}
    for order in (range(len(configs)), reversed(range(len(configs)))):
        for i in order:
            score[i] = max(score[i], _benchmark_tiling(x, w, gs, configs[i], warmup_iters, bench_iters))
    logger.info("  %s heuristic tiling: %.1f GFLOPS", name, score[0])
    best_i = max(score, key=lambda i: (score[i], i == 0))  # ties keep the heuristic
    if best_i:
        logger.info("  best %s: %s -> %.1f GFLOPS", name, configs[best_i], score[best_i])
    return configs[best_i], score[best_i]


def autotune_moe(config: MoETuningConfig, cache_dir: str | None = None, max_trials: int = 20,
                 warmup_iters: int = 3, bench_iters: int = 10) -> MoETuningResult:
    """Tile configurations for the gate_up and down grouped GEMMs (autotuner.py:177-310).

    Times the heuristic configuration (tiling None) and up to ``max_trials`` candidates per
    GEMM on synthetic data with near-uniform expert loads, keeps the fastest, and caches the
    result under ``cache_dir`` when given.  Needs a ROCm device unless the cache already holds
    the result.
    """
    key = _cache_key(config) if cache_dir else None
    if cache_dir:
        cached = _load_cache(cache_dir, key)
        if cached is not None:
            logger.info("MoE autotuner: loaded cached result (%.1f GFLOPS)", cached.throughput_gflops)
            return cached

    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("autotune_moe times the HIP kernels and needs a ROCm GPU (no cached result found)")
    dtype = {"bfloat16": torch.bfloat16, "float32": torch.float32}.get(config.dtype)
    if dtype is None:
        raise ValueError(f"autotune_moe: unsupported dtype {config.dtype!r} (bfloat16 or float32)")
    dev = torch.device("cuda", torch.cuda.current_device())
    E, D, I = config.num_experts, config.hidden_size, config.moe_intermediate_size
    M = config.batch_seq_tokens * config.num_experts_per_tok
    gen = torch.Generator(device=dev)
    gen.manual_seed(42)
    gs = _uniform_group_sizes(M, E, dev)

    def pick(cands):
        if len(cands) > max_trials:
            step = len(cands) // max_trials
            cands = cands[::step][:max_trials]
        return cands

    logger.info("MoE autotuner: tuning gate_up (%d, %d) @ (%d, %d, %d)", M, D, E, D, 2 * I)
    x = torch.randn((M, D), generator=gen, device=dev, dtype=torch.float32).to(dtype)
    w = torch.randn((E, D, 2 * I), generator=gen, device=dev, dtype=torch.float32).mul_(0.02).to(dtype)
    gu_t, gu_g = _tune_one(x, w, gs, pick(_generate_candidates(M, D, 2 * I, E)), warmup_iters, bench_iters,
                           "gate_up")
    del x, w
    logger.info("MoE autotuner: tuning down (%d, %d) @ (%d, %d, %d)", M, I, E, I, D)
    x = torch.randn((M, I), generator=gen, device=dev, dtype=torch.float32).to(dtype)
    w = torch.randn((E, I, D), generator=gen, device=dev, dtype=torch.float32).mul_(0.02).to(dtype)
    dn_t, dn_g = _tune_one(x, w, gs, pick(_generate_candidates(M, I, D, E)), warmup_iters, bench_iters, "down")
    del x, w

    result = MoETuningResult(gate_up_tiling=gu_t, down_tiling=dn_t, backend=BACKEND,
                             throughput_gflops=gu_g + dn_g)
    if cache_dir:
        _save_cache(cache_dir, key, result)
        logger.info("MoE autotuner: saved to cache (%.1f GFLOPS total)", result.throughput_gflops)
    return result

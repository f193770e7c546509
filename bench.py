"""Benchmark of the MoE layer forward on one MI355X (default: the Mixtral-8x7B shape, bf16).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config mixtral|tiny|deepseek|qwen3_fp8|qwen3_bwd|qwen3_bwd_fp8]

A step is one MoE layer forward over one batch of synthetic tokens, inputs resident in HBM:
router top-k on the gate logits -> route (dispatch) -> grouped GEMM gate_up with the fused
SwiGLU -> grouped GEMM down -> weighted combine.  By default the route computes only the
permutation and the gate_up GEMM gathers the token rows itself (the same bits; ``--no-gather``
copies the rows to sorted order first, as ``route`` does).  (The gate GEMM producing the logits
is not part of the path; the logits are an input.)  For ``qwen3_bwd`` a step is the grouped-GEMM
backward (dlhs + tgmm for both expert GEMMs) under Zipf-skewed routing.

Prints ONE JSON line (rank 0).  ``roofline`` is measured live for the dominant kernel with HIP
events on the stream the kernels run on; ``cpu_baseline`` times a torch-CPU restatement of the
reference layer (oracle/cpu_port.py, the reference's arithmetic) on a bounded sample of the same
workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_FP8_TFLOPS = 5000.0    # MI355X dense fp8 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

CONFIGS = {
    "tiny": dict(T=256, D=128, E=8, K=2, I=256, dtype="f32", scoring="softmax", wstd=0.02),
    "mixtral": dict(T=8192, D=4096, E=8, K=2, I=14336, dtype="bf16", scoring="softmax", wstd=0.02),
    "deepseek": dict(T=4096, D=7168, E=256, K=8, I=2048, dtype="bf16", scoring="sigmoid_group", wstd=0.006,
                     n_group=8, topk_group=4, scale=2.5, shared=1),
    "qwen3_fp8": dict(T=16384, D=2048, E=128, K=8, I=768, dtype="fp8", scoring="softmax", wstd=0.02),
    "qwen3_bwd": dict(T=16384, D=2048, E=128, K=8, I=768, dtype="bf16", scoring="softmax", wstd=0.02, zipf=1.2),
    # the C5 backward with fp8 operands (not a BASELINE config: the same shapes and routing)
    "qwen3_bwd_fp8": dict(T=16384, D=2048, E=128, K=8, I=768, dtype="fp8", scoring="softmax", wstd=0.02, zipf=1.2),
}


def _traffic(name: str):
    """(HBM bytes per launch, kernel description) from profiles/traffic_<name>.json, or (None, None)."""
    p = ROOT / "profiles" / f"traffic_{name}.json"
    if p.exists():
        try:
            d = json.loads(p.read_text())
            return d.get("bytes_per_launch"), d.get("kernel")
        except Exception:
            return None, None
    return None, None


class EventTimer:
    """Accumulates HIP-event durations of one region inside the timed loop."""

    def __init__(self, torch):
        self.torch = torch
        self.pairs = []

    def start(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        self.pairs.append([e, None])

    def stop(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        self.pairs[-1][1] = e

    def mean_ms(self):
        return float(np.mean([a.elapsed_time(b) for a, b in self.pairs])) if self.pairs else 0.0


def _cpu_baseline_layer(x, logits, gate_up, down, cfg, shared=None, target_s=4.0):
    """The layer forward on the host CPU in the reference's arithmetic (oracle/cpu_port.py: torch,
    bf16 operands, f32 routing and combine) on the first Ts tokens of the same inputs: one probe
    run sizes Ts for about ``target_s`` per run, then 1 warm-up and the median of 3 timed runs."""
    import torch

    from oracle import cpu_port

    torch.set_num_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    cores = torch.get_num_threads()
    T = x.shape[0]
    kw = dict(k=cfg["K"], scoring=cfg["scoring"], shared=shared, n_group=cfg.get("n_group", 1),
              topk_group=cfg.get("topk_group", 1), routed_scaling_factor=cfg.get("scale", 1.0))

    def once(ts):
        t0 = time.perf_counter()
        cpu_port.moe_layer(x[:ts], logits[:ts], gate_up, down, **kw)
        return time.perf_counter() - t0

    ts = min(T, 256)
    dt = once(ts)
    ts = int(min(T, max(ts, ts * target_s / max(dt, 1e-3))))
    once(ts)  # warm-up at the timed size
    runs = sorted(once(ts) for _ in range(3))
    med = runs[1]
    dt_name = {torch.bfloat16: "bf16", torch.float32: "f32"}[x.dtype]
    return {"value": ts / med, "unit": "tokens/s", "cores": int(cores), "kind": "port",
            "sample": f"torch-CPU restatement of the reference layer (oracle/cpu_port.py; {dt_name} operands, "
                      f"f32 routing and combine) on the first {ts} of {T} tokens of the same inputs; 1 warm-up, "
                      f"median of 3 runs = {med:.2f} s"}


def _zipf_bias(E, s, rng, beta=0.55):
    rank = rng.permutation(E) + 1
    return (-beta * s * np.log(rank)).astype(np.float32)


def layer_inputs(cfg_name, dev, g=None):
    """The synthetic inputs of a config, generated on the device from seed 2: tokens x [T,D],
    gate logits [T,E] (x @ W_g in f32, rounded to the compute dtype; plus the Zipf popularity
    bias for qwen3_bwd), expert weights gate_up [E,D,2I] / down [E,I,D] and, for deepseek, the
    shared expert ([1,D,2I'], [1,I',D]).  Returns (x, logits, gate_up, down, shared, g) with g the
    generator, positioned after the weights (the backward config draws its gradients from it)."""
    import torch

    cfg = CONFIGS[cfg_name]
    T, D, E, I = cfg["T"], cfg["D"], cfg["E"], cfg["I"]
    if g is None:
        g = torch.Generator(device=dev)
        g.manual_seed(2)
    cdt = torch.float32 if cfg["dtype"] == "f32" else torch.bfloat16
    x = torch.randn(T, D, device=dev, generator=g).to(cdt)
    wg = torch.randn(D, E, device=dev, generator=g) * cfg["wstd"]
    logits = (x.float() @ wg).to(cdt)  # the gate GEMM output: an input of the path
    if cfg.get("zipf"):
        bias = torch.from_numpy(_zipf_bias(E, cfg["zipf"], np.random.default_rng(5))).to(dev)
        logits = (logits.float() + bias).to(cdt)
    gate_up = (torch.randn(E, D, 2 * I, device=dev, generator=g) * cfg["wstd"]).to(cdt)
    down = (torch.randn(E, I, D, device=dev, generator=g) * cfg["wstd"]).to(cdt)
    shared = None
    if cfg.get("shared"):
        shared = ((torch.randn(1, D, 2 * I * cfg["shared"], device=dev, generator=g) * cfg["wstd"]).to(cdt),
                  (torch.randn(1, I * cfg["shared"], D, device=dev, generator=g) * cfg["wstd"]).to(cdt))
    return x, logits, gate_up, down, shared, g


def router_kwargs(cfg_name):
    cfg = CONFIGS[cfg_name]
    return dict(scoring=cfg["scoring"], n_group=cfg.get("n_group", 1), topk_group=cfg.get("topk_group", 1),
                routed_scaling_factor=cfg.get("scale", 1.0))


def run(cfg_name, steps, warmup, cpu_baseline=True, shared_mode="separate", use_graph=False, gather=True,
        fp8_scales="amax"):
    import torch

    from mintext_amd import _lib
    from mintext_amd.kernels import grouped_matmul_swiglu, grouped_matmul_vjp, route, route_topk, tgmm, unroute
    from mintext_amd.kernels.grouped_matmul import _gmm_dlhs
    from mintext_amd.kernels.moe_dispatch import unroute_add

    _lib.lib()
    cfg = CONFIGS[cfg_name]
    dev = torch.device("cuda:0")
    T, D, E, K, I = cfg["T"], cfg["D"], cfg["E"], cfg["K"], cfg["I"]
    M = T * K
    cdt = torch.float32 if cfg["dtype"] == "f32" else torch.bfloat16
    x, logits, gate_up, down, shared, g = layer_inputs(cfg_name, dev)
    fold = False
    if shared is not None:
        fold = shared_mode == "folded" and cfg["shared"] == 1
        if fold:
            # load-time transform: the shared expert becomes expert E of the routed weights
            from mintext_amd.moe import fold_shared_expert

            gate_up, down = fold_shared_expert(gate_up, down, shared[0], shared[1])
    rkw = router_kwargs(cfg_name)

    t_gu, t_dn, t_disp, t_comb = EventTimer(torch), EventTimer(torch), EventTimer(torch), EventTimer(torch)
    Mg = M + T if fold else M  # rows through the expert GEMMs (the folded shared expert adds T)
    Kc = K + 1 if fold else K  # rows combined per token
    Eg = E + 1 if fold else E  # groups
    flops_fwd = 2.0 * Mg * D * 2 * I + 2.0 * Mg * I * D
    fp8 = cfg["dtype"] == "fp8"
    if fp8:
        from mintext_amd.kernels.fp8 import (grouped_matmul_fp8, grouped_matmul_fp8_swiglu,
                                             grouped_matmul_fp8_swiglu_gathered, quantize_fp8_rows,
                                             quantize_fp8_weights)
        from mintext_amd.kernels.moe_dispatch import route_quantize_fp8

        f8s = dict(scales=fp8_scales)  # "amax" (scale amax/448) or "pow2" (power-of-two scales, MFMA E8M0)
        guq, gus = quantize_fp8_weights(gate_up, **f8s)
        dnq, dns = quantize_fp8_weights(down, **f8s)
    # the route's row gather inside the gate_up GEMM's operand loads (no sorted copy written)
    from mintext_amd.kernels.grouped_matmul import gathered_swiglu_supported, grouped_matmul_swiglu_gathered
    from mintext_amd.kernels.moe_dispatch import route_indices

    bwd = cfg_name in ("qwen3_bwd", "qwen3_bwd_fp8")
    gather = gather and not bwd and (D >= 256 if fp8 else gathered_swiglu_supported(x, gate_up))
    if fp8 and fp8_scales != "amax" and not gather and not bwd:
        raise SystemExit("--fp8-scales pow2 needs the gathered layer flow (the fused dispatch quantiser is amax-only)")

    def step(timed):
        with torch.no_grad():
            idx, w = route_topk(logits, K, shared_expert=E if fold else None, **rkw)
            if timed:
                t_disp.start()
            if gather:
                # permutation only; fp8: the tokens quantised in token order (1x128 groups)
                if fp8:
                    xq, xs = quantize_fp8_rows(x, **f8s)
                si, gs, _ = route_indices(idx, Eg)
            elif fp8:
                # 1x128 quantisation of the tokens fused into their dispatch
                sq, ss, si, gs, _ = route_quantize_fp8(x, idx, E)
            else:
                st, si, gs = route(x, idx, Eg)
            if timed:
                t_disp.stop()
                t_gu.start()
            if gather:
                if fp8:
                    yq, ys = grouped_matmul_fp8_swiglu_gathered(xq, xs, si, Kc, guq, gus, gs, **f8s)
                else:
                    y = grouped_matmul_swiglu_gathered(x, si, Kc, gate_up, gs)
            elif fp8:
                yq, ys = grouped_matmul_fp8_swiglu(sq, ss, guq, gus, gs)
            else:
                y = grouped_matmul_swiglu(st, gate_up, gs)
            if timed:
                t_gu.stop()
                t_dn.start()
            o = grouped_matmul_fp8(yq, ys, dnq, dns, gs, **f8s) if fp8 else grouped_matmul_vjp(y, down, gs)
            if timed:
                t_dn.stop()
            sh_out = None
            if shared is not None and not fold:
                from mintext_amd.moe import shared_expert_forward

                sh_out = shared_expert_forward(x, shared[0], shared[1])
            if timed:
                t_comb.start()
            # combine; a separate shared expert's output is added in the same pass
            out = unroute(o, si, w, Kc) if sh_out is None else unroute_add(o, si, w, Kc, sh_out)
            if timed:
                t_comb.stop()
            return out

    if bwd:
        with torch.no_grad():
            idx, w = route_topk(logits, K)
            st, si, gs = route(x, idx, E)
            h = grouped_matmul_vjp(st, gate_up, gs)
            y = grouped_matmul_swiglu(st, gate_up, gs)
        gy = torch.randn(M, D, device=dev, generator=g).to(cdt)
        gh = torch.randn(M, 2 * I, device=dev, generator=g).to(cdt)
        flops_fwd = 2 * (2.0 * M * D * 2 * I + 2.0 * M * I * D)
        t_dl, t_tg = t_gu, t_dn

        def step(timed):  # noqa: F811
            with torch.no_grad():
                if timed:
                    t_dl.start()
                a = _gmm_dlhs(gy, down, gs)      # d inter  [M, I]
                b = _gmm_dlhs(gh, gate_up, gs)   # d x      [M, D]
                if timed:
                    t_dl.stop()
                    t_tg.start()
                c = tgmm(y, gy, gs)              # d down   [E, I, D]
                d = tgmm(st, gh, gs)             # d gate_up [E, D, 2I]
                if timed:
                    t_tg.stop()
                return a, b, c, d

    if cfg_name == "qwen3_bwd_fp8":
        # operands quantised once outside the timed region, as a training step quantises each
        # operand once and may reuse it: upstream gradients in 1x128 rows for the dlhs, both tgmm
        # operands in expert-aligned 128-row chunks; weights prepacked in their own layout
        from mintext_amd.kernels.fp8 import (grouped_matmul_fp8_dlhs, quantize_fp8_grouped_t, quantize_fp8_rows,
                                             quantize_fp8_weights_t, tgmm_fp8)

        bf8 = dict(scales=fp8_scales)  # "amax" or "pow2" in every quantisation and GEMM
        with torch.no_grad():
            dnq, dns = quantize_fp8_weights_t(down, **bf8)
            guq, gus = quantize_fp8_weights_t(gate_up, **bf8)
            gyq, gys = quantize_fp8_rows(gy, **bf8)
            ghq, ghs = quantize_fp8_rows(gh, **bf8)
            yt = quantize_fp8_grouped_t(y, gs, **bf8)
            gyt = quantize_fp8_grouped_t(gy, gs, blocks=True, **bf8)
            stt = quantize_fp8_grouped_t(st, gs, **bf8)
            ght = quantize_fp8_grouped_t(gh, gs, blocks=True, **bf8)

        def step(timed):  # noqa: F811
            with torch.no_grad():
                if timed:
                    t_dl.start()
                a = grouped_matmul_fp8_dlhs(gyq, gys, dnq, dns, gs, **bf8)   # d inter [M, I]
                b = grouped_matmul_fp8_dlhs(ghq, ghs, guq, gus, gs, **bf8)   # d x     [M, D]
                if timed:
                    t_dl.stop()
                    t_tg.start()
                c = tgmm_fp8(*yt, *gyt, gs, M, **bf8)                        # d down    [E, I, D]
                d = tgmm_fp8(*stt, *ght, gs, M, **bf8)                       # d gate_up [E, D, 2I]
                if timed:
                    t_tg.stop()
                return a, b, c, d

    for _ in range(warmup):
        step(False)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        step(True)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / steps
    graph_ms = None
    if use_graph:
        # the same step captured once in a HIP graph and replayed: no per-kernel host launches
        from mintext_amd.moe import CapturedLayer

        cap = CapturedLayer(lambda: step(False))
        for _ in range(warmup):
            cap.replay()
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            cap.replay()
        end.record()
        torch.cuda.synchronize()
        graph_ms = start.elapsed_time(end) / steps

    gs_host = None
    with torch.no_grad():
        idx, w = route_topk(logits, K, **rkw)
        gs_host = torch.bincount(idx.reshape(-1).long(), minlength=E).cpu().numpy()

    gu_ms, dn_ms = t_gu.mean_ms(), t_dn.mean_ms()
    peak = PEAK_FP8_TFLOPS if fp8 else PEAK_BF16_TFLOPS
    if bwd:
        kern_flops = 2.0 * M * D * I + 2.0 * M * 2 * I * D  # both dlhs GEMMs
        achieved = kern_flops / (gu_ms * 1e-3) / 1e12
        dominant = "gmm_dlhs (both expert GEMMs)"
    else:
        kern_flops = 2.0 * Mg * D * 2 * I
        achieved = kern_flops / (gu_ms * 1e-3) / 1e12
        dominant = (("gmm_fp8_swiglu_p2 (gate_up + SwiGLU + pow2 requant)" if fp8_scales == "pow2"
                     else "gmm_fp8_swiglu (gate_up + SwiGLU + requant)") if fp8 else "gmm_swiglu (gate_up + fused SwiGLU)")
    tname = cfg_name + ("_pow2" if fp8 and fp8_scales == "pow2" and not bwd else "")
    traffic, tkern = _traffic(tname)
    tsrc = {"traffic_source": f"profiles/traffic_{tname}.json (rocprofv3 FETCH_SIZE/WRITE_SIZE of {tkern}, "
                              "scaled by a plain copy's counters)"} if traffic is not None else {}
    if cfg_name == "deepseek":
        # C3 streams its routed weights once per layer at ~128 rows per expert (arithmetic intensity
        # ~128 FLOP/B < the bf16 ridge of ~315): HBM-bound.  Algorithmic bytes of the gate_up launch:
        # the routed gate_up weights, the token rows (read once each) and the [M, I] bf16 output.
        alg_b = Eg * D * 2 * I * 2 + T * D * 2 + Mg * I * 2
        gbs = alg_b / (gu_ms * 1e-3) / 1e9
        roofline = {"kernel": dominant, "bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic, **tsrc,
                    "bytes_per_launch": alg_b, "mfma": {"achieved": round(achieved, 1), "peak": peak,
                                                        "unit": "TFLOP/s", "frac": round(achieved / peak, 4)}}
    else:
        roofline = {"kernel": dominant, "bound": "mfma", "achieved": round(achieved, 1), "peak": peak,
                    "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": traffic, **tsrc}
    tokens_per_s = T / (ms * 1e-3)
    gemm_ms = gu_ms + dn_ms
    # dispatch: token rows read once (bf16; fp8 runs quantise them in the same pass), sorted rows
    # written (fp8 codes + 1x128 f32 scales for fp8), indices; with the gather in the gate_up
    # GEMM only the indices (permutation + inverse written), plus for fp8 the token-order
    # quantisation (bf16 rows read, codes + scales written).  combine: expert rows, weights,
    # permutation, f32 output (+ the bf16 shared-expert output when it is added in the pass)
    xb = 4 if cfg["dtype"] == "f32" else 2  # bytes per element of the token rows and expert outputs
    if gather:
        disp_b = T * Kc * 4 + 2 * Mg * 4 + Eg * 4 + (T * D * 2 + T * D + T * (D // 128) * 4 if fp8 else 0)
    else:
        disp_b = T * D * xb + Mg * D * (1 if fp8 else xb) + T * Kc * 4 + Mg * 4 + Eg * 4
        if fp8:
            disp_b += Mg * (D // 128) * 4
    comb_b = Mg * D * xb + T * Kc * 4 + Mg * 4 + T * D * 4 + (T * D * xb if shared is not None and not fold else 0)
    res = {
        "metric": "MoE layer fwd tokens/s + grouped-GEMM TFLOP/s (% of peak), 1x MI355X",
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"bf16": "bf16", "f32": "f32", "fp8": "fp8e4m3"}[cfg["dtype"]],
        "data": "synthetic (seeded N(0,1) activations, N(0,%g) weights, random-init experts)" % cfg["wstd"],
        "config": {"workload": f"{cfg_name} MoE layer forward" if not bwd else
                   f"qwen3 grouped-GEMM backward (dlhs+tgmm){', fp8 operands' if fp8 else ''}, Zipf(1.2) skew",
                   "T": T, "d_model": D, "experts": E, "top_k": K, "d_ff": I, "routing": cfg["scoring"],
                   "parallelism": "single GPU",
                   **({"shared_expert": shared_mode if fold else "separate"} if shared is not None else {}),
                   **({"fp8_scales": ("amax/448" if fp8_scales == "amax" else "power of two (MFMA E8M0)")}
                      if fp8 else {})},
        "gemm": {"tflops": round(flops_fwd / (gemm_ms * 1e-3) / 1e12, 1),
                 "frac_of_peak": round((flops_fwd / (gemm_ms * 1e-3) / 1e12) / peak, 4),
                 "gate_up_ms": round(gu_ms, 4), "down_ms": round(dn_ms, 4)},
        "dispatch_combine": {"rows_gathered_in_gate_up": gather,
                             **({"dispatch_note": "route computes the permutation only (index bytes); the token "
                                                  "rows are read by the gate_up GEMM through it"} if gather else {}),
                             "dispatch_ms": round(t_disp.mean_ms(), 4), "combine_ms": round(t_comb.mean_ms(), 4),
                             "dispatch_GBs": round(disp_b / (t_disp.mean_ms() * 1e-3) / 1e9, 1) if t_disp.pairs else None,
                             "combine_GBs": round(comb_b / (t_comb.mean_ms() * 1e-3) / 1e9, 1) if t_comb.pairs else None},
        "roofline": roofline,
        "load": {"min": int(gs_host.min()), "max": int(gs_host.max()), "mean": float(gs_host.mean()),
                 "empty": int((gs_host == 0).sum())},
        "wall_s": round(wall, 3),
    }
    if graph_ms is not None:
        res["hip_graph"] = {"ms_per_step": round(graph_ms, 4), "tokens_per_s": round(T / (graph_ms * 1e-3), 1)}
    if cpu_baseline and not bwd:
        # fp8 has no reference counterpart: the CPU leg runs the reference's bf16 layer on the same tokens
        hdt = torch.float32 if cfg["dtype"] == "f32" else torch.bfloat16
        h = lambda t: t.to(hdt).cpu()
        sh = None if shared is None else (h(shared[0][0]), h(shared[1][0]))
        res["cpu_baseline"] = _cpu_baseline_layer(h(x), logits.float().cpu(), h(gate_up[:E]), h(down[:E]), cfg,
                                                  shared=sh)
    return res


def gemm_power_study(steps=10, warmup=3):
    """C2 gate_up grouped GEMM (fused SwiGLU) and a hipBLASLt dense GEMM of the same FLOPs
    (torch.matmul [16384,4096] x [4096,28672]), each on N(0,1)/N(0,0.02) data and on all-zero
    data: with zeros the MFMA datapath barely toggles, so the clock is not power-limited and
    the difference isolates the data-dependent clock drop from the kernels' issue efficiency.
    Not a benchmark of the path: one JSON line of timings for the DESIGN analysis."""
    import torch

    from mintext_amd import _lib
    from mintext_amd.kernels import grouped_matmul_swiglu

    _lib.lib()
    dev = torch.device("cuda:0")
    M, D, I, E = 16384, 4096, 14336, 8
    gs = torch.full((E,), M // E, dtype=torch.int32, device=dev)
    x = torch.empty(M, D, dtype=torch.bfloat16, device=dev)
    w = torch.empty(E, D, 2 * I, dtype=torch.bfloat16, device=dev)
    flop = 2.0 * M * D * 2 * I

    def t_ms(fn):
        for _ in range(warmup):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        b.synchronize()
        return a.elapsed_time(b) / steps

    out = {"study": "gemm-power", "shape": "C2 gate_up [16384,4096] x [8,4096,28672]", "steps": steps}
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    for data in ("normal", "zeros", "normal"):
        if data == "normal":
            x.copy_(torch.randn(M, D, device=dev, generator=g))
            w.copy_(torch.randn(E, D, 2 * I, device=dev, generator=g) * 0.02)
        else:
            x.zero_()
            w.zero_()
        ours = t_ms(lambda: grouped_matmul_swiglu(x, w, gs))
        dense = t_ms(lambda: torch.matmul(x, w[0]))
        out.setdefault(data, []).append({"gmm_swiglu_ms": round(ours, 4), "gmm_swiglu_tflops": round(flop / ours / 1e9, 1),
                                         "hipblaslt_dense_ms": round(dense, 4),
                                         "hipblaslt_dense_tflops": round(flop / dense / 1e9, 1)})
    print(json.dumps(out))
    return 0


def fp8_vendor_study(steps=10, warmup=3):
    """C4 fp8 grouped GEMMs (blockwise 1x128 / 128x128 scales; gate_up with the fused SwiGLU +
    re-quantisation) beside hipBLASLt's dense fp8 GEMMs of the same shapes through
    torch._scaled_mm with per-tensor and with rowwise scales (hipBLASLt has no blockwise fp8),
    and hipBLASLt's bf16 GEMM.  Not a benchmark of the path: one JSON line of timings that
    places the blockwise kernels against the vendor library on the same box and data."""
    import torch

    from mintext_amd import _lib
    from mintext_amd.kernels.fp8 import (grouped_matmul_fp8, grouped_matmul_fp8_swiglu, quantize_fp8_rows,
                                         quantize_fp8_weights)

    _lib.lib()
    dev = torch.device("cuda:0")
    T, D, E, K, I = 16384, 2048, 128, 8, 768
    M = T * K
    gs = torch.full((E,), M // E, dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(2)

    def t_ms(fn):
        for _ in range(warmup):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        b.synchronize()
        return a.elapsed_time(b) / steps

    out = {"study": "fp8-vendor", "shapes": "C4: gate_up [131072,2048]x[2048,1536], down [131072,768]x[768,2048]",
           "steps": steps, "loads": "uniform (1024 rows per expert)"}
    x = torch.randn(M, D, device=dev, generator=g).bfloat16()
    h = torch.randn(M, I, device=dev, generator=g).bfloat16()
    wgu = (torch.randn(E, D, 2 * I, device=dev, generator=g) * 0.02).bfloat16()
    wdn = (torch.randn(E, I, D, device=dev, generator=g) * 0.02).bfloat16()
    xq, xs = quantize_fp8_rows(x)
    hq, hs = quantize_fp8_rows(h)
    guq, gus = quantize_fp8_weights(wgu)
    dnq, dns = quantize_fp8_weights(wdn)
    one = torch.ones((), device=dev)
    for name, (aq, a_s, wq, w_s, kin, kout, ours) in {
        "gate_up": (xq, xs, guq, gus, D, 2 * I, lambda: grouped_matmul_fp8_swiglu(xq, xs, guq, gus, gs)),
        "down": (hq, hs, dnq, dns, I, D, lambda: grouped_matmul_fp8(hq, hs, dnq, dns, gs)),
    }.items():
        flop = 2.0 * M * kin * kout
        b = wq[0]  # [kout, kin] e4m3, k-contiguous: b.t() is the column-major right operand
        row_a = torch.rand(M, 1, device=dev) + 0.5
        row_b = torch.rand(1, kout, device=dev) + 0.5
        ab = (x if name == "gate_up" else h)
        bb = (wgu[0] if name == "gate_up" else wdn[0]).contiguous()
        res = {"blockwise_grouped_ms": t_ms(ours),
               "hipblaslt_fp8_pertensor_ms": t_ms(lambda: torch._scaled_mm(aq, b.t(), scale_a=one, scale_b=one,
                                                                           out_dtype=torch.bfloat16)),
               "hipblaslt_fp8_rowwise_ms": t_ms(lambda: torch._scaled_mm(aq, b.t(), scale_a=row_a, scale_b=row_b,
                                                                         out_dtype=torch.bfloat16)),
               "hipblaslt_bf16_ms": t_ms(lambda: torch.matmul(ab, bb))}
        out[name] = {k: round(v, 4) for k, v in res.items()}
        out[name].update({k.replace("_ms", "_tflops"): round(flop / v / 1e9, 1) for k, v in res.items()})
    print(json.dumps(out))
    return 0


def grouped_vendor_study(steps=10, warmup=3):
    """The bf16 grouped GEMMs beside the vendor's grouped GEMM on the same ragged problems:
    torch._grouped_mm (on this ROCm build a loop of one hipBLASLt GEMM per group) with the
    weights in the reference's [E, K, N] layout and k-contiguous ([E, N, K] storage), on the C2
    and C3 expert shapes with seeded near-uniform loads.  Not a benchmark of the path: one JSON
    line of timings (and whether the vendor's output equals this library's bit for bit)."""
    import numpy as np
    import torch

    from mintext_amd import _lib
    from mintext_amd.kernels import grouped_matmul
    from mintext_amd.kernels.grouped_matmul import grouped_matmul_swiglu

    _lib.lib()
    dev = torch.device("cuda:0")

    def t_ms(fn):
        for _ in range(warmup):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        b.synchronize()
        return a.elapsed_time(b) / steps

    out = {"study": "grouped-vendor", "steps": steps, "vendor": "torch._grouped_mm (hipBLASLt per group)"}
    rng = np.random.default_rng(1)
    shapes = {  # name: (rows, K, N, experts)
        "c2_gate_up": (16384, 4096, 2 * 14336, 8), "c2_down": (16384, 14336, 4096, 8),
        "c3_gate_up": (32768, 7168, 2 * 2048, 256), "c3_down": (32768, 2048, 7168, 256)}
    loads = {}
    for name, (M, Kin, N, E) in shapes.items():
        if E not in loads:
            loads[E] = torch.from_numpy(rng.multinomial(M, [1.0 / E] * E).astype(np.int32)).to(dev)
        gs = loads[E]
        offs = torch.cumsum(gs, 0).to(torch.int32)
        g = torch.Generator(device=dev)
        g.manual_seed(3)
        x = torch.randn(M, Kin, device=dev, generator=g).bfloat16()
        w = (torch.randn(E, Kin, N, device=dev, generator=g) * 0.02).bfloat16()
        w_kc = w.transpose(1, 2).contiguous().transpose(1, 2)  # same values, k-contiguous storage
        ours = grouped_matmul(x, w, gs)
        res = {"ours_ms": t_ms(lambda: grouped_matmul(x, w, gs))}
        if name.endswith("gate_up"):
            res["ours_with_swiglu_ms"] = t_ms(lambda: grouped_matmul_swiglu(x, w, gs))
        for tag, wv in (("kn", w), ("kcontig", w_kc)):
            v = torch._grouped_mm(x, wv, offs=offs, out_dtype=torch.bfloat16)
            res[f"vendor_{tag}_ms"] = t_ms(lambda: torch._grouped_mm(x, wv, offs=offs, out_dtype=torch.bfloat16))
            res[f"vendor_{tag}_bits_equal"] = bool(torch.equal(v, ours))
        flop = 2.0 * M * Kin * N
        entry = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in res.items()}
        entry.update({k.replace("_ms", "_tflops"): round(flop / v / 1e9, 1) for k, v in res.items() if k.endswith("_ms")})
        entry["loads"] = [int(gs.min()), int(gs.max())]
        out[name] = entry
        del x, w, w_kc, ours
    print(json.dumps(out))
    return 0


def copy_study(steps=20, warmup=3):
    """The practical HBM ceiling for read+write streams on this box: device-to-device copies of
    64 MiB to 1 GiB (bytes read + bytes written per second) by torch's copy_ and by the library's
    streaming copy (mtx_stream_copy: 16-byte loads and stores, 2-16 loads in flight per lane,
    plain or non-temporal, a grid-stride loop over 2-8 workgroups per CU), every variant timed
    and the best one reported per size.  Sizes up to about 128 MiB partly stay in the 256 MB MALL
    between repetitions; the larger ones are HBM.  The dispatch and combine kernels move
    comparable volumes (C2: 201.5 / 268.6 MB)."""
    import torch

    from mintext_amd import _lib as L

    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    variants = [(nt, u, k) for nt in (0, 1) for u in (4, 8, 16) for k in (2, 4, 8)]
    out = {"study": "copy", "unit": "GB/s (read + write)", "cus": ncu, "sizes_MiB": {}}
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        s.record()
        for _ in range(steps):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / steps * 1e-3

    for mib in (64, 128, 256, 512, 1024):
        nbytes = mib << 20
        src = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        src.fill_(1)
        dst = torch.empty_like(src)
        stream = L.stream(src.device)
        row = {"torch_copy_GBs": round(2 * nbytes / timed(lambda: dst.copy_(src)) / 1e9, 1)}
        best = None
        for nt, u, k in variants:
            var = nt | (u << 4 if u < 16 else 15 << 4)
            t = timed(lambda: L.call("mtx_stream_copy", L.ptr(src), L.ptr(dst), nbytes, var, k * ncu, stream))
            gbs = 2 * nbytes / t / 1e9
            if best is None or gbs > best[0]:
                best = (gbs, {"nontemporal": bool(nt), "loads_in_flight": u, "wg_per_cu": k})
        assert torch.equal(dst, src), "streaming copy mismatch"
        row["stream_copy_GBs"] = round(best[0], 1)
        row["stream_copy_best"] = best[1]
        out["sizes_MiB"][mib] = row
        del src, dst
    print(json.dumps(out))
    return 0


def gate_study(steps=20, warmup=5):
    """The router gate GEMM + top-k on the C2, C3 and C4 shapes: hipBLASLt's dense gate GEMM
    (torch.matmul, [T,D] x [D,E]) followed by route_topk, against the fused gate_route_topk (the
    gate weight already in the nn.Linear layout, a load-time transform).  One JSON line of
    timings; not part of the layer bench, whose path starts from the logits."""
    import torch

    from mintext_amd import _lib
    from mintext_amd.kernels import route_topk
    from mintext_amd.kernels.router import gate_route_topk, gate_weight_linear_layout

    _lib.lib()
    dev = torch.device("cuda:0")

    def t_ms(fn):
        for _ in range(warmup):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        b.synchronize()
        return a.elapsed_time(b) / steps

    out = {"study": "gate", "steps": steps}
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    for name in ("mixtral", "deepseek", "qwen3_fp8"):
        cfg = CONFIGS[name]
        T, D, E, K = cfg["T"], cfg["D"], cfg["E"], cfg["K"]
        x = torch.randn(T, D, device=dev, generator=g).bfloat16()
        wg = (torch.randn(D, E, device=dev, generator=g) * cfg["wstd"]).bfloat16()
        wt = gate_weight_linear_layout(wg)
        rkw = dict(scoring=cfg["scoring"], n_group=cfg.get("n_group", 1), topk_group=cfg.get("topk_group", 1),
                   routed_scaling_factor=cfg.get("scale", 1.0))
        unfused = t_ms(lambda: route_topk(torch.matmul(x, wg), K, **rkw))
        gemm_only = t_ms(lambda: torch.matmul(x, wg))
        fused = t_ms(lambda: gate_route_topk(x, wt, K, **rkw))
        xbytes = T * D * 2
        out[name] = {"T": T, "D": D, "E": E, "K": K, "hipblaslt_gate_plus_topk_us": round(unfused * 1e3, 1),
                     "hipblaslt_gate_us": round(gemm_only * 1e3, 1), "fused_us": round(fused * 1e3, 1),
                     "fused_x_read_GBs": round(xbytes / (fused * 1e-3) / 1e9, 1)}
    print(json.dumps(out))
    return 0


KERNEL_STUDY_CONFIGS = {  # benchmarks/benchmark_moe_kernels.py:21-28 (the reference's own kernel benchmark)
    "tiny": {"E": 4, "D": 64, "I": 128, "K": 2, "tokens": 128},
    "small": {"E": 4, "D": 128, "I": 256, "K": 2, "tokens": 256},
    "medium": {"E": 8, "D": 256, "I": 512, "K": 2, "tokens": 1024},
    "dsv3_small": {"E": 64, "D": 512, "I": 1024, "K": 8, "tokens": 2048},
    "dsv3": {"E": 256, "D": 7168, "I": 2048, "K": 8, "tokens": 4096},
    "llama_moe": {"E": 8, "D": 4096, "I": 14336, "K": 2, "tokens": 4096},
}


def kernels_study(steps=20, warmup=5, configs=None):
    """The reference's kernel benchmark (benchmarks/benchmark_moe_kernels.py) on this build: the
    gate_up grouped GEMM [M=tokens*K, D] x [E, D, N=2I] with N(0,1) bf16 operands and uniform groups
    (:31-39), forward, backward (d/dx and d/dw of out.sum(), :68-96) and forward + backward (:99-125),
    for grouped_matmul / grouped_matmul_vjp and, where D and N allow, the blockwise-fp8 VJP.  Times
    are HIP-event means over ``steps`` calls; TFLOP/s counts the GEMMs actually run (forward 2MDN,
    backward 4MDN: dlhs + tgmm, forward + backward 6MDN), not the reference's 3x / 4x approximations."""
    import torch
    from mintext_amd.kernels import grouped_matmul, grouped_matmul_vjp
    from mintext_amd.kernels.fp8 import grouped_matmul_fp8_vjp

    dev = torch.device("cuda:0")

    def t_ms(fn):
        for _ in range(warmup):
            fn()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        b.synchronize()
        return a.elapsed_time(b) / steps

    out = {"study": "kernels", "reference": "benchmarks/benchmark_moe_kernels.py", "steps": steps, "rows": []}
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    for name in configs or list(KERNEL_STUDY_CONFIGS):
        c = KERNEL_STUDY_CONFIGS[name]
        E, D, N, M = c["E"], c["D"], 2 * c["I"], c["tokens"] * c["K"]
        x = torch.randn(M, D, device=dev, generator=g).bfloat16()
        w = torch.randn(E, D, N, device=dev, generator=g).bfloat16()
        gs = torch.tensor([M // E + (1 if i < M % E else 0) for i in range(E)], dtype=torch.int32, device=dev)
        fl = 2.0 * M * D * N
        backends = {"grouped_matmul": grouped_matmul, "grouped_matmul_vjp": grouped_matmul_vjp}
        if D % 256 == 0 and N % 256 == 0:
            backends["fp8_vjp"] = grouped_matmul_fp8_vjp
        row = {"config": name, "M": M, "D": D, "N": N, "E": E}
        for bname, fn in backends.items():
            xr = x.clone().requires_grad_(True)
            wr = w.clone().requires_grad_(True)

            def fwd():
                with torch.no_grad():
                    fn(x, w, gs)

            def bwd():
                o = fn(xr, wr, gs)
                dx, dw = torch.autograd.grad(o.sum(), (xr, wr))
                return dx, dw

            f_ms = t_ms(fwd)
            fb_ms = t_ms(bwd)
            # backward alone: the forward of the same call subtracted
            row[bname] = {"forward_ms": round(f_ms, 4), "forward_TFLOPs": round(fl / f_ms / 1e9, 1),
                          "backward_ms": round(fb_ms - f_ms, 4),
                          "backward_TFLOPs": round(2 * fl / max(fb_ms - f_ms, 1e-6) / 1e9, 1),
                          "fwd_bwd_ms": round(fb_ms, 4), "fwd_bwd_TFLOPs": round(3 * fl / fb_ms / 1e9, 1)}
        out["rows"].append(row)
        del x, w
    print(json.dumps(out))
    return 0


DISPATCH_BWD_CONFIGS = {  # layer shapes of the bench configs: tokens N, top-k K, d_model D, d_ff I
    "mixtral": {"N": 8192, "K": 2, "D": 4096, "I": 14336},
    "deepseek": {"N": 4096, "K": 8, "D": 7168, "I": 2048},
    "qwen3": {"N": 16384, "K": 8, "D": 2048, "I": 768},
}


def dispatch_bwd_study(steps=20, warmup=5):
    """The HBM-bound backward kernels of the layer, as its autograd path calls them: the combine's
    VJP (mtx_unroute_bwd: f32 dout, bf16 expert outputs, f32 router weights -> bf16 d_sorted and
    f32 d_weights; moe_dispatch.py:102-111), the route's VJP (mtx_unroute with unit weights, bf16;
    moe_dispatch.py:33-38,67), and SwiGLU with its VJP (mtx_swiglu / mtx_swiglu_bwd, bf16;
    moe.py:195-196).  Bytes are algorithmic (every input read once, every output written once);
    times are HIP-event means over ``steps`` calls on the current stream, after ``warmup`` calls.
    Before a shape is timed its kernels run in turn for at least 50 ms: on these boxes the first
    few milliseconds after a large buffer is first touched run up to 1.5x slower for any kernel
    that streams it (SwiGLU on the C2 shape: 220 us, then 350, then 280-240 us per call)."""
    import torch
    from mintext_amd import _lib as L

    dev = torch.device("cuda:0")
    st = L.stream(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(0)

    def t_ms(fn):
        for _ in range(warmup):
            fn()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        b.synchronize()
        return a.elapsed_time(b) / steps

    out = {"study": "dispatch-bwd", "steps": steps, "peak_GBs": 8000, "rows": []}
    for name, c in DISPATCH_BWD_CONFIGS.items():
        N, K, D, I = c["N"], c["K"], c["D"], c["I"]
        M = N * K
        inv = torch.randperm(M, device=dev, generator=g).int()
        w = torch.rand(N, K, device=dev, generator=g)
        dout = torch.randn(N, D, device=dev, generator=g)
        Y = torch.randn(M, D, device=dev, generator=g).bfloat16()
        dY = torch.empty_like(Y)
        dw = torch.empty_like(w)
        dx = torch.empty(N, D, dtype=torch.bfloat16, device=dev)
        row = {"config": name, "N": N, "K": K, "D": D, "I": I}

        def ub():
            L.call("mtx_unroute_bwd", L.ptr(dout), L.MTX_F32, L.ptr(Y), L.MTX_BF16, L.ptr(inv), L.ptr(w), L.MTX_F32,
                   N, K, D, L.ptr(dY), L.ptr(dw), st)

        def rv():
            L.call("mtx_unroute", L.ptr(Y), L.MTX_BF16, L.ptr(inv), None, L.MTX_F32, N, K, D, L.ptr(dx), L.MTX_BF16,
                   st)

        kernels = {"unroute_bwd": (ub, N * D * 4 + 2 * M * D * 2 + M * 4 * 3),
                   "route_vjp": (rv, M * D * 2 + N * D * 2 + M * 4)}
        del_after = []
        h = torch.randn(M, 2 * I, device=dev, generator=g).bfloat16()
        dy = torch.randn(M, I, device=dev, generator=g).bfloat16()
        y = torch.empty(M, I, dtype=torch.bfloat16, device=dev)
        dh = torch.empty_like(h)
        del_after += [h, dy, y, dh]

        def sw():
            L.call("mtx_swiglu", L.ptr(h), L.MTX_BF16, M, I, L.ptr(y), st)

        def swb():
            L.call("mtx_swiglu_bwd", L.ptr(h), L.ptr(dy), L.MTX_BF16, M, I, L.ptr(dh), st)

        kernels["swiglu"] = (sw, M * I * 2 * 3)
        kernels["swiglu_bwd"] = (swb, M * I * 2 * 5)
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < 0.05:
            for fn, _ in kernels.values():
                fn()
            torch.cuda.synchronize()
        for kname, (fn, nbytes) in kernels.items():
            ms = t_ms(fn)
            row[kname] = {"us": round(ms * 1e3, 1), "MB": round(nbytes / 1e6, 1),
                          "GBs": round(nbytes / ms / 1e6, 1), "frac": round(nbytes / ms / 1e6 / 8000, 3)}
        out["rows"].append(row)
        del inv, w, dout, Y, dY, dw, dx, del_after
        torch.cuda.empty_cache()
    print(json.dumps(out))
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="mixtral", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--shared", default="separate", choices=["folded", "separate"],
                    help="deepseek: shared expert run as its own one-group GEMMs (default) or folded into the routed GEMMs")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 3 plain 256 MiB device copies (scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--fp8-scales", default="amax", choices=["amax", "pow2"],
                    help="fp8 configs: block scales amax/448 (default) or powers of two applied by the MFMA")
    ap.add_argument("--no-gather", action="store_true",
                    help="materialise the sorted tokens in the dispatch (route) instead of gathering the token "
                         "rows inside the gate_up GEMM")
    ap.add_argument("--graph", action="store_true",
                    help="also time the step captured in a HIP graph and replayed (reported as hip_graph)")
    ap.add_argument("--study", choices=["gemm-power", "fp8-vendor", "grouped-vendor", "gate", "copy", "kernels",
                                        "dispatch-bwd"],
                    default=None,
                    help="gemm-power: GEMM timings on normal vs all-zero data (clock / issue-efficiency study); "
                         "fp8-vendor: C4 blockwise fp8 GEMMs beside hipBLASLt's per-tensor / rowwise fp8 GEMMs; "
                         "grouped-vendor: C2 / C3 bf16 grouped GEMMs beside torch._grouped_mm (hipBLASLt per group); "
                         "gate: router gate GEMM + top-k, hipBLASLt + route_topk vs the fused kernel; "
                         "copy: device-to-device copy bandwidth (the practical read+write HBM ceiling); "
                         "kernels: the reference's benchmarks/benchmark_moe_kernels.py (gate_up grouped GEMM "
                         "forward / backward / fwd+bwd per config); "
                         "dispatch-bwd: the layer's HBM-bound backward kernels (combine and route VJPs, SwiGLU "
                         "and its VJP) at the bench shapes")
    ap.add_argument("--configs", nargs="+", default=None, choices=sorted(KERNEL_STUDY_CONFIGS),
                    help="--study kernels: configs to run (default: all)")
    a = ap.parse_args(argv)
    if a.study == "gemm-power":
        return gemm_power_study(a.steps if a.steps != 20 else 10, a.warmup)
    if a.study == "fp8-vendor":
        return fp8_vendor_study(a.steps if a.steps != 20 else 10, a.warmup)
    if a.study == "grouped-vendor":
        return grouped_vendor_study(a.steps if a.steps != 20 else 10, a.warmup)
    if a.study == "gate":
        return gate_study(a.steps, a.warmup)
    if a.study == "copy":
        return copy_study(a.steps, a.warmup)
    if a.study == "kernels":
        return kernels_study(a.steps, a.warmup, a.configs)
    if a.study == "dispatch-bwd":
        return dispatch_bwd_study(a.steps, a.warmup)
    if a.copy_calibration:
        import torch

        n = 256 << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda")
        src.fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "dispatches": 3}))
        return 0
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (no expert parallelism or "
              "collectives); run with --gpus 1", file=sys.stderr)
        return 2
    res = run(a.config, a.steps, a.warmup, cpu_baseline=not a.no_cpu_baseline, shared_mode=a.shared,
              use_graph=a.graph, gather=not a.no_gather, fp8_scales=a.fp8_scales)
    print(json.dumps(res))
    return 0


if __name__ == "__main__":
    sys.exit(main())

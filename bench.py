"""Benchmark of the HIP GMM EM hot path on one MI355X.

Workload (the headline metric): spherical GMM,
bf16 inputs with fp32 accumulation, N = 4,194,304, D = 128, K = 1024, one
batch.  Synthetic data, seed 1: centres ~ N(0, 4I), per-component std
~ U[0.5, 1.5], Dirichlet(1) weights, labels ~ multinomial(weights),
x = centre + std * N(0, I) rounded to bf16.  Initial means are K distinct
random rows, variances the global spherical variance, weights 1/K.

A "step" is one soft-EM iteration over all N rows (gmmxx_hip_em_step: prelude,
E-step log-normaliser, responsibilities, M-step statistics, finalize), with x
resident in HBM.  ``value`` is EM iterations per second.

Also reported:
  * roofline: the dominant kernel's algorithmic MFMA rate, from its average
    launch time measured with HIP events on its own stream over the timed
    region (each phase of the iteration is launched between events);
  * em_iteration: the whole iteration's algorithmic rate against the bf16
    dense MFMA peak (the BASELINE target is >= 60 %);
  * cpu_baseline: the CPU oracle (a restatement of the reference torch
    fallback) timed on the host on a bounded row sample, scaled to full N.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

N, D, K = 4_194_304, 128, 1024
SEED = 1
PEAK_BF16_TFLOPS = 2516.6            # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
METRIC = "EM iter/s + % bf16 MFMA peak, spherical bf16 N=4M D=128 K=1024"


def algorithmic_flops(n, d, k):
    """Minimal contractions per EM iteration: E-step x·μᵀ (2NKD) and M-step
    rᵀ·[x | ‖x‖² | 1] (2NK(D+2))."""
    return {"lse_tile": 2.0 * n * k * d, "stats_tile": 2.0 * n * k * (d + 2),
            "iteration": 2.0 * n * k * (2 * d + 2)}


def make_data(device, n=N, d=D, k=K, seed=SEED):
    g = torch.Generator(device=device).manual_seed(seed)
    centers = 2.0 * torch.randn((k, d), generator=g, device=device)
    sigma = 0.5 + torch.rand((k,), generator=g, device=device)
    w = -torch.log(torch.rand((k,), generator=g, device=device))
    w = w / w.sum()
    labels = torch.multinomial(w, n, replacement=True, generator=g)
    x = torch.empty((1, n, d), dtype=torch.bfloat16, device=device)
    chunk = 1 << 20
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        lab = labels[s:e]
        noise = torch.randn((e - s, d), generator=g, device=device)
        x[0, s:e] = (centers[lab] + sigma[lab, None] * noise).to(torch.bfloat16)
    idx = torch.randperm(n, generator=g, device=device)[:k]
    means0 = x[0, idx].to(torch.float32).unsqueeze(0).contiguous()
    # Global spherical variance (torch_fallback.py:1348-1363), fixed by the harness.
    s1 = torch.zeros(d, dtype=torch.float64, device=device)
    s2 = torch.zeros((), dtype=torch.float64, device=device)
    for s in range(0, n, chunk):
        xf = x[0, s:s + chunk].to(torch.float64)
        s1 += xf.sum(0)
        s2 += xf.square().sum()
    mean = s1 / n
    gv = float(((s2 / n) - mean.square().sum()).clamp_min(0.0) / d)
    var0 = torch.full((1, k), max(gv, 1e-6), dtype=torch.float32, device=device)
    w0 = torch.full((1, k), 1.0 / k, dtype=torch.float32, device=device)
    return x, means0, var0, w0


def cpu_baseline(x_dev, means0, var0, w0, sample_rows, iters):
    """Oracle EM iterations on the first `sample_rows` rows (fp32 on the
    bf16 values), scaled linearly in N to the full workload."""
    from oracle import torch_ref
    torch.set_num_threads(min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", "64"))))
    xs = x_dev[:, :sample_rows].to(torch.float32).cpu()
    m, v, w = means0.cpu(), var0.cpu(), w0.cpu()
    torch_ref.fit(xs[:, :4096], K, "spherical", max_iters=1, tol=0.0, init_means=m, init_covs=v,
                  init_weights=w, compute_labels=False)  # warm the thread pool
    t0 = time.perf_counter()
    torch_ref.fit(xs, K, "spherical", max_iters=iters, tol=0.0, init_means=m, init_covs=v,
                  init_weights=w, compute_labels=False)
    dt = (time.perf_counter() - t0) / iters
    full_iter_s = dt * (x_dev.shape[1] / sample_rows)
    return {"value": 1.0 / full_iter_s, "unit": "EM iter/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{iters} oracle EM iterations on the first {sample_rows} of {x_dev.shape[1]} rows "
                      f"({dt:.3f} s/iter), scaled linearly in N"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-sample-rows", type=int, default=131072)
    ap.add_argument("--cpu-iters", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the sharding design is described in DESIGN.md); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    from gmmxx_amd import _hip
    _hip.require_hip()
    dev = torch.device("cuda:0")
    print(f"[bench] generating data N={N} D={D} K={K}", file=sys.stderr, flush=True)
    x, means0, var0, w0 = make_data(dev)
    means, var, w = means0.clone(), var0.clone(), w0.clone()
    prob = _hip.problem("spherical", x.dtype, 1, N, D, K)
    ws = _hip.Workspace(prob, dev)
    lb = torch.zeros((max(1, args.steps + args.warmup),), dtype=torch.float32, device=dev)
    phases = _hip.EM_PHASES

    def step(i, events=None):
        for j, ph in enumerate(phases):
            if events is not None:
                events[j].record()
            _hip.em_phase(ph, "spherical", x, means, var, w, lb[i:i + 1], ws)
        if events is not None:
            events[len(phases)].record()

    print(f"[bench] warmup {args.warmup}", file=sys.stderr, flush=True)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(phases) + 1)] for _ in range(args.steps)]
    print(f"[bench] timing {args.steps} EM iterations", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i, evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = 1e3 * wall / args.steps
    phase_ms = {ph: sum(e[j].elapsed_time(e[j + 1]) for e in evs) / args.steps for j, ph in enumerate(phases)}
    flops = algorithmic_flops(N, D, K)
    dominant = max(("lse_tile", "stats_tile"), key=lambda p: phase_ms[p])
    achieved = flops[dominant] / (phase_ms[dominant] * 1e-3) / 1e12
    iter_tflops = flops["iteration"] / (ms_per_step * 1e-3) / 1e12
    lbs = lb[args.warmup:args.warmup + args.steps].tolist()

    result = {
        "metric": METRIC, "value": 1e3 / ms_per_step, "unit": "EM iter/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (BASELINE config 2 recipe, seed 1, generated on device)",
        "config": {"workload": "spherical GMM EM iteration, bf16 x with fp32 accumulation",
                   "B": 1, "N": N, "D": D, "K": K, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": f"em_tile ({dominant})",
                     "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_BF16_TFLOPS, "traffic": None},
        "em_iteration": {"algorithmic_tflop": flops["iteration"] / 1e12, "achieved_tflops": iter_tflops,
                         "frac_of_bf16_peak": iter_tflops / PEAK_BF16_TFLOPS,
                         "phase_ms": phase_ms},
        "lower_bound_last": lbs[-1] if lbs else None,
    }
    if not args.no_cpu_baseline:
        print(f"[bench] cpu baseline on {args.cpu_sample_rows} rows", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(x, means0, var0, w0, args.cpu_sample_rows, args.cpu_iters)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
